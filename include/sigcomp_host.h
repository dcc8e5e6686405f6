/*
 * sigcomp_host.h -- C ABI of the host-side stages either side of the GPU
 * codec: signal split / reassembly (the caller-side token source) and the
 * SIG2 per-chunk framing.  libsigcomp_host.so, plain C++ on the CPU,
 * multithreaded over reads / chunks.  Every function names the reference
 * code it restates (paths relative to the reference's sigcomp/ package).
 *
 * Conventions: all pointers are host pointers, read or written during the
 * call only.  Input reads are given as an array of per-read pointers plus
 * lengths; other per-item data as concatenated arrays plus per-item offsets
 * and lengths.  n_threads <= 0 uses every hardware thread.
 * Return value: SC_OK; SC_ERR_ARG for bad arguments; or an SC_HOST_ERR_*
 * code with *bad set to the index of the first (lowest-numbered) offending
 * item (when `bad` is not NULL); sc_host_last_error() describes the
 * failure.  Items are independent, so a failing item leaves
 * the outputs of other items valid.
 */
#ifndef SIGCOMP_HOST_H
#define SIGCOMP_HOST_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#ifndef SC_OK
#define SC_OK 0
#define SC_ERR_ARG 1
#endif

/* Item failures (the reference's exception for each, as raised by the Python
 * layer, in brackets). */
#define SC_HOST_ERR_FRAME_LENGTH 10  /* truncated uint16 frame length [ValueError] */
#define SC_HOST_ERR_FRAME        11  /* empty, non-multiple-of-4 or truncated frame [ValueError] */
#define SC_HOST_ERR_TRAILING     12  /* bytes after the last frame [ValueError] */
#define SC_HOST_ERR_OVERSIZE     13  /* chunk of more than 65535 bytes [ValueError] */
#define SC_HOST_ERR_COUNTS       14  /* small + large counts != len - 1 [ValueError] */
#define SC_HOST_ERR_POSITION     15  /* large position outside the read [IndexError] */
#define SC_HOST_ERR_EMPTY_READ   16  /* a read of zero samples [IndexError] */

const char *sc_host_last_error(void);

/* Pass 1 of the split.  For each read r (len[r] >= 1 samples at reads[r]):
 * apply the lossy transform when lsb > 0
 * (_lossy_encode(_reduce_lsb(sig, lsb), lsb), main.py:158-167,862-864), then
 * count the small (zigzag delta < 256) and large deltas of _split_signal
 * (main.py:504-521).  Writes sig0[r] (first transformed sample),
 * n_small[r], n_large[r] (n_small + n_large = len - 1).  lsb in [0, 15]. */
int sc_host_split_count(const int16_t *const *reads, const int64_t *len, int64_t n_reads, int32_t lsb,
                        int16_t *sig0, int64_t *n_small, int64_t *n_large, int32_t n_threads, int64_t *bad);

/* Pass 2 of the split: read r's small tokens (uint8, in order) go to
 * small + small_off[r], its large values minus 256 (uint16) to
 * large_adj + large_off[r] and the gap-coded positions (first position,
 * then position differences minus one; uint32) to large_gap + large_off[r].
 * Offsets are the caller's (normally exclusive scans of n_small / n_large). */
int sc_host_split_fill(const int16_t *const *reads, const int64_t *len, int64_t n_reads, int32_t lsb,
                       const int64_t *small_off, const int64_t *large_off, uint8_t *small, uint16_t *large_adj,
                       uint32_t *large_gap, int32_t n_threads, int64_t *bad);

/* Inverse (_reassemble_signal, main.py:524-546, after the Rice decoding of
 * the large values and gaps; then _lossy_decode, main.py:170-171,1164 when
 * lsb > 0): read r (len[r] samples, first sig0[r]) from n_small[r] tokens at
 * small + small_off[r] and n_large[r] large values / gaps at large_off[r];
 * samples to out + out_off[r].  Fails for a read whose counts do not add up
 * to len - 1 or whose positions fall outside the read (the reference raises
 * IndexError / ValueError there).  A length below 1 fails with
 * SC_HOST_ERR_EMPTY_READ before any read is rebuilt (out_off cannot place
 * it); a read's positions are all checked before any of its samples is read
 * or written. */
int sc_host_reassemble(const int16_t *sig0, const int64_t *len, int64_t n_reads, int32_t lsb,
                       const uint8_t *small, const int64_t *small_off, const int64_t *n_small,
                       const uint16_t *large_adj, const uint32_t *large_gap, const int64_t *large_off,
                       const int64_t *n_large, int16_t *out, const int64_t *out_off, int32_t n_threads,
                       int64_t *bad);

/* SIG2 framing of range-coded chunks (ReadFramingMixin.batch_inference_reads,
 * cpu_compression.py:44-52): chunk c = word_cnt[c] little-endian u32 words at
 * words + word_off[c]; its frame (a little-endian uint16 byte length, then the
 * words) goes to out + out_off[c].  A read's payload is the concatenation of
 * its chunks' frames, so out_off is the exclusive scan of 2 + 4*word_cnt.
 * Fails for a chunk of more than 65535 bytes. */
int sc_host_frame(const uint32_t *words, const int64_t *word_off, const int32_t *word_cnt, int64_t n_chunks,
                  uint8_t *out, const int64_t *out_off, int32_t n_threads, int64_t *bad);

/* Parse framed reads (cpu_compression.py:60-84): read r's payload is
 * data[data_off[r] .. data_off[r] + data_len[r]) and holds
 * ceil(tokens[r] / chunk_len) frames, chunk k of it covering
 * min(chunk_len, tokens[r] - k*chunk_len) tokens.  Its chunks are numbered
 * from chunk_begin[r] (the caller's exclusive scan of the frame counts) and
 * their words are copied, in order, to words_out from read_word_off[r] on
 * (data_len[r] / 4 words of room per read always suffice); for each chunk c,
 * word_off[c] (absolute index into words_out), word_cnt[c] and tok_cnt[c] are
 * written.  Fails for a frame of zero bytes or of a byte count that is not a
 * multiple of four, a truncated frame, or trailing bytes after the last
 * frame.  A negative tokens[r] fails with SC_ERR_ARG (*bad = r) before
 * anything is written. */
int sc_host_parse(const uint8_t *data, const int64_t *data_off, const int64_t *data_len, const int64_t *tokens,
                  int64_t n_reads, int32_t chunk_len, const int64_t *chunk_begin, const int64_t *read_word_off,
                  uint32_t *words_out, int64_t *word_off, int32_t *word_cnt, int32_t *tok_cnt, int32_t n_threads,
                  int64_t *bad);

/* sc_host_parse with each read's payload at its own address, payload[r]
 * (data_len[r] bytes): the caller's per-read buffers (the reference's list
 * of bytes objects) are parsed where they are, without first joining them. */
int sc_host_parse_v(const uint8_t *const *payload, const int64_t *data_len, const int64_t *tokens, int64_t n_reads,
                    int32_t chunk_len, const int64_t *chunk_begin, const int64_t *read_word_off, uint32_t *words_out,
                    int64_t *word_off, int32_t *word_cnt, int32_t *tok_cnt, int32_t n_threads, int64_t *bad);

/* ------------------------------------------------------------ SIG2 records
 *
 * A SIG2 archive is MAGIC 'SIG2', a uint32 length and the header blob (the
 * zstd-compressed pickle of the global metadata, main.py:226-246: opaque
 * bytes here), then one record per read (main.py:549-607):
 *   prefix   POD5 source:  REC_FMT '<16sddBBdIIIQ' (62 bytes, sc_pod5_record)
 *            BLOW5 source: read id (16 bytes), uint32 metadata length,
 *                          metadata (a pickle: opaque bytes here)
 *   split header '<hII': sig0 (int16), samples N (uint32), small tokens (uint32)
 *   three blobs, each a uint32 length then the bytes: the framed range-coded
 *   small tokens, the Rice-coded large values, the Rice-coded positions.
 * All integers little-endian, no padding.  The SIDX index (main.py:1451-1502,
 * archive_shards.py:295-304) is 'SIDX', a uint32 count, then per read the
 * 16-byte read id and the uint64 file offset of its record. */

#define SC_SIG2_POD5 0
#define SC_SIG2_BLOW5 1
#define SC_SIG2_POD5_PREFIX 62
#define SC_HOST_ERR_TRUNCATED   20  /* record, header or blob cut short [ValueError] */
#define SC_HOST_ERR_BAD_COUNTS  21  /* N < 1 or small tokens > N - 1 [ValueError] */
#define SC_HOST_ERR_TRAILING_RECORDS 22  /* bytes after the last record [ValueError] */
#define SC_HOST_ERR_INDEX       23  /* bad magic / count / size / offset [ValueError] */
#define SC_HOST_ERR_RICE        24  /* invalid, truncated or trailing Rice blob [ValueError] */
#define SC_HOST_ERR_RICE_RANGE  25  /* value does not fit the fallback width [ValueError] */

/* REC_FMT fields in order (main.py:905-917). */
typedef struct {
    uint8_t read_id[16];
    double calibration_offset, calibration_scale;
    uint8_t end_reason_forced, end_reason_index;
    double median_before;
    uint32_t pore, read_number, run_info;
    uint64_t start_sample;
} sc_pod5_record;

/* Serialize n records (_write_read_payload / _write_read_payload_blow5,
 * main.py:575-597).  Per read r: pod5[r] (POD5) or read_ids[16 r .. +16] and
 * meta[meta_off[r] .. + meta_len[r]] (BLOW5); sig0[r], n_samples[r],
 * n_small[r]; the three blobs at blob_off[3 r + k] with blob_len[3 r + k]
 * bytes in `blobs` (k = 0 small tokens, 1 large values, 2 positions).
 * Record r is written at out + out_off[r]; its size is prefix + 10 + 12 +
 * the blob lengths (+ 20 + meta_len for BLOW5 prefixes). */
int sc_sig2_write_records(int32_t format, int64_t n, const sc_pod5_record *pod5, const uint8_t *read_ids,
                          const uint8_t *meta, const int64_t *meta_off, const int64_t *meta_len,
                          const int16_t *sig0, const uint32_t *n_samples, const uint32_t *n_small,
                          const uint8_t *blobs, const int64_t *blob_off, const int64_t *blob_len, uint8_t *out,
                          const int64_t *out_off, int32_t n_threads, int64_t *bad);

/* Scan n_reads records from data[start .. size) as scan_archive
 * (archive_shards.py:149-175) and cmd_index (main.py:1451-1493) do: writes
 * rec_off[r] (record start; rec_off[n_reads] = end of the last record),
 * read_ids (16 bytes each), sig0 / n_samples / n_small, the blobs' byte
 * offsets and lengths (blob_off / blob_len, 3 per read, offsets into data),
 * meta_off / meta_len (BLOW5; may be NULL for POD5) and pod5 (POD5; may be
 * NULL).  Fails for a truncated record, N < 1 or more small tokens than
 * N - 1, a blob past the end of data, or (require_end != 0) bytes left after
 * the last record. */
int sc_sig2_scan_records(const uint8_t *data, int64_t size, int64_t start, int64_t n_reads, int32_t format,
                         int32_t require_end, int64_t *rec_off, uint8_t *read_ids, int16_t *sig0,
                         uint32_t *n_samples, uint32_t *n_small, int64_t *blob_off, int64_t *blob_len,
                         int64_t *meta_off, int64_t *meta_len, sc_pod5_record *pod5, int64_t *bad);

/* SIDX index of n reads: 8 + 24 n bytes to out. */
int sc_sig2_write_index(int64_t n, const uint8_t *read_ids, const uint64_t *offsets, uint8_t *out);

/* Read an SIDX index of `size` bytes for an archive of n_expected reads whose
 * records span [data_start, file_size) (_checked_index_header and
 * _index_entry, main.py:427-444): checks the magic, count == n_expected,
 * size == 8 + 24 count and every offset inside the records; writes read_ids
 * and offsets.  *bad = the offending entry (-1 for the header). */
int sc_sig2_read_index(const uint8_t *data, int64_t size, int64_t n_expected, int64_t data_start,
                       int64_t file_size, uint8_t *read_ids, uint64_t *offsets, int64_t *bad);

/* ---- Rice coding of the large values and their gap-coded positions ------
 *
 * Replaces fast_rice.rice_encode / rice_decode as the reference calls them
 * through _rice_compress / _rice_decompress (main.py:174-186; call sites
 * main.py:884-885 with fallback_bits 16 for the large values and 32 for the
 * positions, main.py:527-529 to decode, max_quotient 31).  The byte format
 * of fast-rice 0.1.0 is not available here (third-party package, absent
 * from the reference), so this one is this library's own: archives are
 * self-consistent, not byte-identical with the reference's Rice blobs.
 *
 * Blob of n >= 1 values (uint32 v, parameters FB = fallback_bits in 1..32,
 * MQ = max_quotient in 1..64): byte 0 = the Rice parameter k in
 * 0..min(FB, 31), the one minimising the blob's bit count (smallest on
 * ties); then a bit stream, least significant bit of each byte first,
 * zero-padded to a whole byte.  Per value, q = v >> k: if q < MQ, q one
 * bits, a zero bit and the k low bits of v (low bit first); else MQ one bits
 * and v in FB bits (low bit first).  An empty array is the single byte 0,
 * as _rice_compress writes it (main.py:176-177).
 * Decoding is strict: k > min(FB, 31), a quotient whose value would not
 * fit FB bits (q << k >= 2**FB), a stream that ends early, or any byte or
 * non-zero padding bit after the last value is SC_HOST_ERR_RICE. */

/* Largest blob of n values (bytes). */
int64_t sc_rice_bound(int64_t n, int32_t fallback_bits, int32_t max_quotient);

/* Encode n_items arrays: item i = count[i] values at vals + off[i], every
 * value < 2**fallback_bits (else SC_HOST_ERR_RICE_RANGE); blob i is written
 * at out + out_off[i] (room for sc_rice_bound(count[i], ...) bytes) and its
 * length to out_len[i]. */
int sc_rice_encode(const uint32_t *vals, const int64_t *off, const int64_t *count, int64_t n_items,
                   int32_t fallback_bits, int32_t max_quotient, uint8_t *out, const int64_t *out_off,
                   int64_t *out_len, int32_t n_threads, int64_t *bad);

/* Decode n_items blobs: blob i = blob_len[i] bytes at blobs[i], holding
 * count[i] values, written to out + out_off[i]; a count of 0 reads nothing
 * (_rice_decompress returns an empty array without reading, main.py:184-185).
 * A negative count is SC_ERR_ARG (bad = its index), found before any value
 * is written. */
int sc_rice_decode(const uint8_t *const *blobs, const int64_t *blob_len, const int64_t *count, int64_t n_items,
                   int32_t fallback_bits, int32_t max_quotient, uint32_t *out, const int64_t *out_off,
                   int32_t n_threads, int64_t *bad);

#ifdef __cplusplus
}
#endif

#endif /* SIGCOMP_HOST_H */
