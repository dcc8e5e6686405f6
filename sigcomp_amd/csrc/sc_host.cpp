// sc_host.cpp -- host stages either side of the GPU codec (C ABI in
// include/sigcomp_host.h): signal split / reassembly and SIG2 chunk framing,
// multithreaded over reads or chunks.
#include "../../include/sigcomp_host.h"

#include <algorithm>
#include <atomic>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

namespace {

thread_local std::string g_err;

// Runs f(i) for i in [0, n) on up to n_threads threads (dynamic blocks of
// indices); returns after every call ended.
template <class F>
void parallel_for(int64_t n, int32_t n_threads, F f) {
    int64_t hw = (int64_t)std::thread::hardware_concurrency();
    int64_t nt = n_threads > 0 ? n_threads : std::max<int64_t>(hw, 1);
    nt = std::min<int64_t>(nt, std::max<int64_t>(n / 16, 1));
    if (nt <= 1) {
        for (int64_t i = 0; i < n; ++i) f(i);
        return;
    }
    const int64_t block = std::max<int64_t>(1, n / (nt * 8));
    std::atomic<int64_t> next{0};
    auto worker = [&]() {
        for (;;) {
            const int64_t b = next.fetch_add(block);
            if (b >= n) break;
            const int64_t e = std::min(n, b + block);
            for (int64_t i = b; i < e; ++i) f(i);
        }
    };
    std::vector<std::thread> pool;
    pool.reserve((size_t)nt - 1);
    for (int64_t t = 1; t < nt; ++t) pool.emplace_back(worker);
    worker();
    for (auto &th : pool) th.join();
}

// First (lowest-numbered) failing item over all threads.
struct FirstBad {
    std::mutex m;
    int64_t idx = INT64_MAX;
    int code = SC_OK;
    void report(int64_t i, int c) {
        std::lock_guard<std::mutex> g(m);
        if (i < idx) {
            idx = i;
            code = c;
        }
    }
};

const char *err_text(int code) {
    switch (code) {
        case SC_HOST_ERR_FRAME_LENGTH: return "Truncated SIG2 chunk length";
        case SC_HOST_ERR_FRAME: return "Invalid or truncated SIG2 range-coded chunk";
        case SC_HOST_ERR_TRAILING: return "Trailing SIG2 chunk data disagrees with token length";
        case SC_HOST_ERR_OVERSIZE: return "Compressed chunk exceeds the SIG2 uint16 frame";
        case SC_HOST_ERR_COUNTS: return "small and large value counts disagree with the read length";
        case SC_HOST_ERR_POSITION: return "large-value position outside the read";
        case SC_HOST_ERR_EMPTY_READ: return "a read has no samples";
        case SC_HOST_ERR_TRUNCATED: return "Truncated SIG2 read record";
        case SC_HOST_ERR_BAD_COUNTS: return "Invalid sample or token count in SIG2 read record";
        case SC_HOST_ERR_TRAILING_RECORDS: return "SIG2 read count disagrees with trailing file data";
        case SC_HOST_ERR_INDEX: return "Index count/size does not match the archive; rebuild the index";
        case SC_HOST_ERR_RICE: return "Invalid or truncated Rice-coded blob";
        case SC_HOST_ERR_RICE_RANGE: return "value does not fit the Rice fallback width";
        default: return "error";
    }
}

int finish(FirstBad &fb, int64_t *bad) {
    if (fb.idx == INT64_MAX) return SC_OK;
    if (bad) *bad = fb.idx;
    g_err = std::string(err_text(fb.code)) + " (item " + std::to_string(fb.idx) + ")";
    return fb.code;
}

// _reduce_lsb then _lossy_encode (main.py:158-167) on one sample, int16 wrap
inline int16_t lossy_sample(int16_t s, int lsb) {
    if (lsb <= 0) return s;
    const int32_t v = s;
    const int32_t step = 1 << lsb;
    const int32_t rounding = ((v >> (lsb - 1)) & 1) * step;
    const int32_t upper = v & ~(step - 1);
    const int16_t reduced = (int16_t)(uint16_t)(uint32_t)(upper + rounding);
    return (int16_t)(uint16_t)(uint32_t)((int32_t)reduced >> lsb);
}

// zigzag of the int16 delta b - a (np.diff on int16 wraps modulo 2**16)
inline uint16_t zz_delta(int16_t a, int16_t b) {
    const int32_t d = (int16_t)(uint16_t)((uint32_t)(uint16_t)b - (uint32_t)(uint16_t)a);
    return (uint16_t)(((uint32_t)d << 1) ^ (uint32_t)(d >> 31));
}

inline int16_t unzigzag(uint16_t z) {
    const uint32_t v = z;
    return (int16_t)(uint16_t)((v >> 1) ^ (0u - (v & 1u)));
}

}  // namespace

namespace {

// Parse of framed reads (sc_host_parse): `payload(r)` is read r's data.
template <class PayloadFn>
int parse_reads(PayloadFn payload, const int64_t *data_len, const int64_t *tokens, int64_t n_reads, int32_t chunk_len,
                const int64_t *chunk_begin, const int64_t *read_word_off, uint32_t *words_out, int64_t *word_off,
                int32_t *word_cnt, int32_t *tok_cnt, int32_t n_threads, int64_t *bad) {
    if (n_reads < 0 || chunk_len < 1 ||
        (n_reads && (!data_len || !tokens || !chunk_begin || !read_word_off || !word_off || !word_cnt ||
                     !tok_cnt))) {
        g_err = "bad argument";
        return SC_ERR_ARG;
    }
    // a negative token count has no chunk layout (its chunk_begin would point
    // the following reads' chunks outside the caller's arrays): refused
    // before anything is written
    for (int64_t r = 0; r < n_reads; ++r)
        if (tokens[r] < 0) {
            if (bad) *bad = r;
            g_err = "negative token count";
            return SC_ERR_ARG;
        }
    FirstBad fb;
    parallel_for(n_reads, n_threads, [&](int64_t r) {
        const uint8_t *d = payload(r);
        const int64_t size = data_len[r];
        int64_t remaining = tokens[r], pos = 0, c = chunk_begin[r], w = read_word_off[r];
        while (remaining > 0) {
            if (pos + 2 > size) {
                fb.report(r, SC_HOST_ERR_FRAME_LENGTH);
                return;
            }
            const int64_t fbytes = (int64_t)d[pos] | ((int64_t)d[pos + 1] << 8);
            pos += 2;
            if (fbytes == 0 || fbytes % 4 || pos + fbytes > size) {
                fb.report(r, SC_HOST_ERR_FRAME);
                return;
            }
            const int64_t count = std::min<int64_t>(chunk_len, remaining);
            std::memcpy(words_out + w, d + pos, (size_t)fbytes);
            word_off[c] = w;
            word_cnt[c] = (int32_t)(fbytes / 4);
            tok_cnt[c] = (int32_t)count;
            w += fbytes / 4;
            pos += fbytes;
            remaining -= count;
            ++c;
        }
        if (pos != size) fb.report(r, SC_HOST_ERR_TRAILING);
    });
    return finish(fb, bad);
}

}  // namespace

extern "C" {

const char *sc_host_last_error(void) { return g_err.c_str(); }

int sc_host_split_count(const int16_t *const *reads, const int64_t *len, int64_t n_reads, int32_t lsb,
                        int16_t *sig0, int64_t *n_small, int64_t *n_large, int32_t n_threads, int64_t *bad) {
    if (n_reads < 0 || lsb < 0 || lsb > 15 || (n_reads && (!reads || !len || !sig0 || !n_small || !n_large))) {
        g_err = "bad argument";
        return SC_ERR_ARG;
    }
    FirstBad fb;
    parallel_for(n_reads, n_threads, [&](int64_t r) {
        const int64_t n = len[r];
        if (n < 1) {
            fb.report(r, SC_HOST_ERR_EMPTY_READ);
            return;
        }
        const int16_t *s = reads[r];
        int16_t prev = lossy_sample(s[0], lsb);
        int64_t small = 0;
        for (int64_t i = 1; i < n; ++i) {
            const int16_t cur = lossy_sample(s[i], lsb);
            small += zz_delta(prev, cur) < 256;
            prev = cur;
        }
        sig0[r] = lossy_sample(s[0], lsb);
        n_small[r] = small;
        n_large[r] = n - 1 - small;
    });
    return finish(fb, bad);
}

int sc_host_split_fill(const int16_t *const *reads, const int64_t *len, int64_t n_reads, int32_t lsb,
                       const int64_t *small_off, const int64_t *large_off, uint8_t *small, uint16_t *large_adj,
                       uint32_t *large_gap, int32_t n_threads, int64_t *bad) {
    if (n_reads < 0 || lsb < 0 || lsb > 15 ||
        (n_reads && (!reads || !len || !small_off || !large_off || !small || !large_adj || !large_gap))) {
        g_err = "bad argument";
        return SC_ERR_ARG;
    }
    FirstBad fb;
    parallel_for(n_reads, n_threads, [&](int64_t r) {
        const int64_t n = len[r];
        if (n < 1) {
            fb.report(r, SC_HOST_ERR_EMPTY_READ);
            return;
        }
        const int16_t *s = reads[r];
        uint8_t *sm = small + small_off[r];
        uint16_t *la = large_adj + large_off[r];
        uint32_t *lg = large_gap + large_off[r];
        int16_t prev = lossy_sample(s[0], lsb);
        int64_t last = -1;   // position of the previous large value
        for (int64_t i = 1; i < n; ++i) {
            const int16_t cur = lossy_sample(s[i], lsb);
            const uint16_t z = zz_delta(prev, cur);
            prev = cur;
            if (z < 256) {
                *sm++ = (uint8_t)z;
            } else {
                const int64_t pos = i - 1;
                *la++ = (uint16_t)(z - 256);
                *lg++ = (uint32_t)(last < 0 ? pos : pos - last - 1);
                last = pos;
            }
        }
    });
    return finish(fb, bad);
}

int sc_host_reassemble(const int16_t *sig0, const int64_t *len, int64_t n_reads, int32_t lsb, const uint8_t *small,
                       const int64_t *small_off, const int64_t *n_small, const uint16_t *large_adj,
                       const uint32_t *large_gap, const int64_t *large_off, const int64_t *n_large, int16_t *out,
                       const int64_t *out_off, int32_t n_threads, int64_t *bad) {
    if (n_reads < 0 || lsb < 0 || lsb > 15 ||
        (n_reads && (!sig0 || !len || !small_off || !n_small || !large_off || !n_large || !out || !out_off))) {
        g_err = "bad argument";
        return SC_ERR_ARG;
    }
    // an empty or negative length has no place in the output (the caller's
    // out_off, a prefix sum of the lengths, would point the following reads
    // outside `out`): refused before any sample is written
    for (int64_t r = 0; r < n_reads; ++r)
        if (len[r] < 1) {
            if (bad) *bad = r;
            g_err = std::string(err_text(SC_HOST_ERR_EMPTY_READ)) + " (item " + std::to_string(r) + ")";
            return SC_HOST_ERR_EMPTY_READ;
        }
    FirstBad fb;
    parallel_for(n_reads, n_threads, [&](int64_t r) {
        const int64_t n = len[r];
        if (n_small[r] < 0 || n_large[r] < 0 || n_small[r] + n_large[r] != n - 1) {
            fb.report(r, SC_HOST_ERR_COUNTS);
            return;
        }
        const uint8_t *sm = small + small_off[r];
        const uint16_t *la = large_adj + large_off[r];
        const uint32_t *lg = large_gap + large_off[r];
        // positions: first gap, then gap + 1 steps, so strictly increasing.
        // All of them are checked against the read before any sample is
        // rebuilt: the last one inside the read means every large value is
        // placed, and the small values read are then exactly n_small.
        int64_t last = -1;
        for (int64_t k = 0; k < n_large[r]; ++k) {
            last += (int64_t)lg[k] + 1;
            if (last >= n - 1) {
                fb.report(r, SC_HOST_ERR_POSITION);
                return;
            }
        }
        int64_t next_large = n_large[r] ? (int64_t)lg[0] : INT64_MAX, k = 0;
        int16_t *o = out + out_off[r];
        int16_t v = sig0[r];
        o[0] = lsb ? (int16_t)(uint16_t)((uint32_t)(int32_t)v << lsb) : v;
        int64_t js = 0;
        for (int64_t i = 0; i < n - 1; ++i) {
            uint16_t z;
            if (i == next_large) {
                z = (uint16_t)(la[k] + 256u);
                ++k;
                if (k < n_large[r]) next_large += (int64_t)lg[k] + 1;
            } else {
                z = sm[js++];
            }
            v = (int16_t)(uint16_t)((uint32_t)(uint16_t)v + (uint32_t)(uint16_t)unzigzag(z));
            o[i + 1] = lsb ? (int16_t)(uint16_t)((uint32_t)(int32_t)v << lsb) : v;
        }
    });
    return finish(fb, bad);
}

int sc_host_frame(const uint32_t *words, const int64_t *word_off, const int32_t *word_cnt, int64_t n_chunks,
                  uint8_t *out, const int64_t *out_off, int32_t n_threads, int64_t *bad) {
    if (n_chunks < 0 || (n_chunks && (!words || !word_off || !word_cnt || !out || !out_off))) {
        g_err = "bad argument";
        return SC_ERR_ARG;
    }
    FirstBad fb;
    parallel_for(n_chunks, n_threads, [&](int64_t c) {
        const int64_t bytes = (int64_t)word_cnt[c] * 4;
        if (word_cnt[c] < 0 || bytes > 65535) {
            fb.report(c, SC_HOST_ERR_OVERSIZE);
            return;
        }
        uint8_t *o = out + out_off[c];
        o[0] = (uint8_t)(bytes & 0xFF);
        o[1] = (uint8_t)(bytes >> 8);
        std::memcpy(o + 2, words + word_off[c], (size_t)bytes);   // little-endian host
    });
    return finish(fb, bad);
}

int sc_host_parse(const uint8_t *data, const int64_t *data_off, const int64_t *data_len, const int64_t *tokens,
                  int64_t n_reads, int32_t chunk_len, const int64_t *chunk_begin, const int64_t *read_word_off,
                  uint32_t *words_out, int64_t *word_off, int32_t *word_cnt, int32_t *tok_cnt, int32_t n_threads,
                  int64_t *bad) {
    if (n_reads && !data_off) {
        g_err = "bad argument";
        return SC_ERR_ARG;
    }
    return parse_reads([&](int64_t r) { return data + data_off[r]; }, data_len, tokens, n_reads, chunk_len,
                       chunk_begin, read_word_off, words_out, word_off, word_cnt, tok_cnt, n_threads, bad);
}

int sc_host_parse_v(const uint8_t *const *payload, const int64_t *data_len, const int64_t *tokens, int64_t n_reads,
                    int32_t chunk_len, const int64_t *chunk_begin, const int64_t *read_word_off, uint32_t *words_out,
                    int64_t *word_off, int32_t *word_cnt, int32_t *tok_cnt, int32_t n_threads, int64_t *bad) {
    if (n_reads && !payload) {
        g_err = "bad argument";
        return SC_ERR_ARG;
    }
    return parse_reads([&](int64_t r) { return payload[r]; }, data_len, tokens, n_reads, chunk_len, chunk_begin,
                       read_word_off, words_out, word_off, word_cnt, tok_cnt, n_threads, bad);
}

}  // extern "C"

// ---------------------------------------------------------------- SIG2 records

namespace {

template <class T>
inline void put(uint8_t *&o, T v) {
    std::memcpy(o, &v, sizeof(T));   // little-endian host
    o += sizeof(T);
}

template <class T>
inline T get(const uint8_t *p) {
    T v;
    std::memcpy(&v, p, sizeof(T));
    return v;
}

constexpr int64_t SPLIT_HDR = 10;   // '<hII'

}  // namespace

extern "C" {

int sc_sig2_write_records(int32_t format, int64_t n, const sc_pod5_record *pod5, const uint8_t *read_ids,
                          const uint8_t *meta, const int64_t *meta_off, const int64_t *meta_len,
                          const int16_t *sig0, const uint32_t *n_samples, const uint32_t *n_small,
                          const uint8_t *blobs, const int64_t *blob_off, const int64_t *blob_len, uint8_t *out,
                          const int64_t *out_off, int32_t n_threads, int64_t *bad) {
    const bool blow5 = format == SC_SIG2_BLOW5;
    if (n < 0 || (format != SC_SIG2_POD5 && !blow5) ||
        (n && (!sig0 || !n_samples || !n_small || !blobs || !blob_off || !blob_len || !out || !out_off ||
               (blow5 ? (!read_ids || !meta || !meta_off || !meta_len) : !pod5)))) {
        g_err = "bad argument";
        return SC_ERR_ARG;
    }
    FirstBad fb;
    parallel_for(n, n_threads, [&](int64_t r) {
        if (n_samples[r] < 1 || n_small[r] > n_samples[r] - 1) {
            fb.report(r, SC_HOST_ERR_BAD_COUNTS);
            return;
        }
        for (int k = 0; k < 3; ++k)
            if (blob_len[3 * r + k] < 0 || blob_len[3 * r + k] > 0xFFFFFFFFll) {
                fb.report(r, SC_HOST_ERR_OVERSIZE);
                return;
            }
        if (blow5 && (meta_len[r] < 0 || meta_len[r] > 0xFFFFFFFFll)) {
            fb.report(r, SC_HOST_ERR_OVERSIZE);
            return;
        }
        uint8_t *o = out + out_off[r];
        if (blow5) {
            std::memcpy(o, read_ids + 16 * r, 16);
            o += 16;
            put<uint32_t>(o, (uint32_t)meta_len[r]);
            std::memcpy(o, meta + meta_off[r], (size_t)meta_len[r]);
            o += meta_len[r];
        } else {
            const sc_pod5_record &p = pod5[r];
            std::memcpy(o, p.read_id, 16);
            o += 16;
            put<double>(o, p.calibration_offset);
            put<double>(o, p.calibration_scale);
            put<uint8_t>(o, p.end_reason_forced);
            put<uint8_t>(o, p.end_reason_index);
            put<double>(o, p.median_before);
            put<uint32_t>(o, p.pore);
            put<uint32_t>(o, p.read_number);
            put<uint32_t>(o, p.run_info);
            put<uint64_t>(o, p.start_sample);
        }
        put<int16_t>(o, sig0[r]);
        put<uint32_t>(o, n_samples[r]);
        put<uint32_t>(o, n_small[r]);
        for (int k = 0; k < 3; ++k) {
            const int64_t len = blob_len[3 * r + k];
            put<uint32_t>(o, (uint32_t)len);
            std::memcpy(o, blobs + blob_off[3 * r + k], (size_t)len);
            o += len;
        }
    });
    return finish(fb, bad);
}

int sc_sig2_scan_records(const uint8_t *data, int64_t size, int64_t start, int64_t n_reads, int32_t format,
                         int32_t require_end, int64_t *rec_off, uint8_t *read_ids, int16_t *sig0,
                         uint32_t *n_samples, uint32_t *n_small, int64_t *blob_off, int64_t *blob_len,
                         int64_t *meta_off, int64_t *meta_len, sc_pod5_record *pod5, int64_t *bad) {
    const bool blow5 = format == SC_SIG2_BLOW5;
    if (n_reads < 0 || size < 0 || start < 0 || start > size || (format != SC_SIG2_POD5 && !blow5) ||
        !rec_off || (n_reads && (!data || !read_ids || !sig0 || !n_samples || !n_small || !blob_off ||
                                 !blob_len || (blow5 && (!meta_off || !meta_len))))) {
        g_err = "bad argument";
        return SC_ERR_ARG;
    }
    FirstBad fb;
    int64_t pos = start;
    for (int64_t r = 0; r < n_reads; ++r) {
        rec_off[r] = pos;
        if (blow5) {
            if (pos + 20 > size) {
                fb.report(r, SC_HOST_ERR_TRUNCATED);
                break;
            }
            std::memcpy(read_ids + 16 * r, data + pos, 16);
            const int64_t ml = get<uint32_t>(data + pos + 16);
            pos += 20;
            if (pos + ml > size) {
                fb.report(r, SC_HOST_ERR_TRUNCATED);
                break;
            }
            meta_off[r] = pos;
            meta_len[r] = ml;
            pos += ml;
        } else {
            if (pos + SC_SIG2_POD5_PREFIX > size) {
                fb.report(r, SC_HOST_ERR_TRUNCATED);
                break;
            }
            const uint8_t *p = data + pos;
            std::memcpy(read_ids + 16 * r, p, 16);
            if (pod5) {
                sc_pod5_record &q = pod5[r];
                std::memcpy(q.read_id, p, 16);
                q.calibration_offset = get<double>(p + 16);
                q.calibration_scale = get<double>(p + 24);
                q.end_reason_forced = p[32];
                q.end_reason_index = p[33];
                q.median_before = get<double>(p + 34);
                q.pore = get<uint32_t>(p + 42);
                q.read_number = get<uint32_t>(p + 46);
                q.run_info = get<uint32_t>(p + 50);
                q.start_sample = get<uint64_t>(p + 54);
            }
            pos += SC_SIG2_POD5_PREFIX;
        }
        if (pos + SPLIT_HDR > size) {
            fb.report(r, SC_HOST_ERR_TRUNCATED);
            break;
        }
        sig0[r] = get<int16_t>(data + pos);
        n_samples[r] = get<uint32_t>(data + pos + 2);
        n_small[r] = get<uint32_t>(data + pos + 6);
        pos += SPLIT_HDR;
        if (n_samples[r] < 1 || n_small[r] > n_samples[r] - 1) {
            fb.report(r, SC_HOST_ERR_BAD_COUNTS);
            break;
        }
        bool ok = true;
        for (int k = 0; k < 3 && ok; ++k) {
            if (pos + 4 > size) {
                ok = false;
                break;
            }
            const int64_t len = get<uint32_t>(data + pos);
            pos += 4;
            if (pos + len > size) {
                ok = false;
                break;
            }
            blob_off[3 * r + k] = pos;
            blob_len[3 * r + k] = len;
            pos += len;
        }
        if (!ok) {
            fb.report(r, SC_HOST_ERR_TRUNCATED);
            break;
        }
    }
    if (fb.idx == INT64_MAX) {
        rec_off[n_reads] = pos;
        if (require_end && pos != size) fb.report(n_reads, SC_HOST_ERR_TRAILING_RECORDS);
    }
    return finish(fb, bad);
}

int sc_sig2_write_index(int64_t n, const uint8_t *read_ids, const uint64_t *offsets, uint8_t *out) {
    if (n < 0 || n > 0xFFFFFFFFll || !out || (n && (!read_ids || !offsets))) {
        g_err = "bad argument";
        return SC_ERR_ARG;
    }
    uint8_t *o = out;
    std::memcpy(o, "SIDX", 4);
    o += 4;
    put<uint32_t>(o, (uint32_t)n);
    for (int64_t r = 0; r < n; ++r) {
        std::memcpy(o, read_ids + 16 * r, 16);
        o += 16;
        put<uint64_t>(o, offsets[r]);
    }
    return SC_OK;
}

int sc_sig2_read_index(const uint8_t *data, int64_t size, int64_t n_expected, int64_t data_start,
                       int64_t file_size, uint8_t *read_ids, uint64_t *offsets, int64_t *bad) {
    if (size < 0 || n_expected < 0 || (size && !data) || (n_expected && (!read_ids || !offsets))) {
        g_err = "bad argument";
        return SC_ERR_ARG;
    }
    auto fail_at = [&](int64_t i, const char *msg) {
        if (bad) *bad = i;
        g_err = msg;
        return SC_HOST_ERR_INDEX;
    };
    if (size < 8 || std::memcmp(data, "SIDX", 4) != 0) return fail_at(-1, "Not a valid SIDX index");
    const int64_t count = get<uint32_t>(data + 4);
    if (count != n_expected || size != 8 + 24 * count)
        return fail_at(-1, "Index count/size does not match the archive; rebuild the index");
    for (int64_t r = 0; r < count; ++r) {
        const uint8_t *e = data + 8 + 24 * r;
        const uint64_t off = get<uint64_t>(e + 16);
        if (!((uint64_t)data_start <= off && off < (uint64_t)file_size))
            return fail_at(r, "SIDX entry points outside archive records; rebuild the index");
        std::memcpy(read_ids + 16 * r, e, 16);
        offsets[r] = off;
    }
    return SC_OK;
}

}  // extern "C"

// ---------------------------------------------------------------- Rice coder
namespace {

// Bits, least significant first, into a byte buffer.
struct BitWriter {
    uint8_t *p;
    uint64_t acc = 0;
    int n = 0;
    explicit BitWriter(uint8_t *out) : p(out) {}
    void put(uint64_t v, int len) {   // len <= 32, n < 8 on entry
        acc |= (v & ((1ull << len) - 1)) << n;
        n += len;
        while (n >= 8) {
            *p++ = (uint8_t)acc;
            acc >>= 8;
            n -= 8;
        }
    }
    void ones(int len) {
        while (len > 32) {
            put(0xFFFFFFFFull, 32);
            len -= 32;
        }
        put((1ull << len) - 1, len);
    }
    uint8_t *flush() {   // zero padding to the byte
        if (n > 0) *p++ = (uint8_t)acc;
        acc = 0;
        n = 0;
        return p;
    }
};

inline uint64_t shr(uint64_t x, int s) { return s >= 64 ? 0 : x >> s; }

struct BitReader {
    const uint8_t *p, *end;
    uint64_t acc = 0;
    int n = 0;   // valid bits in acc
    BitReader(const uint8_t *b, const uint8_t *e) : p(b), end(e) {}
    void refill() {
        while (n <= 56 && p < end) {
            acc |= (uint64_t)*p++ << n;
            n += 8;
        }
    }
    // false when the stream ends before len bits (len <= 32)
    bool get(int len, uint32_t &v) {
        if (n < len) refill();
        if (n < len) return false;
        v = len ? (uint32_t)(acc & ((1ull << len) - 1)) : 0u;
        acc = shr(acc, len);
        n -= len;
        return true;
    }
    // unary: count of one bits before a zero bit, at most `cap` ones (no
    // zero bit is consumed when the count reaches cap); false when the
    // stream ends first
    bool unary(int cap, int &q) {
        q = 0;
        for (;;) {
            if (n == 0) refill();
            if (n == 0) return false;
            const uint64_t inv = ~acc & (n == 64 ? ~0ull : ((1ull << n) - 1));
            const int run = inv ? __builtin_ctzll(inv) : n;   // ones available in acc
            if (q + run >= cap) {
                const int take = cap - q;
                acc = shr(acc, take);
                n -= take;
                q = cap;
                return true;
            }
            if (run < n) {   // a zero bit ends the run
                q += run;
                acc = shr(acc, run + 1);
                n -= run + 1;
                return true;
            }
            q += run;
            acc = 0;
            n = 0;
        }
    }
    // the rest is zero padding of the last byte, and nothing after it
    bool at_end() const { return p == end && n < 8 && acc == 0; }
};

int rice_kmax(int32_t fb) { return fb < 31 ? fb : 31; }

// bit count of the stream of vals[0..n) with parameter k
uint64_t rice_bits(const uint32_t *v, int64_t n, int k, int32_t fb, int32_t mq) {
    uint64_t bits = 0;
    for (int64_t i = 0; i < n; ++i) {
        const uint32_t q = v[i] >> k;
        bits += q < (uint32_t)mq ? q + 1 + (uint64_t)k : (uint64_t)mq + fb;
    }
    return bits;
}

}  // namespace

extern "C" {

int64_t sc_rice_bound(int64_t n, int32_t fallback_bits, int32_t max_quotient) {
    if (n <= 0) return 1;
    return 1 + (n * ((int64_t)max_quotient + fallback_bits) + 7) / 8;
}

int sc_rice_encode(const uint32_t *vals, const int64_t *off, const int64_t *count, int64_t n_items,
                   int32_t fallback_bits, int32_t max_quotient, uint8_t *out, const int64_t *out_off,
                   int64_t *out_len, int32_t n_threads, int64_t *bad) {
    if (n_items < 0 || fallback_bits < 1 || fallback_bits > 32 || max_quotient < 1 || max_quotient > 64 ||
        (n_items && (!off || !count || !out || !out_off || !out_len))) {
        g_err = "bad argument";
        return SC_ERR_ARG;
    }
    FirstBad fb;
    const int kmax = rice_kmax(fallback_bits);
    const uint64_t lim = fallback_bits == 32 ? 0x100000000ull : (1ull << fallback_bits);
    parallel_for(n_items, n_threads, [&](int64_t i) {
        const int64_t n = count[i];
        uint8_t *o = out + out_off[i];
        if (n <= 0) {
            o[0] = 0;
            out_len[i] = 1;
            if (n < 0) fb.report(i, SC_ERR_ARG);
            return;
        }
        const uint32_t *v = vals + off[i];
        for (int64_t j = 0; j < n; ++j)
            if ((uint64_t)v[j] >= lim) {
                fb.report(i, SC_HOST_ERR_RICE_RANGE);
                out_len[i] = 0;
                return;
            }
        int best_k = 0;
        uint64_t best = rice_bits(v, n, 0, fallback_bits, max_quotient);
        for (int k = 1; k <= kmax; ++k) {
            const uint64_t b = rice_bits(v, n, k, fallback_bits, max_quotient);
            if (b < best) {
                best = b;
                best_k = k;
            }
        }
        o[0] = (uint8_t)best_k;
        BitWriter w(o + 1);
        const uint32_t mq = (uint32_t)max_quotient;
        for (int64_t j = 0; j < n; ++j) {
            const uint32_t q = v[j] >> best_k;
            if (q < mq) {
                w.ones((int)q);
                w.put(0, 1);
                w.put(v[j], best_k);
            } else {
                w.ones(max_quotient);
                w.put(v[j], fallback_bits);
            }
        }
        out_len[i] = w.flush() - o;
    });
    return finish(fb, bad);
}

int sc_rice_decode(const uint8_t *const *blobs, const int64_t *blob_len, const int64_t *count, int64_t n_items,
                   int32_t fallback_bits, int32_t max_quotient, uint32_t *out, const int64_t *out_off,
                   int32_t n_threads, int64_t *bad) {
    if (n_items < 0 || fallback_bits < 1 || fallback_bits > 32 || max_quotient < 1 || max_quotient > 64 ||
        (n_items && (!blobs || !blob_len || !count || !out || !out_off))) {
        g_err = "bad argument";
        return SC_ERR_ARG;
    }
    // every count is checked before anything is written: the output
    // offsets of the items after a negative count would not be valid
    for (int64_t i = 0; i < n_items; ++i)
        if (count[i] < 0) {
            if (bad) *bad = i;
            g_err = "negative value count";
            return SC_ERR_ARG;
        }
    FirstBad fb;
    const int kmax = rice_kmax(fallback_bits);
    const uint64_t lim = fallback_bits == 32 ? 0x100000000ull : (1ull << fallback_bits);
    parallel_for(n_items, n_threads, [&](int64_t i) {
        const int64_t n = count[i];
        if (n == 0) return;
        const uint8_t *b = blobs[i];
        const int64_t len = blob_len[i];
        if (len < 2 || !b || b[0] > kmax) {
            fb.report(i, SC_HOST_ERR_RICE);
            return;
        }
        const int k = b[0];
        BitReader r(b + 1, b + len);
        uint32_t *o = out + out_off[i];
        for (int64_t j = 0; j < n; ++j) {
            int q;
            uint32_t low;
            if (!r.unary(max_quotient, q)) {
                fb.report(i, SC_HOST_ERR_RICE);
                return;
            }
            if (q < max_quotient) {
                if (!r.get(k, low)) {
                    fb.report(i, SC_HOST_ERR_RICE);
                    return;
                }
                if (((uint64_t)q << k) >= lim) {   // no value of the fallback width has this quotient
                    fb.report(i, SC_HOST_ERR_RICE);
                    return;
                }
                o[j] = ((uint32_t)q << k) | low;
            } else {
                if (!r.get(fallback_bits, low)) {
                    fb.report(i, SC_HOST_ERR_RICE);
                    return;
                }
                o[j] = low;
            }
        }
        if (!r.at_end()) fb.report(i, SC_HOST_ERR_RICE);
    });
    return finish(fb, bad);
}

}  // extern "C"
