// sc_kernels.hip -- the C ABI of libsigcomp_hip (include/sigcomp_hip.h) and
// the small kernels around the MLP kernels (tile table, range encoder over
// coded pairs, decode plan statistics, word gather, step-API coder kernels,
// MFMA rate probe).  The MLP kernels are in sc_kernels.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/sigcomp_hip.h"
#include "sc_gen.h"
#include "sc_kernels.h"

using namespace sc;

// =========================================================================
// Kernels
// =========================================================================

namespace {

// ---- compress: teacher-forced MLP fused with the frequency step ----------

// Tiles are 128 consecutive steps of one chunk.  tile_start[c] = number of
// tiles of chunks 0 .. c-1 (exclusive scan of ceil(lengths[c] / 128)),
// tile_start[n_chunks] = total.  One workgroup of 1024 threads: every thread
// scans a contiguous segment, segment sums are scanned in LDS.
constexpr int SCAN_THREADS = 1024;

__global__ __launch_bounds__(SCAN_THREADS) void k_tile_scan(const int32_t *__restrict__ lengths, int64_t n_chunks,
                                                             int32_t *__restrict__ tile_start) {
    __shared__ int32_t s_sum[SCAN_THREADS];
    const int64_t per = (n_chunks + SCAN_THREADS - 1) / SCAN_THREADS;
    const int64_t c0 = threadIdx.x * per, c1 = min(c0 + per, n_chunks);
    int32_t sum = 0;
    // a negative length counts as empty: offsets stay monotone and non-negative
    for (int64_t c = c0; c < c1; ++c) sum += (max(lengths[c], 0) + R_TILE - 1) / R_TILE;
    s_sum[threadIdx.x] = sum;
    __syncthreads();
    for (int d = 1; d < SCAN_THREADS; d <<= 1) {
        const int32_t v = threadIdx.x >= (unsigned)d ? s_sum[threadIdx.x - d] : 0;
        __syncthreads();
        s_sum[threadIdx.x] += v;
        __syncthreads();
    }
    int32_t run = s_sum[threadIdx.x] - sum;
    for (int64_t c = c0; c < c1; ++c) {
        tile_start[c] = run;
        run += (max(lengths[c], 0) + R_TILE - 1) / R_TILE;
    }
    if (threadIdx.x == SCAN_THREADS - 1) tile_start[n_chunks] = s_sum[SCAN_THREADS - 1];
}

// Tile descriptors, one thread per chunk: tile k of chunk c (global index
// tile_start[c] + k) covers steps t0 = 128k .. t0 + 127 and is described by
// {first token's index in the token array (low, high word), L - t0, t0}, so
// that a compress workgroup finds its tile's tokens with one load instead of
// a search over tile_start.
__global__ __launch_bounds__(256) void k_tile_table(const int64_t *__restrict__ tok_off,
                                                    const int32_t *__restrict__ lengths, int64_t n_chunks,
                                                    const int32_t *__restrict__ tile_start, int4 *__restrict__ desc,
                                                    int64_t max_desc) {
    const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= n_chunks) return;
    const int32_t L = lengths[c];
    const int64_t base = tok_off[c];
    int32_t k = tile_start[c];
    // max_desc bounds the table for disjoint chunks inside the token array
    for (int32_t t0 = 0; t0 < L && k < max_desc; t0 += R_TILE, ++k) {
        const int64_t b = base + t0;
        desc[k] = make_int4((int)(uint32_t)b, (int)(b >> 32), L - t0, t0);
    }
}

// One thread per chunk walks its (cum, freq) pairs through the range coder
// and seals the stream (cpu_entropy_coding.py:121-227).
__global__ __launch_bounds__(256) void k_encode_pairs(const uint2 *__restrict__ pairs,
                                                      const int64_t *__restrict__ tok_off,
                                                      const int32_t *__restrict__ lengths, int64_t n_chunks,
                                                      uint32_t *__restrict__ words,
                                                      const int64_t *__restrict__ word_off,
                                                      const int32_t *__restrict__ word_cap,
                                                      int32_t *__restrict__ word_cnt,
                                                      int32_t *__restrict__ status) {
    const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= n_chunks) return;
    const int32_t L = lengths[c];
    const int32_t cap = word_cap[c];
    const uint2 *p = pairs + tok_off[c];
    uint32_t *out = words + word_off[c];
    EncState s{0ull, ~0ull, 0, 0u, 0};
    int st = 0;
    uint2 nxt = L > 0 ? p[0] : make_uint2(0u, 0u);
    for (int32_t t = 0; t < L; ++t) {
        const uint2 cur = nxt;
        if (t + 1 < L) nxt = p[t + 1];
        if (enc_step(s, cur.x, cur.y, out, cap)) { st = SC_STATUS_CAPACITY; break; }
    }
    if (!st && L > 0 && enc_seal(s, out, cap)) st = SC_STATUS_CAPACITY;
    word_cnt[c] = s.pos;
    status[c] = st;
}

// Length statistics for the decode plan, each max(0, ...), one workgroup of
// 1024 threads.  With the last full-wave launch holding chunks g0 .. g0+G-1
// and the `left` chunks after it: out[0] = the longest chunk, out[1] = the
// longest pair (row g0+G-left+i of that launch followed by chunk
// g0+G+left-1-i), out[2] = the longest chunk of that launch, out[3] = the
// longest leftover chunk.
__global__ __launch_bounds__(1024) void k_dec_lengths(const int32_t *__restrict__ lengths, int64_t n, int64_t g0,
                                                      int64_t G, int64_t left, int32_t *__restrict__ out) {
    __shared__ int32_t s_m[4][1024 / 64];
    int32_t m[4] = {0, 0, 0, 0};
    for (int64_t i = threadIdx.x; i < n; i += 1024) {
        const int32_t l = max(lengths[i], 0);
        m[0] = max(m[0], l);
        if (i >= g0 && i < g0 + G) m[2] = max(m[2], l);
        if (i >= g0 + G && i < g0 + G + left) m[3] = max(m[3], l);
    }
    // a pair's second chunk starts one step after its first ends
    for (int64_t i = threadIdx.x; i < left; i += 1024) {
        const int32_t l1 = max(lengths[g0 + G - left + i], 0);
        m[1] = max(m[1], l1 + max(lengths[g0 + G + left - 1 - i], 0) + (l1 > 0 ? 1 : 0));
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        m[k] = wave_max_i32(m[k]);
        if ((threadIdx.x & 63) == 0) s_m[k][threadIdx.x >> 6] = m[k];
    }
    __syncthreads();
    if (threadIdx.x < 4) {
        int32_t r = 0;
        for (int k = 0; k < 1024 / 64; ++k) r = max(r, s_m[threadIdx.x][k]);
        out[threadIdx.x] = r;
    }
}

// Clears n int32 (the split decode's step flags).  A kernel rather than a
// memset, so that a caller may capture the call in a HIP graph.
__global__ __launch_bounds__(256) void k_zero_i32(int32_t *__restrict__ p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0;
}

// ---- word compaction -----------------------------------------------------

// One wavefront per chunk copies its word_cnt[c] words from its capacity slot
// to out + out_off[c] (coalesced 4-byte lanes).
__global__ __launch_bounds__(256) void k_gather_words(const uint32_t *__restrict__ words,
                                                      const int64_t *__restrict__ word_off,
                                                      const int32_t *__restrict__ word_cnt, int64_t n_chunks,
                                                      uint32_t *__restrict__ out,
                                                      const int64_t *__restrict__ out_off) {
    const int64_t c = (int64_t)blockIdx.x * WAVES + (threadIdx.x >> 6);
    if (c >= n_chunks) return;
    const int lane = threadIdx.x & 63;
    const uint32_t *src = words + word_off[c];
    uint32_t *dst = out + out_off[c];
    const int32_t n = word_cnt[c];
    for (int32_t i = lane; i < n; i += 64) dst[i] = src[i];
}

// ---- step-API kernels (GpuRangeStepEncoder / GpuRangeDecoder) ------------
// 256 threads = 16 rows per workgroup (four 16-lane rows per wavefront).  A
// workgroup's rows are a short serial chain (LUT staging, loads, frequency
// step, coder step), run by many workgroups per CU at once (few registers);
// k_logits_to_cdf issues its logits load before the LUT staging barrier.

__device__ __forceinline__ void stage_lut(const uint64_t *lut, double *s_lut) {
    load_lut_lds(lut, s_lut);
    __syncthreads();
}

__device__ __forceinline__ v4i global_logits16(const int8_t *logits, int64_t row, int64_t rows, int u) {
    return row < rows ? *(const v4i *)(logits + row * VOCAB + 16 * u) : v4i{0, 0, 0, 0};
}

// Each wave's 4 rows (4 x 257 int64, one contiguous span of the output)
// are staged in LDS and written out as 16-byte pieces by consecutive lanes:
// written straight from the lanes, each store instruction would scatter 64
// 8-byte pieces 128 bytes apart.  LDS rows hold one pad slot per 16 values,
// so that the 16 lanes of a row (16 values apart) write different banks.
constexpr int CDF_LDS_ROW = VOCAB + 1 + 17;   // 257 values + 16 pads, even
__device__ __forceinline__ int cdf_lds_at(int v) { return v + (v >> 4); }

__global__ __launch_bounds__(256) void k_logits_to_cdf(const int8_t *__restrict__ logits, int64_t rows,
                                                       const uint64_t *__restrict__ lut,
                                                       int64_t *__restrict__ cdf) {
    __shared__ double s_lut[VOCAB];
    __shared__ __attribute__((aligned(16))) int64_t s_out[WAVES][4 * CDF_LDS_ROW];
    const int u = threadIdx.x & 15, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t r = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const v4i raw = global_logits16(logits, r, rows, u);
    stage_lut(lut, s_lut);
    Freq16 fr;
    row_frequencies16(raw, s_lut, u, fr);
    int64_t *so = s_out[wave] + (lane >> 4) * CDF_LDS_ROW;
    uint32_t c = fr.ex;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        so[cdf_lds_at(16 * u + k)] = c;
        c += fr.f[k];
    }
    if (u == 15) so[cdf_lds_at(VOCAB)] = TOTAL;
    // the wave's own LDS writes before its reads (LDS runs a wave's accesses in order)
    slot_sync();
    const int64_t r0 = (int64_t)blockIdx.x * 16 + wave * 4;
    if (r0 >= rows) return;
    const int n = (int)min<int64_t>(4, rows - r0) * (VOCAB + 1);   // values of the span
    int64_t *dst = cdf + r0 * (VOCAB + 1);   // 16-byte aligned: r0 is a multiple of 4, 4 x 2056 = 8224 bytes
    const int64_t *sw = s_out[wave];
    auto at = [&](int i) { return sw[(i / (VOCAB + 1)) * CDF_LDS_ROW + cdf_lds_at(i % (VOCAB + 1))]; };
    for (int i = 2 * lane; i < n; i += 128) {
        if (i + 1 < n) {
            *(longlong2 *)(dst + i) = make_longlong2(at(i), at(i + 1));
        } else {
            dst[i] = at(i);
        }
    }
}

struct EncArrays {
    uint64_t *lower, *range;
    int32_t *inverted;
    uint32_t *first;
    int32_t *write_pos, *status;
};

static_assert(VOCAB == 256, "the step kernels stage one LUT entry per thread of a 256-thread workgroup");

// The encode and decode steps issue every load a row needs (its logits,
// its coder state, the LUT entry of the thread) before the LUT staging
// barrier, so that a workgroup waits for one memory round trip instead of
// three in a row (LUT, then logits, then state); a row's state is read
// whether or not the step codes it (it lies inside the arrays either way).
__global__ __launch_bounds__(256) void k_encode_step(const int8_t *__restrict__ logits,
                                                     const uint64_t *__restrict__ lut,
                                                     const int64_t *__restrict__ symbols,
                                                     const int64_t *__restrict__ valid, int64_t t,
                                                     int64_t B, EncArrays st, uint32_t *__restrict__ words,
                                                     int64_t max_words) {
    __shared__ double s_lut[VOCAB];
    const int u = threadIdx.x & 15;
    const int64_t b = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const bool in = b < B;
    const v4i raw = global_logits16(logits, b, B, u);
    const uint64_t lut_v = lut[threadIdx.x];   // 256 threads, VOCAB entries
    int64_t vb = 0, sym = 0;
    int32_t stb = 0;
    EncState e{};
    if (in) {
        vb = valid[b];
        sym = symbols[b];
        stb = st.status[b];
        e = EncState{st.lower[b], st.range[b], st.inverted[b], st.first[b], st.write_pos[b]};
    }
    s_lut[VOCAB - 1 - threadIdx.x] = (double)lut_v;   // reversed, as load_lut_lds
    __syncthreads();
    Freq16 fr;
    row_frequencies16(raw, s_lut, u, fr);
    if (!in || t >= vb || stb) return;
    if (sym < 0 || sym >= VOCAB) {
        if (u == 0) st.status[b] = SC_STATUS_BAD_TOKEN;
        return;
    }
    const int s = (int)sym;
    if ((s >> 4) != u) return;   // the lane holding the symbol runs the coder
    uint32_t cum, freq;
    freq16_at(fr, s & 15, cum, freq);
    // Every field goes back unconditionally, the status included (0 before
    // this step, since the row is live): the state is unchanged when the step
    // did not fit (enc_step).  One store per field and no branch between
    // them, so that no store's address depends on the path taken.
    const int full = enc_step(e, cum, freq, words + b * max_words, (int32_t)max_words);
    st.lower[b] = e.lower;
    st.range[b] = e.range;
    st.inverted[b] = e.inverted;
    st.first[b] = e.first;
    st.write_pos[b] = e.pos;
    st.status[b] = full ? SC_STATUS_CAPACITY : SC_STATUS_OK;
}

__global__ __launch_bounds__(256) void k_encode_seal(int64_t B, EncArrays st, uint32_t *__restrict__ words,
                                                     int64_t max_words) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= B || st.status[b]) return;
    EncState e{st.lower[b], st.range[b], st.inverted[b], st.first[b], st.write_pos[b]};
    if (enc_seal(e, words + b * max_words, (int32_t)max_words)) {
        st.status[b] = SC_STATUS_CAPACITY;
        return;
    }
    st.lower[b] = e.lower;
    st.range[b] = e.range;
    st.inverted[b] = e.inverted;
    st.write_pos[b] = e.pos;
}

struct DecArrays {
    uint64_t *lower, *range, *point;
    int64_t *read_pos;
    const int64_t *end_pos;
    int32_t *status;
};

__global__ __launch_bounds__(256) void k_decode_step(const int8_t *__restrict__ logits,
                                                     const uint64_t *__restrict__ lut,
                                                     const int64_t *__restrict__ valid, int64_t t,
                                                     int64_t B, DecArrays st,
                                                     const uint32_t *__restrict__ words,
                                                     int64_t *__restrict__ symbols_out) {
    __shared__ double s_lut[VOCAB];
    const int lane = threadIdx.x & 63, u = threadIdx.x & 15;
    const int64_t b = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const bool in_range = b < B;
    const v4i raw = global_logits16(logits, b, B, u);
    const uint64_t lut_v = lut[threadIdx.x];   // 256 threads, VOCAB entries
    int64_t vb = 0, rp = 0, endp = 0;
    int32_t stb = 0;
    uint64_t lower0 = 0, range0 = ~0ull, point0 = 0;
    if (in_range) {
        vb = valid[b];
        stb = st.status[b];
        lower0 = st.lower[b];
        range0 = st.range[b];
        point0 = st.point[b];
        rp = st.read_pos[b];
        endp = st.end_pos[b];
    }
    s_lut[VOCAB - 1 - threadIdx.x] = (double)lut_v;   // reversed, as load_lut_lds
    __syncthreads();
    // the word a renormalisation would shift in, loaded during the frequency step
    const uint32_t wnext = in_range && rp < endp ? words[rp] : 0u;
    Freq16 fr;
    row_frequencies16(raw, s_lut, u, fr);
    const bool active = in_range && t < vb && stb == 0;
    uint64_t lower = 0, range = ~0ull, point = 0;
    if (active) {
        lower = lower0;
        range = range0;
        point = point0;
    }
    const uint64_t scale = range >> 24;
    uint32_t q = 0;
    const bool ok = scale != 0 && dec_quantile(point - lower, scale, q);
    uint32_t cum, freq;
    const int sym = dec_symbol16(fr, q, lane, cum, freq);
    if (!in_range || u != 0) return;
    // an inactive row returns symbol 256; an invalid stream keeps its state
    // and records the status; otherwise the step's new state.  Every field
    // of an active row goes back, the status included (0 before this step),
    // with no branch between the stores.
    const bool step = active && ok;
    if (step) {
        lower += scale * cum;
        range = scale * freq;
        if (range < (1ull << 32)) {
            lower <<= 32;
            range <<= 32;
            point = (point << 32) | wnext;
            rp += 1;
        }
    }
    if (active) {
        st.lower[b] = lower;
        st.range[b] = range;
        st.point[b] = point;
        st.read_pos[b] = rp;
        st.status[b] = ok ? SC_STATUS_OK : SC_STATUS_INVALID_STREAM;
    }
    symbols_out[b] = step ? (int64_t)sym : (int64_t)VOCAB;
}

// Large batches: the kernels above give each row 16 lanes for its frequency
// table and then run the row's coder step (and the decoder's quantile) in
// one of them, so that a wave's coder work uses 4 of its 64 lanes.  The wide
// kernels give each wave 64 rows, in three phases: (A) one lane per row
// loads the row's coder state (coalesced) and, in the decoder, computes its
// quantile; (B) 16 passes of 4 rows, 16 lanes per row, compute the row's
// frequencies and the coded symbol's (cum, freq) (the decoder's symbol
// search), staged in LDS; (C) one lane per row runs the coder step and
// stores the state.  Results are those of the narrow kernels, row by row.
constexpr int WIDE_ROWS = 64;                      // rows per wave
constexpr int WIDE_PASSES = WIDE_ROWS / 4;         // 4 rows per pass
constexpr int64_t STEP_WIDE_MIN_ROWS = 1 << 18;   // below: the narrow kernels fill the GPU better

__global__ __launch_bounds__(256) void k_encode_step_wide(const int8_t *__restrict__ logits,
                                                          const uint64_t *__restrict__ lut,
                                                          const int64_t *__restrict__ symbols,
                                                          const int64_t *__restrict__ valid, int64_t t,
                                                          int64_t B, EncArrays st, uint32_t *__restrict__ words,
                                                          int64_t max_words) {
    __shared__ double s_lut[VOCAB];
    __shared__ uint32_t s_sym[4][WIDE_ROWS];   // the row's symbol, VOCAB when it takes no step
    __shared__ uint32_t s_cum[4][WIDE_ROWS], s_freq[4][WIDE_ROWS];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, u = lane & 15;
    const int64_t base = ((int64_t)blockIdx.x * 4 + wave) * WIDE_ROWS;
    const uint64_t lut_v = lut[threadIdx.x];   // 256 threads, VOCAB entries
    // (A) lane = row
    const int64_t b = base + lane;
    const bool in = b < B;
    int64_t vb = 0, sym = 0;
    int32_t stb = 0;
    EncState e{};
    if (in) {
        vb = valid[b];
        sym = symbols[b];
        stb = st.status[b];
        e = EncState{st.lower[b], st.range[b], st.inverted[b], st.first[b], st.write_pos[b]};
    }
    const bool live = in && t < vb && stb == 0;
    const bool bad = live && (sym < 0 || sym >= VOCAB);
    s_sym[wave][lane] = live && !bad ? (uint32_t)sym : (uint32_t)VOCAB;
    s_lut[VOCAB - 1 - threadIdx.x] = (double)lut_v;   // reversed, as load_lut_lds
    __syncthreads();
    // (B) 16 lanes per row, the next pass's logits loaded during this one
    v4i raw = global_logits16(logits, base + (lane >> 4), B, u);
#pragma unroll 1
    for (int p = 0; p < WIDE_PASSES; ++p) {
        const int r = 4 * p + (lane >> 4);
        const v4i next = p + 1 < WIDE_PASSES ? global_logits16(logits, base + r + 4, B, u) : v4i{0, 0, 0, 0};
        Freq16 fr;
        row_frequencies16(raw, s_lut, u, fr);
        const uint32_t s = s_sym[wave][r];
        if (s < (uint32_t)VOCAB && (int)(s >> 4) == u) {
            uint32_t cum, freq;
            freq16_at(fr, (int)(s & 15), cum, freq);
            s_cum[wave][r] = cum;
            s_freq[wave][r] = freq;
        }
        raw = next;
    }
    slot_sync();   // this wave's LDS writes above, its reads below
    // (C) lane = row; the stores as in k_encode_step
    if (bad) st.status[b] = SC_STATUS_BAD_TOKEN;
    if (!live || bad) return;
    const int full = enc_step(e, s_cum[wave][lane], s_freq[wave][lane], words + b * max_words, (int32_t)max_words);
    st.lower[b] = e.lower;
    st.range[b] = e.range;
    st.inverted[b] = e.inverted;
    st.first[b] = e.first;
    st.write_pos[b] = e.pos;
    st.status[b] = full ? SC_STATUS_CAPACITY : SC_STATUS_OK;
}

__global__ __launch_bounds__(256) void k_decode_step_wide(const int8_t *__restrict__ logits,
                                                          const uint64_t *__restrict__ lut,
                                                          const int64_t *__restrict__ valid, int64_t t,
                                                          int64_t B, DecArrays st,
                                                          const uint32_t *__restrict__ words,
                                                          int64_t *__restrict__ symbols_out) {
    __shared__ double s_lut[VOCAB];
    __shared__ uint32_t s_q[4][WIDE_ROWS];     // the row's quantile
    __shared__ uint32_t s_sym[4][WIDE_ROWS], s_cum[4][WIDE_ROWS], s_freq[4][WIDE_ROWS];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, u = lane & 15;
    const int64_t base = ((int64_t)blockIdx.x * 4 + wave) * WIDE_ROWS;
    const uint64_t lut_v = lut[threadIdx.x];   // 256 threads, VOCAB entries
    // (A) lane = row: the state, the word a renormalisation would shift in,
    // and the quantile (an inactive row's is unused)
    const int64_t b = base + lane;
    const bool in = b < B;
    int64_t vb = 0, rp = 0, endp = 0;
    int32_t stb = 0;
    uint64_t lower = 0, range = ~0ull, point = 0;
    if (in) {
        vb = valid[b];
        stb = st.status[b];
        rp = st.read_pos[b];
        endp = st.end_pos[b];
    }
    const bool active = in && t < vb && stb == 0;
    if (active) {
        lower = st.lower[b];
        range = st.range[b];
        point = st.point[b];
    }
    const uint32_t wnext = active && rp < endp ? words[rp] : 0u;
    const uint64_t scale = range >> 24;
    uint32_t q = 0;
    const bool ok = scale != 0 && dec_quantile(point - lower, scale, q);
    s_q[wave][lane] = q;
    s_lut[VOCAB - 1 - threadIdx.x] = (double)lut_v;   // reversed, as load_lut_lds
    __syncthreads();
    // (B) 16 lanes per row: frequencies and the symbol search
    v4i raw = global_logits16(logits, base + (lane >> 4), B, u);
#pragma unroll 1
    for (int p = 0; p < WIDE_PASSES; ++p) {
        const int r = 4 * p + (lane >> 4);
        const v4i next = p + 1 < WIDE_PASSES ? global_logits16(logits, base + r + 4, B, u) : v4i{0, 0, 0, 0};
        Freq16 fr;
        row_frequencies16(raw, s_lut, u, fr);
        uint32_t cum, freq;
        const int sym = dec_symbol16(fr, s_q[wave][r], lane, cum, freq);
        if (u == 0) {
            s_sym[wave][r] = (uint32_t)sym;
            s_cum[wave][r] = cum;
            s_freq[wave][r] = freq;
        }
        raw = next;
    }
    slot_sync();   // this wave's LDS writes above, its reads below
    // (C) lane = row; the stores as in k_decode_step
    if (!in) return;
    const bool step = active && ok;
    const uint32_t sym = s_sym[wave][lane];
    if (step) {
        lower += scale * s_cum[wave][lane];
        range = scale * s_freq[wave][lane];
        if (range < (1ull << 32)) {
            lower <<= 32;
            range <<= 32;
            point = (point << 32) | wnext;
            rp += 1;
        }
    }
    if (active) {
        st.lower[b] = lower;
        st.range[b] = range;
        st.point[b] = point;
        st.read_pos[b] = rp;
        st.status[b] = ok ? SC_STATUS_OK : SC_STATUS_INVALID_STREAM;
    }
    symbols_out[b] = step ? (int64_t)sym : (int64_t)VOCAB;
}

// ---- measurement: sustained int8 MFMA rate -------------------------------
// Every wave runs 8 independent accumulator chains of v_mfma_i32_32x32x32_i8
// on register operands (4 A and 4 B fragments of `ops`, rotated so that
// consecutive MFMAs see different data; no memory traffic in the loop): the
// int8 MFMA rate the chip sustains at its power limit for the given operand
// data, against which the codec kernels' MFMA rate is read.
__global__ __launch_bounds__(THREADS, 1) void k_mfma_burn(const v4i *__restrict__ ops, int32_t iters,
                                                          v16i *__restrict__ out) {
    const int l = threadIdx.x & 63;
    v4i a[4], b[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        a[j] = ops[j * 64 + l];
        b[j] = ops[256 + j * 64 + l];
    }
    v16i acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = v16i{};
    for (int32_t it = 0; it < iters; ++it) {
        static_for<4>([&](auto ic) {
            constexpr int i2 = decltype(ic)::value;
#pragma unroll
            for (int j = 0; j < 8; ++j)
                acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[j & 3], b[(j + i2) & 3], acc[j], 0, 0, 0);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[(j + 1) & 3], b[(j + 2 + i2) & 3], acc[j], 0, 0, 0);
        });
    }
    v16i s = acc[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) s += acc[j];
    out[(int64_t)blockIdx.x * THREADS + threadIdx.x] = s;
}

}  // namespace


// =========================================================================
// Host side
// =========================================================================

// Read-only after sc_model_create: every call keeps its mutable state in the
// caller's memory (workspace arguments), so calls on different streams or
// threads may share one model.
struct sc_model {
    int device = 0;
    int n_cu = 0;
    ModelDev dev{};
    std::vector<void *> allocs;
};

namespace {

thread_local std::string g_err = "";

int fail(int code, const std::string &msg) {
    g_err = msg;
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    return fail(SC_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

#define SC_HIP(call, what)                          \
    do {                                            \
        hipError_t e_ = (call);                     \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

int check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, what);
    return SC_OK;
}

struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) (void)hipSetDevice(dev);
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

template <class T>
int upload(sc_model *m, const std::vector<T> &host, const T **out) {
    void *p = nullptr;
    SC_HIP(hipMalloc(&p, host.size() * sizeof(T)), "hipMalloc");
    m->allocs.push_back(p);
    SC_HIP(hipMemcpy(p, host.data(), host.size() * sizeof(T), hipMemcpyHostToDevice), "hipMemcpy");
    *out = (const T *)p;
    return SC_OK;
}

// Pack W [n, k] into MFMA A-operand fragments: fragment (nt, kt) holds, for
// lane l, the 16 weights of row nt*32 + l%32 at stored k positions
// kt*32 + (l/32)*16 .. +16.  For layers fed by a hidden layer (perm_k) the
// stored position p of a 32-column block holds column 8*((p%16)/4) +
// 4*(p/16) + p%4, the order in which store_packed_perm lays out activations.
std::vector<int8_t> pack_weight(const int8_t *w, int n, int k, bool perm_k) {
    const int NT = n / 32, KT = k / 32;
    std::vector<int8_t> out((size_t)n * k, 0);
    for (int nt = 0; nt < NT; ++nt)
        for (int kt = 0; kt < KT; ++kt)
            for (int l = 0; l < 64; ++l)
                for (int b = 0; b < 16; ++b) {
                    const int p = (l >> 5) * 16 + b;   // stored position within the block
                    const int col = perm_k ? 8 * ((p & 15) >> 2) + 4 * (p >> 4) + (p & 3) : p;
                    out[(((size_t)nt * KT + kt) * 64 + l) * 16 + b] =
                        w[(size_t)(nt * 32 + (l & 31)) * k + kt * 32 + col];
                }
    return out;
}

// Generic path: W [n, k] into fragments of ceil(n/32) x ceil(k/32) tiles,
// zero beyond n and k, natural column order (fragment (nt, kt), lane l,
// byte b: row nt*32 + l%32, column kt*32 + (l/32)*16 + b).
std::vector<int8_t> pack_weight_padded(const int8_t *w, int n, int k) {
    const int NT = (n + 31) / 32, KT = (k + 31) / 32;
    std::vector<int8_t> out((size_t)NT * KT * 1024, 0);
    for (int nt = 0; nt < NT; ++nt)
        for (int kt = 0; kt < KT; ++kt)
            for (int l = 0; l < 64; ++l)
                for (int b = 0; b < 16; ++b) {
                    const int row = nt * 32 + (l & 31), col = kt * 32 + (l >> 5) * 16 + b;
                    if (row < n && col < k)
                        out[(((size_t)nt * KT + kt) * 64 + l) * 16 + b] = w[(size_t)row * k + col];
                }
    return out;
}

hipStream_t as_stream(void *s) { return (hipStream_t)s; }

// Per-step cost of a full-wave decode launch at rt = 1 .. DEC_RT_MAX row
// tiles per workgroup (MI355X, 512-token chunks, lossless model; us x 10 per
// step, one box; rt <= 4 runs the pipelined core with per-tensor
// requantisation, rt = 2 and 3 with the epilogue beside the next step's
// layer 0).  Per row tile rt = 4 and 3 are cheapest (34.8 and 35.6 us), rt = 1
// the dearest (62.1 us).
constexpr int DEC_STEP_COST[DEC_RT_MAX + 1] = {0, 621, 763, 1067, 1390, 2091};
// Per-step cost of a split decode launch (at most XCH_MAX_GROUPS groups of
// 32 chunks) with 4 and 8 workgroups per group, same unit.
constexpr int DEC_SPLIT_STEP_COST_P4 = 282, DEC_SPLIT_STEP_COST_P8 = 256;

// Split `units` row tiles per CU into launch sizes of least summed step cost
// (largest first, so that they take the longest chunks).
std::vector<int> dec_plan(int64_t units) {
    std::vector<int64_t> best((size_t)units + 1, INT64_MAX);
    std::vector<int> pick((size_t)units + 1, 0);
    best[0] = 0;
    for (int64_t u = 1; u <= units; ++u)
        for (int rt = 1; rt <= DEC_RT_MAX && rt <= u; ++rt)
            if (best[u - rt] + DEC_STEP_COST[rt] < best[u]) {
                best[u] = best[u - rt] + DEC_STEP_COST[rt];
                pick[u] = rt;
            }
    std::vector<int> plan;
    for (int64_t u = units; u > 0; u -= pick[u]) plan.push_back(pick[u]);
    std::sort(plan.rbegin(), plan.rend());
    return plan;
}


// Decode steps per launch.  Within one long launch the workgroups of an XCD
// drift apart (after ~1000 steps by more than the L2 can bridge, and each
// XCD then fetches the 6.2 MB model ~4 times per step from the memory side);
// launches of 256 steps start them together again, so that one fetch serves
// all of them (memory-side traffic of a c3 decode: 530 -> 215 GB).
constexpr int DEC_SEG_STEPS = 256;

// Decode state of sc_decompress_chunks_static: a file-scope device array
// (each GPU the library runs on holds its own copy until the process ends)
// with the coder state of up to SC_STATIC_DEC_MAX_CHUNKS chunks, then the
// launch plan's four length statistics, then the split decode's exchange
// buffers and flags for XCH_MAX_GROUPS groups.  Host code never passes `scratch`
// itself (in host code the name is a stand-in, not a device address): the
// address of the current device's copy comes from hipGetSymbolAddress.
constexpr int64_t SCRATCH_STATE_BYTES = ((int64_t)SC_STATIC_DEC_MAX_CHUNKS * sizeof(DecState) + 255) / 256 * 256;
constexpr int64_t SCRATCH_BYTES = SCRATCH_STATE_BYTES + 256 + xch_bytes(XCH_MAX_GROUPS);
__device__ __align__(256) uint8_t scratch[SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[MAX_DEVICES] = {};

// The current device's copy of `scratch` (resolved once per device, with
// that device current); null on failure, with the error recorded.
void *scratch_ptr(int device, int *rc) {
    *rc = SC_OK;
    if (device < 0 || device >= MAX_DEVICES) {
        *rc = SC_ERR_UNSUPPORTED;
        g_err = "device index beyond the library's static decode state table";
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        void *ptr = nullptr;
        hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            *rc = SC_ERR_HIP;
            g_err = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
            return nullptr;
        }
        g_scratch_ptr[device] = ptr;
    }
    return g_scratch_ptr[device];
}

}  // namespace

extern "C" {

const char *sc_last_error(void) { return g_err.c_str(); }

const char *sc_version(void) { return "sigcomp-hip 0.1 gfx950"; }

int sc_model_create(const int8_t *emb, int32_t emb_rows, int32_t emb_dim, int32_t window,
                    const sc_layer_desc *layers, int32_t n_layers, const int64_t *exp_lut,
                    int32_t device, sc_model **out) {
    if (!out || !emb || !layers || !exp_lut) return fail(SC_ERR_ARG, "null argument");
    *out = nullptr;
    // any architecture whose layers chain from window * emb_dim inputs to 256
    // logits; the bundled one (window 64, 257 x 128 embedding, 8192 -> 512,
    // 512 -> 512 ..., 512 -> 256) runs the specialised kernels, any other
    // the generic path (CORE_GENERIC)
    if (emb_rows != EMB_ROWS) return fail(SC_ERR_UNSUPPORTED, "the embedding needs 257 rows (256 symbols and SOS)");
    if (window < 1 || emb_dim < 1 || (int64_t)window * emb_dim > (int64_t(1) << 20))
        return fail(SC_ERR_UNSUPPORTED, "window and embedding width must be positive, product at most 2**20");
    if (n_layers < 1 || n_layers > MAX_LAYERS) return fail(SC_ERR_UNSUPPORTED, "kernels support 1..16 linear layers");
    bool special = emb_dim == EDIM && window == WIN && n_layers >= 2;
    for (int i = 0; i < n_layers; ++i) {
        const sc_layer_desc &L = layers[i];
        const int64_t want_k = i == 0 ? (int64_t)window * emb_dim : layers[i - 1].n;
        if (L.k != want_k || L.n < 1 || L.n > (1 << 16) || (i == n_layers - 1 && L.n != VOCAB))
            return fail(SC_ERR_UNSUPPORTED, "layers must chain from window * emb_dim inputs to 256 logits");
        special = special && L.k == (i == 0 ? K0 : HID) && L.n == (i == n_layers - 1 ? VOCAB : HID);
        if (!L.weight || !L.bias || !L.m0 || !L.shift) return fail(SC_ERR_ARG, "null layer array");
        for (int j = 0; j < L.n; ++j) {
            if (L.m0[j] < 0 || L.m0[j] > (int64_t(1) << 31))
                return fail(SC_ERR_ARG, "requant multiplier outside [0, 2**31]");
            if (L.shift[j] < 0 || L.shift[j] > 63) return fail(SC_ERR_ARG, "requant shift outside [0, 63]");
        }
    }
    for (int i = 0; i < VOCAB; ++i)
        if (exp_lut[i] < 0 || exp_lut[i] > (int64_t(1) << 38) || (i == 0 && exp_lut[0] <= 0))
            return fail(SC_ERR_ARG, "exp_lut must be nonnegative, at most 2**38, and start positive");
    int n_dev = 0;
    SC_HIP(hipGetDeviceCount(&n_dev), "hipGetDeviceCount");
    if (device < 0 || device >= n_dev) return fail(SC_ERR_ARG, "no such device");
    DeviceGuard guard(device);
    {
        // the static decode state of this device, resolved while it is current
        int src = SC_OK;
        if (!scratch_ptr(device, &src)) return src;
    }
    sc_model *m = new sc_model();
    m->device = device;
    hipDeviceProp_t prop;
    hipError_t pe = hipGetDeviceProperties(&prop, device);
    if (pe != hipSuccess) {
        delete m;
        return hip_fail(pe, "hipGetDeviceProperties");
    }
    m->n_cu = prop.multiProcessorCount;
    int rc = SC_OK;
    {
        std::vector<int8_t> e(emb, emb + (size_t)EMB_ROWS * emb_dim);
        rc = upload(m, e, &m->dev.emb);
    }
    m->dev.window = window;
    m->dev.emb_dim = emb_dim;
    if (rc == SC_OK) {
        std::vector<uint64_t> lut(exp_lut, exp_lut + VOCAB);
        rc = upload(m, lut, &m->dev.lut);
    }
    for (int i = 0; i < n_layers && rc == SC_OK; ++i) {
        const sc_layer_desc &L = layers[i];
        LayerDev &D = m->dev.layer[i];
        std::vector<int8_t> packed = special ? pack_weight(L.weight, L.n, L.k, i > 0) : pack_weight_padded(L.weight, L.n, L.k);
        const int8_t *wdev = nullptr;
        rc = upload(m, packed, &wdev);
        D.w = (const v4i *)wdev;
        if (rc) break;
        // Requant constants.  m0 == 2**31 is rewritten as (2**30, shift - 1)
        // (the same product); layers whose every m0 < 2**31 and shift >= 32
        // take the 32-bit high-product path (requant_u8_fast), with
        // shift - 32 stored.  Packed per 32-output n-tile: bias[32], m0[32],
        // shift[32] (bytes), and for those layers the pre-shift clamp
        // bounds hi[32]; PAR_DWORDS dwords per n-tile.
        std::vector<uint32_t> m0(L.n);
        std::vector<uint8_t> sh(L.n);
        bool fast = true;
        for (int j = 0; j < L.n; ++j) {
            int64_t mj = L.m0[j];
            int32_t sj = L.shift[j];
            if (mj == (int64_t(1) << 31) && sj >= 1) {
                mj >>= 1;
                sj -= 1;
            }
            m0[j] = (uint32_t)mj;
            sh[j] = (uint8_t)sj;
            fast = fast && mj < (int64_t(1) << 31) && sj >= 32;
        }
        fast = fast && special;   // the generic path requantises with the full 64-bit form
        if (fast)
            for (int j = 0; j < L.n; ++j) sh[j] = (uint8_t)(sh[j] - 32);
        D.fast = fast ? 1 : 0;
        // per-tensor constants: one m0 and shift for the whole layer
        bool uni = fast;
        for (int j = 1; j < L.n && uni; ++j) uni = m0[j] == m0[0] && sh[j] == sh[0];
        D.uni = uni ? 1 : 0;
        D.um0 = uni ? (int32_t)m0[0] : 0;
        D.ush = uni ? sh[0] : 0;
        D.uhi = uni ? (int32_t)std::min<int64_t>((int64_t(128) << sh[0]) - 1, INT32_MAX) : 0;
        D.ulo = uni ? (int32_t)std::max<int64_t>(-(int64_t(128) << sh[0]), INT32_MIN) : 0;
        // (padded n-tiles of the generic path: bias, m0 and shift 0)
        const int n_tiles = (L.n + 31) / 32;
        std::vector<uint32_t> par((size_t)n_tiles * PAR_DWORDS, 0u);
        for (int nt = 0; nt < n_tiles; ++nt) {
            uint32_t *blk = par.data() + (size_t)nt * PAR_DWORDS;
            for (int x = 0; x < 32 && nt * 32 + x < L.n; ++x) {
                const int j = nt * 32 + x;
                blk[x] = (uint32_t)L.bias[j];
                blk[32 + x] = m0[j];
                blk[64 + x / 4] |= (uint32_t)sh[j] << (8 * (x % 4));
                if (fast) blk[72 + x] = (uint32_t)std::min<int64_t>((int64_t(128) << sh[j]) - 1, INT32_MAX);
            }
        }
        rc = upload(m, par, &D.par);
        if (rc) break;
        D.n = L.n;
        D.kt = (L.k + 31) / 32;
        D.relu = L.relu ? 1 : 0;
        D.bytes = (int32_t)packed.size();
    }
    m->dev.n_layers = n_layers;
    // SC_HIP_PLAIN_CORE=1 at model creation selects the plain core (testing)
    const char *plain = getenv("SC_HIP_PLAIN_CORE");
    bool pipe = !(plain && plain[0] == '1'), uni = true;
    for (int i = 0; i < n_layers; ++i) {
        if (!m->dev.layer[i].fast || m->dev.layer[i].relu != (i < n_layers - 1 ? 1 : 0)) pipe = false;
        if (!m->dev.layer[i].uni) uni = false;
    }
    m->dev.pipe = !special ? CORE_GENERIC : !pipe ? CORE_PLAIN : uni ? CORE_PIPE_UNI : CORE_PIPE;
    if (rc != SC_OK) {
        sc_model_destroy(m);
        return rc;
    }
    *out = m;
    return SC_OK;
}

int sc_model_destroy(sc_model *m) {
    if (!m) return SC_OK;
    DeviceGuard guard(m->device);
    for (void *p : m->allocs) (void)hipFree(p);
    delete m;
    return SC_OK;
}

const uint64_t *sc_model_lut(const sc_model *m) { return m ? m->dev.lut : nullptr; }

int sc_model_core(const sc_model *m) { return m ? m->dev.pipe : 0; }

static int mlp_context_launch(const sc_model *m, const int64_t *ctx, int64_t rows, int8_t *logits,
                              int32_t *cdf, int32_t *status, void *stream, int mode) {
    if (!m || rows < 0 || !status) return fail(SC_ERR_ARG, "bad argument");
    if (rows == 0) return SC_OK;
    if (!ctx || (mode == OUT_LOGITS && !logits) || (mode == OUT_CDF32 && !cdf))
        return fail(SC_ERR_ARG, "null device pointer");
    DeviceGuard guard(m->device);
    if (m->dev.pipe == CORE_GENERIC) {
        std::string err;
        const int rc = gen_mlp_forward(m->dev, ctx, rows, mode == OUT_LOGITS ? logits : nullptr,
                                       mode == OUT_CDF32 ? cdf : nullptr, status, as_stream(stream), err);
        return rc ? fail(rc, err) : SC_OK;
    }
    const int64_t tiles = (rows + R_TILE - 1) / R_TILE;
    const int grid = (int)std::min<int64_t>(tiles, m->n_cu);
    if (mode == OUT_LOGITS) launch_mlp_context<OUT_LOGITS>(m->dev, grid, as_stream(stream), ctx, rows, logits, cdf, status);
    else launch_mlp_context<OUT_CDF32>(m->dev, grid, as_stream(stream), ctx, rows, logits, cdf, status);
    return check_launch("k_mlp_context");
}

int sc_mlp_forward(const sc_model *m, const int64_t *ctx, int64_t rows, int8_t *logits, int32_t *status,
                   void *stream) {
    return mlp_context_launch(m, ctx, rows, logits, nullptr, status, stream, OUT_LOGITS);
}

int sc_mlp_forward_cdf(const sc_model *m, const int64_t *ctx, int64_t rows, int32_t *cdf, int32_t *status,
                       void *stream) {
    return mlp_context_launch(m, ctx, rows, nullptr, cdf, status, stream, OUT_CDF32);
}

int sc_logits_to_cdf(const int8_t *logits, int64_t rows, const uint64_t *lut, int64_t *cdf, void *stream) {
    if (rows < 0) return fail(SC_ERR_ARG, "rows must be nonnegative");
    if (rows == 0) return SC_OK;
    if (!logits || !lut || !cdf) return fail(SC_ERR_ARG, "null device pointer");
    hipLaunchKernelGGL(k_logits_to_cdf, dim3((unsigned)((rows + 15) / 16)), dim3(256), 0, as_stream(stream),
                       logits, rows, lut, cdf);
    return check_launch("k_logits_to_cdf");
}

// The wide step kernels for batches of at least STEP_WIDE_MIN_ROWS streams;
// SC_HIP_STEP_WIDE = "0" / "1" forces the narrow / wide kernels (comparisons
// and tests of both).
static bool step_wide(int64_t B) {
    const char *env = getenv("SC_HIP_STEP_WIDE");
    if (env && (env[0] == '0' || env[0] == '1') && env[1] == 0) return env[0] == '1';
    return B >= STEP_WIDE_MIN_ROWS;
}

static bool enc_ok(const sc_encoder_state *s) {
    return s && s->lower && s->range && s->inverted && s->first && s->write_pos && s->status;
}

int sc_encode_step(const int8_t *logits, const uint64_t *lut, const int64_t *symbols, const int64_t *valid_lens,
                   int64_t t, int64_t B, const sc_encoder_state *state, uint32_t *words, int64_t max_words,
                   void *stream) {
    if (B < 0 || t < 0 || max_words < 2 || max_words > INT32_MAX) return fail(SC_ERR_ARG, "bad sizes");
    if (B == 0) return SC_OK;
    if (!logits || !lut || !symbols || !valid_lens || !words || !enc_ok(state))
        return fail(SC_ERR_ARG, "null device pointer");
    EncArrays a{state->lower, state->range, state->inverted, state->first, state->write_pos, state->status};
    if (step_wide(B)) {
        hipLaunchKernelGGL(k_encode_step_wide, dim3((unsigned)((B + 4 * WIDE_ROWS - 1) / (4 * WIDE_ROWS))), dim3(256),
                           0, as_stream(stream), logits, lut, symbols, valid_lens, t, B, a, words, max_words);
        return check_launch("k_encode_step_wide");
    }
    hipLaunchKernelGGL(k_encode_step, dim3((unsigned)((B + 15) / 16)), dim3(256), 0, as_stream(stream), logits, lut,
                       symbols, valid_lens, t, B, a, words, max_words);
    return check_launch("k_encode_step");
}

int sc_encode_seal(int64_t B, const sc_encoder_state *state, uint32_t *words, int64_t max_words, void *stream) {
    if (B < 0 || max_words < 2 || max_words > INT32_MAX) return fail(SC_ERR_ARG, "bad sizes");
    if (B == 0) return SC_OK;
    if (!words || !enc_ok(state)) return fail(SC_ERR_ARG, "null device pointer");
    EncArrays a{state->lower, state->range, state->inverted, state->first, state->write_pos, state->status};
    hipLaunchKernelGGL(k_encode_seal, dim3((unsigned)((B + 255) / 256)), dim3(256), 0, as_stream(stream), B, a,
                       words, max_words);
    return check_launch("k_encode_seal");
}

int sc_decode_step(const int8_t *logits, const uint64_t *lut, const int64_t *valid_lens, int64_t t, int64_t B,
                   const sc_decoder_state *state, const uint32_t *words, int64_t *symbols_out, void *stream) {
    if (B < 0 || t < 0) return fail(SC_ERR_ARG, "bad sizes");
    if (B == 0) return SC_OK;
    if (!logits || !lut || !valid_lens || !symbols_out || !state || !state->lower || !state->range ||
        !state->point || !state->read_pos || !state->end_pos || !state->status || !words)
        return fail(SC_ERR_ARG, "null device pointer");
    DecArrays a{state->lower, state->range, state->point, state->read_pos, state->end_pos, state->status};
    if (step_wide(B)) {
        hipLaunchKernelGGL(k_decode_step_wide, dim3((unsigned)((B + 4 * WIDE_ROWS - 1) / (4 * WIDE_ROWS))), dim3(256),
                           0, as_stream(stream), logits, lut, valid_lens, t, B, a, words, symbols_out);
        return check_launch("k_decode_step_wide");
    }
    hipLaunchKernelGGL(k_decode_step, dim3((unsigned)((B + 15) / 16)), dim3(256), 0, as_stream(stream), logits, lut,
                       valid_lens, t, B, a, words, symbols_out);
    return check_launch("k_decode_step");
}

// Workspace: tile_start (int32 [n_chunks + 1]), the tile descriptors (int4
// [at most n_tokens / 128 + n_chunks tiles]), then the (cum, freq) pairs
// (8 bytes per token), each part 256-byte aligned.
static int64_t tile_start_bytes(int64_t n_chunks) { return ((n_chunks + 1) * 4 + 255) / 256 * 256; }
static int64_t tile_desc_bytes(int64_t n_tokens, int64_t n_chunks) {
    return ((n_tokens / R_TILE + n_chunks) * 16 + 255) / 256 * 256;
}

int64_t sc_compress_workspace_bytes(int64_t n_tokens, int64_t n_chunks) {
    if (n_tokens < 0 || n_chunks < 0) return -1;
    return tile_start_bytes(n_chunks) + tile_desc_bytes(n_tokens, n_chunks) + ((n_tokens * 8 + 255) / 256) * 256;
}

int sc_compress_chunks(const sc_model *m, const uint8_t *tokens, const int64_t *tok_off, const int32_t *lengths,
                       int64_t n_chunks, int64_t n_tokens, uint32_t *words, const int64_t *word_off,
                       const int32_t *word_cap, int32_t *word_cnt, int32_t *status, void *workspace,
                       int64_t workspace_bytes, void *stream) {
    if (!m || n_chunks < 0 || n_tokens < 0) return fail(SC_ERR_ARG, "bad argument");
    if (n_chunks == 0) return SC_OK;
    if (!tokens || !tok_off || !lengths || !words || !word_off || !word_cap || !word_cnt || !status || !workspace)
        return fail(SC_ERR_ARG, "null device pointer");
    if (workspace_bytes < sc_compress_workspace_bytes(n_tokens, n_chunks))
        return fail(SC_ERR_ARG, "workspace too small");
    DeviceGuard guard(m->device);
    if (n_tokens / R_TILE + n_chunks >= (int64_t(1) << 31))
        return fail(SC_ERR_UNSUPPORTED, "more than 2**31 tiles");
    const int64_t max_tiles = n_tokens / R_TILE + n_chunks;   // tiles of disjoint chunks of n_tokens tokens
    int32_t *tile_start = (int32_t *)workspace;
    int4 *desc = (int4 *)((char *)workspace + tile_start_bytes(n_chunks));
    uint2 *pairs = (uint2 *)((char *)desc + tile_desc_bytes(n_tokens, n_chunks));
    hipStream_t s = as_stream(stream);
    hipLaunchKernelGGL(k_tile_scan, dim3(1), dim3(SCAN_THREADS), 0, s, lengths, n_chunks, tile_start);
    int rc = check_launch("k_tile_scan");
    if (rc) return rc;
    hipLaunchKernelGGL(k_tile_table, dim3((unsigned)((n_chunks + 255) / 256)), dim3(256), 0, s, tok_off, lengths,
                       n_chunks, tile_start, desc, max_tiles);
    rc = check_launch("k_tile_table");
    if (rc) return rc;
    if (m->dev.pipe == CORE_GENERIC) {
        std::string err;
        rc = gen_compress(m->dev, tokens, tile_start, n_chunks, desc, max_tiles, pairs, s, err);
        if (rc) return fail(rc, err);
    } else {
        // one workgroup per CU (or per tile when there are fewer tiles)
        const int grid = (int)std::max<int64_t>(1, std::min<int64_t>(max_tiles, m->n_cu));
        launch_compress_mlp(m->dev, grid, s, tokens, n_chunks, tile_start, desc, max_tiles, pairs);
        rc = check_launch("k_compress_mlp");
        if (rc) return rc;
    }
    hipLaunchKernelGGL(k_encode_pairs, dim3((unsigned)((n_chunks + 255) / 256)), dim3(256), 0, s, pairs, tok_off,
                       lengths, n_chunks, words, word_off, word_cap, word_cnt, status);
    return check_launch("k_encode_pairs");
}

int sc_gather_words(const uint32_t *words, const int64_t *word_off, const int32_t *word_cnt, int64_t n_chunks,
                    uint32_t *out, const int64_t *out_off, void *stream) {
    if (n_chunks < 0) return fail(SC_ERR_ARG, "bad argument");
    if (n_chunks == 0) return SC_OK;
    if (!words || !word_off || !word_cnt || !out || !out_off) return fail(SC_ERR_ARG, "null device pointer");
    hipLaunchKernelGGL(k_gather_words, dim3((unsigned)((n_chunks + WAVES - 1) / WAVES)), dim3(THREADS), 0,
                       as_stream(stream), words, word_off, word_cnt, n_chunks, out, out_off);
    return check_launch("k_gather_words");
}

int sc_mfma_burn_i8(const int8_t *ops, int32_t iters, int32_t n_groups, int32_t *out, void *stream) {
    if (iters < 0 || n_groups <= 0 || !ops || !out) return fail(SC_ERR_ARG, "bad argument");
    hipLaunchKernelGGL(k_mfma_burn, dim3((unsigned)n_groups), dim3(THREADS), 0, as_stream(stream),
                       (const v4i *)ops, iters, (v16i *)out);
    return check_launch("k_mfma_burn");
}

// Workspace of sc_decompress_chunks: the coder state of every chunk between
// step segments (DecState, 40 bytes each), then the four length statistics
// of the launch plan, each part 256-byte aligned.
static int64_t dec_state_bytes(int64_t n_chunks) {
    return (n_chunks * (int64_t)sizeof(DecState) + 255) / 256 * 256;
}

// then the exchange buffers of a split launch
static int64_t dec_xch_groups(int64_t n_chunks) { return std::min<int64_t>((n_chunks + 31) / 32, XCH_MAX_GROUPS); }

int64_t sc_decompress_workspace_bytes(int64_t n_chunks) {
    if (n_chunks < 0) return -1;
    return dec_state_bytes(n_chunks) + 256 + xch_bytes(dec_xch_groups(n_chunks));
}

// The launch plan's length statistics on the host (k_dec_lengths' rule):
// [0] longest chunk, [1] most steps of a pair (row g0+G-left+i followed by
// chunk g0+G+left-1-i, which starts one step after the first ends), [2]
// longest chunk of the last full-wave launch (g0 .. g0+G-1), [3] longest
// leftover chunk; negative lengths count as 0.
static void host_len_stats(const int32_t *len, int64_t n, int64_t g0, int64_t G, int64_t left, int32_t out[4]) {
    auto at = [&](int64_t i) { return std::max(len[i], 0); };
    out[0] = out[1] = out[2] = out[3] = 0;
    for (int64_t i = 0; i < n; ++i) out[0] = std::max(out[0], at(i));
    for (int64_t i = g0; i < g0 + G && i < n; ++i) out[2] = std::max(out[2], at(i));
    for (int64_t i = g0 + G; i < g0 + G + left && i < n; ++i) out[3] = std::max(out[3], at(i));
    for (int64_t i = 0; i < left; ++i) {
        const int32_t l1 = at(g0 + G - left + i);
        out[1] = std::max(out[1], l1 + at(g0 + G + left - 1 - i) + (l1 > 0 ? 1 : 0));
    }
}

// The decode of sc_decompress_chunks with its buffers given: `state` holds
// DecState for n_chunks rows, `stat_dev` 4 int32 (used only when
// lengths_host is NULL), `xch` xch_bytes(xch_groups) bytes of exchange
// buffers for a split launch of at most xch_groups groups.
static int decompress_run(const sc_model *m, const uint32_t *words, const int64_t *word_off, const int32_t *word_cnt,
                          const int32_t *lengths, int64_t n_chunks, uint8_t *tokens, const int64_t *tok_off,
                          int32_t *status, const int32_t *lengths_host, DecState *state, int32_t *stat_dev,
                          uint8_t *xch, int64_t xch_groups, int32_t options, hipStream_t s) {
    // Under graph capture nothing may wait for the device: the launch plan
    // then needs the caller's host copy of the lengths, checked before
    // anything is enqueued so that a refused call leaves the capture valid.
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    SC_HIP(hipStreamIsCapturing(s, &capture), "hipStreamIsCapturing");
    if (capture != hipStreamCaptureStatusNone && !lengths_host)
        return fail(SC_ERR_ARG, "lengths_host required on a stream under graph capture (the launch plan "
                                "would read the lengths back from the device)");
    if (m->dev.pipe == CORE_GENERIC) {
        // step by step over all chunks: the longest chunk bounds the steps
        int32_t st4[4];
        if (lengths_host) {
            host_len_stats(lengths_host, n_chunks, 0, 0, 0, st4);
        } else {
            hipLaunchKernelGGL(k_dec_lengths, dim3(1), dim3(1024), 0, s, lengths, n_chunks, (int64_t)0, (int64_t)0,
                               (int64_t)0, stat_dev);
            int rc = check_launch("k_dec_lengths");
            if (rc) return rc;
            SC_HIP(hipMemcpyAsync(st4, stat_dev, sizeof(st4), hipMemcpyDeviceToHost, s), "hipMemcpyAsync");
            SC_HIP(hipStreamSynchronize(s), "hipStreamSynchronize");
        }
        std::string err;
        const int rc = gen_decompress(m->dev, words, word_off, word_cnt, lengths, n_chunks, tokens, tok_off, status,
                                      state, st4[0], s, err);
        return rc ? fail(rc, err) : SC_OK;
    }
    // Launch plan.  A workgroup owns 32*rt consecutive chunks for the whole
    // decode, one workgroup per CU, and every launch but the last is one
    // full wave of n_cu workgroups.  The chunks of the full waves make
    // `units` row tiles per CU; with the pipelined core (per-tensor
    // constants: every kernel runs it) they are split into
    // launches by dec_plan (measured step costs), otherwise taken greedily
    // at the largest rt.  The chunks left over (fewer than 32*n_cu) either
    // follow the last rows of the last full-wave launch in the same rows
    // (pairing, pipelined core) or go to a final launch of rt = 1
    // workgroups, whichever the step costs say is cheaper.  With chunks
    // sorted longest first the largest tiles get the longest chunks and the
    // leftover chunks are the shortest ones.
    const int64_t cu = m->n_cu;
    const int64_t units = n_chunks / (32 * cu);
    std::vector<int> plan;
    const char *plan_env = getenv("SC_HIP_DEC_PLAN");   // "greedy": largest rt first (comparisons)
    const char *rt_env = getenv("SC_HIP_DEC_RT");       // n: launches of at most n row tiles (comparisons)
    const int rt_cap = rt_env ? std::min(std::max(atoi(rt_env), 1), DEC_RT_MAX) : 0;
    if (m->dev.pipe == CORE_PIPE_UNI && !rt_cap && !(plan_env && std::strcmp(plan_env, "greedy") == 0)) {
        plan = dec_plan(units);
    } else {
        const int cap = rt_cap ? rt_cap : DEC_RT_MAX;
        for (int64_t u = units; u > 0; u -= std::min<int64_t>(u, cap)) plan.push_back((int)std::min<int64_t>(u, cap));
    }
    const int64_t left = n_chunks - units * 32 * cu;
    const int rt_last = plan.empty() ? 0 : plan.back();
    const int64_t g_count = (int64_t)rt_last * 32 * cu, g0 = units * 32 * cu - g_count;
    const char *pair_env = getenv("SC_HIP_DEC_PAIR");   // "0": never pair (comparisons)
    const bool can_pair = m->dev.pipe == CORE_PIPE_UNI && rt_last >= 1 && rt_last <= 4 && left > 0 && left <= g_count &&
                          !(pair_env && std::strcmp(pair_env, "0") == 0);
    // step segments (SC_HIP_DEC_SEG overrides the length, 0 = one launch per
    // group): the longest row bounds the segments of every group
    const char *seg_env = getenv("SC_HIP_DEC_SEG");
    int64_t seg = seg_env ? std::max(0, atoi(seg_env)) : DEC_SEG_STEPS;
    seg = (seg + WIN - 1) / WIN * WIN;   // segments end where the token ring is flushed
    int32_t st4[4];
    if (lengths_host) {
        // the caller's host copy of the lengths: no wait for the device
        host_len_stats(lengths_host, n_chunks, g0, g_count, can_pair ? left : 0, st4);
    } else {
        hipLaunchKernelGGL(k_dec_lengths, dim3(1), dim3(1024), 0, s, lengths, n_chunks, g0, g_count,
                           can_pair ? left : (int64_t)0, stat_dev);
        int rc = check_launch("k_dec_lengths");
        if (rc) return rc;
        SC_HIP(hipMemcpyAsync(st4, stat_dev, sizeof(st4), hipMemcpyDeviceToHost, s), "hipMemcpyAsync");
        SC_HIP(hipStreamSynchronize(s), "hipStreamSynchronize");
    }
    const int32_t len_max = st4[0], pair_max = st4[1], group_max = st4[2], left_max = st4[3];
    // pairing lengthens the last full-wave launch by the steps its longest
    // pair exceeds its longest chunk; the rt = 1 launch costs the longest
    // leftover chunk's steps
    // the launch of rt = 1 workgroups that takes what the full waves leave
    // runs split when its 32-chunk groups fit: 8 workgroups per group when
    // the CUs hold them, else 4 (SC_HIP_DEC_SPLIT=0: never, 4 or 8: only
    // that split, for comparisons)
    const char *split_env = getenv("SC_HIP_DEC_SPLIT");
    const int split_force = split_env ? atoi(split_env) : -1;
    // (a stream under graph capture gets the unsplit launches: the split
    // one is a cooperative launch)
    const bool split_ok = m->dev.pipe == CORE_PIPE_UNI && xch && split_force != 0 &&
                          !(options & SC_DEC_OPT_NO_SPLIT) && capture == hipStreamCaptureStatusNone;
    // polls before a wait for the peers gives up (SC_HIP_DEC_SPIN: a lower
    // limit, to test the timeout path)
    const char *spin_env = getenv("SC_HIP_DEC_SPIN");
    const int32_t spin_max = spin_env ? std::min(std::max(atoi(spin_env), 0), SYNC_SPIN_MAX) : SYNC_SPIN_MAX;
    auto split_p = [&](int64_t n) {   // workgroups per group of a split launch of n chunks (0: unsplit)
        const int64_t groups = (n + 31) / 32;
        if (!split_ok || groups > std::min<int64_t>(xch_groups, XCH_MAX_GROUPS)) return 0;
        if (split_force != 4 && groups * 8 <= cu) return 8;
        if (split_force != 8 && groups * 4 <= cu) return 4;
        return 0;
    };
    const int p_left = split_p(left);
    const int left_cost = p_left == 8 ? DEC_SPLIT_STEP_COST_P8 : p_left == 4 ? DEC_SPLIT_STEP_COST_P4 : DEC_STEP_COST[1];
    const bool pair = can_pair && (int64_t)std::max(0, pair_max - group_max) * DEC_STEP_COST[rt_last] <
                                      (int64_t)left_max * left_cost;
    const int64_t maxlen = std::max(len_max, pair ? pair_max : 0);
    if (const char *log = getenv("SC_HIP_DEC_LOG"); log && std::strcmp(log, "1") == 0) {
        std::string rts;
        for (int rt : plan) rts += (rts.empty() ? "" : ",") + std::to_string(rt);
        const int64_t rest_last = units == 0 ? n_chunks : pair ? 0 : left;
        const int pl = rest_last ? split_p(rest_last) : 0;
        std::fprintf(stderr, "sc_decompress_chunks: chunks %lld cu %lld plan [%s] leftover %lld %s steps %lld seg %lld\n",
                     (long long)n_chunks, (long long)cu, rts.c_str(), (long long)left,
                     left == 0 ? "none" : pair ? "paired" : pl == 8 ? "split launch p8" : pl == 4 ? "split launch p4" : "launch",
                     (long long)maxlen, (long long)seg);
    }
    int64_t start = 0;
    size_t step = 0;
    while (start < n_chunks) {
        const int64_t rest = n_chunks - start;
        int64_t rt, count, n_second = 0;
        unsigned grid;
        int split = 0;   // workgroups per group of a split launch
        if (step < plan.size()) {
            rt = plan[step++];
            count = cu * 32 * rt;
            grid = (unsigned)cu;
            if (pair && step == plan.size()) n_second = left;
        } else {
            rt = 1;
            count = rest;
            grid = (unsigned)((rest + 31) / 32);
            split = split_p(rest);
        }
        const uint32_t *wds = words;
        const int64_t *woff = word_off + start, *toff = tok_off + start;
        const int32_t *wcnt = word_cnt + start, *len = lengths + start;
        int32_t *st = status + start;
        DecState *ds = seg > 0 ? state + start : nullptr;
        if (split) {
            // step flags of the grid's groups start at zero (they then hold
            // the last step each workgroup published, across segments)
            hipLaunchKernelGGL(k_zero_i32, dim3(1), dim3(256), 0, s, (int32_t *)(xch + grid * (int64_t)XCH_GROUP),
                               (int64_t)grid * split);
            int rc = check_launch("k_zero_i32");
            if (rc) return rc;
        }
        for (int64_t tb = 0; tb == 0 || (seg > 0 && tb < maxlen); tb += (seg > 0 ? seg : INT32_MAX)) {
            const int32_t t0 = (int32_t)tb, t1 = seg > 0 ? (int32_t)std::min<int64_t>(INT32_MAX, tb + seg) : INT32_MAX;
            if (split) {
                const hipError_t e = launch_decompress_split(m->dev, split, grid, s, wds, woff, wcnt, len, count, tokens,
                                                             toff, st, ds, t0, t1, xch, spin_max);
                if (e == hipSuccess) {
                    int rc = check_launch("k_decompress (split)");
                    if (rc) return rc;
                    continue;
                }
                // a device that cannot hold the whole grid at once: the
                // decode runs unsplit (found at the first segment; a later
                // failure is an error)
                (void)hipGetLastError();
                if (tb > 0 || e != hipErrorCooperativeLaunchTooLarge) return hip_fail(e, "k_decompress (split)");
                split = 0;
            }
            switch (rt) {
#define SC_DEC_CASE(N)                                                                                        \
    case N:                                                                                                   \
        launch_decompress<N>(m->dev, grid, s, wds, woff, wcnt, len, count, tokens, toff, st, ds, t0, t1, n_second);       \
        break;
                SC_DEC_CASE(1)
                SC_DEC_CASE(2)
                SC_DEC_CASE(3)
                SC_DEC_CASE(4)
                SC_DEC_CASE(5)
#undef SC_DEC_CASE
            }
            int rc = check_launch("k_decompress");
            if (rc) return rc;
        }
        start += count + n_second;
    }
    return SC_OK;
}

int sc_decompress_chunks(const sc_model *m, const uint32_t *words, const int64_t *word_off, const int32_t *word_cnt,
                         const int32_t *lengths, int64_t n_chunks, uint8_t *tokens, const int64_t *tok_off,
                         int32_t *status, const int32_t *lengths_host, void *workspace, int64_t workspace_bytes,
                         void *stream) {
    return sc_decompress_chunks_opts(m, words, word_off, word_cnt, lengths, n_chunks, tokens, tok_off, status,
                                     lengths_host, workspace, workspace_bytes, 0, stream);
}

int sc_decompress_chunks_opts(const sc_model *m, const uint32_t *words, const int64_t *word_off,
                              const int32_t *word_cnt, const int32_t *lengths, int64_t n_chunks, uint8_t *tokens,
                              const int64_t *tok_off, int32_t *status, const int32_t *lengths_host, void *workspace,
                              int64_t workspace_bytes, int32_t options, void *stream) {
    if (!m || n_chunks < 0 || (options & ~SC_DEC_OPT_NO_SPLIT)) return fail(SC_ERR_ARG, "bad argument");
    if (n_chunks == 0) return SC_OK;
    if (!words || !word_off || !word_cnt || !lengths || !tokens || !tok_off || !status || !workspace)
        return fail(SC_ERR_ARG, "null device pointer");
    if (workspace_bytes < sc_decompress_workspace_bytes(n_chunks)) return fail(SC_ERR_ARG, "workspace too small");
    DeviceGuard guard(m->device);
    DecState *state = (DecState *)workspace;
    int32_t *stat_dev = (int32_t *)((char *)workspace + dec_state_bytes(n_chunks));
    uint8_t *xch = (uint8_t *)workspace + dec_state_bytes(n_chunks) + 256;
    return decompress_run(m, words, word_off, word_cnt, lengths, n_chunks, tokens, tok_off, status, lengths_host,
                          state, stat_dev, xch, dec_xch_groups(n_chunks), options, as_stream(stream));
}

int sc_decompress_chunks_static(const sc_model *m, const uint32_t *words, const int64_t *word_off,
                                const int32_t *word_cnt, const int32_t *lengths, int64_t n_chunks, uint8_t *tokens,
                                const int64_t *tok_off, int32_t *status, const int32_t *lengths_host,
                                void *stream) {
    if (!m || n_chunks < 0) return fail(SC_ERR_ARG, "bad argument");
    if (n_chunks > SC_STATIC_DEC_MAX_CHUNKS)
        return fail(SC_ERR_ARG, "sc_decompress_chunks_static decodes at most SC_STATIC_DEC_MAX_CHUNKS (" +
                                    std::to_string(SC_STATIC_DEC_MAX_CHUNKS) + ") chunks per call; got " +
                                    std::to_string(n_chunks));
    if (n_chunks == 0) return SC_OK;
    if (!words || !word_off || !word_cnt || !lengths || !tokens || !tok_off || !status)
        return fail(SC_ERR_ARG, "null device pointer");
    if (m->dev.pipe == CORE_GENERIC)
        return fail(SC_ERR_UNSUPPORTED, "sc_decompress_chunks_static runs the bundled architecture's kernels only "
                                        "(the generic path allocates scratch memory)");
    DeviceGuard guard(m->device);
    int rc = SC_OK;
    void *base = scratch_ptr(m->device, &rc);
    if (!base) return rc;
    // every DecState is written by a segment before a later one reads it and
    // the statistics are written before they are read; a split launch clears
    // its step flags itself (a kernel, no memset)
    DecState *state = (DecState *)base;
    int32_t *stat_dev = (int32_t *)((char *)base + SCRATCH_STATE_BYTES);
    uint8_t *xch = (uint8_t *)base + SCRATCH_STATE_BYTES + 256;
    return decompress_run(m, words, word_off, word_cnt, lengths, n_chunks, tokens, tok_off, status, lengths_host,
                          state, stat_dev, xch, XCH_MAX_GROUPS, 0, as_stream(stream));
}

}  // extern "C"
