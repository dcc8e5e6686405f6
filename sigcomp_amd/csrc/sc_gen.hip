// sc_gen.hip -- the codec for model architectures other than the bundled one
// (any window, embedding width, hidden width and layer count; the last layer
// gives 256 logits): the reference's GPU codec runs any shapes
// (quant_mlp_export.py:21-101,215-269), and its archives name their model
// dims (main.py:1086-1094).
//
// The specialised kernels keep everything of an evaluation on chip; here
// each stage is its own launch over a batch of rows in device memory:
//   k_gen_embed   token windows -> layer-0 input rows (zero padded to a
//                 multiple of 32 columns)
//   k_gen_linear  one quantised linear layer: v_mfma_i32_32x32x32_i8 over
//                 weights packed in fragment order (zero padded to 32 x 32
//                 tiles) and the rows from memory, then the per-channel
//                 requantisation of cpu_int_kernels.py:5-14 (64-bit form)
//   k_gen_pairs   logits -> (cumulative frequency, frequency) of each coded
//                 token, then the existing range encoder (k_encode_pairs)
//   k_gen_dec_*   one decoder step per chunk from its logits, the coder state
//                 in the caller's workspace
// Padded weight rows and columns are zero, so padded features requantise to
// zero and add nothing to the next layer.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>

#include "sc_gen.h"

namespace sc {
namespace {

// ---- embedding gather ----------------------------------------------------

enum GenSource { SRC_CTX = 0, SRC_TILES = 1, SRC_DECODE = 2 };

// Row r of the batch, window position p: the token, or SOS before the
// sequence start.  SRC_CTX: ctx[r * W + p] (int64, checked); SRC_TILES: row
// r is step t0 + i of the chunk whose step t0 is token `base` (tile
// descriptor r / 128 + tile0, i = r % 128), its context the tokens before it
// in the token array; SRC_DECODE: row r is chunk r at step t, its context
// the tokens it has decoded.
struct GenRows {
    int src;
    const int64_t *ctx;                 // SRC_CTX
    const uint8_t *tokens;              // SRC_TILES / SRC_DECODE
    const int4 *desc;                   // SRC_TILES
    int64_t tile0;
    const int32_t *tile_count;          // SRC_TILES: number of real tiles (device)
    const int64_t *tok_off;             // SRC_DECODE
    const int32_t *lengths;             // SRC_DECODE
    int32_t t;                          // SRC_DECODE
};

__device__ __forceinline__ int gen_token(const GenRows &g, int64_t r, int p, int W, bool &valid_row) {
    if (g.src == SRC_CTX) return (int)g.ctx[r * W + p];
    if (g.src == SRC_TILES) {
        const int64_t tile = g.tile0 + r / R_GEN_TILE;
        const int i = (int)(r % R_GEN_TILE);
        if (tile >= *g.tile_count) {
            valid_row = false;
            return SOS;
        }
        const int4 d = g.desc[tile];
        const int64_t base = (int64_t)(uint32_t)d.x | ((int64_t)d.y << 32);
        if (i >= d.z) valid_row = false;
        const int64_t s = (int64_t)d.w + i - W + p;   // sequence step of window position p
        return s < 0 || !valid_row ? SOS : (int)g.tokens[base + i - W + p];
    }
    const int64_t s = (int64_t)g.t - W + p;
    if (g.t >= g.lengths[r]) valid_row = false;
    return s < 0 || !valid_row ? SOS : (int)g.tokens[g.tok_off[r] + s];
}

// One thread per (row, window position): copies the token's embedding row
// (emb_dim bytes) into X[r][p * emb_dim ..]; the padding columns and rows
// past `rows` are zero.  Out-of-range context tokens set status[0].
__global__ __launch_bounds__(256) void k_gen_embed(const int8_t *__restrict__ emb, int32_t emb_dim, int32_t W,
                                                   GenRows g, int64_t rows, int64_t rows_p, int8_t *__restrict__ X,
                                                   int64_t ldx, int32_t *__restrict__ status) {
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t r = id / (W + 1);
    const int p = (int)(id % (W + 1));
    if (r >= rows_p) return;
    int8_t *row = X + r * ldx;
    if (p == W) {   // this thread clears the padding columns
        for (int64_t k = (int64_t)W * emb_dim; k < ldx; ++k) row[k] = 0;
        return;
    }
    bool valid = r < rows;
    int tok = valid ? gen_token(g, r, p, W, valid) : SOS;
    if (tok < 0 || tok > SOS) {
        if (status) status[0] = SC_STATUS_BAD_TOKEN;
        tok = 0;
    }
    const int8_t *e = emb + (int64_t)tok * emb_dim;
    int8_t *dst = row + (int64_t)p * emb_dim;
    for (int j = 0; j < emb_dim; ++j) dst[j] = r < rows ? e[j] : (int8_t)0;
}

// ---- one linear layer ----------------------------------------------------

// Y[r][n] = requant(sum_k W[n][k] X[r][k] + bias[n]) for rows r < rows of
// the 64-row block and the 64-feature block of the grid; wave w computes
// row tile w & 1, n-tile w >> 1 as one 32 x 32 MFMA tile (transposed:
// D[n][r], A = weight fragment, B = 16 bytes of row r).  X has rows_p
// rows of ldx bytes (ldx = the layer's k-tiles x 32).
__global__ __launch_bounds__(256) void k_gen_linear(LayerDev L, const int8_t *__restrict__ X, int64_t ldx,
                                                    int64_t rows, int8_t *__restrict__ Y, int64_t ldy) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t r0 = (int64_t)blockIdx.x * 64 + (wave & 1) * 32;
    const int nt = blockIdx.y * 2 + (wave >> 1);
    const int NT = (L.n + 31) / 32;
    if (nt >= NT) return;
    const int KT = L.kt;
    const v4i *wf = L.w + (int64_t)nt * KT * 64 + lane;
    const int8_t *xr = X + (r0 + (lane & 31)) * ldx + (lane >> 5) * 16;
    v16i acc = {};
    for (int kt = 0; kt < KT; ++kt) {
        const v4i a = wf[(int64_t)kt * 64];
        const v4i b = *(const v4i *)(xr + kt * 32);
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc, 0, 0, 0);
    }
    const uint32_t *par = L.par + (int64_t)nt * PAR_DWORDS;
    const int64_t r = r0 + (lane & 31);
    const int lo = L.relu ? 0 : -128;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int nl = 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        const uint32_t sh = (par[64 + (nl >> 2)] >> (8 * (nl & 3))) & 0xFFu;
        const uint32_t q = requant_u8(acc[v], (int)par[nl], par[32 + nl], sh, lo);
        if (r < rows) Y[r * ldy + nt * 32 + nl] = (int8_t)(uint8_t)q;
    }
}

// ---- frequencies of the coded tokens (compress) -----------------------------

// 16 rows per workgroup (16-lane rows); row r = step of a tile as in
// k_gen_embed; its token's (cum, freq) go to pairs[token index].
__global__ __launch_bounds__(256) void k_gen_pairs(const int8_t *__restrict__ logits, int64_t rows,
                                                   const uint64_t *__restrict__ lut, const uint8_t *__restrict__ tokens,
                                                   const int4 *__restrict__ desc, int64_t tile0,
                                                   const int32_t *__restrict__ tile_count, uint2 *__restrict__ pairs) {
    __shared__ double s_lut[VOCAB];
    load_lut_lds(lut, s_lut);
    __syncthreads();
    const int u = threadIdx.x & 15;
    const int64_t r = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const v4i raw = r < rows ? *(const v4i *)(logits + r * VOCAB + 16 * u) : v4i{0, 0, 0, 0};
    Freq16 fr;
    row_frequencies16(raw, s_lut, u, fr);
    if (r >= rows) return;
    const int64_t tile = tile0 + r / R_GEN_TILE;
    const int i = (int)(r % R_GEN_TILE);
    if (tile >= *tile_count) return;
    const int4 d = desc[tile];
    if (i >= d.z) return;
    const int64_t g = ((int64_t)(uint32_t)d.x | ((int64_t)d.y << 32)) + i;
    const int s = tokens[g];
    if ((s >> 4) != u) return;   // the lane holding the symbol
    uint32_t cum, freq;
    freq16_at(fr, s & 15, cum, freq);
    pairs[g] = make_uint2(cum, freq);
}

// ---- decoder steps (decompress) ---------------------------------------------

// CpuRangeDecoder.__init__ (cpu_entropy_coding.py:466-474) for every chunk.
__global__ __launch_bounds__(256) void k_gen_dec_init(const uint32_t *__restrict__ words,
                                                      const int64_t *__restrict__ word_off,
                                                      const int32_t *__restrict__ word_cnt, int64_t n,
                                                      DecState *__restrict__ st) {
    const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= n) return;
    const int32_t cnt = word_cnt[c];
    const uint32_t *w = words + word_off[c];
    const int take = cnt < 2 ? cnt : 2;
    uint64_t point = 0;
    for (int i = 0; i < take; ++i) point = (point << 32) | w[i];
    if (cnt == 1) point <<= 32;
    st[c] = DecState{0ull, ~0ull, point, take, 0, 0, 0};
}

// One decoder step at step t for every chunk with t < lengths[c] and a
// valid stream so far (_decode_partition, cpu_entropy_coding.py:230-266):
// 16 chunks per workgroup, the frequency rule on 16-lane rows.
__global__ __launch_bounds__(256) void k_gen_dec_step(const int8_t *__restrict__ logits, int64_t n,
                                                      const uint64_t *__restrict__ lut, int32_t t,
                                                      const int32_t *__restrict__ lengths,
                                                      const uint32_t *__restrict__ words,
                                                      const int64_t *__restrict__ word_off,
                                                      const int32_t *__restrict__ word_cnt,
                                                      uint8_t *__restrict__ tokens, const int64_t *__restrict__ tok_off,
                                                      DecState *__restrict__ st) {
    __shared__ double s_lut[VOCAB];
    load_lut_lds(lut, s_lut);
    __syncthreads();
    const int lane = threadIdx.x & 63, u = threadIdx.x & 15;
    const int64_t c = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const v4i raw = c < n ? *(const v4i *)(logits + c * VOCAB + 16 * u) : v4i{0, 0, 0, 0};
    Freq16 fr;
    row_frequencies16(raw, s_lut, u, fr);
    DecState d{0ull, ~0ull, 0ull, 0, 1, 0, 0};
    const bool active = c < n && t < lengths[c] && (d = st[c]).stat == 0;
    const uint64_t scale = d.range >> 24;
    uint32_t q = 0;
    const bool ok = scale != 0 && dec_quantile(d.point - d.lower, scale, q);
    uint32_t cum, freq;
    const int sym = dec_symbol16(fr, q, lane, cum, freq);
    if (!active || u != 0) return;
    if (!ok) {
        st[c].stat = SC_STATUS_INVALID_STREAM;
        return;
    }
    uint64_t lower = d.lower + mul_scale(scale, cum), range = mul_scale(scale, freq), point = d.point;
    int32_t rp = d.rpos;
    if (range < (1ull << 32)) {
        lower <<= 32;
        range <<= 32;
        point = (point << 32) | (rp < word_cnt[c] ? words[word_off[c] + rp] : 0u);
        rp += 1;
    }
    st[c] = DecState{lower, range, point, rp, 0, 0, 0};
    tokens[tok_off[c] + t] = (uint8_t)sym;
}

__global__ __launch_bounds__(256) void k_gen_dec_status(const DecState *__restrict__ st, int64_t n,
                                                        int32_t *__restrict__ status) {
    const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (c < n) status[c] = st[c].stat;
}

// ---- logits -> int32 CDF (sc_mlp_forward_cdf) ------------------------------

__global__ __launch_bounds__(256) void k_gen_cdf32(const int8_t *__restrict__ logits, int64_t rows,
                                                   const uint64_t *__restrict__ lut, int32_t *__restrict__ cdf) {
    __shared__ double s_lut[VOCAB];
    load_lut_lds(lut, s_lut);
    __syncthreads();
    const int u = threadIdx.x & 15;
    const int64_t r = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const v4i raw = r < rows ? *(const v4i *)(logits + r * VOCAB + 16 * u) : v4i{0, 0, 0, 0};
    Freq16 fr;
    row_frequencies16(raw, s_lut, u, fr);
    if (r >= rows) return;
    int32_t *dst = cdf + r * (VOCAB + 1) + 16 * u;
    uint32_t c = fr.ex;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        dst[k] = (int32_t)c;
        c += fr.f[k];
    }
    if (u == 15) dst[16] = (int32_t)TOTAL;
}

// ---- host side -------------------------------------------------------------

int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

// Widest padded layer input / output of the model (bytes per row).
int64_t max_width(const ModelDev &M) {
    int64_t w = round_up((int64_t)M.window * M.emb_dim, 32);
    for (int i = 0; i < M.n_layers; ++i) w = std::max<int64_t>(w, round_up(M.layer[i].n, 32));
    return w;
}

// Rows per batch of a call that needs `needed` rows: at most
// GEN_BATCH_ROWS, at most what GEN_SCRATCH_BYTES holds at this model's width
// (two activation buffers and the logits per row), and no more than the
// call needs; a multiple of `unit` (64-row MLP tiles, 128-step compress
// tiles).  The widest model sc_model_create accepts (2**20 inputs) still
// gets 384 rows.
int64_t batch_rows(const ModelDev &M, int64_t needed, int64_t unit) {
    const int64_t per_row = 2 * max_width(M) + VOCAB;
    const int64_t fit = std::max<int64_t>(GEN_SCRATCH_BYTES / per_row / unit, 1) * unit;
    return std::min({GEN_BATCH_ROWS / unit * unit, fit, round_up(std::max<int64_t>(needed, 1), unit)});
}

hipError_t launch_check() { return hipGetLastError(); }

// Stream-ordered scratch of one call (hipMallocAsync / hipFreeAsync).
struct Scratch {
    void *p = nullptr;
    hipStream_t s;
    explicit Scratch(hipStream_t st) : s(st) {}
    hipError_t alloc(size_t bytes) { return hipMallocAsync(&p, bytes, s); }
    ~Scratch() {
        if (p) (void)hipFreeAsync(p, s);
    }
};

// The MLP over `rows` rows from `g` -> int8 logits [rows][256] at `logits`
// (row stride 256).  X0 / X1: ping-pong buffers of rows_p x max_width bytes.
hipError_t gen_mlp(const ModelDev &M, const GenRows &g, int64_t rows, int8_t *X0, int8_t *X1, int8_t *logits,
                   int32_t *status, hipStream_t s) {
    const int64_t rows_p = round_up(std::max<int64_t>(rows, 1), 64);
    const int W = M.window;
    const int64_t k0p = round_up((int64_t)W * M.emb_dim, 32);
    const int64_t threads = rows_p * (W + 1);
    hipLaunchKernelGGL(k_gen_embed, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, M.emb, M.emb_dim, W,
                       g, rows, rows_p, X0, k0p, status);
    hipError_t e = launch_check();
    if (e != hipSuccess) return e;
    int8_t *src = X0, *dst = X1;
    int64_t ld = k0p;
    for (int l = 0; l < M.n_layers; ++l) {
        const LayerDev &L = M.layer[l];
        const bool last = l == M.n_layers - 1;
        const int64_t ldy = last ? VOCAB : round_up(L.n, 32);
        int8_t *out = last ? logits : dst;
        const dim3 grid((unsigned)(rows_p / 64), (unsigned)((L.n + 63) / 64));
        hipLaunchKernelGGL(k_gen_linear, grid, dim3(256), 0, s, L, src, ld, last ? rows : rows_p, out, ldy);
        if ((e = launch_check()) != hipSuccess) return e;
        std::swap(src, dst);
        ld = ldy;
    }
    return hipSuccess;
}

}  // namespace

int gen_mlp_forward(const ModelDev &M, const int64_t *ctx, int64_t rows, int8_t *logits, int32_t *cdf,
                    int32_t *status, hipStream_t s, std::string &err) {
    const int64_t B = batch_rows(M, rows, 64);
    const int64_t width = max_width(M), rows_p = B;
    Scratch scr(s);
    hipError_t e = scr.alloc((size_t)(2 * rows_p * width + (cdf ? rows_p * VOCAB : 0)));
    if (e != hipSuccess) {
        err = std::string("hipMallocAsync: ") + hipGetErrorString(e);
        return SC_ERR_HIP;
    }
    int8_t *X0 = (int8_t *)scr.p, *X1 = X0 + rows_p * width, *lg = X1 + rows_p * width;
    for (int64_t r0 = 0; r0 < rows; r0 += B) {
        const int64_t n = std::min(B, rows - r0);
        GenRows g{SRC_CTX, ctx + r0 * M.window, nullptr, nullptr, 0, nullptr, nullptr, nullptr, 0};
        int8_t *out = cdf ? lg : logits + r0 * VOCAB;
        if ((e = gen_mlp(M, g, n, X0, X1, out, status, s)) != hipSuccess) break;
        if (cdf) {
            hipLaunchKernelGGL(k_gen_cdf32, dim3((unsigned)((n + 15) / 16)), dim3(256), 0, s, lg, n, M.lut,
                               cdf + r0 * (VOCAB + 1));
            if ((e = launch_check()) != hipSuccess) break;
        }
    }
    if (e != hipSuccess) {
        err = std::string("generic MLP launch: ") + hipGetErrorString(e);
        return SC_ERR_HIP;
    }
    return SC_OK;
}

int gen_compress(const ModelDev &M, const uint8_t *tokens, const int32_t *tile_start, int64_t n_chunks,
                 const int4 *desc, int64_t max_tiles, uint2 *pairs, hipStream_t s, std::string &err) {
    const int64_t rows_b = batch_rows(M, max_tiles * R_GEN_TILE, R_GEN_TILE), width = max_width(M);
    const int64_t tiles_per = rows_b / R_GEN_TILE;
    Scratch scr(s);
    hipError_t e = scr.alloc((size_t)(2 * rows_b * width + rows_b * VOCAB));
    if (e != hipSuccess) {
        err = std::string("hipMallocAsync: ") + hipGetErrorString(e);
        return SC_ERR_HIP;
    }
    int8_t *X0 = (int8_t *)scr.p, *X1 = X0 + rows_b * width, *lg = X1 + rows_b * width;
    const int32_t *count = tile_start + n_chunks;   // tiles of the call (device)
    for (int64_t t0 = 0; t0 < max_tiles && e == hipSuccess; t0 += tiles_per) {
        const int64_t rows = std::min(tiles_per, max_tiles - t0) * R_GEN_TILE;
        GenRows g{SRC_TILES, nullptr, tokens, desc, t0, count, nullptr, nullptr, 0};
        if ((e = gen_mlp(M, g, rows, X0, X1, lg, nullptr, s)) != hipSuccess) break;
        hipLaunchKernelGGL(k_gen_pairs, dim3((unsigned)((rows + 15) / 16)), dim3(256), 0, s, lg, rows, M.lut, tokens,
                           desc, t0, count, pairs);
        e = launch_check();
    }
    if (e != hipSuccess) {
        err = std::string("generic compress launch: ") + hipGetErrorString(e);
        return SC_ERR_HIP;
    }
    return SC_OK;
}

int gen_decompress(const ModelDev &M, const uint32_t *words, const int64_t *word_off, const int32_t *word_cnt,
                   const int32_t *lengths, int64_t n_chunks, uint8_t *tokens, const int64_t *tok_off,
                   int32_t *status, DecState *state, int32_t max_len, hipStream_t s, std::string &err) {
    const int64_t width = max_width(M);
    const int64_t B = batch_rows(M, n_chunks, 64), rows_p = B;
    Scratch scr(s);
    hipError_t e = scr.alloc((size_t)(2 * rows_p * width + rows_p * VOCAB));
    if (e != hipSuccess) {
        err = std::string("hipMallocAsync: ") + hipGetErrorString(e);
        return SC_ERR_HIP;
    }
    int8_t *X0 = (int8_t *)scr.p, *X1 = X0 + rows_p * width, *lg = X1 + rows_p * width;
    // groups of at most B chunks, each decoded step by step
    for (int64_t c0 = 0; c0 < n_chunks && e == hipSuccess; c0 += B) {
        const int64_t n = std::min(B, n_chunks - c0);
        hipLaunchKernelGGL(k_gen_dec_init, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, words, word_off + c0,
                           word_cnt + c0, n, state + c0);
        if ((e = launch_check()) != hipSuccess) break;
        for (int32_t t = 0; t < max_len && e == hipSuccess; ++t) {
            GenRows g{SRC_DECODE, nullptr, tokens, nullptr, 0, nullptr, tok_off + c0, lengths + c0, t};
            if ((e = gen_mlp(M, g, n, X0, X1, lg, nullptr, s)) != hipSuccess) break;
            hipLaunchKernelGGL(k_gen_dec_step, dim3((unsigned)((n + 15) / 16)), dim3(256), 0, s, lg, n, M.lut, t,
                               lengths + c0, words, word_off + c0, word_cnt + c0, tokens, tok_off + c0, state + c0);
            e = launch_check();
        }
        if (e != hipSuccess) break;
        hipLaunchKernelGGL(k_gen_dec_status, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, state + c0, n,
                           status + c0);
        e = launch_check();
    }
    if (e != hipSuccess) {
        err = std::string("generic decompress launch: ") + hipGetErrorString(e);
        return SC_ERR_HIP;
    }
    return SC_OK;
}

}  // namespace sc
