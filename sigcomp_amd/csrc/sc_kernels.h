// sc_kernels.h -- the MLP kernel templates of libsigcomp_hip (explicit
// context windows, teacher-forced compress, persistent decompress) and the
// host launchers that instantiate them.  Each launcher is defined in a
// translation unit of its own (sc_ctx.hip, sc_comp.hip, sc_dec.hip,
// sc_dec_split.hip), so the large kernels compile in parallel;
// sc_kernels.hip holds the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/sigcomp_hip.h"
#include "sc_device.h"
#include "sc_pipe.h"

namespace sc {

constexpr int RT_TILE = 4;          // rows per MLP tile = 32 * RT_TILE = 128
constexpr int R_TILE = 32 * RT_TILE;
constexpr int DEC_RT_MAX = 5;       // decode: up to 160 chunks per workgroup (LDS)

enum CtxOut { OUT_LOGITS = 0, OUT_CDF32 = 1 };

// Coder state of one row between the step segments of a decode: the state
// of its current chunk, which of its chunks that is and the step it started.
struct DecState {
    uint64_t lower, range, point;
    int32_t rpos, stat, cur, start;
};

// Split decode (small batches): P = 4 or 8 workgroups per 32-chunk group
// share layer 0 (see k_decompress).  Per group the exchange workspace holds
// two parity buffers of 32 rows x 512 feature bytes; after the buffers of
// all groups come P int32 step flags per group (room for SPLIT_P_MAX).
constexpr int SPLIT_P_MAX = 8;
constexpr int XCH_ROW = HID;                 // bytes per row of an exchange buffer
constexpr int XCH_PAR = 32 * XCH_ROW;        // one parity buffer
constexpr int XCH_GROUP = 2 * XCH_PAR;       // both parities of one group
constexpr int XCH_MAX_GROUPS = 64;           // 64 x 4 workgroups fill the 256 CUs
constexpr int64_t xch_bytes(int64_t groups) {
    return groups * XCH_GROUP + (groups * SPLIT_P_MAX * 4 + 255) / 256 * 256;
}

// Host launchers (stream-ordered, no error check: the caller checks
// hipGetLastError).  The MLP core follows M.pipe.
template <int MODE>
void launch_mlp_context(const ModelDev &M, unsigned grid, hipStream_t s, const int64_t *ctx, int64_t rows,
                        int8_t *logits, int32_t *cdf, int32_t *status);
void launch_compress_mlp(const ModelDev &M, unsigned grid, hipStream_t s, const uint8_t *tokens, int64_t n_chunks,
                         const int32_t *tile_start, const int4 *desc, int64_t max_desc, uint2 *pairs);
template <int RT>
void launch_decompress(const ModelDev &M, unsigned grid, hipStream_t s, const uint32_t *words, const int64_t *woff,
                       const int32_t *wcnt, const int32_t *len, int64_t count, uint8_t *tokens, const int64_t *toff,
                       int32_t *st, DecState *state, int32_t t_begin, int32_t t_end, int64_t n_second);
// The split decode of `groups` 32-chunk groups with p = 4 or 8 workgroups
// each (pipelined per-tensor core only): a cooperative launch of groups * p
// workgroups, so that all are resident at once; returns the launch's error
// (the caller falls back when the device cannot hold them).  `xch` =
// xch_bytes(groups) bytes, the flags zeroed before the first step segment
// of a call; each wait for the peers gives up after spin_max polls
// (SYNC_SPIN_MAX).
hipError_t launch_decompress_split(const ModelDev &M, int p, unsigned groups, hipStream_t s, const uint32_t *words,
                                   const int64_t *woff, const int32_t *wcnt, const int32_t *len, int64_t count,
                                   uint8_t *tokens, const int64_t *toff, int32_t *st, DecState *state,
                                   int32_t t_begin, int32_t t_end, uint8_t *xch, int32_t spin_max);

namespace {

// Rows of a tile are post-processed four at a time per wavefront: row
// 4*gi + lane/16 is handled by the 16-lane row lane/16 (see Freq16).

// ---- explicit context windows (GPUBitExactMLPDecoder._ar_step) ----------


// MLP core of one tile: the pipelined core when the model allows it.
template <int CORE, int RT, class AposFn>
__device__ __forceinline__ void mlp_tile(const ModelDev &M, const uint8_t *s_emb, uint8_t *s_act, uint32_t *s_par,
                                         AposFn apos, int wave, int lane) {
    if constexpr (CORE != CORE_PLAIN) mlp_rows_pipe<RT, CORE == CORE_PIPE_UNI>(M, s_emb, s_act, s_par, apos, wave, lane);
    else mlp_rows<RT, (RT <= 4 ? 1 : 2)>(M, s_emb, s_act, s_par, apos, wave, lane);
}
// once per kernel, before the first mlp_tile (and a barrier)
template <int CORE>
__device__ __forceinline__ void mlp_tile_init(const ModelDev &M, uint32_t *s_par, int wave, int lane) {
    if constexpr (CORE != CORE_PLAIN) pipe_params_init<CORE == CORE_PIPE_UNI>(M, s_par, wave, lane);
}
template <int CORE>
constexpr int par_lds_dwords() {
    return CORE == CORE_PLAIN ? PAR_LDS_DWORDS : pipe_par_dwords<CORE == CORE_PIPE_UNI>();
}
// activation row layout of the core: padded rows (pipelined) or swizzled rows
template <bool PIPE>
constexpr int act_row_bytes() { return PIPE ? PACT_ROW : ACT_ROW; }
template <bool PIPE>
__device__ __forceinline__ int act_at(int r, int chunk) { return PIPE ? pact_off(r, chunk) : act_off(r, chunk); }

template <int MODE, int CORE>
__global__ __launch_bounds__(THREADS, 1) void k_mlp_context(ModelDev M, const int64_t *__restrict__ ctx,
                                                            int64_t rows, int8_t *__restrict__ logits,
                                                            int32_t *__restrict__ cdf,
                                                            int32_t *__restrict__ status) {
    constexpr bool PIPE = CORE != CORE_PLAIN;
    __shared__ __attribute__((aligned(16))) uint8_t s_emb[EMB_BYTES];
    __shared__ __attribute__((aligned(16))) uint8_t s_act[R_TILE * act_row_bytes<PIPE>()];
    // rows padded to CTX_STRIDE halfwords: layer 0 reads one position of 32
    // consecutive rows at a time, which a 128-byte row stride would put in
    // one LDS bank
    constexpr int CTX_STRIDE = WIN + 2;
    __shared__ __attribute__((aligned(16))) uint16_t s_ctx[R_TILE * CTX_STRIDE];
    __shared__ __attribute__((aligned(16))) uint32_t s_par[par_lds_dwords<CORE>()];
    __shared__ double s_lut[VOCAB];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int q4 = lane >> 4, u = lane & 15;
    load_emb_lds(M.emb, s_emb);
    load_lut_lds(M.lut, s_lut);
    mlp_tile_init<CORE>(M, s_par, wave, lane);
    const int64_t n_tiles = (rows + R_TILE - 1) / R_TILE;
    // A tile's 128 x 64 context tokens: 32 per thread, all loads issued
    // before the first is used (a load / wait / store loop costs one memory
    // round trip per token).  Element j * THREADS + thread is row 4j + wave,
    // position lane: each load instruction reads 2 KB.  Addresses and row
    // limits are formed from per-tile values, so that none is hoisted out of
    // the tile loop (32 such registers held across the MLP make it spill).
    constexpr int CTX_PER = R_TILE * WIN / THREADS;
    static_assert(THREADS == 4 * WIN, "four context rows per load instruction");
    for (int64_t tile = blockIdx.x; tile < n_tiles; tile += gridDim.x) {
        const int64_t row0 = tile * R_TILE;
        const int64_t *src = ctx + row0 * WIN + threadIdx.x;
        const int64_t lim = rows - row0 - wave;   // element j is in range iff 4j < lim
        int64_t v[CTX_PER];
#pragma unroll
        for (int j = 0; j < CTX_PER; ++j) v[j] = 4 * j < lim ? src[j * THREADS] : 0;
        __syncthreads();
        int bad = 0;
#pragma unroll
        for (int j = 0; j < CTX_PER; ++j) {
            const bool ok = (uint64_t)v[j] <= (uint64_t)SOS;
            bad |= !ok;
            // element j * THREADS + thread: row 4j + wave, position lane
            s_ctx[(4 * j + wave) * CTX_STRIDE + lane] = (uint16_t)emb_off(ok ? (int)v[j] : 0, 0);   // table addresses
        }
        if (bad) status[0] = SC_STATUS_BAD_TOKEN;
        __syncthreads();
        mlp_tile<CORE, RT_TILE>(M, s_emb, s_act, s_par, [&](int r, int p) { return (int)s_ctx[r * CTX_STRIDE + p]; },
                                wave, lane);
        if (MODE == OUT_LOGITS) {
            // 128 rows x 256 bytes, 16-byte chunks, coalesced
            for (int i = threadIdx.x; i < R_TILE * 16; i += THREADS) {
                const int r = i >> 4, c = i & 15;
                if (row0 + r < rows)
                    *(v4i *)(logits + (row0 + r) * VOCAB + c * 16) = *(const v4i *)(s_act + act_at<PIPE>(r, c));
            }
        } else {
            // two row groups (gi, gi + WAVES) per iteration, see row_frequencies16n
            for (int gi = wave; gi < R_TILE / 4; gi += 2 * WAVES) {
                const int rr[2] = {gi * 4 + q4, (gi + WAVES) * 4 + q4};
                const v4i raw[2] = {*(const v4i *)(s_act + act_at<PIPE>(rr[0], u)),
                                    *(const v4i *)(s_act + act_at<PIPE>(rr[1], u))};
                Freq16 fr[2];
                row_frequencies16n<2>(raw, s_lut, u, fr);
#pragma unroll
                for (int n = 0; n < 2; ++n) {
                    if (row0 + rr[n] < rows) {
                        int32_t *dst = cdf + (row0 + rr[n]) * (VOCAB + 1) + 16 * u;
                        uint32_t c = fr[n].ex;
#pragma unroll
                        for (int k = 0; k < 16; ++k) {
                            dst[k] = (int32_t)c;
                            c += fr[n].f[k];
                        }
                        if (u == 15) dst[16] = (int32_t)TOTAL;
                    }
                }
            }
        }
    }
}


// ---- compress: teacher-forced MLP fused with the frequency step ----------

// Workgroup b runs tiles b, b + G, b + 2G, ... (G = grid size) of the global
// tile order.  Every tile costs the same, so the workgroups stay in step and
// stream the same layer's weights at the same time: each XCD's L2 then
// serves one weight fragment to all of its CUs (a work counter lets
// workgroups drift apart, and the L2 cycles through the whole model).  A
// tile's 128 + 64 tokens (64 of left context) are staged in LDS from its
// descriptor (k_tile_table), which is loaded while the previous tile's
// frequency step runs, so a tile waits for one memory round trip.  Output per
// token: (exclusive cumulative frequency, frequency) of the coded token.
template <int CORE>
__global__ __launch_bounds__(THREADS, 1) void k_compress_mlp(ModelDev M, const uint8_t *__restrict__ tokens,
                                                             int64_t n_chunks, const int32_t *__restrict__ tile_start,
                                                             const int4 *__restrict__ desc, int64_t max_desc,
                                                             uint2 *__restrict__ pairs) {
    constexpr bool PIPE = CORE != CORE_PLAIN;
    constexpr int EPI_N = 2;   // row groups per epilogue iteration; R_TILE / 4 is a multiple of EPI_N * WAVES
    static_assert((R_TILE / 4) % (EPI_N * WAVES) == 0, "epilogue iterations must stay inside the tile");
    __shared__ __attribute__((aligned(16))) uint8_t s_emb[EMB_BYTES];
    __shared__ __attribute__((aligned(16))) uint8_t s_act[R_TILE * act_row_bytes<PIPE>()];
    __shared__ __attribute__((aligned(16))) uint32_t s_par[par_lds_dwords<CORE>()];
    __shared__ __attribute__((aligned(16))) uint32_t s_slot[WAVES * EPI_N * 4 * SLOT_DWORDS];
    __shared__ uint16_t s_tok[R_TILE + WIN];
    __shared__ uint16_t s_apos[R_TILE + WIN];   // emb_off(s_tok[i], 0)
    __shared__ double s_lut[VOCAB];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int q4 = lane >> 4, u = lane & 15;
    load_emb_lds(M.emb, s_emb);
    load_lut_lds(M.lut, s_lut);
    mlp_tile_init<CORE>(M, s_par, wave, lane);
    static_assert(R_TILE + WIN <= THREADS, "one staged token per thread");
    const int32_t n_tiles = (int32_t)min<int64_t>(tile_start[n_chunks], max_desc);
    const int32_t G = (int32_t)gridDim.x;
    // This thread's staged token of the tile with descriptor dd: s_tok[i]
    // <-> sequence position t0 - 64 + i (SOS before 0).
    auto stage_token = [&](const int4 &dd) {
        const int64_t b = (int64_t)(uint32_t)dd.x | ((int64_t)dd.y << 32);
        const int32_t p = (int32_t)threadIdx.x - WIN;
        int v = 0;
        if (threadIdx.x < R_TILE + WIN) v = dd.w + p < 0 ? SOS : (p < dd.z ? (int)tokens[b + p] : 0);
        return v;
    };
    // a buffer (vector memory) load: a scalar one, which a load of a
    // uniform address would become, would be waited for with the epilogue's
    // first LDS reads, since they share its counter
    const __amdgpu_buffer_rsrc_t drs = __builtin_amdgcn_make_buffer_rsrc(
        (void *)desc, (short)0, (int)min<int64_t>((int64_t)n_tiles * 16, INT32_MAX), 0x00020000);
    auto desc_at = [&](int32_t k) {
        if (k >= n_tiles) return make_int4(0, 0, 0, 0);
        const v4i x = wload_s(drs, 0, k * 16);
        return make_int4(x[0], x[1], x[2], x[3]);
    };
    // workgroup-uniform: scalar registers across the MLP
    auto uniform = [](int4 x) {
        return make_int4(__builtin_amdgcn_readfirstlane(x.x), __builtin_amdgcn_readfirstlane(x.y),
                         __builtin_amdgcn_readfirstlane(x.z), __builtin_amdgcn_readfirstlane(x.w));
    };
    // Descriptors are loaded two tiles ahead, and the next tile's tokens are
    // loaded right after this tile's MLP: both complete during this tile's
    // epilogue (which waits for no memory load), so a tile starts without a
    // memory round trip.
    int4 d = uniform(desc_at((int32_t)blockIdx.x));
    int v = (int32_t)blockIdx.x < n_tiles ? stage_token(d) : 0;
    int4 dn = uniform(desc_at((int32_t)blockIdx.x + G));
    for (int32_t tile = blockIdx.x; tile < n_tiles; tile += G) {
        const int64_t base = (int64_t)(uint32_t)d.x | ((int64_t)d.y << 32);   // token t0 of the chunk
        const int32_t rem = d.z;                                               // L - t0
        __syncthreads();
        if (threadIdx.x < R_TILE + WIN) {
            s_tok[threadIdx.x] = (uint16_t)v;
            s_apos[threadIdx.x] = (uint16_t)emb_off(v, 0);
        }
        __syncthreads();
        mlp_tile<CORE, RT_TILE>(M, s_emb, s_act, s_par, [&](int r, int p) { return (int)s_apos[r + p]; },
                                wave, lane);
        const int vn = tile + G < n_tiles ? stage_token(dn) : 0;
        const int4 dnn = desc_at(tile + 2 * G);
        uint2 *out = pairs + base;
        const int32_t valid = min(R_TILE, rem);
        // EPI_N row groups (gi + n * WAVES) per iteration, see row_freq.  The
        // lane holding the row's token publishes its 16 symbols in the row's
        // slot; the lane whose index is the token's low 4 bits stores its
        // (cumulative frequency, frequency) pair.
        uint32_t *slots = s_slot + wave * (EPI_N * 4 * SLOT_DWORDS);
        for (int gi = wave; gi * 4 < valid; gi += EPI_N * WAVES) {
            int rr[EPI_N], sym[EPI_N];
            v4i raw[EPI_N];
#pragma unroll
            for (int n = 0; n < EPI_N; ++n) {
                rr[n] = (gi + n * WAVES) * 4 + q4;
                sym[n] = s_tok[rr[n] + WIN];
                raw[n] = *(const v4i *)(s_act + act_at<PIPE>(rr[n], u));
            }
            RowFreq fr[EPI_N];
            row_freq<EPI_N>(raw, s_lut, u, fr);
#pragma unroll
            for (int n = 0; n < EPI_N; ++n)
                if ((sym[n] >> 4) == u) slot_put(slots + (n * 4 + q4) * SLOT_DWORDS, fr[n], u);
            slot_sync();
#pragma unroll
            for (int n = 0; n < EPI_N; ++n) {
                uint32_t cum, freq;
                slot_get(slots + (n * 4 + q4) * SLOT_DWORDS, u, cum, freq);
                if (rr[n] < valid && (sym[n] & 15) == u) out[rr[n]] = make_uint2(cum, freq);
            }
        }
        d = dn;
        dn = uniform(dnn);
        v = vn;
    }
}

// ---- decompress: persistent autoregressive loop per chunk tile ----------

// Workgroup b owns chunks [b*R, b*R + R).  Each step: MLP on the R context
// windows (kept as 64-token rings in LDS), the fused frequency step and one
// decoder step per chunk; the decoded token is appended to the ring.  Chunks
// are independent, so workgroups never synchronise with each other.

// CpuRangeDecoder.__init__ (cpu_entropy_coding.py:466-474): the point is the
// first two words, big-endian combined (one word -> w0 << 32)
__device__ __forceinline__ uint64_t dec_init_point(const uint32_t *w, int cnt, int &take) {
    uint64_t point = 0;
    take = cnt < 2 ? cnt : 2;
    for (int i = 0; i < take; ++i) point = (point << 32) | w[i];
    if (cnt == 1) point <<= 32;
    return point;
}

// ---- split decode: layer 0 shared by the P workgroups of a row group -----
//
// With few chunks a decode has few 32-row workgroups, and each step streams
// the whole model (6.2 MB) through one CU's vector L1 for 32 rows.  In the
// split decode the P workgroups of a group each compute 512 / P of layer
// 0's features (n-tiles 16 / P * slice ..: at P = 4 one n-tile per wave, at
// P = 8 two, each over half of the window positions by a pair of waves whose
// partial sums meet in LDS), exchange them through memory, and then all of
// them run the hidden layers, the output layer and the decoder step on the
// same data: identical integer arithmetic, identical results.  Slice 0
// alone writes tokens, status and coder state.  Workgroup b is slice b % P
// of group b / P: with workgroups placed round-robin on the 8 XCDs, each
// XCD's L2 holds one layer-0 slice (P = 8) or two (P = 4) plus the hidden
// layers.
//
// Exchange of step t: each n-tile's requantised features (32 rows x 32
// bytes) are stored into the group's buffer of parity t & 1 with
// agent-coherent (sc1) stores; once they have completed the workgroup
// publishes
// flags[slice] = t + 1; wave 0 polls the peers' flags (agent-coherent
// loads) until each exceeds t; then every thread copies its share of the
// peers' features into LDS.  A buffer of parity t & 1 is rewritten at step
// t + 2, by a writer that has seen every peer publish step t + 1, which a
// peer does only after its reads of step t have completed.  Every wait is
// bounded (spin_max polls): a workgroup that times out records it and
// stops publishing and waiting, so that its peers time out too and every
// workgroup ends; the group's chunks then report SC_STATUS_SYNC_TIMEOUT.
constexpr int SYNC_SPIN_MAX = 1 << 18;   // ~0.5 s of polls (the default limit)
constexpr int L0_DEPTH = 16;             // layer-0 weight look-ahead of the split decode (k-steps)
constexpr int CPOL_SC1 = 16;             // buffer cache policy: sc1, agent-coherent access

// Layer 0's bias for the wave's n-tile into its slot_p0(0) (once per kernel).
template <int P>
__device__ __forceinline__ int split_ntile(int slice, int wave) { return 16 / P * slice + wave % (16 / P); }
__device__ __forceinline__ void split_params_init(const ModelDev &M, uint32_t *s_par, int nt, int wave, int lane) {
    uint32_t *blk = s_par + wave * PIPE_SLOTS * Slot<true>::BLK + slot_p0(0) * Slot<true>::BLK;
    if (lane < Slot<true>::TD) blk[lane] = M.layer[0].par[nt * PAR_DWORDS + lane];
}

// Layer 0 carried from one step of the split decode to the next: the wave's
// sums over every window position but the last (whose token the step
// decodes), and the last position's weight fragments.
struct L0Carry {
    v16i acc;
    v4i wlast[EDIM / 32];
    bool have;
};

// One MLP evaluation of the group's 32 rows, layer 0 shared (above).  Same
// contract as mlp_rows_pipe<1, true>; `xbuf` / `flags` are the group's
// exchange buffers and step flags, s_err the workgroup's timeout flag,
// s_red (P = 8) 2 x 4 KB of LDS for the partial sums.  Once a step has
// published its features it streams the next step's layer 0 but the last
// position (apos_next, when has_next) into `l0`, so that the next step
// starts with four MFMAs while this step's exchange completes behind that
// work; the first step of a launch computes the whole window.
template <int P, class AposFn, class AposNextFn>
__device__ __forceinline__ void mlp_rows_split(const ModelDev &M, const uint8_t *s_emb, uint8_t *s_act,
                                               uint32_t *s_par, AposFn apos, AposNextFn apos_next, bool has_next,
                                               L0Carry &l0, int wave, int lane, uint8_t *xbuf, int32_t *flags,
                                               int slice, int32_t t, int32_t spin_max, int32_t *s_err,
                                               int32_t *s_red) {
    static_assert(P == 4 || P == 8, "one or two layer-0 n-tiles per wave pair");
    constexpr int NTW = 16 / P;           // layer-0 n-tiles of the workgroup
    constexpr int KSPLIT = WAVES / NTW;   // waves per n-tile, each over WIN / KSPLIT positions
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    constexpr int RT = 1;
    constexpr bool UNI = true;
    wave = __builtin_amdgcn_readfirstlane(wave);
    const int voff = lane * 16, g2 = lane >> 5, rl = lane & 31;
    const int nb0 = 2 * wave;
    constexpr int BLK = Slot<UNI>::BLK;
    uint32_t *s_parw = s_par + wave * PIPE_SLOTS * BLK;
    v16i accA[PNT][RT], accB[PNT][RT];
    constexpr int PPD = ppd<RT>();
    v4i w[2][PPD][PNT];
    uint32_t pk[PNT][RT][4];
    const LayerDev &L0 = M.layer[0];
    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc((void *)(xbuf + (t & 1) * XCH_PAR), (short)0, XCH_PAR, 0x00020000);
    const int nt = split_ntile<P>(slice, wave), kp = wave / NTW;   // n-tile, part of the window
    const bool lastpart = kp == KSPLIT - 1;                          // the part holding the last position
    constexpr int NW = WIN / KSPLIT;
    const WStream ws0 = make_wstream(L0.w, L0.bytes);
    const v16i bias = bias_tile<UNI>(s_parw + slot_p0(0) * BLK, 0, g2);
    const v16i zero = {};
    {
        uint32_t prn[Slot<UNI>::LANE];
        par_fetch<UNI>(M.layer[1].par, nb0, lane, prn);
        v16i a0[1];
        if (l0.have)
            a0[0] = lastpart ? gemm_layer0_position(l0.wlast, WIN - 1, s_emb, apos, l0.acc, lane) : l0.acc;
        else
            a0[0] = gemm_layer0_one<L0_DEPTH, NW>(ws0, nt, kp * NW, s_emb, apos, kp == 0 ? bias : zero, lane);
        par_put<UNI>(s_parw + slot_p0(1) * BLK, prn, lane);
        if constexpr (KSPLIT > 1) {
            // the second half's partial sums -> the first half's wave
            static_assert(KSPLIT == 2, "two waves per n-tile");
            int32_t *red = s_red + (wave % NTW) * 16 * 64 + lane;
            if (kp == 1) {
#pragma unroll
                for (int e = 0; e < 16; ++e) red[e * 64] = a0[0][e];
            }
            __syncthreads();
            if (kp == 0) {
#pragma unroll
                for (int e = 0; e < 16; ++e) a0[0][e] = (int)((uint32_t)a0[0][e] + (uint32_t)red[e * 64]);
            }
        }
        if (kp == 0) {
            uint32_t p0[1][4];
            const RqUni u0 = rq_uni(L0);
            static_for<4>([&](auto gc) __attribute__((always_inline)) {
                rq_words_uni<true, 0, 1>(a0, decltype(gc)::value, u0, p0);
            });
            const v4i v = {(int)p0[0][0], (int)p0[0][1], (int)p0[0][2], (int)p0[0][3]};
            const int chunk = nt * 2 + g2;   // hidden order, as pstore_perm
            *(v4i *)(s_act + pact_off(rl, chunk)) = v;
            __builtin_amdgcn_raw_buffer_store_b128((v4u)v, xr, rl * XCH_ROW + chunk * 16, 0, CPOL_SC1);
        }
    }
    // publish once every wave's stores have completed
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const bool err = *s_err != 0;
    if (threadIdx.x == 0 && !err) __hip_atomic_store(flags + slice, t + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // the next step's layer 0 but its last position while the features travel
    l0.have = has_next;
    if (has_next)
        l0.acc = gemm_layer0_one<L0_DEPTH, NW>(ws0, nt, kp * NW, s_emb, apos_next, kp == 0 ? bias : zero, lane,
                                               lastpart, l0.wlast);
    // the first hidden layer's first weight fragments while the peers finish
    {
        const __amdgpu_buffer_rsrc_t rs1 = layer_rsrc(M.layer[1]);
#pragma unroll
        for (int s = 0; s < PPD; ++s)
#pragma unroll
            for (int j = 0; j < PNT; ++j) w[0][s][j] = wload_s(rs1, voff, ((nb0 + j) * KTH + s) * 1024);
    }
    if (wave == 0 && !err) {
        // at most spin_max polls (none at 0)
        for (int n = 0;; ++n) {
            if (n >= spin_max) {
                if (lane == 0) *s_err = 1;
                break;
            }
            const int32_t f = lane < P && lane != slice
                                  ? __hip_atomic_load(flags + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                  : INT32_MAX;
            if (__builtin_amdgcn_ballot_w64(f <= t) == 0) break;   // every peer has published step t
            __builtin_amdgcn_s_sleep(2);
        }
    }
    __syncthreads();
    // the peers' features: (P - 1) slices x 32 rows x 512 / P bytes, 16-byte pieces
    {
        constexpr int CW = 32 / P;                    // 16-byte chunks per row and slice
        constexpr int ROWP = (P - 1) * CW;            // peer pieces per row
        constexpr int PER = (32 * ROWP + THREADS - 1) / THREADS;   // pieces per thread (the last in part)
        v4i x[PER];
        int dst[PER];
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int i = min(u * THREADS + (int)threadIdx.x, 32 * ROWP - 1);
            const int row = i / ROWP, c = i % ROWP, q = c / CW;
            const int chunk = (q + (q >= slice)) * CW + c % CW;
            x[u] = (v4i)__builtin_amdgcn_raw_buffer_load_b128(xr, row * XCH_ROW + chunk * 16, 0, CPOL_SC1);
            dst[u] = pact_off(row, chunk);
        }
        // (threads past the last piece repeat it: the same bytes to the same place)
#pragma unroll
        for (int u = 0; u < PER; ++u) *(v4i *)(s_act + dst[u]) = x[u];
    }
    __syncthreads();
    const int last = M.n_layers - 1;
    if (last == 1) {
        pipe_hidden<RT, true, UNI, true>(L0, M.layer[1], M.layer[1], s_act, s_parw, 1, accA, accB, w, pk, wave, lane);
        return;
    }
    pipe_hidden<RT, false, UNI, true>(L0, M.layer[1], M.layer[2], s_act, s_parw, 1, accA, accB, w, pk, wave, lane);
#pragma unroll 1
    for (int l = 2; l < last; ++l)
        pipe_hidden<RT, false, UNI>(M.layer[l - 1], M.layer[l], M.layer[l + 1], s_act, s_parw, l, accA, accB, w, pk,
                                    wave, lane);
    pipe_hidden<RT, true, UNI>(M.layer[last - 1], M.layer[last], M.layer[last], s_act, s_parw, last, accA, accB, w,
                               pk, wave, lane);
}

// ---- decoder epilogue pieces ---------------------------------------------
//
// The LDS and global arrays of a k_decompress workgroup that its epilogue
// (frequency table, decoder step, state update) touches.  s_wbuf holds, per
// row, the 64 stream words from s_wbase[r] on (refilled every 64 steps, when
// the token ring is flushed: a row consumes at most one word per step), so
// that the word a renormalisation shifts in is an LDS read.
template <int R>
struct DecCtx {
    const uint8_t *s_act;
    const double *s_lut;
    uint64_t *s_lower, *s_range, *s_point;
    int64_t *s_woff, *s_toff;
    int32_t *s_rpos, *s_wcnt, *s_len, *s_stat, *s_cur, *s_start, *s_wbase;
    uint32_t *s_wbuf;
    uint8_t *s_ring;
    uint16_t *s_apos;
    const uint32_t *words;
    const int64_t *word_off, *tok_off;
    const int32_t *word_cnt, *lengths;
    uint8_t *tokens;
    int32_t *status;
    int64_t n_chunks, c0;
    bool writer;
};
constexpr int WBUF = 64;   // words per row in DecCtx::s_wbuf

// Row r's first chunk ended with step t (16 lanes of the row, lane u): its
// last tokens go out from the ring, its status is written, and the row's
// second chunk (2 * n_chunks - 1 - c) starts at step t + 2 from a
// start-of-sequence context (step t + 1 is idle for the row, so that the
// next step's layer 0, computed beside this epilogue, is never used for
// it).  PIPE: the ring of table addresses is reset; WB: the word buffer
// is refilled.
template <int R, bool PIPE, bool WB>
__device__ __forceinline__ void dec_switch(const DecCtx<R> &c, int r, int u, int32_t t) {
    auto apos_at = [](int rr, int32_t pos) { return (pos & (WIN - 1)) * R + rr; };
    slot_sync();
    const int64_t ch = c.c0 + r;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int32_t pg = (t & ~(WIN - 1)) + 4 * u + k, rs = pg - c.s_start[r];
        if (c.writer && pg <= t && rs >= 0) c.tokens[c.s_toff[r] + rs] = c.s_ring[r * WIN + (pg & (WIN - 1))];
        if constexpr (PIPE) c.s_apos[apos_at(r, 4 * u + k)] = (uint16_t)emb_off(SOS, 0);
    }
    const int64_t c2 = 2 * c.n_chunks - 1 - ch;
    const int32_t cnt = c.word_cnt[c2];
    const int64_t woff = c.word_off[c2];
    int take;
    const uint64_t point = dec_init_point(c.words + woff, cnt, take);
    if (u == 0) {
        if (c.writer) c.status[ch] = c.s_stat[r];
        c.s_point[r] = point;
        c.s_lower[r] = 0ull;
        c.s_range[r] = ~0ull;
        c.s_rpos[r] = take;
        c.s_stat[r] = 0;
        c.s_wcnt[r] = cnt;
        c.s_woff[r] = woff;
        c.s_toff[r] = c.tok_off[c2];
        c.s_len[r] = c.lengths[c2];
        c.s_cur[r] = 3;
        c.s_start[r] = t + 2;
        if constexpr (WB) c.s_wbase[r] = take;
    }
    if constexpr (WB) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int i = 4 * u + k;
            c.s_wbuf[r * WBUF + i] = take + i < cnt ? c.words[woff + take + i] : 0u;
        }
    }
}

// The decoder epilogue of one step for one group of four rows per wave
// (row 4 * (wave + 4 q) + lane / 16), cut into straight-line pieces for
// gemm_layer0_ov: piece<I>(q) runs in k-step region I of body q, after<I>
// between regions (the rare paths).  Each piece's LDS reads are used in a
// later piece (a region starts with a wait for all of them).  The
// arithmetic is row_freq's and the k_decompress epilogue's for one row
// (_frequencies and _decode_partition, cpu_entropy_coding.py:90-110,230-266).
template <int R, bool PIPE>
struct DecEpiSide {
    const DecCtx<R> &c;
    uint32_t *slot;          // the row's slot (SLOT_DWORDS)
    int32_t t;
    int wave, q4, u;
    uint32_t lanebits;
    int r;
    int32_t rs, len, stat, cur, start, rpos, wcnt, wbase;
    uint64_t lower, range, point;
    uint32_t wnext, mcum, mkfix, mffix, mown, fs;
    v4i raw;
    bool active, last1, ok;
    int lm, m;
    double wv[8];
    double T, r24;
    RowFreq fr;
    uint32_t hmin, S, K, qv;

    __device__ DecEpiSide(const DecCtx<R> &ctx, uint32_t *wave_slots, int32_t t_, int wave_, int lane)
        : c(ctx), slot(wave_slots + (lane >> 4) * SLOT_DWORDS), t(t_), wave(wave_), q4(lane >> 4), u(lane & 15),
          lanebits((uint32_t)(15 - (lane & 15)) << 4) {}

    __device__ __forceinline__ int logit(int k) const {
        return (int)(int8_t)((uint32_t)raw[k >> 2] >> (8 * (k & 3)));
    }
    __device__ __forceinline__ void lut8(int k0) {
        const double *p = c.s_lut + (VOCAB - 1 - m);
#pragma unroll
        for (int k = 0; k < 8; ++k) wv[k] = p[logit(k0 + k)];
    }
    __device__ __forceinline__ double sum8() const {
        return ((wv[0] + wv[1]) + (wv[2] + wv[3])) + ((wv[4] + wv[5]) + (wv[6] + wv[7]));
    }
    __device__ __forceinline__ void freq8(int k0) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const double qe = __builtin_fmax(__builtin_fma(wv[k], r24, 0x1p-20), 1.5);
            fr.f[k0 + k] = (uint32_t)qe;
            hmin = min(hmin, (uint32_t)(__builtin_bit_cast(uint64_t, __builtin_amdgcn_fract(qe)) >> 32));
        }
    }

    template <int I>
    __device__ __forceinline__ void piece(int q) {
        if constexpr (I == 0) {
            r = ((wave + q * WAVES) << 2) + q4;
            start = c.s_start[r];
            len = c.s_len[r];
            stat = c.s_stat[r];
            cur = c.s_cur[r];
            lower = c.s_lower[r];
            range = c.s_range[r];
            point = c.s_point[r];
            rpos = c.s_rpos[r];
            wcnt = c.s_wcnt[r];
            wbase = c.s_wbase[r];
            raw = *(const v4i *)(c.s_act + act_at<PIPE>(r, u));
        } else if constexpr (I == 1) {
            rs = t - start;
            active = rs >= 0 && rs < len && stat == 0;
            last1 = cur == 2 && rs == len - 1;   // the row's first chunk ends with this step
            wnext = c.s_wbuf[r * WBUF + ((rpos - wbase) & (WBUF - 1))];
            lm = logit(0);
#pragma unroll
            for (int k = 1; k < 16; ++k) lm = max(lm, logit(k));
        } else if constexpr (I == 2) {
            m = row16_max(lm);
            lut8(0);
        } else if constexpr (I == 3) {
            T = sum8();
            lut8(8);
        } else if constexpr (I == 4) {
            T = row16_sum_f64(T + sum8());
        } else if constexpr (I == 5) {
            r24 = recip_nr(T) * 16777216.0;
            lut8(0);
        } else if constexpr (I == 6) {
            hmin = 0xFFFFFFFFu;
            freq8(0);
            lut8(8);
        } else if constexpr (I == 7) {
            freq8(8);
        } else if constexpr (I == 8) {
            uint32_t sl = 0, km = 0;
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                sl += fr.f[k];
                km = max(km, (fr.f[k] << 4) | (uint32_t)(15 - k));
            }
            fr.tot = sl;
            S = sl;
            K = (((km << 4) - 256u) & 0xFFFFFF00u) | lanebits | (km & 15u);
        } else if constexpr (I == 9) {
            S = row16_sum(S);
            K = row16_max_u32(K);
        } else if constexpr (I == 10) {
            const uint32_t adj = S - TOTAL;
            const bool star = (K & 0xF0u) == lanebits;
            fr.ffix = (K >> 8) + 1u - adj;
            fr.kfix = star ? 15u - (K & 15u) : 16u;
            if (star) fr.tot -= adj;
            fr.ex = row16_excl_scan(fr.tot);
        } else if constexpr (I == 11) {
            const uint64_t scale = range >> 24;
            qv = 0;
            ok = scale != 0 && dec_quantile(point - lower, scale, qv);
        } else if constexpr (I == 12) {
            if (ok && qv - fr.ex < fr.tot) slot_put(slot, fr, u);
        } else if constexpr (I == 13) {
            // slot_get's reads (used in the next piece)
            slot_sync();
            typedef unsigned v4u __attribute__((ext_vector_type(4)));
            const v4u meta = *(const v4u *)(slot + 16);
            mcum = meta[0];
            mkfix = meta[1];
            mffix = meta[2];
            mown = meta[3];
            fs = slot[u];
        } else if constexpr (I == 14) {
            const uint32_t fq = (uint32_t)u == mkfix ? mffix : fs;
            const uint32_t cum = mcum + row16_excl_scan(fq);
            if (active && ok && qv - cum < fq) {
                const uint64_t scale = range >> 24;
                uint64_t lo = lower + mul_scale(scale, cum), ra = mul_scale(scale, fq), pt = point;
                int32_t rp = rpos;
                if (ra < (1ull << 32)) {
                    lo <<= 32;
                    ra <<= 32;
                    pt = (pt << 32) | (rpos < wcnt ? wnext : 0u);
                    rp += 1;
                }
                c.s_lower[r] = lo;
                c.s_range[r] = ra;
                c.s_point[r] = pt;
                c.s_rpos[r] = rp;
                const int sym = (int)mown * 16 + u;
                c.s_ring[r * WIN + (t & (WIN - 1))] = (uint8_t)sym;
                if constexpr (PIPE) c.s_apos[(t & (WIN - 1)) * R + r] = (uint16_t)emb_off(sym, 0);
            }
            if (active && !ok && u == 0) c.s_stat[r] = SC_STATUS_INVALID_STREAM;
        }
    }

    template <int I>
    __device__ __forceinline__ void after(int) {
        if constexpr (I == 7) {
            // high word of 2**-19: the float64 estimate of a frequency is
            // within 2**-19 of an integer -> exact integer division
            if (hmin < 0x3EC00000u) {
                const uint64_t Ti = (uint64_t)T;
                const double rT = r24 * 0x1p-24;
                const double *p = c.s_lut + (VOCAB - 1 - m);
#pragma unroll
                for (int k = 0; k < 16; ++k) {
                    const uint64_t qd = div_floor_est(((uint64_t)p[logit(k)]) << 24, Ti, rT);
                    fr.f[k] = qd < 1 ? 1u : (uint32_t)qd;
                }
            }
        } else if constexpr (I == 15) {
            if (last1) dec_switch<R, PIPE, true>(c, r, u, t);
        }
    }
};

// No side work (gemm_layer0_ov with ng = 0).
struct NoSide {
    template <int I>
    __device__ __forceinline__ void piece(int) {}
    template <int I>
    __device__ __forceinline__ void after(int) {}
};

// P = 1: workgroup b owns chunks [b*R, b*R + R) and never synchronises with
// another.  P > 1 (RT = 1, pipelined per-tensor core): the split decode
// above, workgroup b being slice b % P of the group of chunks
// [(b / P) * 32, (b / P) * 32 + 32).
template <int RT, int CORE, int P = 1>
__global__ __launch_bounds__(THREADS, 1) void k_decompress(ModelDev M, const uint32_t *__restrict__ words,
                                                           const int64_t *__restrict__ word_off,
                                                           const int32_t *__restrict__ word_cnt,
                                                           const int32_t *__restrict__ lengths,
                                                           int64_t n_chunks, uint8_t *__restrict__ tokens,
                                                           const int64_t *__restrict__ tok_off,
                                                           int32_t *__restrict__ status,
                                                           DecState *__restrict__ state, int32_t t_begin,
                                                           int32_t t_end, int64_t n_second, uint8_t *xch,
                                                           int32_t spin_max) {
    // Rows n_chunks - n_second .. n_chunks - 1 each decode a second chunk
    // after their first one ends: row c continues with chunk
    // 2 * n_chunks - 1 - c (the n_second chunks after the launch's own, in
    // reverse order, so that with chunks sorted longest first the longest
    // second chunk follows the shortest first chunk).
    static_assert(P == 1 || (RT == 1 && CORE == CORE_PIPE_UNI), "the split decode runs 32-row groups on the per-tensor core");
    static_assert(P == 1 || P == 4 || P == 8, "split decode: 4 or 8 workgroups per group");
    constexpr bool PIPE = CORE != CORE_PLAIN;
    // the epilogue beside the next step's layer 0 (gemm_layer0_ov)
    constexpr bool OV = P == 1 && PIPE && RT >= 2 && RT <= 3;
    constexpr int R = 32 * RT;
    constexpr int EPI_N = 2;   // row groups per epilogue iteration; R / 4 is a multiple of EPI_N * WAVES
    static_assert((R / 4) % (EPI_N * WAVES) == 0, "epilogue iterations must cover the rows exactly");
    __shared__ __attribute__((aligned(16))) uint8_t s_emb[EMB_BYTES];
    __shared__ __attribute__((aligned(16))) uint8_t s_act[R * act_row_bytes<PIPE>()];
    __shared__ __attribute__((aligned(16))) uint8_t s_ring[R * WIN];
    // the pipelined core also keeps the ring as embedding-table addresses
    // (emb_off(token, 0)), written with the token; the plain core converts.
    // Position-major (apos_at): layer 0 reads one position of 32 consecutive
    // rows at a time, 32 consecutive halfwords instead of 32 reads 128 bytes
    // apart in one LDS bank.
    __shared__ __attribute__((aligned(16))) uint16_t s_apos[PIPE ? R * WIN : 1];
    auto apos_at = [](int r, int32_t pos) { return (pos & (WIN - 1)) * R + r; };
    __shared__ __attribute__((aligned(16))) uint32_t s_slot[WAVES * EPI_N * 4 * SLOT_DWORDS];
    __shared__ __attribute__((aligned(16))) uint32_t s_par[par_lds_dwords<CORE>()];
    __shared__ double s_lut[VOCAB];
    __shared__ uint64_t s_lower[R], s_range[R], s_point[R];
    __shared__ int64_t s_woff[R], s_toff[R];
    __shared__ int32_t s_rpos[R], s_wcnt[R], s_len[R], s_stat[R];
    // which chunk of the row is current (bit 0: the second one; bit 1: the
    // row has a second chunk) and the step at which it started
    __shared__ int32_t s_cur[R], s_start[R];
    __shared__ uint32_t s_wbuf[OV ? R * WBUF : 1];
    __shared__ int32_t s_wbase[OV ? R : 1];
    __shared__ int32_t s_maxlen, s_xerr;
    __shared__ int32_t s_red[P == 8 ? 2 * 16 * 64 : 1];   // partial layer-0 sums of the split decode
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int q4 = lane >> 4, u = lane & 15;
    const int slice = P > 1 ? (int)(blockIdx.x % P) : 0;
    const int64_t group = blockIdx.x / P, c0 = group * R;
    const bool writer = slice == 0;   // the workgroup that writes tokens, status and state
    if (threadIdx.x == 0) {
        s_maxlen = 0;
        s_xerr = 0;
    }
    __syncthreads();
    // The workgroup's step count first, from the lengths alone: a later
    // segment past it returns before reading any coder state, because the
    // segment that finished these rows saved none (the state buffer then
    // holds another call's rows, or nothing).
    for (int r = threadIdx.x; r < R; r += THREADS) {
        const int64_t c = c0 + r;
        const bool in = c < n_chunks;
        // (the plain core's token ring cannot hold the start-of-sequence token)
        const bool paired = PIPE && in && c >= n_chunks - n_second;
        const int32_t len1 = in ? lengths[c] : 0;
        const int32_t len2 = paired ? lengths[2 * n_chunks - 1 - c] : 0;
        // (a second chunk starts one step after the first ends)
        atomicMax(&s_maxlen, max(len1, 0) + max(len2, 0) + (paired && len1 > 0 ? 1 : 0));
    }
    __syncthreads();
    const int32_t maxlen = s_maxlen;
    const int32_t t_stop = min(maxlen, t_end);
    // a later segment past this workgroup's longest row: an earlier one
    // finished its chunks and wrote their status
    if (t_begin > 0 && t_begin >= t_stop) return;
    // Here t_begin < t_stop <= maxlen, so the previous segment (if any) ran
    // this workgroup with t_stop < maxlen and saved every row's state.
    for (int r = threadIdx.x; r < R; r += THREADS) {
        const int64_t c = c0 + r;
        const bool in = c < n_chunks;
        const bool paired = PIPE && in && c >= n_chunks - n_second;
        const int32_t len1 = in ? lengths[c] : 0;
        int32_t cur = 0, start = 0;
        if (t_begin > 0 && in) {
            cur = state[c].cur;
            start = state[c].start;
        } else if (paired && len1 <= 0) {
            if (writer) status[c] = 0;   // an empty first chunk: the second one starts at once
            cur = 1;
        }
        const int64_t cc = cur ? 2 * n_chunks - 1 - c : c;
        int32_t len = 0, cnt = 0;
        int64_t woff = 0, toff = 0;
        if (in) {
            len = lengths[cc];
            cnt = word_cnt[cc];
            woff = word_off[cc];
            toff = tok_off[cc];
        }
        if (t_begin == 0 || !in) {
            int take;
            s_point[r] = dec_init_point(words + woff, cnt, take);
            s_lower[r] = 0ull;
            s_range[r] = ~0ull;
            s_rpos[r] = take;
            s_stat[r] = 0;
        } else {
            // a later segment: the state the previous one left
            const DecState d = state[c];
            s_lower[r] = d.lower;
            s_range[r] = d.range;
            s_point[r] = d.point;
            s_rpos[r] = d.rpos;
            s_stat[r] = d.stat;
        }
        s_wcnt[r] = cnt;
        s_woff[r] = woff;
        s_toff[r] = toff;
        s_len[r] = len;
        s_cur[r] = cur | (paired ? 2 : 0);   // bit 1: the row has a second chunk
        s_start[r] = start;
    }
    load_emb_lds(M.emb, s_emb);
    load_lut_lds(M.lut, s_lut);
    if constexpr (P > 1) split_params_init(M, s_par, split_ntile<P>(slice, wave), wave, lane);
    else mlp_tile_init<CORE>(M, s_par, wave, lane);
    __syncthreads();
    if (t_begin > 0) {
        // the context ring: the 64 tokens before t_begin, already written to
        // `tokens` by the previous segment (segments end on multiples of 64,
        // where the ring is flushed)
        for (int i = threadIdx.x; i < R * WIN; i += THREADS) {
            const int r = i / WIN;
            const int32_t tp = t_begin - WIN + (i % WIN), rs = tp - s_start[r];
            if (tp >= 0 && rs < s_len[r]) {
                // steps before the current chunk started are its start-of-sequence context
                const int v = rs >= 0 ? (int)tokens[s_toff[r] + rs] : SOS;
                s_ring[r * WIN + (tp & (WIN - 1))] = (uint8_t)v;
                if constexpr (PIPE) s_apos[apos_at(r, tp)] = (uint16_t)emb_off(v, 0);
            }
        }
        __syncthreads();
    }
    const DecCtx<R> ctx{s_act, s_lut, s_lower, s_range, s_point, s_woff, s_toff, s_rpos, s_wcnt, s_len, s_stat,
                        s_cur, s_start, s_wbase, s_wbuf, s_ring, s_apos, words, word_off, tok_off, word_cnt,
                        lengths, tokens, status, n_chunks, c0, writer};
    // the epilogue of step t (EPI_N row groups per iteration)
    auto epilogue = [&](int32_t t) {
        // EPI_N row groups (gi + n * WAVES) per iteration, see row_freq.
        // _decode_partition (cpu_entropy_coding.py:230-266): every lane of a
        // row computes the row's quantile; the lane whose 16 symbols hold it
        // publishes them in the row's slot and the lane that finds the
        // symbol there (its interval holds the quantile) stores the new
        // state.  The word a renormalisation would shift in is loaded before
        // the frequency work (whether or not this step needs it) so its
        // latency is hidden.
        uint32_t *slots = s_slot + wave * (EPI_N * 4 * SLOT_DWORDS);
        for (int gi = wave; gi < R / 4; gi += EPI_N * WAVES) {
            int rr[EPI_N];
            uint64_t lower[EPI_N], range[EPI_N], point[EPI_N];
            int32_t rpos[EPI_N];
            uint32_t wnext[EPI_N];
            bool active[EPI_N], last1[EPI_N];
            v4i raw[EPI_N];
#pragma unroll
            for (int n = 0; n < EPI_N; ++n) {
                const int r = (gi + n * WAVES) * 4 + q4;
                rr[n] = r;
                const int32_t rs = t - s_start[r], len = s_len[r];
                active[n] = rs >= 0 && rs < len && s_stat[r] == 0;
                last1[n] = s_cur[r] == 2 && rs == len - 1;   // the row's first chunk ends with this step
                lower[n] = s_lower[r];
                range[n] = s_range[r];
                point[n] = s_point[r];
                rpos[n] = s_rpos[r];
                wnext[n] = rpos[n] < s_wcnt[r] ? words[s_woff[r] + rpos[n]] : 0u;
                raw[n] = *(const v4i *)(s_act + act_at<PIPE>(r, u));
            }
            RowFreq fr[EPI_N];
            row_freq<EPI_N>(raw, s_lut, u, fr);
            uint32_t q[EPI_N];
            bool ok[EPI_N];
#pragma unroll
            for (int n = 0; n < EPI_N; ++n) {
                const uint64_t scale = range[n] >> 24;
                q[n] = 0;
                ok[n] = scale != 0 && dec_quantile(point[n] - lower[n], scale, q[n]);
                if (ok[n] && q[n] - fr[n].ex < fr[n].tot) slot_put(slots + (n * 4 + q4) * SLOT_DWORDS, fr[n], u);
            }
            slot_sync();
#pragma unroll
            for (int n = 0; n < EPI_N; ++n) {
                const int r = rr[n];
                uint32_t cum, freq;
                const uint32_t owner = slot_get(slots + (n * 4 + q4) * SLOT_DWORDS, u, cum, freq);
                if (active[n] && ok[n] && q[n] - cum < freq) {
                    const uint64_t scale = range[n] >> 24;
                    uint64_t lo = lower[n] + mul_scale(scale, cum), ra = mul_scale(scale, freq), pt = point[n];
                    int32_t rp = rpos[n];
                    if (ra < (1ull << 32)) {
                        lo <<= 32;
                        ra <<= 32;
                        pt = (pt << 32) | wnext[n];
                        rp += 1;
                    }
                    s_lower[r] = lo;
                    s_range[r] = ra;
                    s_point[r] = pt;
                    s_rpos[r] = rp;
                    s_ring[r * WIN + (t & (WIN - 1))] = (uint8_t)(owner * 16 + u);
                    if constexpr (PIPE) s_apos[apos_at(r, t)] = (uint16_t)emb_off(owner * 16 + u, 0);
                }
                if (active[n] && !ok[n] && u == 0) s_stat[r] = SC_STATUS_INVALID_STREAM;
                if (last1[n]) dec_switch<R, PIPE, OV>(ctx, r, u, t);
            }
        }
    };
    // the end of step t (after the barrier that ends its epilogue)
    auto flush = [&](int32_t t) {
        // every 64 steps (and at the end) the ring holds the last 64 tokens
        // of each chunk: one wavefront per chunk writes them as one 64-byte
        // run instead of a byte per step
        if (writer && ((t & (WIN - 1)) == WIN - 1 || t == maxlen - 1)) {
            const int32_t p = (t & ~(WIN - 1)) + lane;
            for (int r = wave; r < R; r += WAVES) {
                const int32_t rs = p - s_start[r];
                if (p <= t && rs >= 0 && rs < s_len[r]) tokens[s_toff[r] + rs] = s_ring[r * WIN + lane];
            }
        }
        if constexpr (OV) {
            // the next 64 words of every row
            if ((t & (WIN - 1)) == WIN - 1) {
                for (int r = wave; r < R; r += WAVES) {
                    const int32_t base = s_rpos[r], cnt = s_wcnt[r];
                    s_wbuf[r * WBUF + lane] = base + lane < cnt ? words[s_woff[r] + base + lane] : 0u;
                    if (lane == 0) s_wbase[r] = base;
                }
            }
        }
    };
    if constexpr (OV) {
        // Step t: the MLP after layer 0 (pipe_rest), then layer 0 of step
        // t + 1 with step t's epilogue beside it and, between its last two
        // positions, the barrier that publishes step t's symbols and the
        // end of step t.  The segment's first layer 0 runs alone, its last
        // epilogue after the MLP.
        constexpr bool UNI = CORE == CORE_PIPE_UNI;
        constexpr int NG = R / 16;              // row groups of four rows per wave
        // side VALU instructions per MFMA, and one side piece per layer-0
        // k-step (up to 6 / 8 VALU per MFMA or a piece on every second
        // k-step measured the same, within 0.5%)
        constexpr int XV = RT >= 3 ? 4 : 6;
        constexpr int SP = 1;
        v16i accA[PNT][RT], accB[PNT][RT];
        uint32_t prl[Slot<UNI>::LANE];
        int32_t tl0 = t_begin;                  // the step of the layer 0 in flight
        auto apos0 = [&](int r, int p) {
            if (tl0 + p < WIN) return emb_off(SOS, 0);
            return (int)s_apos[apos_at(r, tl0 + p)];
        };
        for (int r = wave; r < R; r += WAVES) {
            const int32_t base = s_rpos[r], cnt = s_wcnt[r];
            s_wbuf[r * WBUF + lane] = base + lane < cnt ? words[s_woff[r] + base + lane] : 0u;
            if (lane == 0) s_wbase[r] = base;
        }
        {
            NoSide none;
            pipe_layer0_ov<RT, UNI, XV, SP>(M, s_emb, s_par, apos0, accA, accB, prl, wave, lane, 0, none, [] {});
        }
        uint32_t *wslots = s_slot + wave * (EPI_N * 4 * SLOT_DWORDS);
        for (int32_t t = t_begin; t < t_stop; ++t) {
            pipe_rest<RT, UNI>(M, s_act, s_par, accA, accB, prl, wave, lane);
            if (t + 1 < t_stop) {
                tl0 = t + 1;
                DecEpiSide<R, PIPE> side(ctx, wslots, t, wave, lane);
                pipe_layer0_ov<RT, UNI, XV, SP>(M, s_emb, s_par, apos0, accA, accB, prl, wave, lane, NG, side, [&] {
                    __syncthreads();
                    flush(t);
                });
            } else {
                epilogue(t);
                __syncthreads();
                flush(t);
            }
        }
    } else {
        L0Carry l0c;   // (split decode) layer 0 carried between steps
        l0c.have = false;
        for (int32_t t = t_begin; t < t_stop; ++t) {
            auto apos = [&](int r, int p) {
                if (t + p < WIN) return emb_off(SOS, 0);
                if constexpr (PIPE) return (int)s_apos[apos_at(r, t + p)];
                else return emb_off(s_ring[r * WIN + ((t + p) & (WIN - 1))], 0);
            };
            if constexpr (P > 1) {
                // the next step's window, of which all but the last position is known
                auto apos_next = [&](int r, int p) {
                    if (t + 1 + p < WIN) return emb_off(SOS, 0);
                    return (int)s_apos[apos_at(r, t + 1 + p)];
                };
                mlp_rows_split<P>(M, s_emb, s_act, s_par, apos, apos_next, t + 1 < t_stop, l0c, wave, lane,
                                  xch + group * XCH_GROUP, (int32_t *)(xch + (int64_t)gridDim.x / P * XCH_GROUP) + group * P,
                                  slice, t, spin_max, &s_xerr, s_red);
            } else
                mlp_tile<CORE, RT>(M, s_emb, s_act, s_par, apos, wave, lane);
            epilogue(t);
            __syncthreads();
            flush(t);
        }
    }
    if (!writer) return;
    // a split decode whose exchange timed out: every chunk of the group
    // (both of a paired row) fails, and a saved state carries the failure
    // into later segments
    const bool xerr = P > 1 && s_xerr != 0;
    for (int r = threadIdx.x; r < R; r += THREADS)
        if (c0 + r < n_chunks) {
            const int64_t c = c0 + r;
            const int cur = s_cur[r] & 1;
            const int32_t stat = xerr ? SC_STATUS_SYNC_TIMEOUT : s_stat[r];
            status[cur ? 2 * n_chunks - 1 - c : c] = stat;
            if (xerr && (s_cur[r] & 2)) status[cur ? c : 2 * n_chunks - 1 - c] = stat;
            if (t_stop < maxlen)
                state[c0 + r] = DecState{s_lower[r], s_range[r], s_point[r], s_rpos[r], stat, cur, s_start[r]};
        }
}

}  // namespace
}  // namespace sc
