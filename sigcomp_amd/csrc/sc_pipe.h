// sc_pipe.h -- software-pipelined MLP core for tiles of up to 128 rows.
//
// The plain core (mlp_rows) requantises a layer after its GEMM, with the
// matrix cores idle.  Here every layer runs as two passes of two n-tiles per
// wave and the requantisation of one pass is interleaved, instruction by
// instruction, with the MFMA stream of the next GEMM segment:
//
//   pass p of wave w computes n-tiles 8p + 2w, 8p + 2w + 1, so pass 0 of all
//   waves yields features 0..255 (region A of an activation row, the next
//   layer's k-tiles 0..7) and pass 1 features 256..511 (region B, k-tiles
//   8..15).  Per hidden layer l (steps v = 0..31: pass 0 k 0..15, pass 1 k 0..15):
//
//     v  0.. 7  pass 0, k-tiles 0..7 (region A)   || requant of layer l-1 pass 1
//               store layer l-1 pass 1 -> region B; barrier
//     v  8..15  pass 0, k-tiles 8..15 (region B)
//     v 16..31  pass 1, all k-tiles                || requant of layer l pass 0
//               barrier; store layer l pass 0 -> region A; barrier
//
//   A region is overwritten only after a barrier that ends every read of it.
//   Weight fragments are prefetched PPD k-steps ahead across pass and layer
//   boundaries.  Accumulators of the two passes take 2 x 2 x RT x 16 AGPRs
//   (256 for RT = 4).
//
// With UNI (CORE_PIPE_UNI: per-tensor constants on every layer) every
// requantisation is rq_words_uni / rq_pass_uni and the parameter slots hold
// only biases; else the parameter slots hold whole parameter blocks and the
// requantisation is rq_bytes_pc / rq_pass_pc (per-channel constants, the
// same four instructions per value).
// Requires every layer to take the 32-bit requant path (LayerDev::fast), ReLU
// on all layers but the last, and 512-wide hidden layers (ModelDev::pipe).
#pragma once

#include "sc_device.h"

namespace sc {

constexpr int PNT = 2;                               // n-tiles per pass
// Weight prefetch distance in k-steps: 8 where the registers allow (tiles
// of up to 96 rows), else 4.  Both divide the 16 and 32 k-steps of a pass,
// as the two-set register rotation needs.
template <int RT>
constexpr int ppd() { return RT <= 3 ? 8 : 4; }
// Parameter slot geometry.  The per-channel core keeps whole parameter
// blocks (bias, m0, shift) in its slots; the per-tensor core (UNI) only the
// bias of each n-tile, its m0, shift and clamp bounds being per-layer
// scalars (7.7 KB less LDS).
template <bool UNI>
struct Slot {
    static constexpr int TD = UNI ? 32 : PAR_DWORDS;   // dwords per n-tile
    static constexpr int BLK = PNT * TD;               // parameter dwords of one pass
    static constexpr int LANE = (BLK + 63) / 64;       // of them per lane when copied
};
// LDS parameter slots per wave: slot_p0(l) holds the pass-0 parameter blocks
// of layer l, slot_p1(l) its pass-1 blocks.  Layers l >= 1 use four slots by
// parity: layer l's pass-0 blocks are written during layer l-1 (layer l's
// first MFMAs start from their bias tiles), its pass-1 blocks during layer l
// (read until layer l+1 has requantised layer l's pass 1).  Layer 0's two
// slots are written once per kernel (pipe_params_init), before the first MLP
// evaluation, so that its bias tiles are in LDS when each evaluation starts.
constexpr int PIPE_SLOTS = 6;
template <bool UNI>
constexpr int pipe_par_dwords() { return WAVES * PIPE_SLOTS * Slot<UNI>::BLK; }
__device__ __forceinline__ int slot_p0(int l) { return l == 0 ? 4 : (l & 1); }
__device__ __forceinline__ int slot_p1(int l) { return l == 0 ? 5 : 2 + (l & 1); }

// Bias of n-tile j of a parameter block as an accumulator tile: element v of
// a lane in half g (= lane / 32) is the bias of feature 8*(v/4) + 4*g + v%4,
// the feature that accumulator element holds.  A GEMM whose first MFMA
// accumulates onto it ends with acc + bias (int32, wrapping like the
// reference's add), so the requantisation skips the bias add.
template <bool UNI>
__device__ __forceinline__ v16i bias_tile(const uint32_t *blk, int j, int g) {
    const uint32_t *pj = blk + j * Slot<UNI>::TD + 4 * g;
    v16i t;
#pragma unroll
    for (int gg = 0; gg < 4; ++gg) {
        const v4i x = *(const v4i *)(pj + 8 * gg);
#pragma unroll
        for (int e = 0; e < 4; ++e) t[4 * gg + e] = x[e];
    }
    return t;
}

// Requant parameters (M0, clamp bounds and shifts; the bias is already in
// the accumulators) of packed group g of n-tile j (lane half g2).
struct RqPar {
    v4i mm, hi;
    uint32_t sh;   // four shifts - 32, one byte each
};

__device__ __forceinline__ RqPar rq_par(const uint32_t *blk, int j, int g, int g2) {
    const uint32_t *pj = blk + j * PAR_DWORDS;
    const int o = 8 * g + 4 * g2;
    RqPar p;
    p.mm = *(const v4i *)(pj + 32 + o);
    p.hi = *(const v4i *)(pj + 72 + o);
    p.sh = pj[64 + (o >> 2)];
    return p;
}

// Byte E of `packed` = y >> (byte E of sh): the shift amount is read out of
// the packed shifts by the SDWA source select, the result written into its
// byte by the destination select (byte 0 clears the others).  Logical shift
// after a ReLU clamp (y >= 0), else arithmetic.
template <bool RELU, int E>
__device__ __forceinline__ void rq_insert_pc(uint32_t &packed, uint32_t sh, int y) {
#define SC_RQ_INS(OP, B, U, C)                                                                               \
    asm(OP "_sdwa %0, %1, %2 dst_sel:BYTE_" #B " dst_unused:" U " src0_sel:BYTE_" #B " src1_sel:DWORD" \
        : C(packed) : "v"(sh), "v"(y))
    if constexpr (RELU) {
        if constexpr (E == 0) SC_RQ_INS("v_lshrrev_b32", 0, "UNUSED_PAD", "=v");
        else if constexpr (E == 1) SC_RQ_INS("v_lshrrev_b32", 1, "UNUSED_PRESERVE", "+v");
        else if constexpr (E == 2) SC_RQ_INS("v_lshrrev_b32", 2, "UNUSED_PRESERVE", "+v");
        else SC_RQ_INS("v_lshrrev_b32", 3, "UNUSED_PRESERVE", "+v");
    } else {
        if constexpr (E == 0) SC_RQ_INS("v_ashrrev_i32", 0, "UNUSED_PAD", "=v");
        else if constexpr (E == 1) SC_RQ_INS("v_ashrrev_i32", 1, "UNUSED_PRESERVE", "+v");
        else if constexpr (E == 2) SC_RQ_INS("v_ashrrev_i32", 2, "UNUSED_PRESERVE", "+v");
        else SC_RQ_INS("v_ashrrev_i32", 3, "UNUSED_PRESERVE", "+v");
    }
#undef SC_RQ_INS
}

// Bytes E0 <= e < E1 of every row tile's word pk[i][g] (features 8g +
// 4*g2 + e, bias included in the accumulators), per-channel constants of a
// layer on the 32-bit path: x = hi32(a * m0) clamped to [lo, hi] before the
// shift (lo = 0 with ReLU, else -hi - 1 = max(-128 * 2**shift, -2**31)), as
// the per-tensor form below argues; four VALU instructions per value with
// the accumulator read.  The inserts run across the row tiles' words; the
// first byte's (e = 0) clears the rest of its word, so E0 = 0 comes first.
template <bool RELU, int E0, int E1, int RT>
__device__ __forceinline__ void rq_bytes_pc(const v16i (&acc)[RT], int g, const RqPar &p, uint32_t (&pk)[RT][4]) {
    int y[4][RT];
#pragma unroll
    for (int e = E0; e < E1; ++e)
#pragma unroll
        for (int i = 0; i < RT; ++i) {
            const int x = __mulhi(acc[i][4 * g + e], p.mm[e]), hi = p.hi[e];
            if constexpr (RELU) {
                asm("v_med3_i32 %0, %1, 0, %2" : "=v"(y[e][i]) : "v"(x), "v"(hi));
            } else {
                const int lo = ~hi;
                asm("v_med3_i32 %0, %1, %2, %3" : "=v"(y[e][i]) : "v"(x), "v"(lo), "v"(hi));
            }
        }
    static_for<E1 - E0>([&](auto ec) __attribute__((always_inline)) {
        constexpr int e = E0 + decltype(ec)::value;
#pragma unroll
        for (int i = 0; i < RT; ++i) rq_insert_pc<RELU, e>(pk[i][g], p.sh, y[e][i]);
    });
}

// All n-tiles and row tiles of a pass, per-channel constants from the LDS
// parameter blocks at `blk` (the requantisations not interleaved with MFMAs).
template <bool RELU, int RT>
__device__ __forceinline__ void rq_pass_pc(const v16i (&acc)[PNT][RT], const uint32_t *blk, int lane,
                                           uint32_t (&pk)[PNT][RT][4]) {
    const int g2 = lane >> 5;
#pragma unroll
    for (int j = 0; j < PNT; ++j)
        static_for<4>([&](auto gc) __attribute__((always_inline)) {
            constexpr int g = decltype(gc)::value;
            rq_bytes_pc<RELU, 0, 4, RT>(acc[j], g, rq_par(blk, j, g, g2), pk[j]);
#pragma unroll
            for (int i = 0; i < RT; ++i) asm volatile("" : "+v"(pk[j][i][g]));
        });
}

// Per-tensor constants (LayerDev::uni): x = hi32(a * m0) is clamped to
// [0, uhi] BEFORE the shift, uhi = 128 * 2**sh - 1 (or 2**31 - 1 when that
// overflows; then x >> sh < 128 anyway).  floor(x / 2**sh) is monotone in
// x, so this equals min(max(x >> sh, 0), 127) of requant_u8_fast; the shift
// then writes each byte straight into the packed word (SDWA destination
// select; byte 0 clears the others).  Four VALU instructions per value with
// the accumulator read, and no per-channel operands.
// Without ReLU (the output layer) the clamp is to [ulo, uhi], ulo =
// -128 * 2**sh (or -2**31), and the shift is arithmetic.
struct RqUni {
    int m0, hi, sh, lo;
};
__device__ __forceinline__ RqUni rq_uni(const LayerDev &L) {
    return RqUni{__builtin_amdgcn_readfirstlane(L.um0), __builtin_amdgcn_readfirstlane(L.uhi),
                 __builtin_amdgcn_readfirstlane(L.ush), __builtin_amdgcn_readfirstlane(L.ulo)};
}
template <bool RELU, int E>
__device__ __forceinline__ void rq_insert_uni(uint32_t &packed, int sh, int y) {
    if constexpr (RELU) {   // y >= 0
        if constexpr (E == 0)
            asm("v_lshrrev_b32_sdwa %0, %1, %2 dst_sel:BYTE_0 dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:DWORD"
                : "=v"(packed) : "v"(sh), "v"(y));
        else if constexpr (E == 1)
            asm("v_lshrrev_b32_sdwa %0, %1, %2 dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
                : "+v"(packed) : "v"(sh), "v"(y));
        else if constexpr (E == 2)
            asm("v_lshrrev_b32_sdwa %0, %1, %2 dst_sel:BYTE_2 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
                : "+v"(packed) : "v"(sh), "v"(y));
        else
            asm("v_lshrrev_b32_sdwa %0, %1, %2 dst_sel:BYTE_3 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
                : "+v"(packed) : "v"(sh), "v"(y));
    } else {
        if constexpr (E == 0)
            asm("v_ashrrev_i32_sdwa %0, %1, %2 dst_sel:BYTE_0 dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:DWORD"
                : "=v"(packed) : "v"(sh), "v"(y));
        else if constexpr (E == 1)
            asm("v_ashrrev_i32_sdwa %0, %1, %2 dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
                : "+v"(packed) : "v"(sh), "v"(y));
        else if constexpr (E == 2)
            asm("v_ashrrev_i32_sdwa %0, %1, %2 dst_sel:BYTE_2 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
                : "+v"(packed) : "v"(sh), "v"(y));
        else
            asm("v_ashrrev_i32_sdwa %0, %1, %2 dst_sel:BYTE_3 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
                : "+v"(packed) : "v"(sh), "v"(y));
    }
}
// Features 8g + 4*g2 + e (e = 0..3) of accumulator tiles acc[i], I0 <= i <
// I1 -> packed words pk[i][g].  The inserts run byte by byte across the
// words, so that consecutive inserts write different registers.
template <bool RELU, int I0, int I1, int RT>
__device__ __forceinline__ void rq_words_uni(const v16i (&acc)[RT], int g, const RqUni &p, uint32_t (&pk)[RT][4]) {
    int y[4][RT];
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int i = I0; i < I1; ++i) {
            if constexpr (RELU)
                asm("v_med3_i32 %0, %1, 0, %2" : "=v"(y[e][i]) : "v"(__mulhi(acc[i][4 * g + e], p.m0)), "s"(p.hi));
            else
                asm("v_med3_i32 %0, %1, %2, %3"
                    : "=v"(y[e][i]) : "v"(__mulhi(acc[i][4 * g + e], p.m0)), "v"(p.lo), "s"(p.hi));
        }
    static_for<4>([&](auto ec) __attribute__((always_inline)) {
        constexpr int e = decltype(ec)::value;
#pragma unroll
        for (int i = I0; i < I1; ++i) rq_insert_uni<RELU, e>(pk[i][g], p.sh, y[e][i]);
    });
}
// Bytes E0 <= e < E1 of every row tile's word pk[i][g] (features
// 8g + 4*g2 + e), the inserts running across the row tiles' words.  The
// first byte's insert (e = 0) clears the rest of its word, so E0 = 0 comes
// first.
template <bool RELU, int E0, int E1, int RT>
__device__ __forceinline__ void rq_bytes_uni(const v16i (&acc)[RT], int g, const RqUni &p, uint32_t (&pk)[RT][4]) {
    int y[4][RT];
#pragma unroll
    for (int e = E0; e < E1; ++e)
#pragma unroll
        for (int i = 0; i < RT; ++i) {
            if constexpr (RELU)
                asm("v_med3_i32 %0, %1, 0, %2" : "=v"(y[e][i]) : "v"(__mulhi(acc[i][4 * g + e], p.m0)), "s"(p.hi));
            else
                asm("v_med3_i32 %0, %1, %2, %3"
                    : "=v"(y[e][i]) : "v"(__mulhi(acc[i][4 * g + e], p.m0)), "v"(p.lo), "s"(p.hi));
        }
    static_for<E1 - E0>([&](auto ec) __attribute__((always_inline)) {
        constexpr int e = E0 + decltype(ec)::value;
#pragma unroll
        for (int i = 0; i < RT; ++i) rq_insert_uni<RELU, e>(pk[i][g], p.sh, y[e][i]);
    });
}
// All n-tiles and row tiles of a pass (the requantisations that are not
// interleaved with MFMAs: layer 0's pass 0 and the output layer).
template <bool RELU, int RT>
__device__ __forceinline__ void rq_pass_uni(const v16i (&acc)[PNT][RT], const RqUni &p, uint32_t (&pk)[PNT][RT][4]) {
#pragma unroll
    for (int j = 0; j < PNT; ++j)
        static_for<4>([&](auto gc) __attribute__((always_inline)) {
            constexpr int g = decltype(gc)::value;
            rq_words_uni<RELU, 0, RT>(acc[j], g, p, pk[j]);
#pragma unroll
            for (int i = 0; i < RT; ++i) asm volatile("" : "+v"(pk[j][i][g]));
        });
}

__device__ __forceinline__ v4i wload_s(__amdgpu_buffer_rsrc_t rs, int voff, int soff) {
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    v4u x = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, 0);
    return (v4i)x;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t layer_rsrc(const LayerDev &L) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)L.w, (short)0, L.bytes, 0x00020000);
}

// Parameter blocks of one pass (n-tiles nt0, nt0 + 1) into registers / LDS.
// (the first Slot<UNI>::TD dwords of each n-tile's block)
template <bool UNI>
__device__ __forceinline__ void par_fetch(const uint32_t *gpar, int nt0, int lane, uint32_t (&pr)[Slot<UNI>::LANE]) {
    using S = Slot<UNI>;
#pragma unroll
    for (int d = 0; d < S::LANE; ++d) {
        const int idx = d * 64 + lane;
        pr[d] = idx < S::BLK ? gpar[(nt0 + idx / S::TD) * PAR_DWORDS + idx % S::TD] : 0u;
    }
}
template <bool UNI>
__device__ __forceinline__ void par_put(uint32_t *blk, const uint32_t (&pr)[Slot<UNI>::LANE], int lane) {
#pragma unroll
    for (int d = 0; d < Slot<UNI>::LANE; ++d)
        if (d * 64 + lane < Slot<UNI>::BLK) blk[d * 64 + lane] = pr[d];
}

// Layer 0's parameter blocks (read by every MLP evaluation of the kernel)
// into their slots; the caller's next barrier makes them visible.
template <bool UNI>
__device__ __forceinline__ void pipe_params_init(const ModelDev &M, uint32_t *s_par, int wave, int lane) {
    constexpr int BLK = Slot<UNI>::BLK;
    uint32_t *s_parw = s_par + wave * PIPE_SLOTS * BLK;
    uint32_t pr[Slot<UNI>::LANE];
    par_fetch<UNI>(M.layer[0].par, 2 * wave, lane, pr);
    par_put<UNI>(s_parw + slot_p0(0) * BLK, pr, lane);
    par_fetch<UNI>(M.layer[0].par, 8 + 2 * wave, lane, pr);
    par_put<UNI>(s_parw + slot_p1(0) * BLK, pr, lane);
}

// Activation rows of the pipelined core are padded to PACT_ROW bytes instead
// of swizzled: 16 consecutive rows reading the same 16-byte chunk start 16
// bytes apart modulo the 256-byte bank window, so they hit 16 different bank
// groups, and chunk c of a row sits at a constant offset c*16 from the row
// base (an immediate of the LDS instruction).
constexpr int PACT_ROW = ACT_ROW + 16;
__device__ __forceinline__ int pact_off(int r, int chunk) { return r * PACT_ROW + chunk * 16; }

// B fragments of hidden k-tile kt for the RT row tiles; `base` = pact_off(rl, g).
template <int RT>
__device__ __forceinline__ void read_b(const uint8_t *s_act, int base, int kt, v4i (&b)[RT]) {
#pragma unroll
    for (int i = 0; i < RT; ++i) b[i] = *(const v4i *)(s_act + base + i * 32 * PACT_ROW + kt * 32);
}

// Packed results in the padded layout: hidden order (as store_packed_perm)
// and natural order (as store_packed).
template <int RT>
__device__ __forceinline__ void pstore_perm(const uint32_t (&pk)[PNT][RT][4], int nt0, uint8_t *s_act, int lane) {
    const int rl = lane & 31, g2 = lane >> 5;
#pragma unroll
    for (int j = 0; j < PNT; ++j)
#pragma unroll
        for (int i = 0; i < RT; ++i) {
            const v4i v = {(int)pk[j][i][0], (int)pk[j][i][1], (int)pk[j][i][2], (int)pk[j][i][3]};
            *(v4i *)(s_act + pact_off(i * 32 + rl, (nt0 + j) * 2 + g2)) = v;
        }
}
template <int RT>
__device__ __forceinline__ void pstore_natural(const uint32_t (&pk)[PNT][RT][4], int nt0, uint8_t *s_act, int lane) {
    const int rl = lane & 31, g2 = lane >> 5;
#pragma unroll
    for (int j = 0; j < PNT; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int i = 0; i < RT; ++i)
                *(uint32_t *)(s_act + pact_off(i * 32 + rl, 0) + (nt0 + j) * 32 + 8 * g + 4 * g2) = pk[j][i][g];
}

// Instruction order of one pipelined k-step: the step's LDS reads and weight
// loads are spread over its first MFMAs, and VA VALU instructions (the
// interleaved requantisation) follow every MFMA.
template <int MF, int DS, int VM, int VA>
__device__ __forceinline__ void pipe_schedule() {
    static_for<MF>([&](auto mc) __attribute__((always_inline)) {
        constexpr int m = decltype(mc)::value;
        if constexpr (m < DS) __builtin_amdgcn_sched_group_barrier(0x100, DS > MF && m == MF - 1 ? DS - m : 1, 0);
        if constexpr (m < VM) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if constexpr (VA > 0) __builtin_amdgcn_sched_group_barrier(0x002, VA, 0);
    });
}

// One hidden layer l (LASTL = false) or the output layer (LASTL = true, one
// pass: n-tiles 2w, 2w+1 = logits 64w .. 64w+63, stored in natural order).
// Entry: accB = layer l-1 pass 1 (bias included, not yet requantised,
// parameters in slot_p1(l-1)), region A = layer l-1 pass 0 (visible to all
// waves), slot_p0(l) = this layer's pass-0 parameters, w[0][*] = this
// layer's first PPD weight k-steps.  Exit: accB = this layer's pass 1,
// slot_p1(l) = its parameters, slot_p0(l+1) = the next layer's pass-0
// parameters, region A = this layer's pass 0 (visible), w[0][*] = the next
// layer's first k-steps.  Both passes' GEMMs start from their bias tiles.
// FRESH: the whole previous layer is already in regions A and B (visible),
// accB holds nothing to requantise (the first layer after a layer 0 whose
// features were gathered from several workgroups).
template <int RT, bool LASTL, bool UNI, bool FRESH = false>
__device__ __forceinline__ void pipe_hidden(const LayerDev &Lp, const LayerDev &L, const LayerDev &Ln, uint8_t *s_act,
                                            uint32_t *s_parw, int l, v16i (&accA)[PNT][RT],
                                            v16i (&accB)[PNT][RT], v4i (&w)[2][ppd<RT>()][PNT],
                                            uint32_t (&pk)[PNT][RT][4], int wave, int lane) {
    constexpr int PPD = ppd<RT>();
    constexpr int NV = LASTL ? KTH : 2 * KTH;
    constexpr int MF = PNT * RT;
    const int g = lane >> 5, voff = lane * 16;
    const int bbase = pact_off(lane & 31, g);
    const __amdgpu_buffer_rsrc_t rs = layer_rsrc(L);
    const __amdgpu_buffer_rsrc_t rsn = layer_rsrc(Ln);
    const int nb0 = 2 * wave, nb1 = 8 + 2 * wave;   // n-tile bases of pass 0 / pass 1
    constexpr int BLK = Slot<UNI>::BLK;
    const uint32_t *prev1 = s_parw + slot_p1(l - 1) * BLK;
    const uint32_t *cur0 = s_parw + slot_p0(l) * BLK;
    uint32_t *cur1 = s_parw + slot_p1(l) * BLK;
    uint32_t *next0 = s_parw + slot_p0(l + 1) * BLK;
    uint32_t pr1[Slot<UNI>::LANE], prn[Slot<UNI>::LANE];
    if constexpr (!LASTL) {
        par_fetch<UNI>(L.par, nb1, lane, pr1);
        par_fetch<UNI>(Ln.par, nb0, lane, prn);
    }
    v4i b[2][RT];
    read_b<RT>(s_act, bbase, 0, b[0]);
    RqPar pp;
    if constexpr (!UNI) pp = rq_par(prev1, 0, 0, g);
    RqUni up{}, uc{};
    if constexpr (UNI) {
        up = rq_uni(Lp);
        uc = rq_uni(L);
    }
    v16i bias[PNT];
#pragma unroll
    for (int j = 0; j < PNT; ++j) bias[j] = bias_tile<UNI>(cur0, j, g);
    static_for<NV>([&](auto vc) __attribute__((always_inline)) {
        constexpr int v = decltype(vc)::value;
        constexpr int pass = v / KTH, kt = v % KTH, set = (v / PPD) & 1, slot = v % PPD;
        // one wait per k-step for its weight fragments (issued PPD steps
        // ago; the 2 * LANE parameter loads at the top of this function
        // are younger than the first PPD steps' fragments) and its B
        // fragments, instead of the compiler's wait before each first use
        wait_counts<(PPD - 1) * PNT + (v < PPD && !LASTL ? 2 * Slot<UNI>::LANE : 0), 0>();
        // next step's B fragments (none across a barrier)
        if constexpr (v != 7 && v != NV - 1) read_b<RT>(s_act, bbase, (kt + 1) % KTH, b[(kt + 1) & 1]);
        // weights PPD steps ahead: this layer, else the next layer's pass 0
        constexpr int vp = v + PPD;
        if constexpr (vp < NV) {
            constexpr int pp_ = vp / KTH, kp = vp % KTH;
#pragma unroll
            for (int j = 0; j < PNT; ++j)
                w[(vp / PPD) & 1][vp % PPD][j] = wload_s(rs, voff, (((pp_ ? nb1 : nb0) + j) * KTH + kp) * 1024);
        } else if constexpr (!LASTL) {
            constexpr int kn = vp - NV;
#pragma unroll
            for (int j = 0; j < PNT; ++j)
                w[(vp / PPD) & 1][vp % PPD][j] = wload_s(rsn, voff, ((nb0 + j) * KTH + kn) * 1024);
        }
        // side work: parameters one step ahead, then requantised words
        constexpr int VA = v < 8 ? (FRESH ? 0 : 12) : (!LASTL && v >= 16 ? 6 : 0);
        if constexpr (v < 8 && !FRESH) {
            constexpr int j = v / 4, gg = v % 4;
            if constexpr (UNI) {
                rq_words_uni<true, 0, RT>(accB[j], gg, up, pk[j]);
            } else {
                const RqPar cur = pp;
                if constexpr (v + 1 < 8) pp = rq_par(prev1, (v + 1) / 4, (v + 1) % 4, g);
                rq_bytes_pc<true, 0, 4, RT>(accB[j], gg, cur, pk[j]);
            }
        } else if constexpr (!LASTL && v >= 16) {
            constexpr int u = v - 16, j = u / 8, gg = (u / 2) % 4, h = u % 2;
            if constexpr (UNI) {
                rq_bytes_uni<true, 2 * h, 2 * h + 2, RT>(accA[j], gg, uc, pk[j]);
            } else {
                const RqPar cur = pp;
                if constexpr (u + 1 < 16) pp = rq_par(cur0, (u + 1) / 8, ((u + 1) / 2) % 4, g);
                rq_bytes_pc<true, 2 * h, 2 * h + 2, RT>(accA[j], gg, cur, pk[j]);
            }
        }
        // pass 1's bias tiles, one step before its first MFMAs
        if constexpr (!LASTL && v == KTH - 1) {
#pragma unroll
            for (int j = 0; j < PNT; ++j) bias[j] = bias_tile<UNI>(cur1, j, g);
        }
        // this step's MFMAs
        auto &acc = pass == 0 ? accA : accB;
#pragma unroll
        for (int j = 0; j < PNT; ++j)
#pragma unroll
            for (int i = 0; i < RT; ++i)
                acc[j][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(w[set][slot][j], b[kt & 1][i],
                                                                  kt == 0 ? bias[j] : acc[j][i], 0, 0, 0);
        pipe_schedule<MF, (v != 7 && v != NV - 1 ? RT : 0) + (UNI ? 0 : 3) + (v == KTH - 1 ? 4 * PNT : 0), PNT, VA>();
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (v == 7) {
            // layer l-1 pass 1 -> region B; this layer's pass-1 and the next
            // layer's pass-0 parameters -> LDS (the wave's own slots)
            if constexpr (!FRESH) pstore_perm<RT>(pk, nb1, s_act, lane);
            if constexpr (!LASTL) {
                par_put<UNI>(cur1, pr1, lane);
                par_put<UNI>(next0, prn, lane);
                if constexpr (!UNI) pp = rq_par(cur0, 0, 0, g);   // first parameters of the pass-0 requantisation
            }
            if constexpr (!FRESH) __syncthreads();
            read_b<RT>(s_act, bbase, 8, b[0]);
        }
    });
    if constexpr (LASTL) {
        if constexpr (UNI) rq_pass_uni<false, RT>(accA, rq_uni(L), pk);
        else rq_pass_pc<false, RT>(accA, cur0, lane, pk);
        __syncthreads();
        pstore_natural<RT>(pk, nb0, s_act, lane);
    } else {
        __syncthreads();
        pstore_perm<RT>(pk, nb0, s_act, lane);
    }
    __syncthreads();
}

// Layer 0 of ONE n-tile for one row tile (32 rows) over the NW window
// positions pf .. pf + NW - 1 (the whole window, or a part when several
// waves share the n-tile's k-tiles), the operands laid out as in
// gemm_layer0_map, with the weight fragments loaded D k-steps ahead: a wave
// keeps D fragments (D KB) in flight, as many as a wave of gemm_layer0_map
// keeps over its four n-tiles.  With one MFMA per k-step the LDS latency has
// to be hidden as well: a position's four B fragments are read one position
// ahead, its table address two positions ahead.  The accumulator starts
// from `init`.  The look-ahead stops at the range's last k-tile.  With
// `skip_last` (wave-uniform) the range's last position is loaded but not
// multiplied: its fragments are left in `wlast` for gemm_layer0_position
// once its token is known.
template <int D, int NW, class AposFn>
__device__ __forceinline__ v16i gemm_layer0_one(const WStream &ws, int nt, int pf, const uint8_t *s_emb, AposFn apos,
                                                const v16i &init, int lane, bool skip_last = false,
                                                v4i *wlast = nullptr) {
    constexpr int KS = EDIM / 32;   // k-steps per position
    constexpr int NP = D / KS;      // positions per loop body
    static_assert(D % KS == 0 && NP % 2 == 0 && NW % NP == 0 && NW / NP >= 2 && NW <= WIN,
                  "prefetch depth: an even number of positions dividing the range");
    const int voff = nt * KT0 * 1024 + lane * 16;
    v4i w[D];
#pragma unroll
    for (int s = 0; s < D; ++s) w[s] = wload(ws, voff, pf * KS + s);
    const int rl = lane & 31, kg = (lane >> 5) << 4;
    // b[x]: the B fragments of the position with parity x (relative to pf);
    // an: the table address of the next position
    v4i b[2][KS];
    {
        const int e0 = apos(rl, pf) + kg;
#pragma unroll
        for (int q = 0; q < KS; ++q) b[0][q] = *(const v4i *)(s_emb + e0 + q * 32);
    }
    int an = apos(rl, pf + 1);
    v16i acc;
    // D k-steps (NP positions) from position p0; FIRST starts from init,
    // LAST issues no more weight loads (p0 - pf is a multiple of NP, so
    // relative position parity is that of s / KS)
    auto body = [&](int p0, auto firstc, auto lastc) __attribute__((always_inline)) {
        constexpr bool FIRST = decltype(firstc)::value, LAST = decltype(lastc)::value;
        static_for<D>([&](auto sc) __attribute__((always_inline)) {
            constexpr int s = decltype(sc)::value, q = s % KS, h = (s / KS) & 1;
            const int p = p0 + s / KS;
            // this step's weights: issued D loads ago (fewer are outstanding
            // once LAST stops issuing); LDS waits are left to the compiler
            if constexpr (LAST) wait_counts<D - 1 - s, 15>();
            else wait_counts<D - 1, 15>();
            if constexpr (q == 0) {
                // (in the last body, position p is the range's s / KS + 1-th from its end)
                if constexpr (!LAST || s / KS + 1 < NP) {
                    const int e = an + kg;
#pragma unroll
                    for (int qq = 0; qq < KS; ++qq) b[h ^ 1][qq] = *(const v4i *)(s_emb + e + qq * 32);
                }
                if constexpr (!LAST || s / KS + 2 < NP) an = apos(rl, p + 2);
            }
            if constexpr (LAST && s / KS == NP - 1) {
                // the range's last position
                if (skip_last) wlast[q] = w[s];
                else acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(w[s], b[h][q], acc, 0, 0, 0);
            } else {
                acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(w[s], b[h][q], FIRST && s == 0 ? init : acc, 0, 0, 0);
            }
            if constexpr (!LAST) w[s] = wload(ws, voff, p0 * KS + s + D);
            __builtin_amdgcn_sched_barrier(0);
        });
    };
    body(pf, std::true_type{}, std::false_type{});
#pragma unroll 1
    for (int p0 = pf + NP; p0 < pf + NW - NP; p0 += NP) body(p0, std::false_type{}, std::false_type{});
    body(pf + NW - NP, std::false_type{}, std::true_type{});
    return acc;
}

// Position p of layer 0 for one n-tile and row tile, its weight fragments
// already in registers (gemm_layer0_one's `wlast`): acc + W_p . emb(tok(r, p)).
template <class AposFn>
__device__ __forceinline__ v16i gemm_layer0_position(const v4i *wp, int p, const uint8_t *s_emb, AposFn apos,
                                                     v16i acc, int lane) {
    constexpr int KS = EDIM / 32;
    const int e = apos(lane & 31, p) + ((lane >> 5) << 4);
    v4i b[KS];
#pragma unroll
    for (int q = 0; q < KS; ++q) b[q] = *(const v4i *)(s_emb + e + q * 32);
#pragma unroll
    for (int q = 0; q < KS; ++q) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(wp[q], b[q], acc, 0, 0, 0);
    return acc;
}

// ---- layer 0 overlapped with the decoder's epilogue ---------------------
//
// The window of decode step t+1 holds 63 tokens known before step t's
// symbol; only its last position needs that symbol.  gemm_layer0_ov runs
// layer 0 of step t+1 (mlp_rows_pipe's one-pass form over both passes'
// n-tiles) with side work in its first positions and a hook before the
// last one:
//
//   positions 0 .. 4*SP*ng-1 in ng bodies of 4*SP positions (16*SP
//     k-steps): in body k-step SP*I of body q, side.template piece<I>(q)
//     (I = 0..15) runs in the same
//     scheduling region as the k-step's MFMAs (instruction groups of one
//     MFMA and XV other VALU), then side.template after<I>(q) (the side
//     work's rare paths: wave-uniform branches between regions);
//   positions 4*SP*ng .. 62 plain;
//   mid() (the caller's barrier that publishes step t's symbols);
//   position 63, its table addresses read after mid().
//
// Every k-step region starts with an s_waitcnt for all LDS reads of the
// wave (this k-step's B fragments), so a side piece's LDS reads are
// complete in the next region without a wait of their own.  Weight
// fragments are loaded PD = 4 k-steps ahead across the whole range; the
// first k-step accumulates onto init().
template <int XV, int NTP, int RT>
__device__ __forceinline__ void kstep_schedule_side() {
    // LDS reads (the next k-step's B fragments and the side piece's) go in
    // the groups after the first MFMAs, their address arithmetic in the
    // VALU groups before them, so that they complete well before the next
    // region's wait; weight loads and the rest of the side work follow
    static_for<NTP * RT>([&](auto mc) __attribute__((always_inline)) {
        constexpr int m = decltype(mc)::value;
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                   // MFMA
        if constexpr (m >= 1 && m <= 4) __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);   // LDS reads
        if constexpr (m >= 2 && m < 2 + NTP) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // weight load
        __builtin_amdgcn_sched_group_barrier(0x002, XV, 0);                                  // side work
    });
}

template <int NTP, int RT, int XV, int SP, class AposFn, class NtFn, class AccFn, class InitFn, class Side, class Mid>
__device__ __forceinline__ void gemm_layer0_ov(const WStream &ws, NtFn nt, const uint8_t *s_emb, AposFn apos,
                                               AccFn acc, InitFn init, int lane, int ng, Side &side, Mid &&mid) {
    constexpr int PD = 4;
    static_assert(EDIM / 32 == PD && WIN == 64, "four k-steps per position, 64 positions");
    int voff[NTP];
#pragma unroll
    for (int j = 0; j < NTP; ++j) voff[j] = nt(j) * KT0 * 1024 + lane * 16;
    v4i w[2][PD][NTP];
#pragma unroll
    for (int s = 0; s < PD; ++s)
#pragma unroll
        for (int j = 0; j < NTP; ++j) w[0][s][j] = wload(ws, voff[j], s);
    const int rl = lane & 31, kg = (lane >> 5) << 4;
    // ea[x]: this lane's B address of the position with parity x; an[x]: the
    // table address of the next position with parity x (read two ahead)
    int ea[2][RT], an[2][RT];
#pragma unroll
    for (int i = 0; i < RT; ++i) {
        ea[0][i] = apos(i * 32 + rl, 0) + kg;
        an[1][i] = apos(i * 32 + rl, 1);
    }
    v4i b[2][RT];
#pragma unroll
    for (int i = 0; i < RT; ++i) b[0][i] = *(const v4i *)(s_emb + ea[0][i]);
    // k-step S of position p (parity H); FIRST: from init(); PIECE >= 0: with
    // that side piece; NEXTB = false: no B read of the next position
    auto kstep = [&](int p, int q, auto hc, auto sc, auto firstc, auto piecec, auto nextbc) __attribute__((always_inline)) {
        constexpr int h = decltype(hc)::value, s = decltype(sc)::value, hn = h ^ 1;
        constexpr bool FIRST = decltype(firstc)::value, NEXTB = decltype(nextbc)::value;
        constexpr int PIECE = decltype(piecec)::value;
        constexpr int bc = s & 1, bn = bc ^ 1;
        const int kt = p * PD + s;
        wait_counts<NTP * (PD - 1), 0>();
        if constexpr (s == 0) {
            const int p2 = p + 2 < WIN ? p + 2 : WIN - 1;
#pragma unroll
            for (int i = 0; i < RT; ++i) an[h][i] = apos(i * 32 + rl, p2);
        }
        if constexpr (s + 1 < PD) {
#pragma unroll
            for (int i = 0; i < RT; ++i) b[bn][i] = *(const v4i *)(s_emb + ea[h][i] + (s + 1) * 32);
        } else if constexpr (NEXTB) {
#pragma unroll
            for (int i = 0; i < RT; ++i) b[bn][i] = *(const v4i *)(s_emb + ea[hn][i]);
        }
#pragma unroll
        for (int j = 0; j < NTP; ++j) w[hn][s][j] = wload(ws, voff[j], kt + PD);
#pragma unroll
        for (int j = 0; j < NTP; ++j)
#pragma unroll
            for (int i = 0; i < RT; ++i) {
                v16i &a = acc(j, i);
                a = __builtin_amdgcn_mfma_i32_32x32x32_i8(w[h][s][j], b[bc][i], FIRST && s == 0 ? init(j, i) : a,
                                                          0, 0, 0);
            }
        if constexpr (PIECE >= 0) {
            side.template piece<PIECE>(q);
            kstep_schedule_side<XV, NTP, RT>();
        } else {
            kstep_schedule<NTP, RT>();
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (PIECE >= 0) side.template after<PIECE>(q);
    };
    using F = std::false_type;
    using T = std::true_type;
    // position p (parity H): its next position's addresses first.  B0: the
    // body k-step index of its first k-step (-1: no side work); body k-step
    // b carries side piece b / SP when SP divides it
    auto position = [&](int p, int q, auto hc, auto firstc, auto b0c, auto nextbc) __attribute__((always_inline)) {
        constexpr int h = decltype(hc)::value, hn = h ^ 1, B0 = decltype(b0c)::value;
#pragma unroll
        for (int i = 0; i < RT; ++i) ea[hn][i] = an[hn][i] + kg;
        auto pc = [](auto sc) {
            constexpr int b = B0 + decltype(sc)::value;
            return std::integral_constant<int, B0 < 0 || b % SP != 0 ? -1 : b / SP>{};
        };
        kstep(p, q, hc, std::integral_constant<int, 0>{}, firstc, pc(std::integral_constant<int, 0>{}), T{});
        kstep(p, q, hc, std::integral_constant<int, 1>{}, F{}, pc(std::integral_constant<int, 1>{}), T{});
        kstep(p, q, hc, std::integral_constant<int, 2>{}, F{}, pc(std::integral_constant<int, 2>{}), T{});
        kstep(p, q, hc, std::integral_constant<int, 3>{}, F{}, pc(std::integral_constant<int, 3>{}), nextbc);
    };
    using H0 = std::integral_constant<int, 0>;
    using H1 = std::integral_constant<int, 1>;
    using NP = std::integral_constant<int, -1>;
    // a body: 4 * SP positions with side pieces 0..15
    auto body = [&](int q, auto firstc) __attribute__((always_inline)) {
        const int p0 = 4 * SP * q;
        static_for<4 * SP>([&](auto pc) __attribute__((always_inline)) {
            constexpr int pp = decltype(pc)::value;
            using HP = std::integral_constant<int, pp & 1>;
            using FP = std::integral_constant<bool, decltype(firstc)::value && pp == 0>;
            position(p0 + pp, q, HP{}, FP{}, std::integral_constant<int, 4 * pp>{}, T{});
        });
    };
    int pbeg = 0;
    if (ng > 0) {
        body(0, T{});
#pragma unroll 1
        for (int q = 1; q < ng; ++q) body(q, F{});
        pbeg = 4 * SP * ng;
    } else {
        position(0, 0, H0{}, T{}, NP{}, T{});
        position(1, 0, H1{}, F{}, NP{}, T{});
        pbeg = 2;
    }
#pragma unroll 1
    for (int p0 = pbeg; p0 < WIN - 2; p0 += 2) {
        position(p0, 0, H0{}, F{}, NP{}, T{});
        position(p0 + 1, 0, H1{}, F{}, NP{}, T{});
    }
    position(WIN - 2, 0, H0{}, F{}, NP{}, F{});
    mid();
    // position 63: its table addresses and first B fragments now
#pragma unroll
    for (int i = 0; i < RT; ++i) {
        ea[1][i] = apos(i * 32 + rl, WIN - 1) + kg;
        b[0][i] = *(const v4i *)(s_emb + ea[1][i]);
    }
    // (position()'s own first statement would overwrite ea[1] from the
    // stale an[1]: the k-steps are issued directly)
    kstep(WIN - 1, 0, H1{}, std::integral_constant<int, 0>{}, F{}, NP{}, T{});
    kstep(WIN - 1, 0, H1{}, std::integral_constant<int, 1>{}, F{}, NP{}, T{});
    kstep(WIN - 1, 0, H1{}, std::integral_constant<int, 2>{}, F{}, NP{}, T{});
    kstep(WIN - 1, 0, H1{}, std::integral_constant<int, 3>{}, F{}, NP{}, F{});
}

// Layer 0 of mlp_rows_pipe with the epilogue of the previous decode step
// beside it (gemm_layer0_ov): accA / accB receive both passes' layer-0
// accumulators (bias included), pr the first hidden layer's pass-0
// parameter block (pipe_rest stores it).
template <int RT, bool UNI, int XV, int SP, class AposFn, class Side, class Mid>
__device__ __forceinline__ void pipe_layer0_ov(const ModelDev &M, const uint8_t *s_emb, const uint32_t *s_par,
                                               AposFn apos, v16i (&accA)[PNT][RT], v16i (&accB)[PNT][RT],
                                               uint32_t (&pr)[Slot<UNI>::LANE], int wave, int lane, int ng,
                                               Side &side, Mid &&mid) {
    wave = __builtin_amdgcn_readfirstlane(wave);
    const int nb0 = 2 * wave, nb1 = 8 + 2 * wave, g = lane >> 5;
    constexpr int BLK = Slot<UNI>::BLK;
    const uint32_t *s_parw = s_par + wave * PIPE_SLOTS * BLK;
    const uint32_t *p00 = s_parw + slot_p0(0) * BLK, *p10 = s_parw + slot_p1(0) * BLK;
    par_fetch<UNI>(M.layer[1].par, nb0, lane, pr);
    const LayerDev &L0 = M.layer[0];
    const WStream ws = make_wstream(L0.w, L0.bytes);
    gemm_layer0_ov<2 * PNT, RT, XV, SP>(
        ws, [&](int j) { return j < PNT ? nb0 + j : nb1 + j - PNT; }, s_emb, apos,
        [&](int j, int i) -> v16i & { return j < PNT ? accA[j][i] : accB[j - PNT][i]; },
        [&](int j, int) { return j < PNT ? bias_tile<UNI>(p00, j, g) : bias_tile<UNI>(p10, j - PNT, g); }, lane, ng,
        side, mid);
}

// mlp_rows_pipe after its layer 0 (accA / accB from pipe_layer0_ov, pr its
// parameter block): entered when no wave reads s_act any more, leaves the
// logits in s_act after a barrier.
template <int RT, bool UNI>
__device__ __forceinline__ void pipe_rest(const ModelDev &M, uint8_t *s_act, uint32_t *s_par, v16i (&accA)[PNT][RT],
                                          v16i (&accB)[PNT][RT], const uint32_t (&pr)[Slot<UNI>::LANE], int wave,
                                          int lane) {
    wave = __builtin_amdgcn_readfirstlane(wave);
    const int voff = lane * 16;
    const int nb0 = 2 * wave;
    constexpr int BLK = Slot<UNI>::BLK;
    uint32_t *s_parw = s_par + wave * PIPE_SLOTS * BLK;
    constexpr int PPD = ppd<RT>();
    v4i w[2][PPD][PNT];
    uint32_t pk[PNT][RT][4];
    {
        const LayerDev &L0 = M.layer[0];
        par_put<UNI>(s_parw + slot_p0(1) * BLK, pr, lane);
        if constexpr (UNI) rq_pass_uni<true, RT>(accA, rq_uni(L0), pk);
        else rq_pass_pc<true, RT>(accA, s_parw + slot_p0(0) * BLK, lane, pk);
        pstore_perm<RT>(pk, nb0, s_act, lane);
        const __amdgpu_buffer_rsrc_t rs1 = layer_rsrc(M.layer[1]);
#pragma unroll
        for (int s = 0; s < PPD; ++s)
#pragma unroll
            for (int j = 0; j < PNT; ++j) w[0][s][j] = wload_s(rs1, voff, ((nb0 + j) * KTH + s) * 1024);
        __syncthreads();
    }
    const int last = M.n_layers - 1;
#pragma unroll 1
    for (int l = 1; l < last; ++l)
        pipe_hidden<RT, false, UNI>(M.layer[l - 1], M.layer[l], M.layer[l + 1], s_act, s_parw, l, accA, accB, w, pk,
                                    wave, lane);
    pipe_hidden<RT, true, UNI>(M.layer[last - 1], M.layer[last], M.layer[last], s_act, s_parw, last, accA, accB, w,
                               pk, wave, lane);
}

// One MLP evaluation of R = 32*RT rows (RT <= 4), same contract as mlp_rows
// but in the padded row layout: entered after a barrier that ends every read
// of s_act (R * PACT_ROW bytes), leaves the int8 logits in bytes 0..255 of
// each row (natural order) after a barrier.  s_par holds pipe_par_dwords<UNI>(),
// layer 0's slots filled by pipe_params_init.
template <int RT, bool UNI, class AposFn>
__device__ __forceinline__ void mlp_rows_pipe(const ModelDev &M, const uint8_t *s_emb, uint8_t *s_act,
                                              uint32_t *s_par, AposFn apos, int wave, int lane) {
    static_assert(RT >= 1 && RT <= 4, "two passes of accumulators must fit the AGPRs");
    static_assert(WAVES * 2 * PNT * 32 == HID && WAVES * PNT * 32 == VOCAB, "tile split assumes 4 waves");
    // wave-uniform in a scalar register: weight offsets go to the scalar
    // offset of the buffer loads
    wave = __builtin_amdgcn_readfirstlane(wave);
    const int voff = lane * 16;
    const int nb0 = 2 * wave, nb1 = 8 + 2 * wave;
    constexpr int BLK = Slot<UNI>::BLK;
    uint32_t *s_parw = s_par + wave * PIPE_SLOTS * BLK;
    v16i accA[PNT][RT], accB[PNT][RT];
    constexpr int PPD = ppd<RT>();
    v4i w[2][PPD][PNT];
    uint32_t pk[PNT][RT][4];
    // layer 0 in one pass over both passes' n-tiles (each embedding B
    // fragment is read from LDS once), starting from the bias tiles, then
    // the pass-0 requantisation and store (no wave reads s_act during layer
    // 0); pass 1 stays in accB for the first hidden layer; then that layer's
    // pass-0 parameters and first weights
    {
        const LayerDev &L0 = M.layer[0];
        const int g = lane >> 5;
        const uint32_t *p00 = s_parw + slot_p0(0) * BLK, *p10 = s_parw + slot_p1(0) * BLK;
        uint32_t prn[Slot<UNI>::LANE];
        par_fetch<UNI>(M.layer[1].par, nb0, lane, prn);
        v16i bias[2 * PNT];
#pragma unroll
        for (int j = 0; j < PNT; ++j) {
            bias[j] = bias_tile<UNI>(p00, j, g);
            bias[PNT + j] = bias_tile<UNI>(p10, j, g);
        }
        const WStream ws = make_wstream(L0.w, L0.bytes);
        gemm_layer0_map<2 * PNT, RT>(
            ws, [&](int j) { return j < PNT ? nb0 + j : nb1 + j - PNT; }, s_emb, apos,
            [&](int j, int i) -> v16i & { return j < PNT ? accA[j][i] : accB[j - PNT][i]; },
            [&](int j, int) { return bias[j]; }, lane);
        par_put<UNI>(s_parw + slot_p0(1) * BLK, prn, lane);
        if constexpr (UNI) rq_pass_uni<true, RT>(accA, rq_uni(L0), pk);
        else rq_pass_pc<true, RT>(accA, p00, lane, pk);
        pstore_perm<RT>(pk, nb0, s_act, lane);
        const __amdgpu_buffer_rsrc_t rs1 = layer_rsrc(M.layer[1]);
#pragma unroll
        for (int s = 0; s < PPD; ++s)
#pragma unroll
            for (int j = 0; j < PNT; ++j) w[0][s][j] = wload_s(rs1, voff, ((nb0 + j) * KTH + s) * 1024);
        __syncthreads();
    }
    const int last = M.n_layers - 1;
#pragma unroll 1
    for (int l = 1; l < last; ++l)
        pipe_hidden<RT, false, UNI>(M.layer[l - 1], M.layer[l], M.layer[l + 1], s_act, s_parw, l, accA, accB, w, pk,
                                    wave, lane);
    pipe_hidden<RT, true, UNI>(M.layer[last - 1], M.layer[last], M.layer[last], s_act, s_parw, last, accA, accB, w,
                               pk, wave, lane);
}

}  // namespace sc
