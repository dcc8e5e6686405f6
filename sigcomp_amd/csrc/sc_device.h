// sc_device.h -- device building blocks of the gfx950 SigComp codec.
//
//  * int8 MFMA GEMM (v_mfma_i32_32x32x32_i8) for the quantised MLP, computed
//    transposed: D[n][r] = sum_k W[n][k] * act[r][k], so that a lane's 16
//    accumulators hold 4 groups of 4 consecutive output features of one
//    activation row -> one packed 32-bit LDS write per group;
//  * fused requantisation epilogue (cpu_int_kernels.py:5-14);
//  * logits -> frequency table rule on one wavefront per row
//    (cpu_entropy_coding.py:90-110), exact 64-bit floor divisions via a
//    float64 reciprocal estimate and one integer correction step;
//  * range-coder encoder / seal / decoder steps
//    (cpu_entropy_coding.py:121-266, gpu_entropy_coding.py:78-397).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace sc {

constexpr int VOCAB = 256;
constexpr int SOS = 256;
constexpr int WIN = 64;                 // context window (tokens)
constexpr int EDIM = 128;               // embedding width
constexpr int EMB_ROWS = 257;
constexpr int HID = 512;                // hidden width
constexpr int K0 = WIN * EDIM;          // 8192, layer-0 input width
constexpr int KT0 = K0 / 32;            // 256 k-tiles
constexpr int KTH = HID / 32;           // 16 k-tiles
constexpr int WAVES = 4;
constexpr int THREADS = WAVES * 64;
constexpr int MAX_LAYERS = 16;
constexpr uint32_t TOTAL = 1u << 24;    // frequency precision 2**24
constexpr int ACT_ROW = 512;            // bytes per activation row in LDS
constexpr int EMB_STRIDE = EDIM + 16;   // bytes per embedding row in LDS (see emb_off)
constexpr int EMB_BYTES = EMB_ROWS * EMB_STRIDE;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// Requant parameters of one 32-output n-tile, 104 dwords: bias[32] (int32),
// m0[32] (uint32), shift[32] (uint8, packed four per dword), then for
// layers on the 32-bit path (LayerDev::fast) hi[32] (int32): each output's
// pre-shift clamp bound min(128 * 2**shift - 1, 2**31 - 1), shift - 32 as
// stored (the per-channel form of LayerDev::uhi).
constexpr int PAR_DWORDS = 104;
constexpr int PAR_LDS_DWORDS = 4 * PAR_DWORDS * 4;   // 4 waves x up to 4 n-tiles

struct LayerDev {
    const v4i *w;            // packed weight fragments (pack order: pack_weight in sc_kernels.hip)
    const uint32_t *par;     // [n/32][PAR_DWORDS] requant parameter blocks
    int32_t n, kt;           // output width, k-tiles of 32
    int32_t relu;
    int32_t bytes;           // size of the packed weight buffer
    int32_t fast;            // every m0 < 2**31 and shift >= 32; shift[] holds shift - 32
    int32_t uni;             // fast, and one m0 and shift for every output (per-tensor constants):
    int32_t um0, ush;        //   that m0 and shift - 32
    int32_t uhi;             //   the pre-shift clamp bounds min(128 * 2**ush - 1, 2**31 - 1)
    int32_t ulo;             //   and max(-128 * 2**ush, -2**31) (layers without ReLU)
};

struct ModelDev {
    LayerDev layer[MAX_LAYERS];
    const int8_t *emb;       // [257][128] row-major
    const uint64_t *lut;     // [256]
    int32_t n_layers;
    int32_t pipe;            // MLP core: CORE_PLAIN, CORE_PIPE, CORE_PIPE_UNI or CORE_GENERIC (sc_model_create)
    int32_t window, emb_dim; // context tokens per row and embedding width (64 and 128 but for CORE_GENERIC)
};

// MLP cores.  CORE_PIPE (sc_pipe.h) needs every layer fast with ReLU on all
// but the last; CORE_PIPE_UNI additionally per-tensor constants on every
// layer (their requantisation then takes four VALU instructions per value,
// rq_words_uni, and the LDS parameter slots hold only biases).  All three
// give identical results.
constexpr int CORE_PLAIN = 0, CORE_PIPE = 1, CORE_PIPE_UNI = 2;
// CORE_GENERIC: any other architecture (window, embedding width, layer
// widths and count), one launch per stage (sc_gen.hip).
constexpr int CORE_GENERIC = 3;

// ---------------------------------------------------------------- LDS layouts

// Activation rows: 512 bytes per row, 16-byte chunks XOR-swizzled with the
// row's low 4 bits so that 16 consecutive rows reading the same chunk hit 16
// different 16-byte bank groups.
__device__ __forceinline__ int act_off(int r, int chunk) {
    return r * ACT_ROW + ((chunk ^ (r & 15)) << 4);
}

// Embedding rows: 128 bytes per token at a stride of 144 bytes, so that
// chunk c of token t starts at 9*t + c 16-byte units: lanes reading chunk c
// of different tokens spread over the bank groups, and the chunks of one
// token stay in order (chunk c is a constant c*16 bytes from the row start,
// an immediate of the LDS instruction).
__device__ __forceinline__ int emb_off(int tok, int chunk) { return tok * EMB_STRIDE + chunk * 16; }

__device__ __forceinline__ void load_emb_lds(const int8_t *__restrict__ emb, uint8_t *s_emb) {
    for (int idx = threadIdx.x; idx < EMB_ROWS * (EDIM / 16); idx += blockDim.x) {
        const int tok = idx >> 3, c = idx & 7;
        *(v4i *)(s_emb + emb_off(tok, c)) = *(const v4i *)(emb + tok * EDIM + c * 16);
    }
}

// The exp-LUT is staged in LDS reversed, s_rlut[j] = LUT[255 - j], as
// float64 (entries <= 2**38 are exact): LUT[max - l] = s_rlut[255 - max + l]
// is then one shift-add from the signed logit l (see row_freq).
__device__ __forceinline__ void load_lut_lds(const uint64_t *__restrict__ lut, double *s_rlut) {
    for (int i = threadIdx.x; i < VOCAB; i += blockDim.x) s_rlut[VOCAB - 1 - i] = (double)lut[i];
}

// ---------------------------------------------------------------- wave primitives

__device__ __forceinline__ int wave_max_i32(int v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = max(v, __shfl_xor(v, m));
    return v;
}
__device__ __forceinline__ int wave_min_i32(int v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = min(v, __shfl_xor(v, m));
    return v;
}
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += (uint32_t)__shfl_xor((int)v, m);
    return v;
}
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += (uint64_t)__shfl_xor((unsigned long long)v, m);
    return v;
}
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v, int lane) {
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        uint32_t t = (uint32_t)__shfl_up((int)v, d);
        if (lane >= d) v += t;
    }
    return v;
}

// ---------------------------------------------------------------- requant

// cpu_int_kernels.py:5-14: int32 wrapping bias add, int64 product with M0,
// arithmetic (floor) right shift, clamp to [relu ? 0 : -128, 127].
__device__ __forceinline__ uint32_t requant_u8(int acc, int bias, uint32_t m0, uint32_t shift,
                                               int lo) {
    const int biased = (int)((uint32_t)acc + (uint32_t)bias);
    const long long prod = (long long)biased * (long long)m0;
    long long s = prod >> shift;
    s = s < lo ? lo : s;
    s = s > 127 ? 127 : s;
    return (uint32_t)(uint8_t)(int8_t)s;
}

// The same function when m0 < 2**31 and shift >= 32 (layers flagged `fast`,
// whose shift array then holds shift - 32): writing the 64-bit product as
// hi*2**32 + lo with 0 <= lo < 2**32, floor(prod / 2**shift) equals
// floor(hi / 2**(shift-32)) because the low part adds less than one unit.
__device__ __forceinline__ uint32_t requant_u8_fast(int acc, int bias, int m0, uint32_t shift32,
                                                    int lo) {
    const int biased = (int)((uint32_t)acc + (uint32_t)bias);
    const int s = __mulhi(biased, m0) >> shift32;
    return (uint32_t)(uint8_t)(int8_t)min(max(s, lo), 127);
}

// Compile-time loop: f(std::integral_constant<int, I>) for I = 0 .. N-1, so
// that arrays indexed by I stay in registers however large the body is.
template <int N, int I = 0, class F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<N, I + 1>(f);
    }
}

// ---------------------------------------------------------------- MFMA GEMMs

// s_waitcnt until at most VM vector-memory and LG LDS/scalar-memory
// operations of this wave are outstanding (gfx9 encoding: vmcnt in bits 3:0
// and 15:14, expcnt 6:4 left at its maximum, lgkmcnt 11:8).  The compiler's
// own waits still guard every use; this only merges them.
template <int VM, int LG>
__device__ __forceinline__ void wait_counts() {
    static_assert(VM >= 0 && VM < 64 && LG >= 0 && LG < 16, "counter range");
    __builtin_amdgcn_s_waitcnt((VM & 15) | ((VM >> 4) << 14) | (7 << 4) | (LG << 8));
}

template <int NTP, int RT>
__device__ __forceinline__ void zero_acc(v16i (&acc)[NTP][RT]) {
#pragma unroll
    for (int j = 0; j < NTP; ++j)
#pragma unroll
        for (int i = 0; i < RT; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[j][i][v] = 0;
}

// Weight fragments are streamed with raw buffer loads: the per-lane offset
// of fragment (nt, kt) is (nt*KT)*1024 + lane*16 and the k-tile offset
// kt*1024 goes into the scalar offset.  Loads are issued PD k-tiles ahead
// of their MFMAs; out-of-range look-ahead reads return zero.
struct WStream {
    __amdgpu_buffer_rsrc_t rsrc;
};

__device__ __forceinline__ WStream make_wstream(const v4i *w, int bytes) {
    return WStream{__builtin_amdgcn_make_buffer_rsrc((void *)w, (short)0, bytes, 0x00020000)};
}

__device__ __forceinline__ v4i wload(const WStream &ws, int voff, int kt) {
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    v4u x = __builtin_amdgcn_raw_buffer_load_b128(ws.rsrc, voff, kt * 1024, 0);
    return (v4i)x;
}


// Pin the instruction order of one k-step: the RT LDS reads of the next
// step's B fragments and the NTP weight loads are spread between this
// step's MFMAs, so their latency overlaps the MFMA pipeline.
template <int NTP, int RT>
__device__ __forceinline__ void kstep_schedule() {
    constexpr int MF = NTP * RT;
    constexpr int per = MF / (RT + NTP) > 0 ? MF / (RT + NTP) : 1;
#pragma unroll
    for (int i = 0; i < RT; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
        __builtin_amdgcn_sched_group_barrier(0x008, per, 0); // MFMA
    }
#pragma unroll
    for (int j = 0; j < NTP; ++j) {
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // VMEM read
        __builtin_amdgcn_sched_group_barrier(0x008, per, 0); // MFMA
    }
    if constexpr (MF - per * (RT + NTP) > 0)
        __builtin_amdgcn_sched_group_barrier(0x008, MF - per * (RT + NTP), 0);
}

// Hidden / output layer: B operand from the activation rows in LDS.
// The wave computes output n-tiles [nt0, nt0 + NTP) for all RT row tiles.
//
// Software pipeline (per k-step): the B fragments of the next k-step are
// read from LDS and the weight fragments PD k-steps ahead are loaded while
// this step's MFMAs run.  Weights live in two register sets w[0], w[1] of PD
// k-steps each and B in two buffers; the loop body covers 2*PD k-steps so
// every register keeps one role across the back-edge (no copies that would
// wait on in-flight loads).
template <int NTP, int RT, int KT>
__device__ __forceinline__ void gemm_hidden(const WStream &ws, int nt0, const uint8_t *s_act,
                                            v16i (&acc)[NTP][RT], int lane) {
    constexpr int PD = 4;
    static_assert(KT % (2 * PD) == 0 && (KT & (KT - 1)) == 0, "k-tiles: power of two, multiple of 2*PD");
    int voff[NTP];
#pragma unroll
    for (int j = 0; j < NTP; ++j) voff[j] = (nt0 + j) * KT * 1024 + lane * 16;
    v4i w[2][PD][NTP];
#pragma unroll
    for (int s = 0; s < PD; ++s)
#pragma unroll
        for (int j = 0; j < NTP; ++j) w[0][s][j] = wload(ws, voff[j], s);
    const int rl = lane & 31, g = lane >> 5;
    int roff[RT];
#pragma unroll
    for (int i = 0; i < RT; ++i) roff[i] = (i * 32 + rl) * ACT_ROW;
    const int key = rl & 15;   // act_off swizzle key; (i*32 + rl) & 15 == rl & 15
    v4i b[2][RT];
#pragma unroll
    for (int i = 0; i < RT; ++i) b[0][i] = *(const v4i *)(s_act + roff[i] + ((g ^ key) << 4));
#pragma unroll 1
    for (int kt0 = 0; kt0 < KT; kt0 += 2 * PD) {
#pragma unroll
        for (int s = 0; s < 2 * PD; ++s) {
            const int kt = kt0 + s;
            const int ws_cur = s / PD, ws_nxt = ws_cur ^ 1, slot = s % PD;
            const int bc = s & 1, bn = bc ^ 1;
            const int cn = (((kt + 1) & (KT - 1)) * 2 + g) ^ key;
#pragma unroll
            for (int i = 0; i < RT; ++i) b[bn][i] = *(const v4i *)(s_act + roff[i] + (cn << 4));
#pragma unroll
            for (int j = 0; j < NTP; ++j) w[ws_nxt][slot][j] = wload(ws, voff[j], kt + PD);
#pragma unroll
            for (int j = 0; j < NTP; ++j)
#pragma unroll
                for (int i = 0; i < RT; ++i)
                    acc[j][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(w[ws_cur][slot][j], b[bc][i],
                                                                      acc[j][i], 0, 0, 0);
            kstep_schedule<NTP, RT>();
            __builtin_amdgcn_sched_barrier(0);   // one scheduling region per k-step
        }
    }
}

// Layer 0: the B operand row r, k = p*128 + j is emb[tok(r, p)][j], gathered
// from the LDS embedding table; a k-tile of 32 never straddles a position,
// so a position is PD = 4 k-steps.  Same pipeline as gemm_hidden over pairs
// of positions.  apos(r, p) = emb_off(tok(r, p), 0), the table address of
// the token's row (the callers keep tokens in that form): a lane's chunk
// 2q + g of a position is at apos + 16 g + 32 q.  Addresses are read two
// positions ahead.  Each k-step starts with one wait for its own weight
// fragments and B fragments (loads complete in order), instead of one wait
// per first use.
//
// General form: n-tile of accumulator j is nt(j), accumulator tile (j, i) is
// acc(j, i) (a reference), and the first k-step accumulates onto init(j, i)
// (zero, a bias tile, or acc(j, i) itself), so the accumulators need no
// separate initialisation; the form below it covers n-tiles nt0 .. nt0+NTP-1.
template <int NTP, int RT, class AposFn, class NtFn, class AccFn, class InitFn>
__device__ __forceinline__ void gemm_layer0_map(const WStream &ws, NtFn nt, const uint8_t *s_emb, AposFn apos,
                                                AccFn acc, InitFn init, int lane) {
    constexpr int PD = 4;
    static_assert(WIN % 2 == 0, "positions are processed in pairs");
    int voff[NTP];
#pragma unroll
    for (int j = 0; j < NTP; ++j) voff[j] = nt(j) * KT0 * 1024 + lane * 16;
    v4i w[2][PD][NTP];
#pragma unroll
    for (int s = 0; s < PD; ++s)
#pragma unroll
        for (int j = 0; j < NTP; ++j) w[0][s][j] = wload(ws, voff[j], s);
    const int rl = lane & 31, kg = (lane >> 5) << 4;
    // ea[x]: address of this lane's chunk g of the position with parity x
    // (chunk 2q + g is at ea + 32 q); an[x]: apos of the next position with
    // parity x
    int ea[2][RT], an[2][RT];
#pragma unroll
    for (int i = 0; i < RT; ++i) {
        ea[0][i] = apos(i * 32 + rl, 0) + kg;
        an[1][i] = apos(i * 32 + rl, 1);
    }
    v4i b[2][RT];
#pragma unroll
    for (int i = 0; i < RT; ++i) b[0][i] = *(const v4i *)(s_emb + ea[0][i]);
    // one pair of positions; the first pair is a separate copy whose first
    // k-step takes init() as the accumulator input
    auto pair = [&](int p0, auto firstc) __attribute__((always_inline)) {
        constexpr bool FIRST = decltype(firstc)::value;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int p = p0 + h, hn = h ^ 1;
            const int p2 = p + 2 < WIN ? p + 2 : WIN - 1;
#pragma unroll
            for (int i = 0; i < RT; ++i) ea[hn][i] = an[hn][i] + kg;   // position p + 1
#pragma unroll
            for (int s = 0; s < PD; ++s) {
                const int kt = p * PD + s;
                const int bc = s & 1, bn = bc ^ 1;
                // this step's weights (issued PD steps ago, NTP per step) and B fragments
                wait_counts<NTP * (PD - 1), 0>();
                if (s == 0) {
#pragma unroll
                    for (int i = 0; i < RT; ++i) an[h][i] = apos(i * 32 + rl, p2);   // position p + 2
                }
#pragma unroll
                for (int i = 0; i < RT; ++i) {
                    const int e = s + 1 < PD ? ea[h][i] : ea[hn][i];
                    b[bn][i] = *(const v4i *)(s_emb + e + ((s + 1) % PD) * 32);
                }
#pragma unroll
                for (int j = 0; j < NTP; ++j) w[hn][s][j] = wload(ws, voff[j], kt + PD);
#pragma unroll
                for (int j = 0; j < NTP; ++j)
#pragma unroll
                    for (int i = 0; i < RT; ++i) {
                        v16i &a = acc(j, i);
                        a = __builtin_amdgcn_mfma_i32_32x32x32_i8(w[h][s][j], b[bc][i],
                                                                  FIRST && h == 0 && s == 0 ? init(j, i) : a,
                                                                  0, 0, 0);
                    }
                kstep_schedule<NTP, RT>();
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };
    pair(0, std::true_type{});
#pragma unroll 1
    for (int p0 = 2; p0 < WIN; p0 += 2) pair(p0, std::false_type{});
}

template <int NTP, int RT, class AposFn>
__device__ __forceinline__ void gemm_layer0(const WStream &ws, int nt0, const uint8_t *s_emb,
                                            AposFn apos, v16i (&acc)[NTP][RT], int lane) {
    const v16i zero = {};
    gemm_layer0_map<NTP, RT>(
        ws, [&](int j) { return nt0 + j; }, s_emb, apos,
        [&](int j, int i) -> v16i & { return acc[j][i]; }, [&](int, int) { return zero; }, lane);
}

// Requantise accumulators to packed int8.  Accumulator element v of tile
// (j, i) is output feature n = (nt0 + j)*32 + 8*(v/4) + 4*(lane/32) + v%4 of
// row r = i*32 + lane%32, so pk[j][i][g] holds features n0 .. n0+3 with
// n0 = (nt0 + j)*32 + 8*g + 4*(lane/32).  `par` points at the LDS copy of
// the parameter block of n-tile nt0.
//
// BIAS = false: the accumulators already hold the bias (their GEMM started
// from the bias tile), the bias add is skipped.
template <int NTP, int RT, bool FAST, bool RELU, bool BIAS = true>
__device__ __forceinline__ void requant_pack_t(const v16i (&acc)[NTP][RT], const uint32_t *par, int lane,
                                               uint32_t (&pk)[NTP][RT][4]) {
    const int g2 = lane >> 5;
    constexpr int lo = RELU ? 0 : -128;
#pragma unroll
    for (int j = 0; j < NTP; ++j) {
        const uint32_t *pj = par + j * PAR_DWORDS;
        v4i bb[4] = {}, mm[4];
        uint32_t sh[4][4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int o = 8 * g + 4 * g2;
            if constexpr (BIAS) bb[g] = *(const v4i *)(pj + o);
            mm[g] = *(const v4i *)(pj + 32 + o);
            const uint32_t ss = pj[64 + (o >> 2)];
#pragma unroll
            for (int e = 0; e < 4; ++e) sh[g][e] = (ss >> (8 * e)) & 63u;
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
#pragma unroll
            for (int i = 0; i < RT; ++i) {
                uint32_t packed = 0;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    // read the accumulator out of its AGPR here, one at a
                    // time (otherwise every accumulator is copied to VGPRs
                    // at the end of the k loop, which spills)
                    int a;
                    asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(a) : "a"(acc[j][i][4 * g + e]));
                    const uint32_t q = FAST ? requant_u8_fast(a, bb[g][e], mm[g][e], sh[g][e], lo)
                                            : requant_u8(a, bb[g][e], (uint32_t)mm[g][e], sh[g][e], lo);
                    packed |= q << (8 * e);
                }
                // materialise the packed word here: without this the compiler
                // sinks the requantisation below the next pass's GEMM and keeps
                // every accumulator and parameter alive across it (spills)
                asm volatile("" : "+v"(packed));
                pk[j][i][g] = packed;
            }
        }
    }
}

// One uniform branch per layer selects the requantisation variant.
template <int NTP, int RT>
__device__ __forceinline__ void requant_pack(const v16i (&acc)[NTP][RT], const LayerDev &L,
                                             const uint32_t *par, int lane, uint32_t (&pk)[NTP][RT][4]) {
    if (L.fast) {
        if (L.relu) requant_pack_t<NTP, RT, true, true>(acc, par, lane, pk);
        else requant_pack_t<NTP, RT, true, false>(acc, par, lane, pk);
    } else {
        if (L.relu) requant_pack_t<NTP, RT, false, true>(acc, par, lane, pk);
        else requant_pack_t<NTP, RT, false, false>(acc, par, lane, pk);
    }
}

// Natural feature order: pk[j][i][g] -> bytes n0 .. n0+3 of row r.
template <int NTP, int RT>
__device__ __forceinline__ void store_packed(const uint32_t (&pk)[NTP][RT][4], int nt0, uint8_t *s_act,
                                             int lane) {
    const int rl = lane & 31, g2 = lane >> 5;
#pragma unroll
    for (int j = 0; j < NTP; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int n0 = (nt0 + j) * 32 + 8 * g + 4 * g2;
#pragma unroll
            for (int i = 0; i < RT; ++i)
                *(uint32_t *)(s_act + act_off(i * 32 + rl, n0 >> 4) + (n0 & 15)) = pk[j][i][g];
        }
}

// Hidden-layer order: within each 32-feature block, feature 8g + 4h + e is
// stored at byte 16h + 4g + e, so a lane's 16 results of one tile row form
// one 16-byte chunk (one ds_write_b128).  The next layer's weight columns
// are packed in the same order (pack_weight), so the products are unchanged.
template <int NTP, int RT>
__device__ __forceinline__ void store_packed_perm(const uint32_t (&pk)[NTP][RT][4], int nt0,
                                                  uint8_t *s_act, int lane) {
    const int rl = lane & 31, g2 = lane >> 5;
#pragma unroll
    for (int j = 0; j < NTP; ++j)
#pragma unroll
        for (int i = 0; i < RT; ++i) {
            const v4i v = {(int)pk[j][i][0], (int)pk[j][i][1], (int)pk[j][i][2], (int)pk[j][i][3]};
            *(v4i *)(s_act + act_off(i * 32 + rl, (nt0 + j) * 2 + g2)) = v;
        }
}

// One layer over R = 32*RT rows.  Wave w owns n-tiles
// [w*NTP*PASSES, (w+1)*NTP*PASSES), computed NTP at a time; the int8 results
// of every pass are held in registers until all waves have finished reading
// the layer input, then written over it.  The wave's requant parameter
// blocks are loaded before its GEMM and copied to its LDS slot `s_par`
// afterwards.  Leaves with a barrier.
template <int NTP, int PASSES, int RT, bool FIRST, bool LAST, class AposFn>
__device__ __forceinline__ void mlp_layer(const LayerDev &L, const uint8_t *s_emb, uint8_t *s_act,
                                          uint32_t *s_par, AposFn apos, int wave, int lane) {
    constexpr int NTW = NTP * PASSES;                 // n-tiles per wave
    constexpr int PW = NTW * PAR_DWORDS;              // parameter dwords per wave
    constexpr int PL = (PW + 63) / 64;                // per lane
    static_assert(NTW <= 4, "LDS parameter slot holds 4 n-tiles per wave");
    const int ntw0 = wave * NTW;
    uint32_t pr[PL];
#pragma unroll
    for (int d = 0; d < PL; ++d) {
        const int idx = d * 64 + lane;
        pr[d] = idx < PW ? L.par[ntw0 * PAR_DWORDS + idx] : 0u;
    }
    uint32_t *par = s_par + wave * 4 * PAR_DWORDS;
    uint32_t pk[PASSES][NTP][RT][4];
    static_for<PASSES>([&](auto pc) __attribute__((always_inline)) {
        constexpr int pass = decltype(pc)::value;
        const int nt0 = ntw0 + pass * NTP;
        v16i acc[NTP][RT];
        if constexpr (!FIRST) zero_acc(acc);   // layer 0 starts its accumulators from zero itself
        const WStream ws = make_wstream(L.w, L.bytes);
        if constexpr (FIRST) gemm_layer0<NTP, RT>(ws, nt0, s_emb, apos, acc, lane);
        else gemm_hidden<NTP, RT, KTH>(ws, nt0, s_act, acc, lane);
        if constexpr (pass == 0) {
#pragma unroll
            for (int d = 0; d < PL; ++d)
                if (d * 64 + lane < PW) par[d * 64 + lane] = pr[d];
        }
        requant_pack(acc, L, par + pass * NTP * PAR_DWORDS, lane, pk[pass]);
    });
    if constexpr (!FIRST) __syncthreads();
    static_for<PASSES>([&](auto pc) __attribute__((always_inline)) {
        constexpr int pass = decltype(pc)::value;
        if constexpr (LAST) store_packed(pk[pass], ntw0 + pass * NTP, s_act, lane);
        else store_packed_perm(pk[pass], ntw0 + pass * NTP, s_act, lane);
    });
    __syncthreads();
}

// One MLP evaluation of R = 32*RT rows: tokens -> int8 logits in s_act rows
// (bytes 0..255 of each row in natural symbol order, same swizzle; hidden
// activations use the store_packed_perm order).  Must be entered after a barrier
// that ends every read of s_act; leaves with a barrier.  HP = passes per
// hidden layer (1: 4 n-tiles per pass; 2: 2 n-tiles per pass, fewer registers).
template <int RT, int HP, class AposFn>
__device__ __forceinline__ void mlp_rows(const ModelDev &M, const uint8_t *s_emb, uint8_t *s_act,
                                         uint32_t *s_par, AposFn apos, int wave, int lane) {
    static_assert(WAVES * 4 * 32 == HID && WAVES * 2 * 32 == VOCAB, "tile split assumes 4 waves");
    constexpr int HN = 4 / HP;
    mlp_layer<HN, HP, RT, true, false>(M.layer[0], s_emb, s_act, s_par, apos, wave, lane);
#pragma unroll 1
    for (int l = 1; l < M.n_layers - 1; ++l)
        mlp_layer<HN, HP, RT, false, false>(M.layer[l], s_emb, s_act, s_par, apos, wave, lane);
    mlp_layer<2, 1, RT, false, true>(M.layer[M.n_layers - 1], s_emb, s_act, s_par, apos, wave, lane);
}

// ---------------------------------------------------------------- frequencies

// floor(n / d) for n < 2**63, 0 < d < 2**53, given rd ~ 1/d: the float64
// estimate is within one of the quotient (both roundings are relative
// 2**-53 and quotients here are below 2**25), one integer step corrects it.
__device__ __forceinline__ uint64_t div_floor_est(uint64_t n, uint64_t d, double rd) {
    uint64_t q = (uint64_t)((double)n * rd);
    const long long r = (long long)(n - q * d);
    if (r < 0) q -= 1;
    else if ((uint64_t)r >= d) q += 1;
    return q;
}

// DPP moves within 16-lane rows (gfx9 encodings): quad_perm xor 1 / xor 2,
// row_half_mirror, row_mirror, row_shr:n.  Lanes whose source is outside
// the row read 0.
template <int CTRL>
__device__ __forceinline__ int dpp(int x) {
    return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xF, 0xF, false);
}
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140;

__device__ __forceinline__ int row16_max(int x) {
    x = max(x, dpp<DPP_XOR1>(x));
    x = max(x, dpp<DPP_XOR2>(x));
    x = max(x, dpp<DPP_HALF_MIRROR>(x));
    return max(x, dpp<DPP_MIRROR>(x));
}
__device__ __forceinline__ int row16_min(int x) {
    x = min(x, dpp<DPP_XOR1>(x));
    x = min(x, dpp<DPP_XOR2>(x));
    x = min(x, dpp<DPP_HALF_MIRROR>(x));
    return min(x, dpp<DPP_MIRROR>(x));
}
__device__ __forceinline__ uint32_t row16_sum(uint32_t x) {
    x += (uint32_t)dpp<DPP_XOR1>((int)x);
    x += (uint32_t)dpp<DPP_XOR2>((int)x);
    x += (uint32_t)dpp<DPP_HALF_MIRROR>((int)x);
    return x + (uint32_t)dpp<DPP_MIRROR>((int)x);
}
template <int CTRL>
__device__ __forceinline__ uint64_t dpp64(uint64_t x) {
    const uint32_t lo = (uint32_t)dpp<CTRL>((int)(uint32_t)x);
    const uint32_t hi = (uint32_t)dpp<CTRL>((int)(uint32_t)(x >> 32));
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t row16_sum64(uint64_t x) {
    x += dpp64<DPP_XOR1>(x);
    x += dpp64<DPP_XOR2>(x);
    x += dpp64<DPP_HALF_MIRROR>(x);
    return x + dpp64<DPP_MIRROR>(x);
}
// exclusive prefix sum over the 16 lanes of a row
__device__ __forceinline__ uint32_t row16_excl_scan(uint32_t x) {
    uint32_t v = x;
    v += (uint32_t)dpp<0x111>((int)v);   // row_shr:1
    v += (uint32_t)dpp<0x112>((int)v);   // row_shr:2
    v += (uint32_t)dpp<0x114>((int)v);   // row_shr:4
    v += (uint32_t)dpp<0x118>((int)v);   // row_shr:8
    return v - x;
}

// Frequency table of one row held by a 16-lane row of the wavefront: lane u
// (= lane % 16) owns symbols 16u .. 16u+15.  f[k] = frequency of symbol
// 16u+k, ex = exclusive cumulative frequency of symbol 16u.
struct Freq16 {
    uint32_t f[16];
    uint32_t ex;
};

template <int CTRL>
__device__ __forceinline__ double dpp_f64(double x) {
    return __builtin_bit_cast(double, dpp64<CTRL>(__builtin_bit_cast(uint64_t, x)));
}
__device__ __forceinline__ double row16_sum_f64(double x) {
    x += dpp_f64<DPP_XOR1>(x);
    x += dpp_f64<DPP_XOR2>(x);
    x += dpp_f64<DPP_HALF_MIRROR>(x);
    return x + dpp_f64<DPP_MIRROR>(x);
}

// cpu_entropy_coding.py:90-110: w = LUT[max - l]; T = sum w;
// f = max(w*2**24 // T, 1); the first argmax absorbs sum(f) - 2**24.
//
// Exactness.  w and every partial sum of T are integers below 2**53, exact
// in float64 (s_rlut is the reversed LUT, see load_lut_lds).  r24 = 2**24/T
// is the hardware reciprocal refined by two Newton-Raphson steps
// (r += r (1 - T r)), relative error below 2**-50, and qe = w r24 + 2**-20
// (one fma) lies within 2**-26 of Q + 2**-20, Q = w 2**24 / T the exact
// quotient.  So floor(qe) = floor(Q) unless Q lies less than 2**-20 + 2**-26
// below an integer, which needs fract(qe) < 2**-19.  Below 2 either floor
// gives f = max(., 1) = 1, so qe is clamped to >= 1.5 first and only
// quotients >= 2 are checked (w = 0, the LUT's zero tail, never is).  A lane
// with a flagged quotient redoes its 16 with exact integer division
// (div_floor_est).
//
// The argmax correction stays per-lane data instead of a per-symbol update:
// the row's first argmax is the row maximum of the key
// (f - 1) << 8 | (15 - u) << 4 | (15 - k) (higher f first, then the lower
// symbol index 16u + k; f <= 2**24 so the key fits 32 bits), and only the
// lane that holds it gets kfix < 16.
struct RowFreq {
    uint32_t f[16];   // symbols 16u .. 16u+15 before the argmax correction
    uint32_t ex;      // corrected exclusive cumulative frequency of symbol 16u
    uint32_t tot;     // corrected sum of this lane's 16 frequencies
    uint32_t kfix;    // k of the row's first argmax if this lane holds it, else 16
    uint32_t ffix;    // corrected frequency of the first argmax
};

__device__ __forceinline__ uint32_t row16_max_u32(uint32_t x) {
    x = max(x, (uint32_t)dpp<DPP_XOR1>((int)x));
    x = max(x, (uint32_t)dpp<DPP_XOR2>((int)x));
    x = max(x, (uint32_t)dpp<DPP_HALF_MIRROR>((int)x));
    return max(x, (uint32_t)dpp<DPP_MIRROR>((int)x));
}

// reciprocal of a float64 in [1, 2**64): the hardware estimate refined by
// two Newton-Raphson steps
__device__ __forceinline__ double recip_nr(double x) {
    double r = __builtin_amdgcn_rcp(x);
    r = __builtin_fma(r, __builtin_fma(-x, r, 1.0), r);
    return __builtin_fma(r, __builtin_fma(-x, r, 1.0), r);
}

// N rows at once (N independent 16-lane rows per lane group): the phases of
// the N rows are interleaved in straight-line code so that their latency
// chains (LDS lookups, DPP reductions, float64 arithmetic) overlap.
template <int N>
__device__ __forceinline__ void row_freq(const v4i (&raw)[N], const double *s_rlut, int u, RowFreq (&o)[N]) {
    int l[N][16];
    int m[N];
#pragma unroll
    for (int n = 0; n < N; ++n) {
#pragma unroll
        for (int k = 0; k < 16; ++k) l[n][k] = (int)(int8_t)((uint32_t)raw[n][k >> 2] >> (8 * (k & 3)));
        int lm = l[n][0];
#pragma unroll
        for (int k = 1; k < 16; ++k) lm = max(lm, l[n][k]);
        m[n] = lm;
    }
#pragma unroll
    for (int n = 0; n < N; ++n) m[n] = row16_max(m[n]);
    double w[N][16];
    double T[N];
#pragma unroll
    for (int n = 0; n < N; ++n) {
        const double *p = s_rlut + (VOCAB - 1 - m[n]);
#pragma unroll
        for (int k = 0; k < 16; ++k) w[n][k] = p[l[n][k]];
        double s[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) s[k] = w[n][2 * k] + w[n][2 * k + 1];
        T[n] = ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
    }
#pragma unroll
    for (int n = 0; n < N; ++n) T[n] = row16_sum_f64(T[n]);
    double r24[N];
#pragma unroll
    for (int n = 0; n < N; ++n) r24[n] = recip_nr(T[n]) * 16777216.0;
    uint32_t hmin = 0xFFFFFFFFu;
#pragma unroll
    for (int n = 0; n < N; ++n) {
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const double qe = __builtin_fmax(__builtin_fma(w[n][k], r24[n], 0x1p-20), 1.5);
            o[n].f[k] = (uint32_t)qe;
            hmin = min(hmin, (uint32_t)(__builtin_bit_cast(uint64_t, __builtin_amdgcn_fract(qe)) >> 32));
        }
    }
    // high word of 2**-19: a non-negative double is below 2**-19 iff its
    // high word is below this
    if (hmin < 0x3EC00000u) {
#pragma unroll
        for (int n = 0; n < N; ++n) {
            const uint64_t Ti = (uint64_t)T[n];
            const double rT = r24[n] * 0x1p-24;
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const uint64_t q = div_floor_est(((uint64_t)w[n][k]) << 24, Ti, rT);
                o[n].f[k] = q < 1 ? 1u : (uint32_t)q;
            }
        }
    }
    const uint32_t lanebits = (uint32_t)(15 - u) << 4;
    uint32_t S[N], K[N];
#pragma unroll
    for (int n = 0; n < N; ++n) {
        uint32_t sl = 0, km = 0;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            sl += o[n].f[k];
            km = max(km, (o[n].f[k] << 4) | (uint32_t)(15 - k));
        }
        o[n].tot = sl;
        S[n] = sl;
        K[n] = (((km << 4) - 256u) & 0xFFFFFF00u) | lanebits | (km & 15u);
    }
#pragma unroll
    for (int n = 0; n < N; ++n) {
        S[n] = row16_sum(S[n]);
        K[n] = row16_max_u32(K[n]);
    }
#pragma unroll
    for (int n = 0; n < N; ++n) {
        const uint32_t adj = S[n] - TOTAL;   // sum(f) - 2**24, mod 2**32
        const bool star = (K[n] & 0xF0u) == lanebits;
        o[n].ffix = (K[n] >> 8) + 1u - adj;
        o[n].kfix = star ? 15u - (K[n] & 15u) : 16u;
        if (star) o[n].tot -= adj;
    }
#pragma unroll
    for (int n = 0; n < N; ++n) o[n].ex = row16_excl_scan(o[n].tot);
}

// corrected frequency of symbol 16u + k
__device__ __forceinline__ uint32_t row_freq_at(const RowFreq &o, int k) {
    return (uint32_t)k == o.kfix ? o.ffix : o.f[k];
}

// The whole corrected table, lane u's 16 entries (full-CDF and step paths).
template <int N>
__device__ __forceinline__ void row_frequencies16n(const v4i (&raw)[N], const double *s_rlut, int u,
                                                   Freq16 (&o)[N]) {
    RowFreq rf[N];
    row_freq<N>(raw, s_rlut, u, rf);
#pragma unroll
    for (int n = 0; n < N; ++n) {
#pragma unroll
        for (int k = 0; k < 16; ++k) o[n].f[k] = row_freq_at(rf[n], k);
        o[n].ex = rf[n].ex;
    }
}

__device__ __forceinline__ void row_frequencies16(v4i raw, const double *s_rlut, int u, Freq16 &o) {
    const v4i r[1] = {raw};
    Freq16 f[1];
    row_frequencies16n<1>(r, s_rlut, u, f);
    o = f[0];
}

// ---- symbol lookups through a per-row LDS slot --------------------------
//
// A row's 16 lanes hold 16 symbols each.  To find the cumulative frequency
// of a given symbol (encoder) or the symbol whose interval holds a quantile
// (decoder) without a 16-step select chain in every lane, the lane whose
// segment holds it (the owner) writes its 16 frequencies and
// {ex, kfix, ffix, owner} to the row's slot; lane j of the row then reads
// frequency j of that segment, applies the argmax correction and a 16-lane
// prefix sum gives each lane its symbol's cumulative frequency.  The owner's
// write and the row's reads are in one wavefront: LDS executes a
// wavefront's accesses in order, slot_sync only keeps the compiler from
// moving them.
constexpr int SLOT_DWORDS = 20;

__device__ __forceinline__ void slot_put(uint32_t *slot, const RowFreq &o, int u) {
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    v4u *s = (v4u *)slot;
#pragma unroll
    for (int j = 0; j < 4; ++j) s[j] = v4u{o.f[4 * j], o.f[4 * j + 1], o.f[4 * j + 2], o.f[4 * j + 3]};
    s[4] = v4u{o.ex, o.kfix, o.ffix, (uint32_t)u};
}

__device__ __forceinline__ void slot_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// lane u's symbol of the slot's segment: its cumulative frequency and
// frequency; returns the owner lane (the symbol is 16 * owner + u)
__device__ __forceinline__ uint32_t slot_get(const uint32_t *slot, int u, uint32_t &cum, uint32_t &freq) {
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    const v4u meta = *(const v4u *)(slot + 16);
    uint32_t f = slot[u];
    if ((uint32_t)u == meta[1]) f = meta[2];
    cum = meta[0] + row16_excl_scan(f);
    freq = f;
    return meta[3];
}

// cumulative frequency and frequency of local symbol k (0..15) of this lane
__device__ __forceinline__ void freq16_at(const Freq16 &fr, int k, uint32_t &cum, uint32_t &freq) {
    uint32_t c = fr.ex, f = fr.f[0];
#pragma unroll
    for (int x = 0; x < 16; ++x) {
        if (x < k) c += fr.f[x];
        if (x == k) f = fr.f[x];
    }
    cum = c;
    freq = f;
}

// logits of row r (in s_act) as the 16 bytes of lane u's symbols
__device__ __forceinline__ v4i row_logits16(const uint8_t *s_act, int r, int u) {
    return *(const v4i *)(s_act + act_off(r, u));
}

// ---------------------------------------------------------------- range coder

struct EncState {
    uint64_t lower, range;
    int32_t inverted;
    uint32_t first;
    int32_t pos;
};

// _encode_one (cpu_entropy_coding.py:121-161) after the frequency lookup.
// Returns 0 or 1 (capacity exceeded; state left as before the step).
__device__ __forceinline__ int enc_step(EncState &s, uint64_t cum, uint64_t freq,
                                        uint32_t *__restrict__ out, int32_t cap) {
    const uint64_t scale = s.range >> 24;
    const uint64_t new_range = scale * freq;
    const uint64_t new_lower = s.lower + scale * cum;
    int32_t pos = s.pos, inv = s.inverted;
    if (inv > 0 && new_lower + new_range > new_lower) {
        uint32_t emit_first, emit_rest;
        if (new_lower < s.lower) { emit_first = s.first + 1u; emit_rest = 0u; }
        else { emit_first = s.first; emit_rest = 0xFFFFFFFFu; }
        if (pos + inv > cap) return 1;
        out[pos++] = emit_first;
        for (int32_t i = 0; i < inv - 1; ++i) out[pos++] = emit_rest;
        inv = 0;
    }
    uint64_t lower = new_lower, range = new_range;
    if (range < (1ull << 32)) {
        range <<= 32;
        const uint32_t word = (uint32_t)(lower >> 32);
        lower <<= 32;
        if (inv > 0) {
            inv += 1;
        } else if (lower + range > lower) {
            if (pos >= cap) return 1;
            out[pos++] = word;
        } else {
            inv = 1;
            s.first = word;
        }
    }
    s.lower = lower;
    s.range = range;
    s.inverted = inv;
    s.pos = pos;
    return 0;
}

// _seal (cpu_entropy_coding.py:206-227).  A sealed state has range 2**64-1
// so that sealing again emits nothing.
__device__ __forceinline__ int enc_seal(EncState &s, uint32_t *__restrict__ out, int32_t cap) {
    if (s.range == ~0ull) return 0;
    const uint64_t point = s.lower + 0xFFFFFFFFull;
    int32_t pos = s.pos;
    if (s.inverted > 0) {
        uint32_t emit_first, emit_rest;
        if (point < s.lower) { emit_first = s.first + 1u; emit_rest = 0u; }
        else { emit_first = s.first; emit_rest = 0xFFFFFFFFu; }
        if (pos + s.inverted > cap) return 1;
        out[pos++] = emit_first;
        for (int32_t i = 0; i < s.inverted - 1; ++i) out[pos++] = emit_rest;
    }
    const uint32_t point_word = (uint32_t)(point >> 32);
    const uint32_t upper_word = (uint32_t)((s.lower + s.range) >> 32);
    const int need = upper_word == point_word ? 2 : 1;
    if (pos + need > cap) return 1;
    out[pos++] = point_word;
    if (need == 2) out[pos++] = 0u;
    s.pos = pos;
    s.inverted = 0;
    s.range = ~0ull;
    return 0;
}

// a * b for a < 2**40, b < 2**24 (a coder scale times a frequency or a
// cumulative frequency): the high word of a times b fits the 24-bit multiply
__device__ __forceinline__ uint64_t mul_scale(uint64_t a, uint32_t b) {
    return (uint64_t)(uint32_t)a * b + ((uint64_t)__umul24((uint32_t)(a >> 32), b) << 32);
}

// Decoder quantile (point - lower) // scale for 0 < scale < 2**40 (range >>
// 24), exact for quotients below 2**24; false when the quotient is >= 2**24
// (an invalid stream, cpu_entropy_coding.py:240-248).  The float64 estimate
// D * (1/scale) (D rounded once, the reciprocal within 2**-50) is within one
// of the quotient; it is clamped to 2**24 - 1 so that q0 * scale never wraps,
// and one integer step corrects it (a quotient >= 2**24 ends at 2**24).
__device__ __forceinline__ bool dec_quantile(uint64_t D, uint64_t scale, uint32_t &q) {
    const double Df = __builtin_fma((double)(uint32_t)(D >> 32), 0x1p32, (double)(uint32_t)D);
    const double sf = __builtin_fma((double)(uint32_t)(scale >> 32), 0x1p32, (double)(uint32_t)scale);
    uint32_t q0 = (uint32_t)__builtin_fmin(Df * recip_nr(sf), 16777215.0);
    const uint64_t prod = mul_scale(scale, q0);
    if (prod > D) q0 -= 1;
    else if (D - prod >= scale) q0 += 1;
    q = q0;
    return q0 < TOTAL;
}

// Symbol search on a 16-lane row: largest v with excl_cdf[v] <= q (the
// cumulative frequencies are strictly increasing since every f >= 1), as the
// CPU loop (cpu_entropy_coding.py:251-254) and the Triton count
// (gpu_entropy_coding.py:370-374).  All 16 lanes return the symbol and its
// cum / freq.
__device__ __forceinline__ int dec_symbol16(const Freq16 &fr, uint32_t q, int lane, uint32_t &cum,
                                            uint32_t &freq) {
    uint32_t cnt = 0, c = fr.ex;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        cnt += c <= q ? 1u : 0u;
        c += fr.f[k];
    }
    int s = (int)row16_sum(cnt) - 1;
    s = s < 0 ? 0 : (s > 255 ? 255 : s);
    uint32_t mc, mf;
    freq16_at(fr, s & 15, mc, mf);
    const int src = (lane & ~15) | (s >> 4);
    cum = (uint32_t)__shfl((int)mc, src);
    freq = (uint32_t)__shfl((int)mf, src);
    return s;
}

}  // namespace sc
