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
constexpr int EMB_BYTES = EMB_ROWS * EDIM;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

struct LayerDev {
    const v4i *w;            // packed weight fragments (pack order: pack_weight in sc_kernels.hip)
    const int32_t *bias;     // [n]
    const uint32_t *m0;      // [n]
    const uint8_t *shift;    // [n]
    int32_t n, kt;           // output width, k-tiles of 32
    int32_t relu;
    int32_t bytes;           // size of the packed weight buffer
    int32_t fast;            // every m0 < 2**31 and shift >= 32; shift[] holds shift - 32
    int32_t pad;
};

struct ModelDev {
    LayerDev layer[MAX_LAYERS];
    const int8_t *emb;       // [257][128] row-major
    const uint64_t *lut;     // [256]
    int32_t n_layers;
    int32_t pad;
};

// ---------------------------------------------------------------- LDS layouts

// Activation rows: 512 bytes per row, 16-byte chunks XOR-swizzled with the
// row's low 4 bits so that 16 consecutive rows reading the same chunk hit 16
// different 16-byte bank groups.
__device__ __forceinline__ int act_off(int r, int chunk) {
    return r * ACT_ROW + ((chunk ^ (r & 15)) << 4);
}

// Embedding rows: 128 bytes per token, chunks swizzled with the token's low 3 bits.
__device__ __forceinline__ int emb_off(int tok, int chunk) {
    return tok * EDIM + ((chunk ^ (tok & 7)) << 4);
}

__device__ __forceinline__ void load_emb_lds(const int8_t *__restrict__ emb, uint8_t *s_emb) {
    for (int idx = threadIdx.x; idx < EMB_ROWS * (EDIM / 16); idx += blockDim.x) {
        const int tok = idx >> 3, c = idx & 7;
        *(v4i *)(s_emb + emb_off(tok, c)) = *(const v4i *)(emb + tok * EDIM + c * 16);
    }
}

__device__ __forceinline__ void load_lut_lds(const uint64_t *__restrict__ lut, uint64_t *s_lut) {
    for (int i = threadIdx.x; i < VOCAB; i += blockDim.x) s_lut[i] = lut[i];
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
    int s = __mulhi(biased, m0) >> shift32;
    s = s < lo ? lo : s;
    s = s > 127 ? 127 : s;
    return (uint32_t)(uint8_t)(int8_t)s;
}

// ---------------------------------------------------------------- MFMA GEMMs

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

// Hidden / output layer: B operand from the activation rows in LDS.
// The wave computes output n-tiles [nt0, nt0 + NTP) for all RT row tiles.
// B fragments are read one k-tile ahead of their MFMAs (the read for the
// step past the end wraps to k-tile 0 and is unused).
template <int NTP, int RT, int KT>
__device__ __forceinline__ void gemm_hidden(const WStream &ws, int nt0, const uint8_t *s_act,
                                            v16i (&acc)[NTP][RT], int lane) {
    constexpr int PD = 4;
    static_assert(KT % PD == 0 && (KT & (KT - 1)) == 0, "k-tiles: power of two, multiple of PD");
    int voff[NTP];
#pragma unroll
    for (int j = 0; j < NTP; ++j) voff[j] = (nt0 + j) * KT * 1024 + lane * 16;
    v4i ring[PD][NTP];
#pragma unroll
    for (int s = 0; s < PD; ++s)
#pragma unroll
        for (int j = 0; j < NTP; ++j) ring[s][j] = wload(ws, voff[j], s);
    const int rl = lane & 31, g = lane >> 5;
    int roff[RT];
#pragma unroll
    for (int i = 0; i < RT; ++i) roff[i] = (i * 32 + rl) * ACT_ROW;
    const int key = rl & 15;   // act_off swizzle key; (i*32 + rl) & 15 == rl & 15
    v4i bcur[RT];
#pragma unroll
    for (int i = 0; i < RT; ++i) bcur[i] = *(const v4i *)(s_act + roff[i] + ((g ^ key) << 4));
#pragma unroll 1
    for (int kt0 = 0; kt0 < KT; kt0 += PD) {
#pragma unroll
        for (int s = 0; s < PD; ++s) {
            const int kt = kt0 + s;
            v4i a[NTP];
#pragma unroll
            for (int j = 0; j < NTP; ++j) a[j] = ring[s][j];
            v4i bnxt[RT];
            const int cn = (((kt + 1) & (KT - 1)) * 2 + g) ^ key;
#pragma unroll
            for (int i = 0; i < RT; ++i) bnxt[i] = *(const v4i *)(s_act + roff[i] + (cn << 4));
#pragma unroll
            for (int j = 0; j < NTP; ++j) ring[s][j] = wload(ws, voff[j], kt + PD);
#pragma unroll
            for (int j = 0; j < NTP; ++j)
#pragma unroll
                for (int i = 0; i < RT; ++i)
                    acc[j][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[j], bcur[i], acc[j][i], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < RT; ++i) bcur[i] = bnxt[i];
        }
    }
}

// Layer 0: the B operand row r, k = p*128 + j is emb[tok(r, p)][j], gathered
// from the LDS embedding table; a k-tile of 32 never straddles a position.
// Tokens are looked up one position ahead and B fragments one k-tile ahead.
template <int NTP, int RT, class TokFn>
__device__ __forceinline__ void gemm_layer0(const WStream &ws, int nt0, const uint8_t *s_emb,
                                            TokFn tok, v16i (&acc)[NTP][RT], int lane) {
    constexpr int PD = 4;   // = k-tiles per position, so one position per outer step
    int voff[NTP];
#pragma unroll
    for (int j = 0; j < NTP; ++j) voff[j] = (nt0 + j) * KT0 * 1024 + lane * 16;
    v4i ring[PD][NTP];
#pragma unroll
    for (int s = 0; s < PD; ++s)
#pragma unroll
        for (int j = 0; j < NTP; ++j) ring[s][j] = wload(ws, voff[j], s);
    const int rl = lane & 31, g = lane >> 5;
    int ebase[RT], ekey[RT];
#pragma unroll
    for (int i = 0; i < RT; ++i) {
        const int t = tok(i * 32 + rl, 0);
        ebase[i] = t * EDIM;
        ekey[i] = t & 7;
    }
    v4i bcur[RT];
#pragma unroll
    for (int i = 0; i < RT; ++i) bcur[i] = *(const v4i *)(s_emb + ebase[i] + ((g ^ ekey[i]) << 4));
#pragma unroll 1
    for (int p = 0; p < WIN; ++p) {
        int nbase[RT], nkey[RT];
        const int pn = p + 1 < WIN ? p + 1 : WIN - 1;
#pragma unroll
        for (int i = 0; i < RT; ++i) {
            const int t = tok(i * 32 + rl, pn);
            nbase[i] = t * EDIM;
            nkey[i] = t & 7;
        }
#pragma unroll
        for (int s = 0; s < PD; ++s) {
            const int kt = p * PD + s;
            v4i a[NTP];
#pragma unroll
            for (int j = 0; j < NTP; ++j) a[j] = ring[s][j];
            v4i bnxt[RT];
            if (s + 1 < PD) {
                const int c = (s + 1) * 2 + g;
#pragma unroll
                for (int i = 0; i < RT; ++i)
                    bnxt[i] = *(const v4i *)(s_emb + ebase[i] + ((c ^ ekey[i]) << 4));
            } else {
#pragma unroll
                for (int i = 0; i < RT; ++i)
                    bnxt[i] = *(const v4i *)(s_emb + nbase[i] + ((g ^ nkey[i]) << 4));
            }
#pragma unroll
            for (int j = 0; j < NTP; ++j) ring[s][j] = wload(ws, voff[j], kt + PD);
#pragma unroll
            for (int j = 0; j < NTP; ++j)
#pragma unroll
                for (int i = 0; i < RT; ++i)
                    acc[j][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[j], bcur[i], acc[j][i], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < RT; ++i) bcur[i] = bnxt[i];
        }
#pragma unroll
        for (int i = 0; i < RT; ++i) {
            ebase[i] = nbase[i];
            ekey[i] = nkey[i];
        }
    }
}

// Requantise accumulators to packed int8.  Accumulator element v of tile
// (j, i) is output feature n = (nt0 + j)*32 + 8*(v/4) + 4*(lane/32) + v%4 of
// row r = i*32 + lane%32, so pk[j][i][g] holds features n0 .. n0+3 with
// n0 = (nt0 + j)*32 + 8*g + 4*(lane/32).
template <int NTP, int RT>
__device__ __forceinline__ void requant_pack(const v16i (&acc)[NTP][RT], const LayerDev &L, int nt0,
                                             int lane, uint32_t (&pk)[NTP][RT][4]) {
    const int g2 = lane >> 5;
    const int lo = L.relu ? 0 : -128;
#pragma unroll
    for (int j = 0; j < NTP; ++j) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int n0 = (nt0 + j) * 32 + 8 * g + 4 * g2;
            const v4i bb = *(const v4i *)(L.bias + n0);
            const v4i mm = *(const v4i *)(L.m0 + n0);
            const uint32_t ss = *(const uint32_t *)(L.shift + n0);
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
                    const uint32_t sh = (ss >> (8 * e)) & 63u;
                    packed |= (L.fast ? requant_u8_fast(a, bb[e], mm[e], sh, lo)
                                      : requant_u8(a, bb[e], (uint32_t)mm[e], sh, lo)) << (8 * e);
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

// One layer over R = 32*RT rows.  Wave w owns n-tiles
// [w*NTP*PASSES, (w+1)*NTP*PASSES), computed NTP at a time; the int8 results
// of every pass are held in registers until all waves have finished reading
// the layer input, then written over it.  Leaves with a barrier.
template <int NTP, int PASSES, int RT, bool FIRST, class TokFn>
__device__ __forceinline__ void mlp_layer(const LayerDev &L, const uint8_t *s_emb, uint8_t *s_act,
                                          TokFn tok, int wave, int lane) {
    uint32_t pk[PASSES][NTP][RT][4];
#pragma unroll
    for (int pass = 0; pass < PASSES; ++pass) {
        const int nt0 = (wave * PASSES + pass) * NTP;
        v16i acc[NTP][RT];
        zero_acc(acc);
        const WStream ws = make_wstream(L.w, L.bytes);
        if constexpr (FIRST) gemm_layer0<NTP, RT>(ws, nt0, s_emb, tok, acc, lane);
        else gemm_hidden<NTP, RT, KTH>(ws, nt0, s_act, acc, lane);
        requant_pack(acc, L, nt0, lane, pk[pass]);
    }
    if constexpr (!FIRST) __syncthreads();
#pragma unroll
    for (int pass = 0; pass < PASSES; ++pass) store_packed(pk[pass], (wave * PASSES + pass) * NTP, s_act, lane);
    __syncthreads();
}

// One MLP evaluation of R = 32*RT rows: tokens -> int8 logits in s_act rows
// (bytes 0..255 of each row, same swizzle).  Must be entered after a barrier
// that ends every read of s_act; leaves with a barrier.  HP = passes per
// hidden layer (1: 4 n-tiles per pass; 2: 2 n-tiles per pass, fewer registers).
template <int RT, int HP, class TokFn>
__device__ __forceinline__ void mlp_rows(const ModelDev &M, const uint8_t *s_emb, uint8_t *s_act,
                                         TokFn tok, int wave, int lane) {
    static_assert(WAVES * 4 * 32 == HID && WAVES * 2 * 32 == VOCAB, "tile split assumes 4 waves");
    constexpr int HN = 4 / HP;
    mlp_layer<HN, HP, RT, true>(M.layer[0], s_emb, s_act, tok, wave, lane);
#pragma unroll 1
    for (int l = 1; l < M.n_layers - 1; ++l)
        mlp_layer<HN, HP, RT, false>(M.layer[l], s_emb, s_act, tok, wave, lane);
    mlp_layer<2, 1, RT, false>(M.layer[M.n_layers - 1], s_emb, s_act, tok, wave, lane);
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

struct RowFreq {
    uint32_t f[4];   // frequencies of symbols 4*lane .. 4*lane+3
    uint32_t e[4];   // exclusive cumulative frequencies of the same symbols
};

// cpu_entropy_coding.py:90-110 on one wavefront: lane holds logits of
// symbols 4*lane .. 4*lane+3.  u = LUT[max - l]; T = sum u;
// f = max(u*2**24 // T, 1); the first argmax absorbs sum(f) - 2**24.
__device__ __forceinline__ void row_frequencies(uint32_t packed_logits, const uint64_t *s_lut,
                                                int lane, RowFreq &o) {
    int l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) l[i] = (int)(int8_t)(packed_logits >> (8 * i));
    const int m = wave_max_i32(max(max(l[0], l[1]), max(l[2], l[3])));
    uint64_t u[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) u[i] = s_lut[m - l[i]];
    const uint64_t T = wave_sum_u64(u[0] + u[1] + u[2] + u[3]);
    const double rT = 1.0 / (double)T;
    uint32_t f[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint64_t q = div_floor_est(u[i] << 24, T, rT);
        f[i] = q < 1 ? 1u : (uint32_t)q;
    }
    const uint32_t S = wave_sum_u32(f[0] + f[1] + f[2] + f[3]);
    const int fm = wave_max_i32((int)max(max(f[0], f[1]), max(f[2], f[3])));
    int cand = 1 << 20;
#pragma unroll
    for (int i = 3; i >= 0; --i)
        if ((int)f[i] == fm) cand = 4 * lane + i;
    const int idx = wave_min_i32(cand);
    if ((idx >> 2) == lane) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if ((idx & 3) == i) f[i] -= S - TOTAL;
    }
    const uint32_t tot = f[0] + f[1] + f[2] + f[3];
    uint32_t ex = wave_incl_scan_u32(tot, lane) - tot;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        o.f[i] = f[i];
        o.e[i] = ex;
        ex += f[i];
    }
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

// Decoder quantile (point - lower) // scale, exact for quotients below
// 2**24; false when the quotient is >= 2**24 (an invalid stream,
// cpu_entropy_coding.py:240-248).  q0 is clamped to 2**24 before the
// product so that q0*scale <= 2**24*scale <= range never wraps.
__device__ __forceinline__ bool dec_quantile(uint64_t D, uint64_t scale, uint32_t &q) {
    const double qe = (double)D * (1.0 / (double)scale);
    uint64_t q0 = qe >= 16777216.0 ? 16777216ull : (uint64_t)qe;
    const uint64_t prod = q0 * scale;
    if (prod > D) q0 -= 1;
    else if (D - prod >= scale) q0 += 1;
    if (q0 >= TOTAL) return false;
    q = (uint32_t)q0;
    return true;
}

// Symbol search on one wavefront: largest v with excl_cdf[v] <= q (the
// cumulative frequencies are strictly increasing since every f >= 1), as the
// CPU loop (cpu_entropy_coding.py:251-254) and the Triton count
// (gpu_entropy_coding.py:370-374).  Returns the symbol, its cum and freq.
__device__ __forceinline__ int dec_symbol(const RowFreq &fr, uint32_t q, int lane,
                                          uint32_t &cum, uint32_t &freq) {
    uint32_t cnt = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) cnt += fr.e[i] <= q ? 1u : 0u;
    int s = (int)wave_sum_u32(cnt) - 1;
    s = s < 0 ? 0 : (s > 255 ? 255 : s);
    const int src = s >> 2, sel = s & 3;
    uint32_t ce = fr.e[0], cf = fr.f[0];
#pragma unroll
    for (int i = 1; i < 4; ++i)
        if (sel == i) { ce = fr.e[i]; cf = fr.f[i]; }
    cum = (uint32_t)__shfl((int)ce, src);
    freq = (uint32_t)__shfl((int)cf, src);
    return s;
}

}  // namespace sc
