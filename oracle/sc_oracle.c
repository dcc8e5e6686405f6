/*
 * sc_oracle.c -- CPU restatement of SigComp's integer codec path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * product in sigcomp_amd/ and the CPU baseline timed by bench.py.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * The product path never calls it.
 *
 * Every function cites the reference source it restates (paths relative to
 * the reference's sigcomp/ package).  Pinning of each function (golden vectors
 * written from the reference, closed forms, invariants) is listed in the
 * header comment of oracle/oracle.py.
 *
 * Build: oracle/Makefile  ->  oracle/libsc_oracle.so
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#if defined(__x86_64__)
#include <immintrin.h>
#endif
#ifdef _OPENMP
#include <omp.h>
#endif

#define SCO_VOCAB 256
#define SCO_PRECISION 24
#define SCO_TOTAL ((int64_t)1 << SCO_PRECISION)
#define SCO_U32_MASK 0xFFFFFFFFull
#define SCO_U64_MAX 0xFFFFFFFFFFFFFFFFull
#define SCO_RENORM ((uint64_t)1 << 32)
#define SCO_MAX_LAYERS 16
#define SCO_ROW_BLOCK 64

/* Status codes shared with the HIP library (include/sigcomp_hip.h). */
#define SCO_OK 0
#define SCO_CAPACITY 1      /* cpu_entropy_coding.py:137-138 (OverflowError) */
#define SCO_INVALID 2       /* cpu_entropy_coding.py:240-248 (ValueError)    */
#define SCO_BAD_TOKEN 3     /* cpu_int_kernels.py:87-89                       */
#define SCO_BAD_ARG 4

/* ------------------------------------------------------------------------ */
/* Integer MLP                                                               */
/* ------------------------------------------------------------------------ */

typedef struct {
    int32_t n, k;               /* weight is [n, k] row-major (nn.Linear)      */
    const int8_t *w;
    const int32_t *bias;        /* [n]                                         */
    const int64_t *m0;          /* [n] requant multiplier (per-tensor: equal)  */
    const int32_t *shift;       /* [n] requant right shift                     */
    int32_t relu;
} sco_layer;

typedef struct {
    int32_t n_layers;
    int32_t window;             /* context tokens per row (64)                 */
    int32_t emb_rows, emb_dim;  /* 257 x 128                                   */
    const int8_t *emb;
    sco_layer layers[SCO_MAX_LAYERS];
} sco_model;

/* cpu_int_kernels.py:5-14 (_requantize): int32 wrapping bias add, int64
 * product with the multiplier, arithmetic (floor) right shift, clamp. */
static inline int8_t sco_requant(int32_t acc, int32_t bias, int64_t m0,
                                 int32_t shift, int32_t relu)
{
    int32_t biased = (int32_t)((uint32_t)acc + (uint32_t)bias);
    int64_t scaled = ((int64_t)biased * m0) >> shift;
    int64_t lo = relu ? 0 : -128;
    if (scaled < lo) scaled = lo;
    if (scaled > 127) scaled = 127;
    return (int8_t)scaled;
}

int8_t sco_requantize(int32_t acc, int32_t bias, int64_t m0, int32_t shift, int32_t relu)
{
    return sco_requant(acc, bias, m0, shift, relu);
}

/* int8 x int8 -> int32 dot product with int32 wrap-around accumulation, as
 * in cpu_int_kernels.py:143-156 (_linear_cell).  Partial sums are kept in
 * uint32 so that wrapping is defined behaviour in C. */
static inline uint32_t sco_dot(const int8_t *x, const int8_t *w, int32_t k)
{
    uint32_t acc = 0;
    for (int32_t i = 0; i < k; ++i)
        acc += (uint32_t)((int32_t)x[i] * (int32_t)w[i]);
    return acc;
}

/* Four rows against one weight row; the weight row is loaded once. */
static inline void sco_dot4(const int8_t *x0, const int8_t *x1, const int8_t *x2,
                            const int8_t *x3, const int8_t *w, int32_t k, uint32_t out[4])
{
    uint32_t a0 = 0, a1 = 0, a2 = 0, a3 = 0;
    for (int32_t i = 0; i < k; ++i) {
        int32_t wv = w[i];
        a0 += (uint32_t)((int32_t)x0[i] * wv);
        a1 += (uint32_t)((int32_t)x1[i] * wv);
        a2 += (uint32_t)((int32_t)x2[i] * wv);
        a3 += (uint32_t)((int32_t)x3[i] * wv);
    }
    out[0] = a0; out[1] = a1; out[2] = a2; out[3] = a3;
}

/* One quantised linear layer on `rows` activations (cpu_int_inference.py
 * :125-256 CPUBitExactInt8Linear; quant_mlp_export.py:21-76 on the GPU),
 * portable C. */
static void sco_linear_rows_c(const int8_t *x, int64_t rows, const sco_layer *L, int8_t *out)
{
    const int32_t k = L->k, n = L->n;
    int64_t r = 0;
    for (; r + 4 <= rows; r += 4) {
        const int8_t *x0 = x + (r + 0) * k, *x1 = x + (r + 1) * k;
        const int8_t *x2 = x + (r + 2) * k, *x3 = x + (r + 3) * k;
        for (int32_t j = 0; j < n; ++j) {
            uint32_t acc[4];
            sco_dot4(x0, x1, x2, x3, L->w + (int64_t)j * k, k, acc);
            for (int q = 0; q < 4; ++q)
                out[(r + q) * n + j] = sco_requant((int32_t)acc[q], L->bias[j], L->m0[j],
                                                   L->shift[j], L->relu);
        }
    }
    for (; r < rows; ++r)
        for (int32_t j = 0; j < n; ++j)
            out[r * n + j] = sco_requant((int32_t)sco_dot(x + r * k, L->w + (int64_t)j * k, k),
                                         L->bias[j], L->m0[j], L->shift[j], L->relu);
}

#if defined(__x86_64__)
/* The same layer with AVX-512 VNNI, as the reference's int_mm backend runs on
 * such hosts (oneDNN u8 x s8 dot products, cpu_int_inference.py:24-82):
 * vpdpbusd multiplies unsigned by signed bytes, so each activation byte is
 * offset by 128 (x ^ 0x80 = x + 128 as u8) and 128 * sum(w) is taken off
 * again.  Exact: |sum| < 2**31 for k <= 65536, so the int32 accumulators
 * never wrap, and the int32 result equals the wrapping sum of cpu_int_kernels.
 * k must be a multiple of 64; wsum[j] = sum of weight row j. */
__attribute__((target("avx512f,avx512bw,avx512vnni")))
static void sco_linear_rows_vnni(const int8_t *x, int64_t rows, const sco_layer *L, const int32_t *wsum,
                                 int8_t *out)
{
    const int32_t k = L->k, n = L->n;
    const __m512i flip = _mm512_set1_epi8((char)0x80);
    int64_t r = 0;
    for (; r < rows; r += 4) {
        const int nr = rows - r < 4 ? (int)(rows - r) : 4;
        const int8_t *xr[4];
        for (int q = 0; q < 4; ++q) xr[q] = x + (r + (q < nr ? q : 0)) * k;
        for (int32_t j = 0; j + 1 < n; j += 2) {
            const int8_t *w0 = L->w + (int64_t)j * k, *w1 = w0 + k;
            __m512i a[4][2];
            for (int q = 0; q < 4; ++q) a[q][0] = a[q][1] = _mm512_setzero_si512();
            for (int32_t i = 0; i < k; i += 64) {
                const __m512i b0 = _mm512_loadu_si512((const void *)(w0 + i));
                const __m512i b1 = _mm512_loadu_si512((const void *)(w1 + i));
                for (int q = 0; q < 4; ++q) {
                    const __m512i xv = _mm512_xor_si512(_mm512_loadu_si512((const void *)(xr[q] + i)), flip);
                    a[q][0] = _mm512_dpbusd_epi32(a[q][0], xv, b0);
                    a[q][1] = _mm512_dpbusd_epi32(a[q][1], xv, b1);
                }
            }
            for (int q = 0; q < nr; ++q)
                for (int h = 0; h < 2; ++h) {
                    const int32_t acc = _mm512_reduce_add_epi32(a[q][h]) - 128 * wsum[j + h];
                    out[(r + q) * n + j + h] = sco_requant(acc, L->bias[j + h], L->m0[j + h], L->shift[j + h],
                                                           L->relu);
                }
        }
        if (n & 1) {
            const int32_t j = n - 1;
            for (int q = 0; q < nr; ++q)
                out[(r + q) * n + j] = sco_requant((int32_t)sco_dot(xr[q], L->w + (int64_t)j * k, k), L->bias[j],
                                                   L->m0[j], L->shift[j], L->relu);
        }
    }
}
#endif

int sco_num_threads(void);

/* 1 when the VNNI path runs (x86-64 host with AVX-512 VNNI, and
 * SCO_NO_VNNI unset or 0). */
int sco_uses_vnni(void)
{
#if defined(__x86_64__)
    static int state = -1;
    if (state < 0) {
        const char *e = getenv("SCO_NO_VNNI");
        __builtin_cpu_init();
        state = (!e || e[0] == '0') && __builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512bw");
    }
    return state;
#else
    return 0;
#endif
}

/* Weight row sums of a layer (for the VNNI offset), malloc'ed. */
static int32_t *sco_row_sums(const sco_layer *L)
{
    int32_t *ws = (int32_t *)malloc(sizeof(int32_t) * (size_t)L->n);
    for (int32_t j = 0; j < L->n; ++j) {
        int32_t t = 0;
        for (int32_t i = 0; i < L->k; ++i) t += L->w[(int64_t)j * L->k + i];
        ws[j] = t;
    }
    return ws;
}

static void sco_linear_rows(const int8_t *x, int64_t rows, const sco_layer *L, const int32_t *wsum, int8_t *out)
{
#if defined(__x86_64__)
    if (wsum && L->k % 64 == 0) {
        sco_linear_rows_vnni(x, rows, L, wsum, out);
        return;
    }
#endif
    (void)wsum;
    sco_linear_rows_c(x, rows, L, out);
}

void sco_linear(const int8_t *x, int64_t rows, int32_t k, const int8_t *w, int32_t n,
                const int32_t *bias, const int64_t *m0, const int32_t *shift, int32_t relu,
                int8_t *out)
{
    sco_layer L = {n, k, w, bias, m0, shift, relu};
    int32_t *wsum = sco_uses_vnni() ? sco_row_sums(&L) : NULL;
#pragma omp parallel for schedule(static)
    for (int64_t r0 = 0; r0 < rows; r0 += SCO_ROW_BLOCK) {
        int64_t cnt = rows - r0 < SCO_ROW_BLOCK ? rows - r0 : SCO_ROW_BLOCK;
        sco_linear_rows(x + r0 * k, cnt, &L, wsum, out + r0 * n);
    }
    free(wsum);
}

/* Embedding gather of a token window into one flat activation row,
 * position-major (cpu_int_kernels.py:81-92 _embedding_row;
 * quant_mlp_export.py:133-135).  Out-of-range tokens flag an error. */
static int sco_embed_row(const sco_model *M, const int32_t *window, int8_t *out)
{
    for (int32_t p = 0; p < M->window; ++p) {
        int32_t tok = window[p];
        if (tok < 0 || tok >= M->emb_rows) return SCO_BAD_TOKEN;
        memcpy(out + (int64_t)p * M->emb_dim, M->emb + (int64_t)tok * M->emb_dim,
               (size_t)M->emb_dim);
    }
    return SCO_OK;
}

static int64_t sco_max_width(const sco_model *M)
{
    int64_t w = (int64_t)M->window * M->emb_dim;
    for (int i = 0; i < M->n_layers; ++i)
        if (M->layers[i].n > w) w = M->layers[i].n;
    return w;
}

/* Forward pass over up to SCO_ROW_BLOCK rows whose windows are given
 * explicitly (GPUBitExactMLPDecoder._ar_step, quant_mlp_export.py:133-138;
 * CPUBitExactMLPDecoder._ar_step, cpu_int_inference.py:323-343). */
static int sco_mlp_block(const sco_model *M, int32_t *const *wsum, const int32_t *ctx, int64_t rows,
                         int8_t *buf0, int8_t *buf1, int8_t *logits)
{
    const int64_t in_w = (int64_t)M->window * M->emb_dim;
    for (int64_t r = 0; r < rows; ++r) {
        int st = sco_embed_row(M, ctx + r * M->window, buf0 + r * in_w);
        if (st) return st;
    }
    int8_t *src = buf0, *dst = buf1;
    for (int i = 0; i < M->n_layers; ++i) {
        const int last = i == M->n_layers - 1;
        sco_linear_rows(src, rows, &M->layers[i], wsum ? wsum[i] : NULL, last ? logits : dst);
        if (!last) { int8_t *t = src; src = dst; dst = t; }
    }
    return SCO_OK;
}

int sco_mlp_forward(const sco_model *M, const int32_t *ctx, int64_t rows, int8_t *logits)
{
    if (!M || M->n_layers < 1 || M->n_layers > SCO_MAX_LAYERS) return SCO_BAD_ARG;
    const int64_t wmax = sco_max_width(M);
    const int32_t n_out = M->layers[M->n_layers - 1].n;
    int status = SCO_OK;
    int32_t *wsum[SCO_MAX_LAYERS];
    const int vnni = sco_uses_vnni();
    for (int i = 0; i < M->n_layers; ++i) wsum[i] = vnni ? sco_row_sums(&M->layers[i]) : NULL;
    /* row blocks of at most SCO_ROW_BLOCK, small enough that every thread
     * gets about two (batches of a few hundred rows keep all threads busy) */
    int64_t blk = (rows + 2 * (int64_t)sco_num_threads() - 1) / (2 * (int64_t)sco_num_threads());
    blk = (blk + 3) / 4 * 4;
    if (blk < 4) blk = 4;
    if (blk > SCO_ROW_BLOCK) blk = SCO_ROW_BLOCK;
#pragma omp parallel
    {
        int8_t *b0 = (int8_t *)malloc((size_t)(SCO_ROW_BLOCK * wmax));
        int8_t *b1 = (int8_t *)malloc((size_t)(SCO_ROW_BLOCK * wmax));
#pragma omp for schedule(dynamic, 1)
        for (int64_t r0 = 0; r0 < rows; r0 += blk) {
            int64_t cnt = rows - r0 < blk ? rows - r0 : blk;
            int st = sco_mlp_block(M, vnni ? wsum : NULL, ctx + r0 * M->window, cnt, b0, b1, logits + r0 * n_out);
            if (st) {
#pragma omp atomic write
                status = st;
            }
        }
        free(b0);
        free(b1);
    }
    for (int i = 0; i < M->n_layers; ++i) free(wsum[i]);
    return status;
}

/* ------------------------------------------------------------------------ */
/* logits -> frequency table (cpu_entropy_coding.py:90-110 _frequencies;      */
/* gpu_entropy_coding.py:163-188 inside the Triton step kernels)             */
/* ------------------------------------------------------------------------ */

void sco_frequencies(const int8_t *logits, const int64_t *lut, int64_t *freq)
{
    int32_t maximum = -128;
    for (int v = 0; v < SCO_VOCAB; ++v)
        if (logits[v] > maximum) maximum = logits[v];
    int64_t total = 0;
    for (int v = 0; v < SCO_VOCAB; ++v) {
        freq[v] = lut[maximum - (int32_t)logits[v]];
        total += freq[v];
    }
    int64_t total_freq = 0, max_freq = 0;
    int max_index = 0;
    for (int v = 0; v < SCO_VOCAB; ++v) {
        int64_t f = (freq[v] * SCO_TOTAL) / total;   /* both nonnegative: floor */
        if (f < 1) f = 1;
        freq[v] = f;
        total_freq += f;
        if (f > max_freq) { max_freq = f; max_index = v; }   /* first argmax */
    }
    freq[max_index] -= total_freq - SCO_TOTAL;
}

/* int8_logits_to_cdf (cpu_entropy_coding.py:73-87): [rows, 257] int64 with
 * cdf[0] = 0 and cdf[256] = 2**24. */
void sco_logits_to_cdf(const int8_t *logits, int64_t rows, const int64_t *lut, int64_t *cdf)
{
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        int64_t f[SCO_VOCAB];
        sco_frequencies(logits + r * SCO_VOCAB, lut, f);
        int64_t *c = cdf + r * (SCO_VOCAB + 1);
        c[0] = 0;
        for (int v = 0; v < SCO_VOCAB; ++v) c[v + 1] = c[v] + f[v];
    }
}

/* ------------------------------------------------------------------------ */
/* Range coder (cpu_entropy_coding.py:121-266; Triton twin                    */
/* gpu_entropy_coding.py:78-397)                                             */
/* ------------------------------------------------------------------------ */

typedef struct {
    uint64_t lower, range;
    int64_t inverted;           /* pending "inverted" words                     */
    uint32_t first;             /* first pending word                           */
    int64_t pos;                /* words written                                */
} sco_enc;

void sco_enc_init(sco_enc *e)
{
    e->lower = 0;
    e->range = SCO_U64_MAX;
    e->inverted = 0;
    e->first = 0;
    e->pos = 0;
}

/* One encoder step given the symbol's cumulative frequency and frequency
 * (_encode_one, cpu_entropy_coding.py:121-161). */
static int sco_enc_step(sco_enc *e, uint64_t cum, uint64_t freq, uint32_t *out, int64_t cap)
{
    uint64_t scale = e->range >> SCO_PRECISION;
    uint64_t new_range = scale * freq;
    uint64_t new_lower = e->lower + scale * cum;
    if (e->inverted > 0 && new_lower + new_range > new_lower) {
        uint64_t emit_first, emit_rest;
        if (new_lower < e->lower) { emit_first = (uint64_t)e->first + 1; emit_rest = 0; }
        else { emit_first = e->first; emit_rest = SCO_U32_MASK; }
        if (e->pos + e->inverted > cap) return SCO_CAPACITY;
        out[e->pos++] = (uint32_t)(emit_first & SCO_U32_MASK);
        for (int64_t i = 0; i < e->inverted - 1; ++i) out[e->pos++] = (uint32_t)emit_rest;
        e->inverted = 0;
    }
    e->lower = new_lower;
    e->range = new_range;
    if (e->range < SCO_RENORM) {
        e->range <<= 32;
        uint32_t word = (uint32_t)(e->lower >> 32);
        e->lower <<= 32;
        if (e->inverted > 0) {
            e->inverted += 1;
        } else if (e->lower + e->range > e->lower) {
            if (e->pos >= cap) return SCO_CAPACITY;
            out[e->pos++] = word;
        } else {
            e->inverted = 1;
            e->first = word;
        }
    }
    return SCO_OK;
}

int sco_enc_symbol(sco_enc *e, const int8_t *logits, const int64_t *lut, int32_t symbol,
                   uint32_t *out, int64_t cap)
{
    if (symbol < 0 || symbol >= SCO_VOCAB) return SCO_BAD_TOKEN;
    int64_t f[SCO_VOCAB];
    sco_frequencies(logits, lut, f);
    uint64_t cum = 0;
    for (int v = 0; v < symbol; ++v) cum += (uint64_t)f[v];
    return sco_enc_step(e, cum, (uint64_t)f[symbol], out, cap);
}

/* _seal (cpu_entropy_coding.py:206-227). */
int sco_enc_seal(sco_enc *e, uint32_t *out, int64_t cap)
{
    if (e->range == SCO_U64_MAX) return SCO_OK;
    uint64_t point = e->lower + SCO_U32_MASK;
    if (e->inverted > 0) {
        uint64_t emit_first, emit_rest;
        if (point < e->lower) { emit_first = (uint64_t)e->first + 1; emit_rest = 0; }
        else { emit_first = e->first; emit_rest = SCO_U32_MASK; }
        if (e->pos + e->inverted > cap) return SCO_CAPACITY;
        out[e->pos++] = (uint32_t)(emit_first & SCO_U32_MASK);
        for (int64_t i = 0; i < e->inverted - 1; ++i) out[e->pos++] = (uint32_t)emit_rest;
        e->inverted = 0;
    }
    uint64_t point_word = point >> 32;
    if (e->pos >= cap) return SCO_CAPACITY;
    out[e->pos++] = (uint32_t)point_word;
    uint64_t upper_word = (e->lower + e->range) >> 32;
    if (upper_word == point_word) {
        if (e->pos >= cap) return SCO_CAPACITY;
        out[e->pos++] = 0;
    }
    e->range = SCO_U64_MAX;   /* sealed: a second seal emits nothing */
    return SCO_OK;
}

/* Encode a whole stream from precomputed logits, then seal
 * (CpuRangeStepEncoder.encode_logits + seal + get_compressed,
 * cpu_entropy_coding.py:410-448). Returns the status; *n_words = words. */
int sco_encode_stream(const int8_t *logits, const int32_t *symbols, int64_t length,
                      const int64_t *lut, uint32_t *out, int64_t cap, int64_t *n_words)
{
    sco_enc e;
    sco_enc_init(&e);
    for (int64_t t = 0; t < length; ++t) {
        int st = sco_enc_symbol(&e, logits + t * SCO_VOCAB, lut, symbols[t], out, cap);
        if (st) { *n_words = e.pos; return st; }
    }
    int st = sco_enc_seal(&e, out, cap);
    *n_words = e.pos;
    return st;
}

typedef struct {
    uint64_t lower, range, point;
    int64_t read_pos, end_pos;  /* indices into the stream's own words          */
} sco_dec;

/* Decoder construction (CpuRangeDecoder.__init__, cpu_entropy_coding.py
 * :454-478): the point is the first two words, big-word first. */
void sco_dec_init(sco_dec *d, const uint32_t *words, int64_t n_words)
{
    uint64_t point = 0;
    int64_t take = n_words < 2 ? n_words : 2;
    for (int64_t i = 0; i < take; ++i) point = (point << 32) | words[i];
    if (n_words == 1) point <<= 32;
    d->lower = 0;
    d->range = SCO_U64_MAX;
    d->point = point;
    d->read_pos = take;
    d->end_pos = n_words;
}

/* One decoder step (_decode_partition, cpu_entropy_coding.py:230-266).
 * Returns the status; the symbol goes to *symbol. */
int sco_dec_step(sco_dec *d, const int8_t *logits, const int64_t *lut, const uint32_t *words,
                 int32_t *symbol)
{
    uint64_t scale = d->range >> SCO_PRECISION;
    if (scale == 0) { *symbol = SCO_VOCAB; return SCO_INVALID; }
    uint64_t quantile = (d->point - d->lower) / scale;
    if (quantile >= (uint64_t)SCO_TOTAL) { *symbol = SCO_VOCAB; return SCO_INVALID; }
    int64_t f[SCO_VOCAB];
    sco_frequencies(logits, lut, f);
    uint64_t cum = 0;
    int32_t s = 0;
    while (s < SCO_VOCAB - 1 && cum + (uint64_t)f[s] <= quantile) {
        cum += (uint64_t)f[s];
        ++s;
    }
    d->lower += scale * cum;
    d->range = scale * (uint64_t)f[s];
    if (d->range < SCO_RENORM) {
        d->lower <<= 32;
        d->range <<= 32;
        d->point <<= 32;
        if (d->read_pos < d->end_pos) d->point |= words[d->read_pos];
        d->read_pos += 1;
    }
    *symbol = s;
    return SCO_OK;
}

/* Decode a stream whose per-step logits are known in advance (the coder in
 * isolation; the AR driver below computes them from the decoded context). */
int sco_decode_stream(const uint32_t *words, int64_t n_words, const int8_t *logits,
                      int64_t length, const int64_t *lut, int32_t *symbols)
{
    sco_dec d;
    sco_dec_init(&d, words, n_words);
    for (int64_t t = 0; t < length; ++t) {
        int st = sco_dec_step(&d, logits + t * SCO_VOCAB, lut, words, symbols + t);
        if (st) return st;
    }
    return SCO_OK;
}

/* ------------------------------------------------------------------------ */
/* Chunk drivers                                                             */
/* ------------------------------------------------------------------------ */

/* Window of step t over a chunk: context_buf = [SOS x window | symbols], the
 * window of step t is context_buf[t : t + window]
 * (quant_mlp_export.py:296-309; cpu_compression.py:217-226). */
static inline int32_t sco_window_token(const uint8_t *tokens, int64_t t, int32_t p,
                                       int32_t window, int32_t sos)
{
    int64_t j = t + p - window;
    return j < 0 ? sos : (int32_t)tokens[j];
}

/* Compress one chunk: teacher-forced MLP over every step, then the range
 * encoder and seal (CPUQuantMLPCompression.compress_chunks,
 * cpu_compression.py:178-257). */
static int sco_compress_one(const sco_model *M, int32_t *const *wsum, const int64_t *lut,
                            const uint8_t *tokens, int64_t length, uint32_t *out, int64_t cap,
                            int64_t *n_words, int32_t *ctx, int8_t *b0, int8_t *b1, int8_t *logits)
{
    const int32_t sos = M->emb_rows - 1;
    sco_enc e;
    sco_enc_init(&e);
    for (int64_t t0 = 0; t0 < length; t0 += SCO_ROW_BLOCK) {
        int64_t cnt = length - t0 < SCO_ROW_BLOCK ? length - t0 : SCO_ROW_BLOCK;
        for (int64_t r = 0; r < cnt; ++r)
            for (int32_t p = 0; p < M->window; ++p)
                ctx[r * M->window + p] = sco_window_token(tokens, t0 + r, p, M->window, sos);
        int st = sco_mlp_block(M, wsum, ctx, cnt, b0, b1, logits);
        if (st) return st;
        for (int64_t r = 0; r < cnt; ++r) {
            st = sco_enc_symbol(&e, logits + r * SCO_VOCAB, lut, tokens[t0 + r], out, cap);
            if (st) { *n_words = e.pos; return st; }
        }
    }
    int st = sco_enc_seal(&e, out, cap);
    *n_words = e.pos;
    return st;
}

/* Compress n_chunks chunks in parallel.  Chunk c has lengths[c] tokens at
 * tokens + tok_off[c]; its words go to words + word_off[c] with capacity
 * word_cap[c]; the word count goes to word_cnt[c] and the status to
 * status[c].  Returns the first nonzero status. */
int sco_compress_chunks(const sco_model *M, const int64_t *lut, const uint8_t *tokens,
                        const int64_t *tok_off, const int32_t *lengths, int64_t n_chunks,
                        uint32_t *words, const int64_t *word_off, const int64_t *word_cap,
                        int32_t *word_cnt, int32_t *status)
{
    const int64_t wmax = sco_max_width(M);
    int result = SCO_OK;
    int32_t *wsum[SCO_MAX_LAYERS];
    const int vnni = sco_uses_vnni();
    for (int i = 0; i < M->n_layers; ++i) wsum[i] = vnni ? sco_row_sums(&M->layers[i]) : NULL;
#pragma omp parallel
    {
        int32_t *ctx = (int32_t *)malloc(sizeof(int32_t) * SCO_ROW_BLOCK * M->window);
        int8_t *b0 = (int8_t *)malloc((size_t)(SCO_ROW_BLOCK * wmax));
        int8_t *b1 = (int8_t *)malloc((size_t)(SCO_ROW_BLOCK * wmax));
        int8_t *lg = (int8_t *)malloc((size_t)SCO_ROW_BLOCK * SCO_VOCAB);
#pragma omp for schedule(dynamic, 1)
        for (int64_t c = 0; c < n_chunks; ++c) {
            int64_t nw = 0;
            int st = sco_compress_one(M, vnni ? wsum : NULL, lut, tokens + tok_off[c], lengths[c],
                                      words + word_off[c], word_cap[c], &nw, ctx, b0, b1, lg);
            word_cnt[c] = (int32_t)nw;
            status[c] = st;
            if (st) {
#pragma omp atomic write
                result = st;
            }
        }
        free(ctx); free(b0); free(b1); free(lg);
    }
    for (int i = 0; i < M->n_layers; ++i) free(wsum[i]);
    return result;
}

/* Decompress n_chunks chunks.  The decode is autoregressive in time and
 * batched across chunks: every step runs one MLP row per active chunk, as
 * CPUQuantMLPCompression.decompress_chunks does (cpu_compression.py:259-332).
 * Chunk c's words are words + word_off[c] (word_cnt[c] of them); its
 * lengths[c] decoded tokens go to tokens + tok_off[c]. */
int sco_decompress_chunks(const sco_model *M, const int64_t *lut, const uint32_t *words,
                          const int64_t *word_off, const int32_t *word_cnt,
                          const int32_t *lengths, int64_t n_chunks, uint8_t *tokens,
                          const int64_t *tok_off, int32_t *status)
{
    const int32_t sos = M->emb_rows - 1;
    const int32_t W = M->window;
    int32_t max_len = 0;
    for (int64_t c = 0; c < n_chunks; ++c) if (lengths[c] > max_len) max_len = lengths[c];
    sco_dec *dec = (sco_dec *)malloc(sizeof(sco_dec) * (size_t)(n_chunks ? n_chunks : 1));
    int64_t *active = (int64_t *)malloc(sizeof(int64_t) * (size_t)(n_chunks ? n_chunks : 1));
    int32_t *ctx = (int32_t *)malloc(sizeof(int32_t) * (size_t)(n_chunks ? n_chunks : 1) * W);
    int8_t *logits = (int8_t *)malloc((size_t)(n_chunks ? n_chunks : 1) * SCO_VOCAB);
    for (int64_t c = 0; c < n_chunks; ++c) {
        sco_dec_init(&dec[c], words + word_off[c], word_cnt[c]);
        status[c] = SCO_OK;
    }
    int result = SCO_OK;
    for (int32_t t = 0; t < max_len; ++t) {
        int64_t n_act = 0;
        for (int64_t c = 0; c < n_chunks; ++c)
            if (t < lengths[c] && status[c] == SCO_OK) active[n_act++] = c;
        if (!n_act) break;
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < n_act; ++i) {
            int64_t c = active[i];
            for (int32_t p = 0; p < W; ++p)
                ctx[i * W + p] = sco_window_token(tokens + tok_off[c], t, p, W, sos);
        }
        int st = sco_mlp_forward(M, ctx, n_act, logits);
        if (st) { result = st; break; }
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < n_act; ++i) {
            int64_t c = active[i];
            int32_t s;
            int st2 = sco_dec_step(&dec[c], logits + i * SCO_VOCAB, lut, words + word_off[c], &s);
            if (st2) status[c] = st2;
            else tokens[tok_off[c] + t] = (uint8_t)s;
        }
    }
    for (int64_t c = 0; c < n_chunks && result == SCO_OK; ++c)
        if (status[c]) result = status[c];
    free(dec); free(active); free(ctx); free(logits);
    return result;
}

int sco_num_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void sco_set_num_threads(int n)
{
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}
