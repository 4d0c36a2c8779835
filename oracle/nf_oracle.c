/*
 * nf_oracle.c — CPU oracle for the quantized linear path.
 *
 * TEST INFRASTRUCTURE ONLY (see nf_oracle.h): the checker and the timed CPU
 * baseline, never part of the product path.  Built with -ffp-contract=off so
 * every `acc += a * b` is a separately rounded multiply and add, in k order,
 * exactly as the reference's loop is written (dequant_test.cpp:313-319).
 */
#include "nf_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* fp16 bits -> fp32, restating dequant_test.cpp:77-98 (exact for every
 * input, subnormals normalised, Inf/NaN payload kept). */
float nf_oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t mant = h & 0x3FFu;
    uint32_t f;
    if (exp == 0) {
        if (mant == 0) {
            f = sign;
        } else {
            exp = 1;
            while (!(mant & 0x400u)) {
                mant <<= 1;
                exp--;
            }
            mant &= 0x3FFu;
            f = sign | ((exp + 127 - 15) << 23) | (mant << 13);
        }
    } else if (exp == 31) {
        f = sign | 0x7F800000u | (mant << 13);
    } else {
        f = sign | ((exp + 127 - 15) << 23) | (mant << 13);
    }
    float r;
    memcpy(&r, &f, 4);
    return r;
}

/* fp32 -> fp16 with IEEE 754 roundTiesToEven, gradual underflow and
 * overflow to infinity; NaN stays NaN (quiet bit set, top payload kept). */
uint16_t nf_oracle_f32_to_f16_rne(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 rounds to inf */
    const int e = (int)(ax >> 23) - 127;
    if (e < -25 - 1) return sign; /* below a quarter of the smallest subnormal */
    /* significand with the implicit bit (f32 subnormals never reach here
     * in a way that matters: they are far below the fp16 range) */
    const uint32_t m = (ax & 0x7FFFFFu) | ((ax >> 23) ? 0x800000u : 0u);
    uint32_t shift, base;
    if (e >= -14) { /* fp16 normal: keep 11 significant bits */
        shift = 13;
        base = (uint32_t)(e + 15) << 10;
    } else { /* fp16 subnormal: value / 2^-24 = m * 2^(e+1) */
        shift = (uint32_t)(-(e + 1));
        base = 0;
    }
    uint32_t h = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) h++;
    /* normal: h carries the implicit bit (0x400..0x800); adding to the
     * biased exponent field handles a carry into the next binade. */
    return (uint16_t)(sign | (e >= -14 ? base + (h - 0x400u) : h));
}

/* The reference tests' own encoder (dequant_test.cpp:100-109): truncates
 * the mantissa and flushes anything below the fp16 normal range to zero.
 * Only used to rebuild those tests' input blocks bit for bit. */
uint16_t nf_oracle_f32_to_f16_trunc(float val) {
    uint32_t f;
    memcpy(&f, &val, 4);
    uint16_t sign = (uint16_t)((f >> 16) & 0x8000u);
    int exp = (int)((f >> 23) & 0xFFu) - 127 + 15;
    uint32_t mant = f & 0x7FFFFFu;
    if (exp <= 0) return sign;
    if (exp >= 31) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | (uint16_t)(exp << 10) | (uint16_t)(mant >> 13));
}

void nf_oracle_f16_to_f32_n(const uint16_t *in, float *out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = nf_oracle_f16_to_f32(in[i]);
}

void nf_oracle_f32_to_f16_rne_n(const float *in, uint16_t *out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = nf_oracle_f32_to_f16_rne(in[i]);
}

/* ---- element decode (flat index e into the block stream) ----------- */

static inline float scale_of(const uint8_t *blk) {
    return nf_oracle_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
}

/* ref_dequant_q4_0 (dequant_test.cpp:112-120) for one element. */
static inline float q4_0_elem(const uint8_t *W, uint64_t e) {
    const uint8_t *blk = W + (e / 32) * 18;
    const int i = (int)(e % 32);
    const int nibble = (i < 16) ? (blk[2 + i] & 0xF) : (blk[2 + i - 16] >> 4);
    return scale_of(blk) * (float)(nibble - 8);
}

/* ref_dequant_q8_0 (dequant_test.cpp:123-128) for one element. */
static inline float q8_0_elem(const uint8_t *W, uint64_t e) {
    const uint8_t *blk = W + (e / 32) * 34;
    return scale_of(blk) * (float)(int8_t)blk[2 + (e % 32)];
}

void nf_oracle_dequant_q4_0_f32(const uint8_t *blocks, uint64_t count, float *out) {
    for (uint64_t e = 0; e < count; ++e) out[e] = q4_0_elem(blocks, e);
}

void nf_oracle_dequant_q8_0_f32(const uint8_t *blocks, uint64_t count, float *out) {
    for (uint64_t e = 0; e < count; ++e) out[e] = q8_0_elem(blocks, e);
}

void nf_oracle_dequant_q4_0_f16(const uint8_t *blocks, uint64_t count, uint16_t *out) {
    for (uint64_t e = 0; e < count; ++e) out[e] = nf_oracle_f32_to_f16_rne(q4_0_elem(blocks, e));
}

void nf_oracle_dequant_q8_0_f16(const uint8_t *blocks, uint64_t count, uint16_t *out) {
    for (uint64_t e = 0; e < count; ++e) out[e] = nf_oracle_f32_to_f16_rne(q8_0_elem(blocks, e));
}

/* ---- the other GGUF block formats (dequant_<fmt>[_f16]) ------------- */
/*
 * The reference's layouts are simplified ones (not llama.cpp's interleaved
 * K-quant order): element i of a block reads its code bits at the plain
 * positions written below.  Offsets are byte offsets inside one block.
 */

static const struct { uint32_t bytes, elems; } kq_geom[NF_ORACLE_NFMT] = {
    [NF_ORACLE_Q4_0] = {18, 32},  [NF_ORACLE_Q8_0] = {34, 32},  [NF_ORACLE_Q4_1] = {20, 32},
    [NF_ORACLE_Q5_0] = {22, 32},  [NF_ORACLE_Q5_1] = {24, 32},  [NF_ORACLE_Q2_K] = {84, 256},
    [NF_ORACLE_Q3_K] = {110, 256}, [NF_ORACLE_Q4_K] = {144, 256}, [NF_ORACLE_Q5_K] = {176, 256},
    [NF_ORACLE_Q6_K] = {210, 256},
};

static inline float half_at(const uint8_t *blk, int off) {
    return nf_oracle_f16_to_f32((uint16_t)(blk[off] | (blk[off + 1] << 8)));
}

/* Low nibble of qs[i] for i < 16, high nibble of qs[i-16] otherwise. */
static inline int nib32(const uint8_t *qs, int i) { return i < 16 ? (qs[i] & 0xF) : (qs[i - 16] >> 4); }

/* Bit i of the 32-bit high-bit mask qh (little-endian bytes). */
static inline int bit_of(const uint8_t *qh, int i) { return (qh[i / 8] >> (i % 8)) & 1; }

/* ref_dequant_q4_1 (kquant_dequant_test.cpp:118-125): {d, m, qs[16]}. */
static float q4_1_elem(const uint8_t *b, int i) {
    return half_at(b, 0) * (float)nib32(b + 4, i) + half_at(b, 2);
}

/* ref_dequant_q5_0 (kquant_dequant_test.cpp:127-134): {d, qh[4], qs[16]}. */
static float q5_0_elem(const uint8_t *b, int i) {
    return half_at(b, 0) * (float)((nib32(b + 6, i) | (bit_of(b + 2, i) << 4)) - 16);
}

/* ref_dequant_q5_1 (kquant_dequant_test.cpp:136-144): {d, m, qh[4], qs[16]}. */
static float q5_1_elem(const uint8_t *b, int i) {
    return half_at(b, 0) * (float)(nib32(b + 8, i) | (bit_of(b + 4, i) << 4)) + half_at(b, 2);
}

/* ref_dequant_q2_k (kquant_dequant_test.cpp:148-160): {scales[16], qs[64],
 * d, dmin}; 16 sub-blocks of 16, scale byte = (min << 4) | scale. */
static float q2_k_elem(const uint8_t *b, int i) {
    const uint8_t s = b[i / 16];
    const float sc = (float)(s & 0xF) * half_at(b, 80);
    const float mn = (float)(s >> 4) * half_at(b, 82);
    const int q2 = (b[16 + i / 4] >> ((i % 4) * 2)) & 3;
    return sc * (float)q2 - mn;
}

static inline int q3_code(const uint8_t *b, int i) {
    return (((b[32 + i / 4] >> ((i % 4) * 2)) & 3) | (bit_of(b, i) << 2)) - 4;
}

/* ref_dequant_q3_k (kquant_dequant_test.cpp:162-183): {hmask[32], qs[64],
 * scales[12], d}; 6-bit signed sub-block scales, low nibbles of bytes 0..7
 * (sub < 8) or high nibbles (sub >= 8), top two bits from bytes 8..11. */
static float q3_k_elem(const uint8_t *b, int i) {
    const uint8_t *sc = b + 96;
    const int sub = i / 16;
    int scale;
    if (sub < 8)
        scale = (sc[sub] & 0xF) | (((sc[8 + sub / 2] >> (4 * (sub % 2))) & 3) << 4);
    else
        scale = (sc[sub - 8] >> 4) | (((sc[8 + (sub - 8) / 2] >> (4 * ((sub - 8) % 2) + 2)) & 3) << 4);
    return half_at(b, 108) * (float)(scale - 32) * (float)q3_code(b, i);
}

/* dequant_q3_k_f16 (metal_provider.mm:833-848) takes the raw byte at
 * scales[sub] - 32 as the scale, for sub = 0..15 of a 12-byte array: sub 12
 * and 13 read the bytes of d, sub 14 and 15 the first two bytes of the next
 * block.  `at(off)` is the byte at flat stream offset `off`, 0 past the end
 * of the input buffer (the Metal read there is out of bounds). */
static float q3_k_f16_elem(const uint8_t *W, uint64_t in_bytes, uint64_t blk_off, int i) {
    const uint64_t off = blk_off + 96 + (uint64_t)(i / 16);
    const int raw = off < in_bytes ? W[off] : 0;
    const uint8_t *b = W + blk_off;
    return half_at(b, 108) * (float)(raw - 32) * (float)q3_code(b, i);
}

/* Scale / min of sub-block `sub` (0..7) from the 12 packed bytes
 * (kquant_dequant_test.cpp:190-198). */
static inline void k_scale_min(const uint8_t *sc, int sub, int *s, int *m) {
    if (sub < 4) {
        *s = sc[sub] & 0x3F;
        *m = sc[sub + 4] & 0x3F;
    } else {
        *s = (sc[sub - 4] >> 6) | ((sc[sub + 4] & 0x0F) << 2);
        *m = (sc[sub] >> 6) | ((sc[sub + 4] >> 4) << 2);
    }
}

/* ref_dequant_q4_k (kquant_dequant_test.cpp:185-203): {d, dmin, scales[12],
 * qs[128]}; 8 sub-blocks of 32, element i = nibble (i odd: high) of qs[i/2]. */
static float q4_k_elem(const uint8_t *b, int i) {
    int s, m;
    k_scale_min(b + 4, i / 32, &s, &m);
    const int q = (i & 1) ? (b[16 + i / 2] >> 4) : (b[16 + i / 2] & 0xF);
    return half_at(b, 0) * (float)s * (float)q - half_at(b, 2) * (float)m;
}

/* ref_dequant_q5_k (kquant_dequant_test.cpp:205-224): q4_k plus bit i of qh. */
static float q5_k_elem(const uint8_t *b, int i) {
    int s, m;
    k_scale_min(b + 4, i / 32, &s, &m);
    const int q = ((i & 1) ? (b[16 + i / 2] >> 4) : (b[16 + i / 2] & 0xF)) | (bit_of(b + 144, i) << 4);
    return half_at(b, 0) * (float)s * (float)q - half_at(b, 2) * (float)m;
}

/* dequant_q6_k (metal_provider.mm:534-573): {ql[128], qh[64], int8
 * scales[16], d}; low nibble from ql[i/2] (i odd: high), two high bits from
 * qh[i/4] at bit 2*(i%4); scale = scales[i/16] * d. */
static float q6_k_elem(const uint8_t *b, int i) {
    const float scale = (float)(int8_t)b[192 + i / 16] * half_at(b, 208);
    const int lo = (i & 1) ? (b[i / 2] >> 4) : (b[i / 2] & 0xF);
    const int hi = (b[128 + i / 4] >> ((i % 4) * 2)) & 3;
    return scale * (float)(((hi << 4) | lo) - 32);
}

uint32_t nf_oracle_block_bytes(int fmt) {
    return (fmt >= 0 && fmt < NF_ORACLE_NFMT) ? kq_geom[fmt].bytes : 0;
}

uint32_t nf_oracle_block_elems(int fmt) {
    return (fmt >= 0 && fmt < NF_ORACLE_NFMT) ? kq_geom[fmt].elems : 0;
}

static float elem_of(int fmt, const uint8_t *W, uint64_t in_bytes, uint64_t e, int f16) {
    const uint64_t be = kq_geom[fmt].elems;
    const uint64_t off = (e / be) * kq_geom[fmt].bytes;
    const uint8_t *b = W + off;
    const int i = (int)(e % be);
    switch (fmt) {
        case NF_ORACLE_Q4_0: return q4_0_elem(W, e);
        case NF_ORACLE_Q8_0: return q8_0_elem(W, e);
        case NF_ORACLE_Q4_1: return q4_1_elem(b, i);
        case NF_ORACLE_Q5_0: return q5_0_elem(b, i);
        case NF_ORACLE_Q5_1: return q5_1_elem(b, i);
        case NF_ORACLE_Q2_K: return q2_k_elem(b, i);
        case NF_ORACLE_Q3_K: return f16 ? q3_k_f16_elem(W, in_bytes, off, i) : q3_k_elem(b, i);
        case NF_ORACLE_Q4_K: return q4_k_elem(b, i);
        case NF_ORACLE_Q5_K: return q5_k_elem(b, i);
        default: return q6_k_elem(b, i);
    }
}

int nf_oracle_dequant(int fmt, const uint8_t *blocks, uint64_t in_bytes, uint64_t count, int f16_out,
                      void *out) {
    if (fmt < 0 || fmt >= NF_ORACLE_NFMT) return -1;
    const uint64_t be = kq_geom[fmt].elems;
    if ((count + be - 1) / be * kq_geom[fmt].bytes > in_bytes) return -1;
    if (f16_out) {
        uint16_t *o = (uint16_t *)out;
        for (uint64_t e = 0; e < count; ++e)
            o[e] = nf_oracle_f32_to_f16_rne(elem_of(fmt, blocks, in_bytes, e, 1));
    } else {
        float *o = (float *)out;
        for (uint64_t e = 0; e < count; ++e) o[e] = elem_of(fmt, blocks, in_bytes, e, 0);
    }
    return 0;
}

/* ---- dense linear ----------------------------------------------------- */

void nf_oracle_linear_f32(const float *A, const float *B, float *C, uint32_t M, uint32_t N,
                          uint32_t K) {
    for (uint32_t r = 0; r < M; ++r)
        for (uint32_t c = 0; c < N; ++c) {
            float acc = 0.0f;
            for (uint32_t k = 0; k < K; ++k) acc += A[(uint64_t)r * K + k] * B[(uint64_t)c * K + k];
            C[(uint64_t)r * N + c] = acc;
        }
}

void nf_oracle_linear_f16(const uint16_t *A, const uint16_t *B, uint16_t *C, uint32_t M,
                          uint32_t N, uint32_t K) {
    for (uint32_t r = 0; r < M; ++r)
        for (uint32_t c = 0; c < N; ++c) {
            float acc = 0.0f;
            for (uint32_t k = 0; k < K; ++k)
                acc += nf_oracle_f16_to_f32(A[(uint64_t)r * K + k]) *
                       nf_oracle_f16_to_f32(B[(uint64_t)c * K + k]);
            C[(uint64_t)r * N + c] = nf_oracle_f32_to_f16_rne(acc);
        }
}

/* ---- fused dequant + linear --------------------------------------------- */

typedef struct {
    const float *A; /* f16 path: the fp16 activations widened exactly to fp32, once per call */
    const uint8_t *W;
    int qfmt;
    int f16;
    void *C;
    uint32_t M, N, K, n0, n1;
} fused_job;

/* One weight row n: flat elements n*K .. n*K+K-1, dequantized exactly as the
 * reference kernels do (f16 path: rounded to fp16 first). */
static void dequant_row(const uint8_t *W, int qfmt, int f16, uint64_t n, uint32_t K, float *row) {
    const uint64_t e0 = n * (uint64_t)K;
    for (uint32_t k = 0; k < K; ++k) {
        float w = (qfmt == NF_ORACLE_Q4_0) ? q4_0_elem(W, e0 + k) : q8_0_elem(W, e0 + k);
        row[k] = f16 ? nf_oracle_f16_to_f32(nf_oracle_f32_to_f16_rne(w)) : w;
    }
}

static void *fused_worker(void *arg) {
    const fused_job *j = (const fused_job *)arg;
    float *row = (float *)malloc(sizeof(float) * (j->K ? j->K : 1));
    if (!row) return (void *)1;
    for (uint32_t n = j->n0; n < j->n1; ++n) {
        dequant_row(j->W, j->qfmt, j->f16, n, j->K, row);
        for (uint32_t m = 0; m < j->M; ++m) {
            const float *a = j->A + (uint64_t)m * j->K;
            float acc = 0.0f;
            for (uint32_t k = 0; k < j->K; ++k) acc += a[k] * row[k];
            if (j->f16)
                ((uint16_t *)j->C)[(uint64_t)m * j->N + n] = nf_oracle_f32_to_f16_rne(acc);
            else
                ((float *)j->C)[(uint64_t)m * j->N + n] = acc;
        }
    }
    free(row);
    return NULL;
}

/* 0 on success; -1 when a working buffer could not be allocated (the
 * output is then incomplete, and the caller must not use it). */
static int fused_run(const void *A, const uint8_t *W, int qfmt, int f16, void *C, uint32_t M,
                     uint32_t N, uint32_t K, uint32_t n0, uint32_t n1, uint32_t threads) {
    if (n1 > N) n1 = N;
    if (n0 >= n1) return 0;
    if (threads < 1) threads = 1;
    if (threads > n1 - n0) threads = n1 - n0;
    if (threads > 256) threads = 256;
    /* fp16 activations widened once (exact), shared by every worker */
    float *a32 = NULL;
    if (f16) {
        const uint64_t n = (uint64_t)M * K;
        a32 = (float *)malloc(sizeof(float) * (n ? n : 1));
        if (!a32) return -1;
        for (uint64_t i = 0; i < n; ++i) a32[i] = nf_oracle_f16_to_f32(((const uint16_t *)A)[i]);
    }
    fused_job jobs[256];
    pthread_t tids[256];
    const uint32_t span = n1 - n0;
    for (uint32_t t = 0; t < threads; ++t) {
        fused_job *j = &jobs[t];
        j->A = f16 ? a32 : (const float *)A;
        j->W = W;
        j->qfmt = qfmt;
        j->f16 = f16;
        j->C = C;
        j->M = M;
        j->N = N;
        j->K = K;
        j->n0 = n0 + (uint32_t)((uint64_t)span * t / threads);
        j->n1 = n0 + (uint32_t)((uint64_t)span * (t + 1) / threads);
    }
    int failed = 0;
    if (threads == 1) {
        failed = fused_worker(&jobs[0]) != NULL;
    } else {
        uint32_t started = 0;
        for (uint32_t t = 0; t < threads; ++t) {
            if (pthread_create(&tids[t], NULL, fused_worker, &jobs[t]) != 0) {
                failed = 1;
                break;
            }
            ++started;
        }
        for (uint32_t t = 0; t < started; ++t) {
            void *r = NULL;
            pthread_join(tids[t], &r);
            failed |= r != NULL;
        }
    }
    free(a32);
    return failed ? -1 : 0;
}

int nf_oracle_fused_f32(const float *A, const uint8_t *W, int qfmt, float *C, uint32_t M,
                        uint32_t N, uint32_t K, uint32_t n0, uint32_t n1, uint32_t threads) {
    return fused_run(A, W, qfmt, 0, C, M, N, K, n0, n1, threads);
}

int nf_oracle_fused_f16(const uint16_t *A, const uint8_t *W, int qfmt, uint16_t *C, uint32_t M,
                        uint32_t N, uint32_t K, uint32_t n0, uint32_t n1, uint32_t threads) {
    return fused_run(A, W, qfmt, 1, C, M, N, K, n0, n1, threads);
}

/* ---- layer ops around the linears ---------------------------------------- */
/*
 * Each loop below follows the reference kernel's per-thread code
 * (plugins/metal/src/metal_provider.mm) in fp32, with libm's expf / tanhf /
 * powf / cosf / sinf / sqrtf for Metal's exp / tanh / pow / cos / sin / rsqrt.
 * f16 inputs and outputs are fp16 bits (uint16), converted exactly on load
 * and rounded to nearest even on store.
 */

static inline float ld_t(const void *p, uint64_t i, int f16) {
    return f16 ? nf_oracle_f16_to_f32(((const uint16_t *)p)[i]) : ((const float *)p)[i];
}

static inline void st_t(void *p, uint64_t i, float v, int f16) {
    if (f16)
        ((uint16_t *)p)[i] = nf_oracle_f32_to_f16_rne(v);
    else
        ((float *)p)[i] = v;
}

/* silu :1032-1037 (f16 :1108-1113), gelu :1039-1045 (:1115-1121), relu :51-54 */
void nf_oracle_unary(int fn, const void *in, void *out, uint64_t n, int f16) {
    for (uint64_t i = 0; i < n; ++i) {
        const float x = ld_t(in, i, f16);
        float y;
        if (fn == 0) {
            y = x / (1.0f + expf(-x));
        } else if (fn == 1) {
            const float x3 = x * x * x;
            y = 0.5f * x * (1.0f + tanhf(0.7978845608f * (x + 0.044715f * x3)));
        } else {
            y = x > 0.0f ? x : 0.0f;
        }
        st_t(out, i, y, f16);
    }
}

/* metal_vector_add / elementwise_mul :44-49, 1047-1052 (f16 :1123-1135: the
 * product / sum of two halves rounded once to half). */
void nf_oracle_binary(int fn, const void *a, const void *b, void *out, uint64_t n, int f16) {
    for (uint64_t i = 0; i < n; ++i) {
        const float x = ld_t(a, i, f16), y = ld_t(b, i, f16);
        /* for halves, x*y and x+y in fp32 round to the same half as a native
         * half operation: the fp32 result is exact (product) or rounds far
         * below half precision without creating a tie (sum) */
        st_t(out, i, fn == 0 ? x + y : x * y, f16);
    }
}

/* rms_norm :85-102 (f16 :1069-1084, weights f32) */
void nf_oracle_rms_norm(const void *in, const float *w, void *out, uint32_t rows, uint32_t dim, float eps,
                        int f16) {
    for (uint32_t r = 0; r < rows; ++r) {
        const uint64_t base = (uint64_t)r * dim;
        float sum_sq = 0.0f;
        for (uint32_t j = 0; j < dim; ++j) {
            const float v = ld_t(in, base + j, f16);
            sum_sq += v * v;
        }
        const float rms = 1.0f / sqrtf(sum_sq / (float)dim + eps);
        for (uint32_t j = 0; j < dim; ++j) st_t(out, base + j, ld_t(in, base + j, f16) * rms * w[j], f16);
    }
}

/* rope_batch :125-147 (f16 :1086-1106); rope :104-122 with pos = step for
 * every row (batch = 0).  row_span = n_heads * head_dim for rope_batch. */
void nf_oracle_rope(const void *in, void *out, uint64_t n, uint32_t n_heads, uint32_t head_dim, uint32_t step,
                    float theta, int batch, int f16) {
    const uint32_t half = head_dim / 2;
    const uint64_t span = batch ? (uint64_t)n_heads * head_dim : head_dim;
    for (uint64_t id = 0; id < n; ++id) {
        const uint32_t e = (uint32_t)(id % head_dim);
        const uint32_t pair = e % half;
        const uint64_t pos = batch ? id / span + step : step;
        const float freq = 1.0f / powf(theta, (float)(2 * pair) / (float)head_dim);
        const float angle = (float)pos * freq;
        const float c = cosf(angle), sn = sinf(angle);
        const uint64_t base = id - e;
        const float x0 = ld_t(in, base + pair, f16), x1 = ld_t(in, base + pair + half, f16);
        st_t(out, id, e < half ? x0 * c - x1 * sn : x0 * sn + x1 * c, f16);
    }
}

/* softmax :1002-1030 */
void nf_oracle_softmax(const float *in, float *out, uint32_t rows, uint32_t dim) {
    for (uint32_t r = 0; r < rows; ++r) {
        const uint64_t base = (uint64_t)r * dim;
        float mx = in[base];
        for (uint32_t j = 1; j < dim; ++j)
            if (in[base + j] > mx) mx = in[base + j];
        float sum = 0.0f;
        for (uint32_t j = 0; j < dim; ++j) {
            const float e = expf(in[base + j] - mx);
            out[base + j] = e;
            sum += e;
        }
        const float inv = 1.0f / sum;
        for (uint32_t j = 0; j < dim; ++j) out[base + j] *= inv;
    }
}

/* argmax_rows :1601-1619 */
void nf_oracle_argmax(const float *in, int32_t *out, uint32_t rows, uint32_t dim) {
    for (uint32_t r = 0; r < rows; ++r) {
        const uint64_t base = (uint64_t)r * dim;
        if (dim == 0) { /* the kernel's start value, never replaced */
            out[r] = 0;
            continue;
        }
        float best = in[base];
        int32_t idx = 0;
        for (uint32_t j = 1; j < dim; ++j)
            if (in[base + j] > best) {
                best = in[base + j];
                idx = (int32_t)j;
            }
        out[r] = idx;
    }
}

/* moe_top_k_gating :1907-1962.  Per token: max over all n_experts logits,
 * softmax over the first min(n_experts, 64), insertion of each probability
 * into a descending top_k (<= 8) list at the first slot it strictly exceeds,
 * renormalization by the selected sum.  n_experts = 0 selects nothing (the
 * reference reads logits[0] there, which is out of bounds). */
void nf_oracle_moe_gate(const float *logits, int32_t *ids, float *w, uint32_t batch, uint32_t n_experts,
                        uint32_t top_k) {
    if (top_k > 8) top_k = 8;
    for (uint32_t b = 0; b < batch; ++b) {
        const float *l = logits + (uint64_t)b * n_experts;
        float max_val = n_experts ? l[0] : 0.0f;
        for (uint32_t i = 1; i < n_experts; ++i)
            if (l[i] > max_val) max_val = l[i];
        float probs[64], sum = 0.0f;
        for (uint32_t i = 0; i < n_experts && i < 64; ++i) {
            probs[i] = expf(l[i] - max_val);
            sum += probs[i];
        }
        for (uint32_t i = 0; i < n_experts && i < 64; ++i) probs[i] /= sum;
        int32_t sel_ids[8] = {-1, -1, -1, -1, -1, -1, -1, -1};
        float sel_p[8] = {0};
        for (uint32_t i = 0; i < n_experts && i < 64; ++i)
            for (uint32_t k = 0; k < top_k; ++k)
                if (probs[i] > sel_p[k]) {
                    for (uint32_t j = top_k - 1; j > k; --j) {
                        sel_ids[j] = sel_ids[j - 1];
                        sel_p[j] = sel_p[j - 1];
                    }
                    sel_ids[k] = (int32_t)i;
                    sel_p[k] = probs[i];
                    break;
                }
        float sel_sum = 0.0f;
        for (uint32_t k = 0; k < top_k; ++k) sel_sum += sel_p[k];
        for (uint32_t k = 0; k < top_k; ++k) {
            ids[(uint64_t)b * top_k + k] = sel_ids[k];
            w[(uint64_t)b * top_k + k] = sel_sum > 0.0f ? sel_p[k] / sel_sum : 0.0f;
        }
    }
}

/* moe_scatter_gather :1964-1997.  out[b, d] = sum over k of w[b,k] *
 * experts[ids[b,k], d], k in order; ids < 0 are skipped, and so are ids at or
 * past `rows` (the expert rows present; the reference reads out of bounds). */
void nf_oracle_moe_scatter(const float *experts, uint32_t rows, const int32_t *ids, const float *w, float *out,
                           uint32_t batch, uint32_t top_k, uint32_t dim) {
    for (uint32_t b = 0; b < batch; ++b)
        for (uint32_t d = 0; d < dim; ++d) {
            float val = 0.0f;
            for (uint32_t k = 0; k < top_k; ++k) {
                const int32_t e = ids[(uint64_t)b * top_k + k];
                if (e < 0 || (uint32_t)e >= rows) continue;
                val += w[(uint64_t)b * top_k + k] * experts[(uint64_t)e * dim + d];
            }
            out[(uint64_t)b * dim + d] = val;
        }
}

/* embedding_lookup :1054-1067 (f16 :1137-1150); a token outside the table's
 * `vocab` rows yields zeros (the reference reads out of bounds there). */
void nf_oracle_embedding(const void *w, uint32_t vocab, const int32_t *ids, void *out, uint64_t n, uint32_t dim,
                         uint32_t seq_len, int f16) {
    for (uint64_t id = 0; id < n; ++id) {
        const uint64_t t = id / dim;
        if (t >= seq_len) continue;
        const int32_t tok = ids[t];
        float v = 0.0f;
        if (tok >= 0 && (uint32_t)tok < vocab) v = ld_t(w, (uint64_t)tok * dim + id % dim, f16);
        st_t(out, id, v, f16);
    }
}

/* ---- attention ----------------------------------------------------------------
 * prm[] = {mode, variant, n_heads, n_kv, head_dim, seq_len, step, max_seq,
 *          window, block_size, n_blocks, q_offset, pool_blocks}
 * mode:    0 causal_attention [heads, seq, dim]            (:166-213)
 *          1 cached: Q/out [seq, heads, dim], cache [kv, max_seq, dim] (:217-341, 344-497)
 *          2 gqa: Q/out [heads, seq, dim]                   (:1715-1806)
 *          3 paged: pools [block][kv][bs][dim] + table       (:1622-1712)
 * variant: 0 two-pass (causal_attention, causal_attention_cached)
 *          1 32-key tiles, online (flash_attention_cached / _f16)
 *          2 per-key online (flash_attention_gqa)
 *          3 per-block online (flash_attention_paged)
 * The cached modes append K_new / V_new to the caches first (all appended
 * rows are visible to every query, the intent of the reference kernels).
 * A paged block index at or past pool_blocks is skipped. */

#define NF_NEG_INF (-1e30f)

static inline uint64_t attn_q_row(const uint32_t *P, uint32_t q, uint32_t h) {
    const uint32_t mode = P[0], H = P[2], D = P[4], S = P[5], step = P[6];
    if (mode == 0) return ((uint64_t)h * S + q) * D;
    if (mode == 1) return step ? (uint64_t)h * D : ((uint64_t)q * H + h) * D;
    if (mode == 2) return step ? (uint64_t)h * D : ((uint64_t)h * S + q) * D;
    return ((uint64_t)(P[11] + q) * H + h) * D;
}

static inline int64_t attn_kv_row(const uint32_t *P, const uint32_t *table, uint32_t kvh, uint32_t pos) {
    const uint32_t mode = P[0], KV = P[3], D = P[4], S = P[5], max_seq = P[7], bs = P[9];
    if (mode == 0) return (int64_t)(((uint64_t)kvh * S + pos) * D);
    if (mode == 1 || mode == 2) return (int64_t)(((uint64_t)kvh * max_seq + pos) * D);
    const uint32_t phys = table[pos / bs];
    if (phys >= P[12]) return -1;
    return (int64_t)((((uint64_t)phys * KV + kvh) * bs + pos % bs) * D);
}

static float attn_dot(const void *Q, uint64_t qrow, const void *K, int64_t krow, uint32_t D, int f16) {
    float dot = 0.0f;
    for (uint32_t d = 0; d < D; ++d) dot += ld_t(Q, qrow + d, f16) * ld_t(K, (uint64_t)krow + d, f16);
    return dot;
}

int nf_oracle_attention(const uint32_t *P, int f16, const void *Q, const void *K_new, const void *V_new, void *K,
                        void *V, const uint32_t *table, void *out) {
    const uint32_t mode = P[0], variant = P[1], H = P[2], KV = P[3], D = P[4], S = P[5], step = P[6];
    const uint32_t max_seq = P[7], window = P[8], bs = P[9], n_blocks = P[10];
    const int decode = mode != 0 && step > 0;
    if (mode == 1 || mode == 2) {
        if (decode && step >= max_seq) return 0;
        const uint32_t tokens = decode ? 1 : S, first = decode ? step : 0;
        for (uint32_t kvh = 0; kvh < KV; ++kvh)
            for (uint32_t t = 0; t < tokens; ++t)
                for (uint32_t d = 0; d < D; ++d) {
                    const uint64_t src = mode == 1 ? ((uint64_t)t * KV + kvh) * D + d : ((uint64_t)kvh * tokens + t) * D + d;
                    const uint64_t dst = ((uint64_t)kvh * max_seq + first + t) * D + d;
                    st_t(K, dst, ld_t(K_new, src, f16), f16);
                    st_t(V, dst, ld_t(V_new, src, f16), f16);
                }
    }
    const float scale = 1.0f / sqrtf((float)D);
    const uint32_t nq = decode ? 1 : S;
    float *acc = (float *)malloc(sizeof(float) * (D ? D : 1));
    if (!acc) return -1;
    for (uint32_t q = 0; q < nq; ++q)
        for (uint32_t h = 0; h < H; ++h) {
            const uint32_t kvh = (uint32_t)((uint64_t)h * KV / H);
            const uint32_t pos = decode ? step : q;
            uint32_t lo = 0;
            if (mode == 1 && window > 0 && pos >= window) lo = pos - window + 1;
            int64_t hi = pos;
            if (mode == 3) {
                const int64_t cap = (int64_t)n_blocks * bs - 1;
                if (hi > cap) hi = cap;
            }
            const uint64_t qrow = attn_q_row(P, q, h);
            for (uint32_t d = 0; d < D; ++d) acc[d] = 0.0f;
            float res_scale;
            if (variant == 0) {
                float mx = NF_NEG_INF;
                for (int64_t k = lo; k <= hi; ++k) {
                    const float dot = attn_dot(Q, qrow, K, attn_kv_row(P, table, kvh, (uint32_t)k), D, f16) * scale;
                    if (dot > mx) mx = dot;
                }
                float sum = 0.0f;
                for (int64_t k = lo; k <= hi; ++k)
                    sum += expf(attn_dot(Q, qrow, K, attn_kv_row(P, table, kvh, (uint32_t)k), D, f16) * scale - mx);
                for (int64_t k = lo; k <= hi; ++k) {
                    const int64_t row = attn_kv_row(P, table, kvh, (uint32_t)k);
                    const float w = expf(attn_dot(Q, qrow, K, row, D, f16) * scale - mx) / sum;
                    for (uint32_t d = 0; d < D; ++d) acc[d] += w * ld_t(V, (uint64_t)row + d, f16);
                }
                res_scale = 1.0f;
            } else {
                float m = NF_NEG_INF, l = 0.0f;
                const uint32_t tile = variant == 1 ? 32u : variant == 2 ? 1u : bs;
                /* paged tiles are the logical blocks, aligned at 0 */
                for (int64_t t0 = lo; t0 <= hi; t0 += tile) {
                    int64_t t1 = t0 + tile - 1;
                    if (t1 > hi) t1 = hi;
                    float tmax = NF_NEG_INF;
                    int any = 0;
                    for (int64_t k = t0; k <= t1; ++k) {
                        const int64_t row = attn_kv_row(P, table, kvh, (uint32_t)k);
                        if (row < 0) continue;
                        any = 1;
                        const float dot = attn_dot(Q, qrow, K, row, D, f16) * scale;
                        if (dot > tmax) tmax = dot;
                    }
                    if (!any) continue;
                    const float m_new = m > tmax ? m : tmax;
                    const float corr = expf(m - m_new);
                    if (variant == 2) {
                        const int64_t row = attn_kv_row(P, table, kvh, (uint32_t)t0);
                        const float e = expf(tmax - m_new);
                        l = l * corr + e;
                        for (uint32_t d = 0; d < D; ++d) acc[d] = acc[d] * corr + e * ld_t(V, (uint64_t)row + d, f16);
                    } else {
                        for (uint32_t d = 0; d < D; ++d) acc[d] *= corr;
                        l *= corr;
                        for (int64_t k = t0; k <= t1; ++k) {
                            const int64_t row = attn_kv_row(P, table, kvh, (uint32_t)k);
                            if (row < 0) continue;
                            const float w = expf(attn_dot(Q, qrow, K, row, D, f16) * scale - m_new);
                            l += w;
                            for (uint32_t d = 0; d < D; ++d) acc[d] += w * ld_t(V, (uint64_t)row + d, f16);
                        }
                    }
                    m = m_new;
                }
                res_scale = l > 0.0f ? 1.0f / l : 0.0f;
            }
            for (uint32_t d = 0; d < D; ++d) st_t(out, qrow + d, acc[d] * res_scale, f16);
        }
    free(acc);
    return 0;
}
