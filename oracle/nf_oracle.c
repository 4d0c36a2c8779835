/*
 * nf_oracle.c — CPU oracle for the quantized linear path.
 *
 * TEST INFRASTRUCTURE ONLY (see nf_oracle.h): the checker and the timed CPU
 * baseline, never part of the product path.  Built with -ffp-contract=off so
 * every `acc += a * b` is a separately rounded multiply and add, in k order,
 * exactly as the reference's loop is written (dequant_test.cpp:313-319).
 */
#include "nf_oracle.h"

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
    const void *A;
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
    float *arow = j->f16 ? (float *)malloc(sizeof(float) * (j->K ? j->K : 1)) : NULL;
    if (!row || (j->f16 && !arow)) {
        free(row);
        free(arow);
        return (void *)1;
    }
    for (uint32_t n = j->n0; n < j->n1; ++n) {
        dequant_row(j->W, j->qfmt, j->f16, n, j->K, row);
        for (uint32_t m = 0; m < j->M; ++m) {
            float acc = 0.0f;
            if (j->f16) {
                const uint16_t *a = (const uint16_t *)j->A + (uint64_t)m * j->K;
                for (uint32_t k = 0; k < j->K; ++k) arow[k] = nf_oracle_f16_to_f32(a[k]);
                for (uint32_t k = 0; k < j->K; ++k) acc += arow[k] * row[k];
                ((uint16_t *)j->C)[(uint64_t)m * j->N + n] = nf_oracle_f32_to_f16_rne(acc);
            } else {
                const float *a = (const float *)j->A + (uint64_t)m * j->K;
                for (uint32_t k = 0; k < j->K; ++k) acc += a[k] * row[k];
                ((float *)j->C)[(uint64_t)m * j->N + n] = acc;
            }
        }
    }
    free(row);
    free(arow);
    return NULL;
}

static void fused_run(const void *A, const uint8_t *W, int qfmt, int f16, void *C, uint32_t M,
                      uint32_t N, uint32_t K, uint32_t n0, uint32_t n1, uint32_t threads) {
    if (n1 > N) n1 = N;
    if (n0 >= n1) return;
    if (threads < 1) threads = 1;
    if (threads > n1 - n0) threads = n1 - n0;
    if (threads > 256) threads = 256;
    fused_job jobs[256];
    pthread_t tids[256];
    const uint32_t span = n1 - n0;
    for (uint32_t t = 0; t < threads; ++t) {
        fused_job *j = &jobs[t];
        j->A = A;
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
    if (threads == 1) {
        fused_worker(&jobs[0]);
        return;
    }
    for (uint32_t t = 0; t < threads; ++t) pthread_create(&tids[t], NULL, fused_worker, &jobs[t]);
    for (uint32_t t = 0; t < threads; ++t) pthread_join(tids[t], NULL);
}

void nf_oracle_fused_f32(const float *A, const uint8_t *W, int qfmt, float *C, uint32_t M,
                         uint32_t N, uint32_t K, uint32_t n0, uint32_t n1, uint32_t threads) {
    fused_run(A, W, qfmt, 0, C, M, N, K, n0, n1, threads);
}

void nf_oracle_fused_f16(const uint16_t *A, const uint8_t *W, int qfmt, uint16_t *C, uint32_t M,
                         uint32_t N, uint32_t K, uint32_t n0, uint32_t n1, uint32_t threads) {
    fused_run(A, W, qfmt, 1, C, M, N, K, n0, n1, threads);
}
