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
