/*
 * nf_oracle.h — CPU oracle for the quantized linear path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: tests/, the
 * smoke() entry and bench.py's cpu_baseline leg call it to compute expected
 * results and to time the reference's CPU algorithm.  The product path
 * (libnf_plugin_hip.so) never links, loads or calls it.
 *
 * Each function restates the reference's CPU code or kernel semantics
 * (citations below are relative to the reference repository):
 *   nf_oracle_f16_to_f32      tests/driver/dequant_test.cpp:77-98
 *   nf_oracle_f32_to_f16_trunc tests/driver/dequant_test.cpp:100-109 (the
 *                             tests' truncating, flush-to-zero input encoder;
 *                             used only to rebuild the tests' own inputs)
 *   nf_oracle_f32_to_f16_rne  IEEE 754 roundTiesToEven with subnormals — the
 *                             conversion the kernels' half(x) performs
 *                             (plugins/metal/src/metal_provider.mm:749,758,1457,1467)
 *   nf_oracle_dequant_*_f32   ref_dequant_q4_0/q8_0, dequant_test.cpp:112-128
 *   nf_oracle_dequant_*_f16   dequant_q4_0_f16/q8_0_f16, metal_provider.mm:741-759
 *   nf_oracle_dequant         every dequant_<fmt>[_f16] op:
 *                             q4_1/q5_0/q5_1/q2_k/q3_k/q4_k/q5_k f32 follow
 *                             the CPU refs of tests/driver/kquant_dequant_test.cpp:118-224;
 *                             q6_k follows metal_provider.mm:534-573 (no CPU
 *                             ref exists); the _f16 ops are the RNE half of
 *                             the same f32 value (metal_provider.mm:761-900),
 *                             except q3_k_f16, whose kernel reads raw bytes
 *                             as scales (metal_provider.mm:833-848)
 *   nf_oracle_unary/binary/rms_norm/rope/softmax/argmax/embedding/attention
 *                             the layer-op kernels, metal_provider.mm:44-497,
 *                             1002-1150, 1273-1394, 1601-1906, in their loop
 *                             order (pins: tests/test_oracle_layer.py)
 *   nf_oracle_linear_*        naive sequential-k loop, dequant_test.cpp:313-319,
 *                             with B stored [N,K] (dequant_test.cpp:321-325)
 *   nf_oracle_fused_*         dequant_q4_0_linear_tiled[_f16] semantics,
 *                             metal_provider.mm:1396-1468: weight element (n,k)
 *                             is flat element n*K+k of the block stream.
 *
 * Parity pins are in tests/test_oracle.py.
 */
#ifndef NF_ORACLE_H
#define NF_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    NF_ORACLE_Q4_0 = 0, NF_ORACLE_Q8_0 = 1, NF_ORACLE_Q4_1 = 2, NF_ORACLE_Q5_0 = 3,
    NF_ORACLE_Q5_1 = 4, NF_ORACLE_Q2_K = 5, NF_ORACLE_Q3_K = 6, NF_ORACLE_Q4_K = 7,
    NF_ORACLE_Q5_K = 8, NF_ORACLE_Q6_K = 9, NF_ORACLE_NFMT = 10
};

float nf_oracle_f16_to_f32(uint16_t h);
uint16_t nf_oracle_f32_to_f16_rne(float f);
uint16_t nf_oracle_f32_to_f16_trunc(float f);

void nf_oracle_f16_to_f32_n(const uint16_t *in, float *out, uint64_t n);
void nf_oracle_f32_to_f16_rne_n(const float *in, uint16_t *out, uint64_t n);

/* Dequantize `count` elements (blocks are consumed in order; a trailing
 * partial block is allowed). */
void nf_oracle_dequant_q4_0_f32(const uint8_t *blocks, uint64_t count, float *out);
void nf_oracle_dequant_q8_0_f32(const uint8_t *blocks, uint64_t count, float *out);
void nf_oracle_dequant_q4_0_f16(const uint8_t *blocks, uint64_t count, uint16_t *out);
void nf_oracle_dequant_q8_0_f16(const uint8_t *blocks, uint64_t count, uint16_t *out);

/* Any of the ten block formats: `count` elements to f32 (f16_out = 0) or
 * fp16 bits (f16_out = 1) with the semantics of dequant_<fmt>[_f16].
 * `in_bytes` is the size of the input buffer: dequant_q3_k_f16 reads two
 * bytes past its last block, taken as 0 beyond `in_bytes`.  Returns -1 for an
 * unknown format or an input shorter than ceil(count / elems) blocks. */
int nf_oracle_dequant(int fmt, const uint8_t *blocks, uint64_t in_bytes, uint64_t count, int f16_out,
                      void *out);
uint32_t nf_oracle_block_bytes(int fmt);
uint32_t nf_oracle_block_elems(int fmt);

/* Layer ops around the linears (metal_provider.mm line ranges in
 * nf_oracle.c).  f16 = 1: inputs and outputs are fp16 bits.
 * unary fn: 0 silu, 1 gelu, 2 relu; binary fn: 0 add, 1 mul. */
void nf_oracle_unary(int fn, const void *in, void *out, uint64_t n, int f16);
void nf_oracle_binary(int fn, const void *a, const void *b, void *out, uint64_t n, int f16);
void nf_oracle_rms_norm(const void *in, const float *w, void *out, uint32_t rows, uint32_t dim, float eps,
                        int f16);
void nf_oracle_rope(const void *in, void *out, uint64_t n, uint32_t n_heads, uint32_t head_dim, uint32_t step,
                    float theta, int batch, int f16);
void nf_oracle_softmax(const float *in, float *out, uint32_t rows, uint32_t dim);
void nf_oracle_argmax(const float *in, int32_t *out, uint32_t rows, uint32_t dim);
void nf_oracle_moe_gate(const float *logits, int32_t *ids, float *w, uint32_t batch, uint32_t n_experts,
                        uint32_t top_k);
void nf_oracle_moe_scatter(const float *experts, uint32_t rows, const int32_t *ids, const float *w, float *out,
                           uint32_t batch, uint32_t top_k, uint32_t dim);
void nf_oracle_embedding(const void *w, uint32_t vocab, const int32_t *ids, void *out, uint64_t n, uint32_t dim,
                         uint32_t seq_len, int f16);
/* prm = {mode, variant, n_heads, n_kv, head_dim, seq_len, step, max_seq,
 * window, block_size, n_blocks, q_offset, pool_blocks}; see nf_oracle.c. */
int nf_oracle_attention(const uint32_t *prm, int f16, const void *Q, const void *K_new, const void *V_new,
                        void *K, void *V, const uint32_t *table, void *out);

/* C[M,N] = A[M,K] * B[N,K]^T, fp32 accumulation in k order. */
void nf_oracle_linear_f32(const float *A, const float *B, float *C,
                          uint32_t M, uint32_t N, uint32_t K);
/* f16 A and B, fp32 accumulation of exact products, C rounded to fp16. */
void nf_oracle_linear_f16(const uint16_t *A, const uint16_t *B, uint16_t *C,
                          uint32_t M, uint32_t N, uint32_t K);

/* Fused dequant + linear over the output columns n in [n0, n1); the other
 * columns of C are left untouched.  qfmt is NF_ORACLE_Q4_0 / NF_ORACLE_Q8_0.
 * threads > 1 partitions the columns across pthreads (same arithmetic).
 * Returns 0, or -1 when a working buffer or thread could not be had (the
 * output is then incomplete). */
int nf_oracle_fused_f32(const float *A, const uint8_t *W, int qfmt, float *C,
                        uint32_t M, uint32_t N, uint32_t K,
                        uint32_t n0, uint32_t n1, uint32_t threads);
int nf_oracle_fused_f16(const uint16_t *A, const uint8_t *W, int qfmt, uint16_t *C,
                        uint32_t M, uint32_t N, uint32_t K,
                        uint32_t n0, uint32_t n1, uint32_t threads);

#ifdef __cplusplus
}
#endif
#endif
