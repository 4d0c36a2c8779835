// launch.hpp — host entry points of the kernel translation units.
//
// Each function validates nothing (plan.cpp already did) and enqueues on
// `s`.  Shapes: A[M,K] row-major, W[N,K] as 32-element blocks along K,
// C[M,N] row-major.
#pragma once

#include <hip/hip_runtime.h>

#include "plan.hpp"

namespace nfhip {

// Device workspace owned by the provider (allocated at init): fp32 partial
// tiles of split-K launches and one counter per output tile.  Counters start
// at zero and every split-K launch leaves them at zero again (the last
// workgroup of a tile resets its counter), so no per-launch clearing is
// needed.  Launches on the provider's single stream never overlap, so they
// share it.
struct Workspace {
  float* part = nullptr;
  uint32_t* cnt = nullptr;
  size_t part_floats = 0;
  uint32_t cnt_len = 0;
};

// Every block format; `in_bytes` (the input buffer size) bounds every read of `w`.
hipError_t launch_dequant(QFmt q, EType out_t, const void* w, uint64_t in_bytes, void* out, uint64_t count,
                          hipStream_t s);

hipError_t launch_gemv(QFmt q, EType t, const void* A, const void* W, void* C, uint32_t M,
                       uint32_t N, uint32_t K, hipStream_t s);

// Launch-floor calibration: stream `bytes` from `src` (read only, nothing
// stored), or an empty kernel when bytes < 16.
hipError_t launch_diag_read(const void* src, uint64_t bytes, hipStream_t s);

// Several decode GEMVs over the same activations A (same format, dtype, M
// and K; each with its own weights, output and N) in one launch, each job
// computed exactly as launch_gemv would.  hipErrorNotSupported when the
// jobs do not suit one launch (the caller then launches them one by one).
constexpr int kGemvGroupMax = 4;
struct GemvJob {
  const void* W;
  void* C;
  uint32_t N;
};
hipError_t launch_gemv_group(QFmt q, EType t, const void* A, const GemvJob* jobs, uint32_t n, uint32_t M,
                             uint32_t K, hipStream_t s);
hipError_t launch_skinny_group(QFmt q, EType t, const void* A, const GemvJob* jobs, uint32_t n, uint32_t M,
                               uint32_t K, const Workspace& ws, hipStream_t s);

// Small-batch (M <= 64) MFMA kernel; skinny_fits() says whether a shape and
// operand alignment suit it.
bool skinny_fits(uint32_t M, uint32_t N, uint32_t K, const void* A, const void* W);
uint32_t skinny_max_rows(EType t);  // activation rows per launch
hipError_t launch_skinny(QFmt q, EType t, const void* A, const void* W, void* C, uint32_t M, uint32_t N,
                         uint32_t K, const Workspace& ws, hipStream_t s);
// Several small-batch linears over the same activations (M <= 32, same
// format, dtype and K) in one launch, each computed exactly as launch_skinny
// would; hipErrorNotSupported when they would not get the same kernel
// variant and K split on their own (the caller launches them one by one).

// tile: Tuning::gemm_tile (-1 = register-dequantizing kernel, 0..6 = an
// LDS-staged tile shape).
hipError_t launch_gemm_mfma(QFmt q, EType t, const void* A, const void* W, void* C, uint32_t M,
                            uint32_t N, uint32_t K, int tile, const Workspace& ws, hipStream_t s);

hipError_t launch_generic(QFmt q, EType t, const void* A, const void* W, void* C, uint32_t M,
                          uint32_t N, uint32_t K, hipStream_t s);

// Dense fp16 x fp16 linear on the tiled MFMA kernel, fp16 or fp32 output;
// hipErrorInvalidValue when the shape/alignment does not fit it (K % 64,
// 16-B aligned operands).
hipError_t launch_dense_mfma_f16(const void* A, const void* B, void* C, uint32_t M, uint32_t N, uint32_t K,
                                 bool out_f32, hipStream_t s);

// Dense linear with at least one fp32 operand (fp16 operands widened
// exactly) on the fp32 MFMA; hipErrorNotSupported when K % 32 != 0 or an
// operand is not 16-B aligned.
hipError_t launch_dense_mfma_f32(EType a, EType b, EType c, const void* A, const void* B, void* C, uint32_t M,
                                 uint32_t N, uint32_t K, const Workspace& ws, hipStream_t s);

hipError_t launch_dense(EType a, EType b, EType c, const void* A, const void* B, void* C,
                        uint32_t M, uint32_t N, uint32_t K, const Workspace& ws, hipStream_t s);

// ---- layer ops (kernels/layer.hip) -------------------------------------------
hipError_t launch_binary(EwFn fn, EType t, const void* a, const void* b, void* out, uint64_t n, hipStream_t s);
hipError_t launch_unary(EwFn fn, EType t, const void* in, void* out, uint64_t n, hipStream_t s);
hipError_t launch_mock_prefill(const void* in, void* k, void* v, uint64_t nk, uint64_t nv, hipStream_t s);
hipError_t launch_rms_norm(EType t, const void* in, const void* w, void* out, uint32_t rows, uint32_t dim, float eps,
                           hipStream_t s);
// batch: rope_batch ([seq, n_heads, head_dim], pos = token + step); else rope (pos = step).
hipError_t launch_rope(EType t, bool batch, const void* in, void* out, uint64_t n, uint32_t n_heads,
                       uint32_t head_dim, uint32_t step, float theta, hipStream_t s);
// ws: the provider workspace (partials of rows split into chunks), may be null
hipError_t launch_softmax(const void* in, void* out, uint32_t rows, uint32_t dim, float* ws, size_t ws_floats,
                          hipStream_t s);
hipError_t launch_argmax(const void* in, void* out, uint32_t rows, uint32_t dim, float* ws, size_t ws_floats,
                         hipStream_t s);
// MoE (metal_provider.mm:1907-1997): per token, softmax over the first
// min(n_experts, 64) gate logits, the top_k (<= 8) largest in index order of
// ties, renormalized; and the weighted sum of the selected experts' rows.
hipError_t launch_moe_gate(const void* logits, void* ids, void* weights, uint32_t batch, uint32_t n_experts,
                           uint32_t top_k, hipStream_t s);
hipError_t launch_moe_scatter(const void* experts, uint32_t expert_rows, const void* ids, const void* weights,
                              void* out, uint32_t batch, uint32_t top_k, uint32_t dim, hipStream_t s);
hipError_t launch_embedding(EType t, const void* w, uint32_t vocab, const void* ids, void* out, uint64_t n,
                            uint32_t dim, uint32_t seq_len, hipStream_t s);

// ---- attention (kernels/attention.hip) ---------------------------------------
struct AttnArgs {
  const void* q = nullptr;
  const void* k_new = nullptr;  // Cached / Gqa: rows appended to the cache first
  const void* v_new = nullptr;
  void* k = nullptr;  // Plain: K; Cached / Gqa: cache_k; Paged: K pool
  void* v = nullptr;
  const uint32_t* block_table = nullptr;  // Paged
  void* out = nullptr;
  LayerParams lp;
  uint64_t pool_blocks = 0;  // Paged: whole blocks the pools hold
  float* ws = nullptr;       // decode partials (the provider's split-K workspace)
  size_t ws_floats = 0;
};
hipError_t launch_attention(EType t, const AttnArgs& a, hipStream_t s);

}  // namespace nfhip
