// plan.hpp — host-side op planning for the HIP provider.
//
// Turns (op name, operand descriptors, push constants) into a validated
// execution plan: which kernel family runs, with which M/N/K and how much
// algorithmic work it represents.  No HIP types appear here, so the same
// logic backs dispatch() and the GPU-free nf_hip_plan_dispatch() query.
#pragma once

#include <cstdint>
#include <string>

#include "nf_abi.h"

namespace nfhip {

enum class OpKind { Dequant, FusedLinear, DenseLinear, Layer };
// Q4_0 and Q8_0 serve the fused linear kernels; every format serves the
// standalone dequant ops.
enum class QFmt { None, Q4_0, Q8_0, Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K };
enum class EType { F32, F16 };
enum class Path {
  Dequant,   // standalone dequantization
  Gemv,      // VALU decode kernel, M <= gemv crossover
  Skinny,    // small-batch MFMA kernel, gemv crossover < M <= skinny crossover
  GemmMfma,  // LDS-tiled MFMA kernel (prefill, f16), M > skinny crossover
  Generic,   // flat-index fallback for K % 32 != 0
  Dense,     // dense linear (weights already dequantized)
  // the layer ops around the linears (plan_layer.cpp)
  Binary,      // metal_vector_add, elementwise_mul
  Unary,       // silu, gelu, mock_relu
  MockPrefill, // attention_prefill (k = x/2, v = -x/4)
  RmsNorm,
  Rope,        // single-token rope
  RopeBatch,
  Softmax,
  Embedding,
  Argmax,
  Attention,   // every attention op (causal, cached, flash, gqa, paged)
  MoeGate,     // moe_top_k_gating
  MoeScatter   // moe_scatter_gather
};

// Element-wise functions of the Binary / Unary paths.
enum class EwFn { Add, Mul, Silu, Gelu, Relu };

// KV addressing and query layout of an attention op.
enum class AttnMode {
  Plain,   // causal_attention: Q, K, V, out [n_heads, seq_len, head_dim]
  Cached,  // causal_attention_cached, flash_attention_cached: Q/out [seq, n_heads, dim],
           // K_new/V_new [seq, n_kv, dim], cache [n_kv, max_seq, dim]
  Gqa,     // flash_attention_gqa: Q/out [n_heads, seq, dim], K_new/V_new [n_kv, seq, dim]
  Paged    // flash_attention_paged: pools [block][n_kv][block_size][dim] + block table
};

// Parameters of the layer ops, from the push constants
// {seq_len@0, n_heads@4, head_dim@8, epsilon@12, theta@16, M@20, N@24, K@28,
//  step_idx@32, max_seq_len@36, window_size@40} (metal_provider.mm:71-84).
struct LayerParams {
  EwFn fn = EwFn::Add;
  AttnMode attn = AttnMode::Plain;
  uint32_t rows = 0, dim = 0;  // rms_norm / softmax / argmax / embedding
  uint32_t seq_len = 0, n_heads = 0, n_kv = 0, head_dim = 0;
  uint32_t step = 0, max_seq = 0, window = 0;
  uint32_t n_blocks = 0, block_size = 0, q_offset = 0;  // paged attention
  uint32_t n_experts = 0, top_k = 0;                     // MoE gating / scatter-gather
  uint64_t count2 = 0;  // attention_prefill: elements of the second output
  float eps = 0.f, theta = 0.f;
  bool decode = false;  // attention with step_idx > 0 (one query token)
  bool append = false;  // attention op that first writes K_new / V_new into the cache
  bool noop = false;    // nothing to launch (decode at step >= max_seq_len, as the reference)
};

// Switch points between the kernel families of the fused op: the VALU GEMV
// while M <= gemv_max_m (and its activation stage fits in LDS), the
// small-batch MFMA kernel while M <= skinny_max_m (f16 and f32 activations
// each have their own; the f32 ring kernel takes all 64 rows in one launch),
// the tiled MFMA GEMM above (f16: fp16 MFMA; f32: bf16-piece MFMA, K % 64 == 0, else the GEMV).
// Defaults from measured sweeps on MI355X (graph replay over 4 rotated weight
// copies).  bench.py's configs[4] section (28672x8192 and 8192x28672 Q4_0,
// f16 activations): the GEMV is fastest up to M = 2 (31.0 / 38.8 us against
// 46.3 / 47.1 us for the small-batch kernel at 28672x8192) while two of its
// workgroups fit a CU's LDS (at 8192x28672 M = 2 its 112 KB activation stage
// leaves one: 47.9 against 46.3 us; plan.cpp), the small-batch kernel for M = 4..16 (58.6 and
// 61.6 us at M = 16 against 67.6 and 69.2 us for the tiled GEMM), the tiled
// GEMM from M = 32 (70.2 vs 88.8 us and 69.4 vs 88.7 us).  f32 activations
// (configs[3] Llama-3-8B Q8_0 step): the small-batch ring kernel up to
// M = 64, all rows in one launch (5.12 against 11.75 ms per M = 64 step and
// 4.86 against 11.64 ms at M = 48 with the bf16-piece tiled GEMM), the tiled
// GEMM above, where the ring kernel does not go.
// At M = 3..4 the winner depends on the weight size: the GEMV wins on
// matrices up to about 10 MB, where the small-batch kernel's fixed
// per-launch cost dominates (f32 M = 4: 2048x2048 4.9 vs 8.6 us, 4096x4096
// 10.4 vs 11.4 us; f16 5632x2048 6.5 vs 8.7 us), they tie at 25 MB
// (11008x4096 f32 20.2 vs 18.5, 4096x11008 19.5 vs 19.2 us) and the
// small-batch kernel wins beyond (32000x2048 f32 25.0 vs 21.4 us,
// 32000x4096 49.3 vs 36.2 us; f16 alike).  Hence the GEMV takes M = 3..4
// only while the weights are at most gemv_m4_max_weight_bytes (16 MB).
// skinny_f16_max_k caps K for f16 batches above M = 4 on the small-batch
// kernel (longer K goes to the tiled GEMM); no cap by default, since the
// small-batch kernel's K split over workgroups (skinny_split) makes it the
// faster one at K = 28672 too (M = 8: 52.8 against 68.1 us).
struct Tuning {
  uint32_t gemv_max_m_f32 = 4;
  uint32_t gemv_max_m_f16 = 4;
  uint32_t skinny_max_m_f16 = 16;
  uint32_t skinny_max_m_f32 = 64;
  uint64_t gemv_m4_max_weight_bytes = 16ull << 20;
  uint32_t gemv_m2_max_stage_bytes = 80 * 1024;
  uint32_t skinny_f16_max_k = 1u << 30;
  // Kernel of the f16 GEMM path: -1 = the register-dequantizing kernels,
  // picked by M (launch_gemm_mfma); 0..6 = one of the LDS-staged tile
  // shapes; 7 = the register-dequantizing kernel with one wave per SIMD;
  // 8 / 9 / 10 = the two-wave kernel with 128 / 64 / 32-row waves wherever
  // it applies (K % 128 == 0; 8: Q4_0 only); 11 = its 128-row waves on
  // 128-column tiles (Q4_0, K % 128 == 0).
  int32_t gemm_tile = -1;
};

// "256x256" -> 0, "256x128" -> 1, "128x128" -> 2, "256x128w4" -> 3,
// "256x128w4s3" -> 4, "128x128s3" -> 5, "128x256" -> 6, "wq1" -> 7,
// "wq2" -> 8, "wq2m64" -> 9, "wq2m32" -> 10, "wq2n128" -> 11, or the number
// 0..11; anything else (including null) -> -1.
int gemm_tile_from_name(const char* name);

struct Plan {
  OpKind op = OpKind::Dequant;
  QFmt q = QFmt::None;
  EType a = EType::F32, b = EType::F32, c = EType::F32;
  Path path = Path::Dequant;
  uint32_t M = 0, N = 0, K = 0;
  uint64_t count = 0;     // dequant: output elements
  uint64_t in_bytes = 0;  // dequant: size of the quantized input buffer
  uint64_t weight_bytes = 0, act_bytes = 0, out_bytes = 0, flops = 0;
  std::string kernel;
  LayerParams lp;
  uint32_t writes_inputs = 0;  // bit i: the op writes input i (KV cache append, in-place relu)
};

// Bytes and elements of one block (gguf_loader.hpp:64-74): Q4_0 = 2 (fp16
// scale) + 16, Q8_0 = 2 + 32, Q4_1 20, Q5_0 22, Q5_1 24 (32 elements);
// Q2_K 84, Q3_K 110, Q4_K 144, Q5_K 176, Q6_K 210 (256 elements).
inline uint32_t block_bytes(QFmt q) {
  switch (q) {
    case QFmt::Q4_0: return 18u;
    case QFmt::Q8_0: return 34u;
    case QFmt::Q4_1: return 20u;
    case QFmt::Q5_0: return 22u;
    case QFmt::Q5_1: return 24u;
    case QFmt::Q2_K: return 84u;
    case QFmt::Q3_K: return 110u;
    case QFmt::Q4_K: return 144u;
    case QFmt::Q5_K: return 176u;
    case QFmt::Q6_K: return 210u;
    default: return 0u;
  }
}
inline uint32_t block_elems(QFmt q) {
  return (q == QFmt::Q2_K || q == QFmt::Q3_K || q == QFmt::Q4_K || q == QFmt::Q5_K || q == QFmt::Q6_K)
             ? 256u
             : 32u;
}
inline uint32_t elt_bytes(EType t) { return t == EType::F16 ? 2u : 4u; }

// Validates and plans one dispatch.  `ins`/`outs` are descriptor pointers
// (may be null when n == 0).  `pc` points at the task's push-constant bytes
// or is null.  Returns NF_OK, NF_ERROR_UNSUPPORTED_OP (unknown name) or
// NF_ERROR_INVALID_ARG (arity, dtype or size mismatch); `why` receives a
// human-readable reason on error.
nf_status make_plan(const char* op_name, const nf_tensor_desc* const* ins, uint32_t n_in,
                    const nf_tensor_desc* const* outs, uint32_t n_out, const uint8_t* pc,
                    uint32_t pc_size, const Tuning& tuning, Plan* plan, std::string* why);

// True when `op_name` is served by this provider.
bool op_known(const char* op_name);

// True when the op reads the task descriptor's push constants.
bool op_reads_push_constants(const char* op_name);

// The layer ops (plan_layer.cpp).  `pc` is the whole push-constant block
// (fields past pc_size read as zero).
bool layer_op_known(const char* op_name);
bool layer_op_reads_push_constants(const char* op_name);
nf_status make_layer_plan(const char* op_name, const nf_tensor_desc* const* ins, uint32_t n_in,
                          const nf_tensor_desc* const* outs, uint32_t n_out, const uint8_t* pc,
                          uint32_t pc_size, Plan* plan, std::string* why);

}  // namespace nfhip
