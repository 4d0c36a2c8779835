// plan.cpp — validation and kernel selection for every op the provider serves.
//
// Semantics follow the reference's Metal host code:
//   * dequant ops write count = out.size_bytes / element-size elements
//     (metal_provider.mm:2654-2684);
//   * the fused dequant+linear op picks its f16 path from the OUTPUT dtype
//     (metal_provider.mm:2997) and reads M, N, K from push-constant bytes
//     20/24/28 (metal_provider.mm:2301-2307, 3006-3007);
//   * dense linear picks its path from A's and C's dtypes
//     (metal_provider.mm:2551-2552).
// Where the reference would read out of bounds or reinterpret a buffer with
// the wrong element type, this provider returns NF_ERROR_INVALID_ARG instead.
#include "plan.hpp"

#include <cstring>
#include <unordered_map>

namespace nfhip {
namespace {

struct OpInfo {
  OpKind kind;
  QFmt q;
  bool f16_out;  // dequant only: op name carries the _f16 suffix
};

const std::unordered_map<std::string, OpInfo>& op_table() {
  static const std::unordered_map<std::string, OpInfo> t = {
      {"dequant_q4_0", {OpKind::Dequant, QFmt::Q4_0, false}},
      {"dequant_q4_0_f16", {OpKind::Dequant, QFmt::Q4_0, true}},
      {"dequant_q8_0", {OpKind::Dequant, QFmt::Q8_0, false}},
      {"dequant_q8_0_f16", {OpKind::Dequant, QFmt::Q8_0, true}},
      // metal_provider.mm:3159-3176
      {"dequant_q4_1", {OpKind::Dequant, QFmt::Q4_1, false}},
      {"dequant_q4_1_f16", {OpKind::Dequant, QFmt::Q4_1, true}},
      {"dequant_q5_0", {OpKind::Dequant, QFmt::Q5_0, false}},
      {"dequant_q5_0_f16", {OpKind::Dequant, QFmt::Q5_0, true}},
      {"dequant_q5_1", {OpKind::Dequant, QFmt::Q5_1, false}},
      {"dequant_q5_1_f16", {OpKind::Dequant, QFmt::Q5_1, true}},
      {"dequant_q2_k", {OpKind::Dequant, QFmt::Q2_K, false}},
      {"dequant_q2_k_f16", {OpKind::Dequant, QFmt::Q2_K, true}},
      {"dequant_q3_k", {OpKind::Dequant, QFmt::Q3_K, false}},
      {"dequant_q3_k_f16", {OpKind::Dequant, QFmt::Q3_K, true}},
      {"dequant_q4_k", {OpKind::Dequant, QFmt::Q4_K, false}},
      {"dequant_q4_k_f16", {OpKind::Dequant, QFmt::Q4_K, true}},
      {"dequant_q5_k", {OpKind::Dequant, QFmt::Q5_K, false}},
      {"dequant_q5_k_f16", {OpKind::Dequant, QFmt::Q5_K, true}},
      {"dequant_q6_k", {OpKind::Dequant, QFmt::Q6_K, false}},
      {"dequant_q6_k_f16", {OpKind::Dequant, QFmt::Q6_K, true}},
      {"dequant_q4_0_linear", {OpKind::FusedLinear, QFmt::Q4_0, false}},
      {"dequant_q4_0_linear_f16", {OpKind::FusedLinear, QFmt::Q4_0, false}},
      {"dequant_q8_0_linear", {OpKind::FusedLinear, QFmt::Q8_0, false}},
      {"dequant_q8_0_linear_f16", {OpKind::FusedLinear, QFmt::Q8_0, false}},
      {"linear", {OpKind::DenseLinear, QFmt::None, false}},
      {"linear_tiled", {OpKind::DenseLinear, QFmt::None, false}},
  };
  return t;
}

const char* qname(QFmt q) {
  switch (q) {
    case QFmt::Q4_0: return "q4_0";
    case QFmt::Q8_0: return "q8_0";
    case QFmt::Q4_1: return "q4_1";
    case QFmt::Q5_0: return "q5_0";
    case QFmt::Q5_1: return "q5_1";
    case QFmt::Q2_K: return "q2_k";
    case QFmt::Q3_K: return "q3_k";
    case QFmt::Q4_K: return "q4_k";
    case QFmt::Q5_K: return "q5_k";
    case QFmt::Q6_K: return "q6_k";
    default: return "none";
  }
}
const char* ename(EType e) { return e == EType::F16 ? "f16" : "f32"; }

nf_status fail(std::string* why, const std::string& msg) {
  if (why) *why = msg;
  return NF_ERROR_INVALID_ARG;
}

// Reads M, N, K from the push-constant block (bytes 20, 24, 28).
nf_status read_mnk(const uint8_t* pc, uint32_t pc_size, uint32_t* M, uint32_t* N, uint32_t* K,
                   std::string* why) {
  if (!pc || pc_size < 32 || pc_size > 64)
    return fail(why, "matmul ops need push constants carrying M, N, K (bytes 20..31)");
  std::memcpy(M, pc + 20, 4);
  std::memcpy(N, pc + 24, 4);
  std::memcpy(K, pc + 28, 4);
  if (*M == 0 || *N == 0 || *K == 0) return fail(why, "M, N and K must be non-zero");
  if (*M > (1u << 30) || *N > (1u << 30) || *K > (1u << 30))
    return fail(why, "M, N, K beyond 2^30 are not supported");
  return NF_OK;
}

}  // namespace

bool op_known(const char* op_name) {
  return op_name && (op_table().count(op_name) != 0 || layer_op_known(op_name));
}

bool op_reads_push_constants(const char* op_name) {
  if (!op_name) return false;
  auto it = op_table().find(op_name);
  if (it != op_table().end()) return it->second.kind != OpKind::Dequant;
  return layer_op_reads_push_constants(op_name);
}

nf_status make_plan(const char* op_name, const nf_tensor_desc* const* ins, uint32_t n_in,
                    const nf_tensor_desc* const* outs, uint32_t n_out, const uint8_t* pc,
                    uint32_t pc_size, const Tuning& tuning, Plan* plan, std::string* why) {
  if (!op_name) return fail(why, "null op name");
  if (layer_op_known(op_name)) return make_layer_plan(op_name, ins, n_in, outs, n_out, pc, pc_size, plan, why);
  auto it = op_table().find(op_name);
  if (it == op_table().end()) {
    if (why) *why = std::string("unsupported op '") + op_name + "'";
    return NF_ERROR_UNSUPPORTED_OP;
  }
  const OpInfo& info = it->second;
  Plan p;
  p.op = info.kind;
  p.q = info.q;

  if (info.kind == OpKind::Dequant) {
    if (n_in < 1 || n_out < 1 || !ins || !outs || !ins[0] || !outs[0])
      return fail(why, "dequant ops take 1 input and 1 output");
    p.c = info.f16_out ? EType::F16 : EType::F32;
    p.path = Path::Dequant;
    p.count = outs[0]->size_bytes / elt_bytes(p.c);
    const uint64_t be = block_elems(p.q);
    const uint64_t blocks = (p.count + be - 1) / be;
    p.weight_bytes = blocks * block_bytes(p.q);
    p.in_bytes = ins[0]->size_bytes;
    p.out_bytes = p.count * elt_bytes(p.c);
    if (ins[0]->size_bytes < p.weight_bytes)
      return fail(why, "quantized input holds fewer blocks than the output needs");
    p.kernel = std::string("dequant_") + qname(p.q) + "_" + ename(p.c);
    *plan = p;
    return NF_OK;
  }

  if (n_in < 2 || n_out < 1 || !ins || !outs || !ins[0] || !ins[1] || !outs[0])
    return fail(why, "linear ops take 2 inputs (A, W) and 1 output");
  nf_status st = read_mnk(pc, pc_size, &p.M, &p.N, &p.K, why);
  if (st != NF_OK) return st;
  const uint64_t M = p.M, N = p.N, K = p.K;
  p.flops = 2ull * M * N * K;

  if (info.kind == OpKind::FusedLinear) {
    // Path from the output dtype (metal_provider.mm:2997).
    if (outs[0]->dtype == NF_DTYPE_F16) {
      p.a = p.b = p.c = EType::F16;
      if (ins[0]->dtype != NF_DTYPE_F16)
        return fail(why, "f16 output requires f16 activations (A dtype must be F16)");
    } else {
      if (outs[0]->dtype != NF_DTYPE_F32)
        return fail(why, "fused linear output must be F32 or F16");
      if (ins[0]->dtype != NF_DTYPE_F32)
        return fail(why, "f32 output requires f32 activations (A dtype must be F32)");
      p.a = p.b = p.c = EType::F32;
    }
    const uint64_t blocks = (K % 32 == 0) ? N * (K / 32) : (N * K + 31) / 32;
    p.weight_bytes = blocks * block_bytes(p.q);
    p.act_bytes = M * K * elt_bytes(p.a);
    p.out_bytes = M * N * elt_bytes(p.c);
    if (ins[0]->size_bytes < p.act_bytes) return fail(why, "A is smaller than M*K elements");
    if (ins[1]->size_bytes < p.weight_bytes)
      return fail(why, "W holds fewer quantized blocks than N*K/32");
    if (outs[0]->size_bytes < p.out_bytes) return fail(why, "C is smaller than M*N elements");
    const std::string tag = std::string(qname(p.q)) + "_" + ename(p.c);
    if (K % 32 != 0) {
      p.path = Path::Generic;
      p.kernel = "generic_" + tag;
    } else {
      const bool f16 = p.c == EType::F16;
      const uint32_t gemv_max = f16 ? tuning.gemv_max_m_f16 : tuning.gemv_max_m_f32;
      // The GEMV stages M' x K activations per workgroup (M' = M rounded up
      // to 1, 2 or 4), each 64-element pair followed by one 16-byte padding
      // chunk (kernels/gemv.hip: xslot), plus f32 Q4_0 block sums; beyond
      // 136 KB of LDS it would fall back to its slow block kernel, so the
      // MFMA kernel takes over.
      const uint64_t mm = p.M <= 2 ? p.M : 4;
      const uint64_t stage = mm * (K / 64) * (64 * elt_bytes(p.a) + 16) +
                             ((!f16 && p.q == QFmt::Q4_0) ? mm * (K / 64) * 8 : 0);
      const bool gemv_fits = K % 64 != 0 || stage <= 136 * 1024;
      // Two rows: the GEMV only while two of its workgroups fit a CU's LDS
      // (stage <= gemv_m2_max_stage_bytes, 80 KB); past that the small-batch kernel is as fast
      // (8192x28672 f16, 112 KB stage: 46.3 against 47.9 us; 28672x8192
      // f32, 66 KB: the GEMV 44.5 against 57.0 us).  Three or four rows:
      // the GEMV only while the weights are small enough that the
      // small-batch kernel's fixed per-launch cost dominates it.
      const bool gemv_rows_ok = p.M == 1 || (p.M == 2 ? (stage <= tuning.gemv_m2_max_stage_bytes || K % 256 != 0)
                                                      : p.weight_bytes <= tuning.gemv_m4_max_weight_bytes);
      if (p.M <= gemv_max && gemv_rows_ok && (gemv_fits || K % 256 != 0)) {
        p.path = Path::Gemv;
        p.kernel = "gemv_" + tag;
      } else if (K % 256 == 0 && p.M <= (f16 ? tuning.skinny_max_m_f16 : tuning.skinny_max_m_f32) &&
                 (!f16 || p.M <= 4 || K <= tuning.skinny_f16_max_k)) {
        p.path = Path::Skinny;
        p.kernel = "skinny_mfma_" + tag;
      } else if (f16 || K % 64 == 0) {
        p.path = Path::GemmMfma;
        p.kernel = "gemm_mfma_" + tag;
      } else {
        p.path = Path::Gemv;  // f32 with K % 64 != 0
        p.kernel = "gemv_" + tag;
      }
    }
    *plan = p;
    return NF_OK;
  }

  // Dense linear: dtype-driven (metal_provider.mm:2551-2552).
  auto etype_of = [](nf_dtype d, bool* ok) {
    *ok = (d == NF_DTYPE_F16 || d == NF_DTYPE_F32);
    return d == NF_DTYPE_F16 ? EType::F16 : EType::F32;
  };
  bool ok_a = false, ok_b = false, ok_c = false;
  p.a = etype_of(ins[0]->dtype, &ok_a);
  p.b = etype_of(ins[1]->dtype, &ok_b);
  p.c = etype_of(outs[0]->dtype, &ok_c);
  if (!ok_a || !ok_c) return fail(why, "linear needs F32 or F16 activations and output");
  if (!ok_b) p.b = p.a;  // untyped weight buffer: same element type as A
  p.weight_bytes = N * K * elt_bytes(p.b);
  p.act_bytes = M * K * elt_bytes(p.a);
  p.out_bytes = M * N * elt_bytes(p.c);
  if (ins[0]->size_bytes < p.act_bytes) return fail(why, "A is smaller than M*K elements");
  if (ins[1]->size_bytes < p.weight_bytes) return fail(why, "B is smaller than N*K elements");
  if (outs[0]->size_bytes < p.out_bytes) return fail(why, "C is smaller than M*N elements");
  p.path = Path::Dense;
  p.kernel = std::string("linear_") + ename(p.a) + ename(p.b) + "_" + ename(p.c);
  *plan = p;
  return NF_OK;
}

int gemm_tile_from_name(const char* name) {
  if (!name) return -1;
  static const char* const kNames[] = {"256x256", "256x128", "128x128", "256x128w4",
                                       "256x128w4s3", "128x128s3", "128x256", "wq1", "wq2", "wq2m64", "wq2m32", "wq2n128"};
  for (int i = 0; i < 12; ++i)
    if (std::strcmp(name, kNames[i]) == 0) return i;
  if (name[0] >= '0' && name[0] <= '9' && name[1] == '\0') return name[0] - '0';
  if (std::strcmp(name, "10") == 0) return 10;
  if (std::strcmp(name, "11") == 0) return 11;
  return -1;
}

}  // namespace nfhip
