// model_ops.cpp — op selection for a model layer that drives this provider
// (declared in nf_hip_model.h): which op a projection with weights of a
// given dtype runs as, and which warm-up dequantization it needs.
//
// The reference's model layer fuses Q4_0 only and always runs the output
// projection as a dense `linear` (quant_registry.hpp:84-88;
// llama_dag_builder.hpp:1025-1039, 1411-1422, 1520-1523).  Here both fused
// formats the provider serves are named, and the output projection is a
// projection like any other.
#include <cstdint>

#include "nf_hip_model.h"

namespace {

// nf_dtype codes (neuro_fabric_abi.h:124-141): Q4_0 .. Q6_K are 6 .. 15.
constexpr uint32_t kQ4_0 = 6, kQ8_0 = 7, kFirstQuant = 6, kLastQuant = 15;

const char* const kDequant[] = {"dequant_q4_0", "dequant_q8_0", "dequant_q4_1", "dequant_q5_0", "dequant_q5_1",
                                "dequant_q2_k", "dequant_q3_k", "dequant_q4_k", "dequant_q5_k", "dequant_q6_k"};
const char* const kDequantF16[] = {"dequant_q4_0_f16", "dequant_q8_0_f16", "dequant_q4_1_f16", "dequant_q5_0_f16",
                                   "dequant_q5_1_f16", "dequant_q2_k_f16", "dequant_q3_k_f16", "dequant_q4_k_f16",
                                   "dequant_q5_k_f16", "dequant_q6_k_f16"};

bool quantized(uint32_t t) { return t >= kFirstQuant && t <= kLastQuant; }

}  // namespace

extern "C" {

NF_API const char* nf_hip_fused_linear_op_name(uint32_t wtype, bool fp16) {
  if (wtype == kQ4_0) return fp16 ? "dequant_q4_0_linear_f16" : "dequant_q4_0_linear";
  if (wtype == kQ8_0) return fp16 ? "dequant_q8_0_linear_f16" : "dequant_q8_0_linear";
  return nullptr;
}

NF_API const char* nf_hip_projection_op_name(uint32_t wtype, bool fp16) {
  const char* fused = nf_hip_fused_linear_op_name(wtype, fp16);
  return fused ? fused : "linear";
}

NF_API bool nf_hip_projection_needs_dequant(uint32_t wtype) {
  return quantized(wtype) && nf_hip_fused_linear_op_name(wtype, false) == nullptr;
}

NF_API const char* nf_hip_dequant_op_name(uint32_t wtype, bool fp16) {
  if (!quantized(wtype)) return nullptr;
  return fp16 ? kDequantF16[wtype - kFirstQuant] : kDequant[wtype - kFirstQuant];
}

}  // extern "C"
