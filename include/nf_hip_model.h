/*
 * nf_hip_model.h — op selection for a model layer that drives this provider.
 *
 * The reference's model layer picks the op of every projection from the
 * weight's dtype: a fused dequant + linear op only for Q4_0
 * (model/model/quant_registry.hpp:84-88, nf_fused_linear_op_name), a
 * warm-up dequant to dense weights plus `linear` for every other quantized
 * format (llama_dag_builder.hpp:1025-1039, maybe_dq; :1411-1422,
 * fused_or_linear), and always a warm-up dequant plus `linear` for the
 * output projection (lm_head, :1050-1056 and :1520-1523).  This provider
 * also fuses Q8_0, so a model layer that asks these functions instead runs
 * Q8_0 projections and a Q4_0 / Q8_0 lm_head straight from the quantized
 * blocks: no dense fp32 copy (3.8x the Q8_0 bytes, 7.1x the Q4_0 bytes) is
 * made at load and none is streamed per token.
 *
 * Self-contained C (no other header of this library), so it can be included
 * next to the reference's own neuro_fabric_abi.h: dtypes are the numeric
 * nf_dtype codes both define (F32 = 0, F16 = 1, Q4_0 = 6, Q8_0 = 7,
 * Q4_1 .. Q6_K = 8 .. 15).
 */
#ifndef NF_HIP_MODEL_H
#define NF_HIP_MODEL_H

#include <stdbool.h>
#include <stdint.h>

#ifndef NF_API
#define NF_API __attribute__((visibility("default")))
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* Fused dequant + linear op for weights of dtype `wtype`, or NULL when the
 * provider has none: "dequant_q4_0_linear[_f16]", "dequant_q8_0_linear[_f16]"
 * (fp16 = f16 activations and output).  Replaces nf_fused_linear_op_name
 * (quant_registry.hpp:84-88), which names Q4_0 only. */
NF_API const char *nf_hip_fused_linear_op_name(uint32_t wtype, bool fp16);

/* The op a model layer emits for a projection (attention and FFN linears and
 * the output projection alike) whose weight is stored as `wtype`: the fused
 * op when nf_hip_fused_linear_op_name has one, else "linear" on a dense copy
 * (F32 / F16 weights as stored, other quantized formats after the warm-up
 * dequantization below).  Replaces fused_or_linear
 * (llama_dag_builder.hpp:1411-1422) and the lm_head's fixed "linear"
 * (:1520-1523). */
NF_API const char *nf_hip_projection_op_name(uint32_t wtype, bool fp16);

/* True when a projection weight of dtype `wtype` needs a warm-up
 * dequantization to a dense copy before its "linear": quantized formats the
 * provider does not fuse (maybe_dq, llama_dag_builder.hpp:1025-1039). */
NF_API bool nf_hip_projection_needs_dequant(uint32_t wtype);

/* The dequantization op of a quantized dtype, "dequant_<fmt>" or
 * "dequant_<fmt>_f16", or NULL for a dense dtype (nf_dequant_op_name[_f16],
 * quant_registry.hpp:50-81, keyed by nf_dtype instead of the GGUF code). */
NF_API const char *nf_hip_dequant_op_name(uint32_t wtype, bool fp16);

#ifdef __cplusplus
}
#endif
#endif /* NF_HIP_MODEL_H */
