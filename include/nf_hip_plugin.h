/*
 * nf_hip_plugin.h — exported C entry points of libnf_plugin_hip.so, the
 * MI355X (gfx950) execution provider for NeuralOS's quantized linear path.
 *
 * The provider is a drop-in for the reference's plugins/metal (and the
 * plugins/cuda slot): an engine that links or dlopen()s this library and
 * calls nf_plugin_register / nf_plugin_register_mem gets the same op names,
 * argument conventions and error codes.  Everything else in the library has
 * hidden visibility.
 *
 * Ops served by dispatch() (op name -> inputs -> outputs):
 *   dequant_q4_0 / dequant_q8_0             W(quant) -> f32[count]
 *   dequant_q4_0_f16 / dequant_q8_0_f16     W(quant) -> f16[count]
 *       count = output size_bytes / element size (metal_provider.mm:2654-2684)
 *   dequant_q4_0_linear / dequant_q4_0_linear_f16
 *   dequant_q8_0_linear / dequant_q8_0_linear_f16   (Q8_0: new, additive)
 *       A[M,K], W[N,K] quant -> C[M,N]; path chosen by the OUTPUT dtype:
 *       F16 output => f16 activations, weights rounded to f16, fp32 accumulate,
 *       f16 result; otherwise f32 in/out with exact f32 weights
 *       (metal_provider.mm:1396-1468, 2990-3031).
 *   linear / linear_tiled                   A[M,K], B[N,K] dense -> C[M,N]
 *       (metal_provider.mm:2544-2613; f16 A with f32 C is computed correctly)
 * M, N, K come from the push constants of the enclosing nf_task_desc
 * (bytes 20, 24, 28), recovered through the offsetof bridge
 * (metal_provider.mm:2301-2307).
 */
#ifndef NF_HIP_PLUGIN_H
#define NF_HIP_PLUGIN_H

#include <stdbool.h>
#include "nf_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* 48-byte push-constant block carried in nf_task_desc.push_constants.
 * Layout of metal_provider.mm:70-83 / llama_dag_builder.hpp:105-111. */
typedef struct nf_push_constants {
    uint32_t seq_len;
    uint32_t n_heads;
    uint32_t head_dim;
    float epsilon;
    float theta;
    uint32_t M; /* byte 20 */
    uint32_t N; /* byte 24 */
    uint32_t K; /* byte 28 */
    uint32_t step_idx;
    uint32_t max_seq_len;
    uint32_t window_size;
    uint32_t _pad1;
} nf_push_constants;

/* ---- plugin entry points -------------------------------------------- */

/* Fill the provider vtable and return the provider handle (a process-wide
 * singleton).  Replaces metal_provider.mm:3266-3281 (and the plugins/cuda
 * slot, cuda_provider.cpp:188-202); contract neuro_fabric_abi.h:233-254. */
NF_API nf_status nf_plugin_register(nf_provider_vtable *vt, nf_provider *out);

/* Fill the memory vtable (alloc / import_buffer / can_import).  One-argument
 * form of metal_provider.mm:3283-3289; contract neuro_buffer_abi.h:262-271.
 * Callers that declare it with a second argument (nf_generate.cpp:62) are
 * harmless under the SysV calling convention. */
NF_API nf_status nf_plugin_register_mem(nf_provider_mem_vtable *mem_vt);

/* Optional async DDI (dispatch_async / wait / poll / query_caps).
 * Contract neuro_ddi.h:51-84; the Metal plugin does not export it. */
NF_API nf_status nf_plugin_register_ddi(nf_ddi_vtable *ddi_vt);

/* ---- per-dispatch GPU timing ring ------------------------------------ */
/* Same signatures and ring semantics (1024 entries, oldest overwritten) as
 * metal_provider.mm:2149-2189, measured with HIP events on the provider's
 * stream.  Enabling clears the ring. */
NF_API void nf_hip_enable_timing(bool enable);
NF_API uint32_t nf_hip_get_timing_count(void);
NF_API void nf_hip_get_timings(char (*op_names)[64], double *gpu_ms, uint32_t max_count);
NF_API void nf_hip_get_timings_ext(char (*op_names)[64], double *gpu_ms, uint8_t *dtypes,
                                   uint32_t *elem_counts, uint32_t max_count);

/* The same four entry points under the Metal plugin's names
 * (metal_provider.mm:2149-2189), for code that binds them by name:
 * model/model/trace_export.hpp:20-25, tests/driver/benchmark_kernels.cpp,
 * tests/driver/real_model_test.cpp. */
NF_API void nf_metal_enable_timing(bool enable);
NF_API uint32_t nf_metal_get_timing_count(void);
NF_API void nf_metal_get_timings(char (*op_names)[64], double *gpu_ms, uint32_t max_count);
NF_API void nf_metal_get_timings_ext(char (*op_names)[64], double *gpu_ms, uint8_t *dtypes,
                                     uint32_t *elem_counts, uint32_t max_count);

/* ---- MI355X extensions (no counterpart in the reference) -------------- */

/* Which kernel a dispatch would run and the work it represents.  Pure host
 * logic: validates exactly like dispatch() and needs no GPU, so callers
 * (and tests) can inspect kernel selection and size checks. */
typedef struct nf_hip_plan {
    char kernel[64];       /* kernel family, e.g. "gemv_q4_0_f32" */
    uint32_t M, N, K;
    uint64_t count;        /* dequant ops: elements written */
    uint64_t weight_bytes; /* algorithmic bytes, each operand counted once */
    uint64_t act_bytes;
    uint64_t out_bytes;
    uint64_t flops;        /* 2*M*N*K for matmul ops, 0 otherwise */
} nf_hip_plan;

NF_API nf_status nf_hip_plan_dispatch(const char *op_name,
                                      const nf_tensor_desc *in_descs, uint32_t n_in,
                                      const nf_tensor_desc *out_descs, uint32_t n_out,
                                      const void *push_constants, uint32_t push_constants_size,
                                      nf_hip_plan *plan);

/* Batch-size switch points between the kernel families of the fused ops:
 * the VALU decode GEMV while M <= gemv_max_m, the small-batch MFMA kernel
 * above it up to skinny_max_m (at most 32 f32 / 64 f16 activation rows per
 * launch), the tiled MFMA GEMM beyond (f16 activations: fp16 MFMA; f32
 * activations: exact bf16 pieces on bf16 MFMA, K % 64 == 0).  f16 and f32
 * activations each have their own switch points.  Defaults come from
 * measurement; environment overrides NF_HIP_GEMV_MAX_M_F32,
 * NF_HIP_GEMV_MAX_M_F16, NF_HIP_SKINNY_MAX_M_F16 and NF_HIP_SKINNY_MAX_M_F32
 * are read at nf_plugin_register.  No counterpart in the reference: its
 * Metal provider runs one kernel for every M (metal_provider.mm:3009-3019,
 * the simdgroup variant disabled). */
NF_API void nf_hip_set_gemv_max_m(uint32_t f32_path, uint32_t f16_path);
NF_API void nf_hip_get_gemv_max_m(uint32_t *f32_path, uint32_t *f16_path);
/* Further limits on the GEMV at M <= gemv_max_m: two rows only while the
 * activation stage (2 x K x element size, plus the f32 Q4_0 path's
 * partial sums) is at most m2_max_stage_bytes (default 80 KB: two
 * workgroups per CU), three or four rows only while the weights are at
 * most m34_max_weight_bytes (default 16 MB); past either the small-batch
 * kernel takes the rows.  Environment overrides NF_HIP_GEMV_M2_MAX_STAGE
 * and NF_HIP_GEMV_M4_MAX_WEIGHT (bytes).  No counterpart in the reference
 * (one kernel for every M, metal_provider.mm:3009-3019). */
NF_API void nf_hip_set_gemv_row_limits(uint32_t m2_max_stage_bytes, uint64_t m34_max_weight_bytes);
NF_API void nf_hip_get_gemv_row_limits(uint32_t *m2_max_stage_bytes, uint64_t *m34_max_weight_bytes);
NF_API void nf_hip_set_skinny_max_m(uint32_t f16_path);
NF_API uint32_t nf_hip_get_skinny_max_m(void);
NF_API void nf_hip_set_skinny_max_m_f32(uint32_t f32_path);
NF_API uint32_t nf_hip_get_skinny_max_m_f32(void);
/* f16 activations: above M = 4 the small-batch kernel serves only rows of
 * K <= skinny_f16_max_k (default 2^30, no cap: with its K split over
 * workgroups the small-batch kernel measured faster than the tiled GEMM at
 * K = 28672 too); environment override NF_HIP_SKINNY_F16_MAX_K. */
NF_API void nf_hip_set_skinny_f16_max_k(uint32_t k);
NF_API uint32_t nf_hip_get_skinny_f16_max_k(void);

/* Kernel of the fused f16 GEMM path (M above the small-batch range): -1
 * (default) = the kernels that dequantize weights in registers, picked by M
 * from measurement on MI355X (two waves per SIMD with 32-row waves up to
 * M = 32 and 64-row waves up to M = 64 or while ceil(M/64) x ceil(N/256) is
 * at most 80 (Q4_0) / 64 (Q8_0) with K <= 16384; 128-row waves for the other
 * Q4_0 batches, on 128-column tiles when ceil(M/128) x ceil(N/256) x K/128 <=
 * 4096;
 * one wave per SIMD otherwise; the two-wave kernels need K % 128 == 0); 0..6 = the kernel that dequantizes weight tiles into LDS,
 * tile shape 256x256, 256x128, 128x128, 256x128 with 4 waves, 256x128 with
 * 4 waves and 3 stages, 128x128 with 3 stages, 128x256; 7 = the
 * register-dequantizing kernel with one wave per SIMD for every shape;
 * 8 / 9 / 10 = the two-wave kernel with 128 / 64 / 32-row waves wherever it
 * applies (K % 128 == 0; 8: Q4_0 only), else as 7; 11 = its 128-row waves
 * on 128-column tiles (Q4_0 only), else as 7.  With f32 activations
 * (the bf16-piece kernel) 8 / 9 force its 128- / 64-row waves.
 * Other values mean -1.  Environment override NF_HIP_GEMM_TILE (the shape
 * name or number) is read at nf_plugin_register.  No counterpart in the
 * reference (its Metal provider has one fused GEMM kernel); this is
 * process-wide tuning like the switch points above. */
NF_API void nf_hip_set_gemm_tile(int32_t tile);
NF_API int32_t nf_hip_get_gemm_tile(void);

/* Dispatch `n_tasks` prepared task descriptors in order, `repeat` times —
 * a compiled step submitted with one call, the way Session::step walks its
 * plan (PipelineEngine.hpp:518-561) but without a thread hop per node.  Each
 * element goes through the same validation as vtable.dispatch, on the same
 * stream; returns the first non-NF_OK status.  Because the whole batch is
 * known, adjacent decode GEMVs and small-batch (M <= 32) linears that read
 * the same activation buffer (same fused op, M and K; no output overlapping
 * another member's inputs or output) are launched as one grouped kernel, up
 * to four at a time: the results are bit-identical to dispatching them one
 * by one, in order.  Not done while per-dispatch timing is enabled.
 * vtable.dispatch itself never defers or merges anything. */
NF_API nf_status nf_hip_run_tasks(nf_provider self, const nf_task_desc *tasks, uint32_t n_tasks,
                                  uint32_t repeat);

/* Launches enqueued since nf_plugin_register: one per dispatch, and one per
 * group of decode GEMVs that nf_hip_run_tasks merged into a single launch
 * (adjacent tasks of the same fused op reading the same activation buffer
 * with the same M and K, with no buffer hazard between them: q/k/v,
 * gate/up).  No counterpart in the reference; lets a caller relate a step's
 * time to its kernel launches. */
NF_API uint64_t nf_hip_launch_count(nf_provider self);

/* Per-launch floor calibration for benchmarks: enqueues on `stream` (a
 * hipStream_t, or NULL for the null stream) one kernel that reads the
 * `bytes` at `src` (16-byte aligned; every 16-byte chunk loaded once, all
 * loads of a thread in flight together, nothing stored), or an empty kernel
 * when bytes < 16.  Timing it beside a fused GEMV over the same bytes
 * separates the cost of moving the weights from the GEMV's own work.
 * NF_ERROR_INVALID_ARG for a null or misaligned src.  No counterpart in
 * the reference. */
NF_API nf_status nf_hip_diag_stream_read(const void *src, uint64_t bytes, void *stream);

/* The in-order hipStream_t (as void*) every dispatch is launched on, so a
 * caller can time or capture (hipStreamBeginCapture) a run of dispatches.
 * A buffer that a captured dispatch writes is marked for good: map,
 * cache_sync(INVALIDATE) and nf_hip_buffer_read of it drain this stream
 * first, so they see the results of every graph replay the caller launched
 * on it.  Work the caller enqueues on any other stream is the caller's to
 * synchronize before such a read.  NF_ERROR_INVALID_ARG before init. */
NF_API nf_status nf_hip_get_stream(nf_provider self, void **stream);

/* Device pointer behind one of this provider's buffers (for zero-copy
 * hand-off to other HIP code in the same process). */
NF_API nf_status nf_hip_buffer_device_ptr(nf_buffer buf, void **dev_ptr);

/* Copy `bytes` bytes between host memory of any kind (pageable, such as an
 * mmap of a GGUF file, or pinned) and the byte range [offset, offset+bytes)
 * of a buffer; complete on return.  A write is ordered on the provider
 * stream after every dispatch already issued; a read waits for the last
 * dispatch that wrote the buffer (every dispatch for a buffer whose device
 * address was handed out by export, get_info or nf_hip_buffer_device_ptr).  NF_ERROR_INVALID_ARG for a range outside the
 * buffer or a mapped buffer.  No counterpart in the reference's ABI: it is
 * the one-copy form of the weight upload the reference's model layer does
 * with map + memcpy + unmap (model/model/llama_dag_builder.hpp:146-156,
 * load_weight), which costs a staging copy here (31 GB/s from pageable
 * memory on MI355X against ~15 GB/s for map/memcpy/unmap with a warm
 * staging pool). */
NF_API nf_status nf_hip_buffer_write(nf_buffer buf, uint64_t offset, const void *src, uint64_t bytes);
NF_API nf_status nf_hip_buffer_read(nf_buffer buf, uint64_t offset, void *dst, uint64_t bytes);

/* Frees the pinned staging blocks that unmapping large buffers (>= 64 MiB)
 * leaves in the provider's pool for reuse (at most 2 GiB), e.g. once model
 * weights are uploaded.  Shutdown frees them too.  NULL = the provider this
 * library registers. */
NF_API void nf_hip_release_staging(nf_provider self);

/* Last error text recorded by the provider (thread-local, never NULL). */
NF_API const char *nf_hip_last_error(void);

/* Fused dequant + linear that allocates nothing.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same computation and kernel choice as dispatch() of
 * dequant_q4_0_linear[_f16] / dequant_q8_0_linear[_f16] (wtype Q4_0 or
 * Q8_0; f16 = f16 activations and output, else f32), on caller-owned device
 * pointers A [M,K], W [N,K] (blocks along K) and C [M,N], enqueued on
 * `stream` (a hipStream_t; NULL = the null stream); needs no init.
 * Split-K partials and tile counters come from a static device array of the
 * library (4 MiB of partial tiles plus 4096 counters, held on every GPU the
 * library runs on until the process ends), not from the provider workspace:
 * a shape whose K split would need more partial tiles than that runs with
 * fewer splits, so no size is refused for scratch and results agree with
 * dispatch() within the fp32 accumulation tolerance.  Calls on one GPU share
 * that array: calls that overlap in time on one GPU (different streams or
 * threads) race; calls in order on one stream do not.  Returns
 * NF_ERROR_INVALID_ARG for a bad dtype, null operand, zero size or a shape
 * dispatch() would reject. */
NF_API nf_status nf_hip_fused_linear_noalloc(nf_dtype wtype, const void *A, const void *W, void *C, uint32_t M,
                                             uint32_t N, uint32_t K, bool f16, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* NF_HIP_PLUGIN_H */
