/*
 * nf_abi.h — the NeuralOS plugin waist, restated for the MI355X provider.
 *
 * Every type below crosses a shared-library boundary between the engine
 * (scheduler, model layer, tools) and an execution provider such as
 * libnf_plugin_hip.so.  The sizes, field orders and enum values are part
 * of the binary contract: a provider built from this header must be
 * loadable by an engine built from the reference's own headers, so every
 * layout is pinned with a static assertion.
 *
 * Reference interface restated here (layouts and values only):
 *   core/include/neuralOS/ddi/neuro_fabric_abi.h:45-254   (status, dtype,
 *       tensor desc, provider vtable, nf_plugin_register)
 *   core/include/neuralOS/ddi/neuro_buffer_abi.h:36-271   (memory domains,
 *       buffer info/ops, alloc request, mem vtable)
 *   core/include/neuralOS/ddi/neuro_scheduler_abi.h:86-127 (task desc; the
 *       push-constant "offsetof bridge" depends on its layout)
 *   core/include/neuralOS/ddi/neuro_ddi.h:33-84            (driver caps,
 *       async DDI vtable)
 *
 * Plain C11 / C++ — no vtables, no exceptions, opaque handles only.
 */
#ifndef NF_ABI_H
#define NF_ABI_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define NF_API __attribute__((visibility("default")))
#else
#define NF_API
#endif

#ifdef __cplusplus
#define NF_STATIC_ASSERT(c, m) static_assert(c, m)
extern "C" {
#else
#define NF_STATIC_ASSERT(c, m) _Static_assert(c, m)
#endif

/* ABI version 0.2.0, packed as 0x00MMNNPP.  A loader rejects a provider
 * whose get_abi_version() differs (core/src/plugin_loader.cpp:48-54). */
#define NF_ABI_VERSION_MAJOR 0
#define NF_ABI_VERSION_MINOR 2
#define NF_ABI_VERSION_PATCH 0
#define NF_ABI_VERSION                                   \
    (((uint32_t)NF_ABI_VERSION_MAJOR << 16) |            \
     ((uint32_t)NF_ABI_VERSION_MINOR << 8) |             \
     ((uint32_t)NF_ABI_VERSION_PATCH))

/* ---- opaque handles ------------------------------------------------ */
typedef struct nf_context_t  *nf_context;
typedef struct nf_node_t     *nf_node;
typedef struct nf_provider_t *nf_provider;
typedef struct nf_buffer_t   *nf_buffer;

/* ---- status codes -------------------------------------------------- */
typedef enum nf_status {
    NF_OK                   = 0,
    NF_ERROR_INVALID_ARG    = 1,
    NF_ERROR_OUT_OF_MEMORY  = 2,
    NF_ERROR_NOT_FOUND      = 3,
    NF_ERROR_ABI_MISMATCH   = 4,
    NF_ERROR_PLUGIN_LOAD    = 5,
    NF_ERROR_DEVICE_LOST    = 6,
    NF_ERROR_UNSUPPORTED_OP = 7,
    NF_ERROR_TIMEOUT        = 8,
    NF_ERROR_INVALID_INPUT  = 9,
    NF_ERROR_INTERNAL       = 255
} nf_status;

/* ---- element types ------------------------------------------------- */
/* Q4_0: 18-byte block = fp16 scale + 16 bytes of packed 4-bit codes.
 * Q8_0: 34-byte block = fp16 scale + 32 signed 8-bit codes.
 * Both cover 32 consecutive elements along the fastest dimension. */
typedef enum nf_dtype {
    NF_DTYPE_F32  = 0,
    NF_DTYPE_F16  = 1,
    NF_DTYPE_BF16 = 2,
    NF_DTYPE_I8   = 3,
    NF_DTYPE_I32  = 4,
    NF_DTYPE_U8   = 5,
    NF_DTYPE_Q4_0 = 6,
    NF_DTYPE_Q8_0 = 7,
    NF_DTYPE_Q4_1 = 8,
    NF_DTYPE_Q5_0 = 9,
    NF_DTYPE_Q5_1 = 10,
    NF_DTYPE_Q2_K = 11,
    NF_DTYPE_Q3_K = 12,
    NF_DTYPE_Q4_K = 13,
    NF_DTYPE_Q5_K = 14,
    NF_DTYPE_Q6_K = 15
} nf_dtype;

#define NF_MAX_DIMS 8

/* POD tensor description; does not own memory.  144 bytes. */
typedef struct nf_tensor_desc {
    nf_dtype dtype;
    uint32_t ndim;
    uint64_t shape[NF_MAX_DIMS];
    uint64_t strides[NF_MAX_DIMS]; /* bytes; 0 = contiguous */
    uint64_t size_bytes;
} nf_tensor_desc;
NF_STATIC_ASSERT(sizeof(nf_tensor_desc) == 144, "nf_tensor_desc must be 144 bytes");

/* ---- provider vtable (the compute contract) ------------------------ */
typedef struct nf_provider_vtable {
    const char *(*get_name)(nf_provider self);
    uint32_t (*get_abi_version)(nf_provider self);
    nf_status (*init)(nf_provider self);
    void (*shutdown)(nf_provider self);
    nf_status (*buffer_alloc)(nf_provider self, const nf_tensor_desc *desc, nf_buffer *out);
    void (*buffer_free)(nf_provider self, nf_buffer buf);
    nf_status (*buffer_map)(nf_provider self, nf_buffer buf, void **out_ptr);
    nf_status (*buffer_unmap)(nf_provider self, nf_buffer buf);
    /* Enqueue a named operator.  A return of NF_OK means "enqueued";
     * synchronize() (or a buffer fence) waits for completion. */
    nf_status (*dispatch)(nf_provider self, const char *op_name,
                          const nf_buffer *inputs, uint32_t n_in,
                          nf_buffer *outputs, uint32_t n_out);
    nf_status (*synchronize)(nf_provider self);
} nf_provider_vtable;

typedef nf_status (*nf_plugin_register_fn)(nf_provider_vtable *vtable, nf_provider *provider);
#define NF_PLUGIN_ENTRY_SYMBOL "nf_plugin_register"

/* ---- buffer protocol ------------------------------------------------ */
typedef enum nf_mem_domain {
    NF_MEM_DOMAIN_CPU        = 0,
    NF_MEM_DOMAIN_UNIFIED    = 1,
    NF_MEM_DOMAIN_DEVICE     = 2,
    NF_MEM_DOMAIN_DMA_BUF    = 3,
    NF_MEM_DOMAIN_EXTERNAL   = 4,
    NF_MEM_DOMAIN_MMAP       = 5,
    NF_MEM_DOMAIN_CXL        = 6,
    NF_MEM_DOMAIN_CXL_SHARED = 7
} nf_mem_domain;

typedef enum nf_cache_op {
    NF_CACHE_FLUSH            = 0x01, /* host writes -> device */
    NF_CACHE_INVALIDATE       = 0x02, /* device writes -> host */
    NF_CACHE_FLUSH_INVALIDATE = 0x03
} nf_cache_op;

/* 176 bytes. */
typedef struct nf_buffer_info {
    nf_tensor_desc desc;
    nf_mem_domain domain;
    uint64_t offset_bytes;
    uint64_t share_token;
    uint32_t refcount;
    uint32_t _reserved;
} nf_buffer_info;
NF_STATIC_ASSERT(sizeof(nf_buffer_info) == 176, "nf_buffer_info must be 176 bytes");

typedef struct nf_buffer_ops {
    uint32_t (*retain)(nf_buffer self);
    uint32_t (*release)(nf_buffer self); /* returns the new count; 0 = freed */
    nf_status (*map)(nf_buffer self, void **out_ptr);
    nf_status (*unmap)(nf_buffer self);
    nf_status (*cache_sync)(nf_buffer self, nf_cache_op op, uint64_t offset, uint64_t size);
    nf_status (*get_info)(nf_buffer self, nf_buffer_info *info);
    nf_status (*export_handle)(nf_buffer self, uint64_t *token, nf_mem_domain *domain);
    nf_status (*import_handle)(nf_provider provider, uint64_t token, nf_mem_domain domain,
                               const nf_tensor_desc *desc, nf_buffer *out);
} nf_buffer_ops;

/* 160 bytes. */
typedef struct nf_buffer_alloc_request {
    nf_tensor_desc desc;
    nf_mem_domain preferred;
    uint32_t flags;
    uint32_t _reserved;
} nf_buffer_alloc_request;
NF_STATIC_ASSERT(sizeof(nf_buffer_alloc_request) == 160, "nf_buffer_alloc_request must be 160 bytes");

#define NF_BUFFER_USAGE_WEIGHT_MMAP 0x01u

typedef struct nf_provider_mem_vtable {
    nf_status (*alloc)(nf_provider self, const nf_buffer_alloc_request *req,
                       nf_buffer_ops *ops, nf_buffer *buf);
    nf_status (*import_buffer)(nf_provider self, uint64_t token, nf_mem_domain domain,
                               const nf_tensor_desc *desc, nf_buffer_ops *ops, nf_buffer *buf);
    nf_status (*can_import)(nf_provider self, nf_mem_domain domain);
} nf_provider_mem_vtable;

typedef nf_status (*nf_plugin_register_mem_fn)(nf_provider_mem_vtable *mem_vt);
#define NF_PLUGIN_MEM_ENTRY_SYMBOL "nf_plugin_register_mem"

/* ---- task descriptor (scheduler side) ------------------------------ */
typedef enum nf_task_priority {
    NF_PRIORITY_LOW = 0, NF_PRIORITY_NORMAL = 1, NF_PRIORITY_HIGH = 2, NF_PRIORITY_CRITICAL = 3
} nf_task_priority;

typedef enum nf_task_flags {
    NF_TASK_NONE = 0, NF_TASK_ASYNC = 0x01, NF_TASK_FENCE = 0x02,
    NF_TASK_REMOTE = 0x04, NF_TASK_CACHEABLE = 0x08
} nf_task_flags;

typedef enum nf_affinity {
    NF_AFFINITY_ANY = 0, NF_AFFINITY_CPU = 1, NF_AFFINITY_GPU = 2,
    NF_AFFINITY_NPU = 3, NF_AFFINITY_REMOTE = 4
} nf_affinity;

#define NF_MAX_TASK_INPUTS    16
#define NF_MAX_TASK_OUTPUTS   8
#define NF_MAX_OP_NAME        64
#define NF_MAX_PUSH_CONSTANTS 64

/* 3056 bytes.  The engine passes &desc.inputs[0] as dispatch()'s `inputs`
 * argument; a provider recovers the descriptor (and its push constants)
 * by stepping back offsetof(nf_task_desc, inputs) bytes. */
typedef struct nf_task_desc {
    char op_name[NF_MAX_OP_NAME];
    nf_buffer inputs[NF_MAX_TASK_INPUTS];
    nf_buffer_ops input_ops[NF_MAX_TASK_INPUTS];
    uint32_t n_inputs;
    nf_buffer outputs[NF_MAX_TASK_OUTPUTS];
    nf_buffer_ops output_ops[NF_MAX_TASK_OUTPUTS];
    uint32_t n_outputs;
    nf_tensor_desc output_descs[NF_MAX_TASK_OUTPUTS];
    nf_affinity affinity;
    nf_task_priority priority;
    uint32_t flags;
    void *user_data;
    uint32_t push_constants_size;
    uint8_t push_constants[NF_MAX_PUSH_CONSTANTS];
} nf_task_desc;
NF_STATIC_ASSERT(sizeof(nf_task_desc) == 3056, "nf_task_desc must be 3056 bytes");
NF_STATIC_ASSERT(offsetof(nf_task_desc, inputs) == 64, "inputs must follow op_name");
NF_STATIC_ASSERT(offsetof(nf_task_desc, push_constants_size) == 2984, "push-constant size offset");
NF_STATIC_ASSERT(offsetof(nf_task_desc, push_constants) == 2988, "push-constant offset");

/* ---- optional async DDI -------------------------------------------- */
typedef struct nf_completion_token_t *nf_completion_token;

/* 32 bytes. */
typedef struct nf_driver_caps {
    uint32_t max_concurrent;
    uint64_t memory_bytes;
    uint64_t flops;
    uint32_t supported_dtypes; /* bit i set <=> nf_dtype i supported */
    uint32_t flags;
} nf_driver_caps;
NF_STATIC_ASSERT(sizeof(nf_driver_caps) == 32, "nf_driver_caps must be 32 bytes");

#define NF_CAP_ASYNC 0x01
#define NF_CAP_RDMA  0x02
#define NF_CAP_FP16  0x04
#define NF_CAP_INT8  0x08
#define NF_CAP_PAGED 0x10

typedef struct nf_ddi_vtable {
    nf_status (*dispatch_async)(nf_provider self, const char *op_name,
                                const nf_buffer *inputs, uint32_t n_in,
                                nf_buffer *outputs, uint32_t n_out,
                                nf_completion_token *token);
    nf_status (*wait_completion)(nf_provider self, nf_completion_token token, uint64_t timeout_ms);
    nf_status (*poll_completion)(nf_provider self, nf_completion_token token);
    nf_status (*query_caps)(nf_provider self, nf_driver_caps *caps);
} nf_ddi_vtable;

typedef nf_status (*nf_plugin_register_ddi_fn)(nf_ddi_vtable *ddi_vt);
#define NF_PLUGIN_DDI_ENTRY_SYMBOL "nf_plugin_register_ddi"

#ifdef __cplusplus
}
#endif
#endif /* NF_ABI_H */
