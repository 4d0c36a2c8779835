"""ctypes mirror of the NeuralOS plugin ABI (include/nf_abi.h).

Layouts match the reference waist byte for byte
(core/include/neuralOS/ddi/neuro_fabric_abi.h:123-229,
neuro_buffer_abi.h:36-261, neuro_scheduler_abi.h:86-127, neuro_ddi.h:33-76);
`check_layout()` asserts the pinned sizes and offsets.
"""
from __future__ import annotations

import ctypes as C

# ---- enums ------------------------------------------------------------
NF_OK = 0
NF_ERROR_INVALID_ARG = 1
NF_ERROR_OUT_OF_MEMORY = 2
NF_ERROR_NOT_FOUND = 3
NF_ERROR_ABI_MISMATCH = 4
NF_ERROR_PLUGIN_LOAD = 5
NF_ERROR_DEVICE_LOST = 6
NF_ERROR_UNSUPPORTED_OP = 7
NF_ERROR_TIMEOUT = 8
NF_ERROR_INVALID_INPUT = 9
NF_ERROR_INTERNAL = 255

STATUS_NAMES = {
    0: "NF_OK", 1: "NF_ERROR_INVALID_ARG", 2: "NF_ERROR_OUT_OF_MEMORY", 3: "NF_ERROR_NOT_FOUND",
    4: "NF_ERROR_ABI_MISMATCH", 5: "NF_ERROR_PLUGIN_LOAD", 6: "NF_ERROR_DEVICE_LOST",
    7: "NF_ERROR_UNSUPPORTED_OP", 8: "NF_ERROR_TIMEOUT", 9: "NF_ERROR_INVALID_INPUT",
    255: "NF_ERROR_INTERNAL",
}

NF_DTYPE_F32 = 0
NF_DTYPE_F16 = 1
NF_DTYPE_BF16 = 2
NF_DTYPE_I8 = 3
NF_DTYPE_I32 = 4
NF_DTYPE_U8 = 5
NF_DTYPE_Q4_0 = 6
NF_DTYPE_Q8_0 = 7
NF_DTYPE_Q4_1 = 8
NF_DTYPE_Q5_0 = 9
NF_DTYPE_Q5_1 = 10
NF_DTYPE_Q2_K = 11
NF_DTYPE_Q3_K = 12
NF_DTYPE_Q4_K = 13
NF_DTYPE_Q5_K = 14
NF_DTYPE_Q6_K = 15

NF_MEM_DOMAIN_CPU = 0
NF_MEM_DOMAIN_UNIFIED = 1
NF_MEM_DOMAIN_DEVICE = 2
NF_MEM_DOMAIN_DMA_BUF = 3
NF_MEM_DOMAIN_EXTERNAL = 4
NF_MEM_DOMAIN_MMAP = 5
NF_MEM_DOMAIN_CXL = 6
NF_MEM_DOMAIN_CXL_SHARED = 7

NF_CACHE_FLUSH = 0x01
NF_CACHE_INVALIDATE = 0x02
NF_CACHE_FLUSH_INVALIDATE = 0x03

NF_AFFINITY_GPU = 2

NF_CAP_ASYNC = 0x01
NF_CAP_RDMA = 0x02
NF_CAP_FP16 = 0x04
NF_CAP_INT8 = 0x08
NF_CAP_PAGED = 0x10

NF_MAX_DIMS = 8
NF_MAX_TASK_INPUTS = 16
NF_MAX_TASK_OUTPUTS = 8
NF_MAX_OP_NAME = 64
NF_MAX_PUSH_CONSTANTS = 64

NF_ABI_VERSION = (0 << 16) | (2 << 8) | 0

nf_status = C.c_int
nf_provider = C.c_void_p
nf_buffer = C.c_void_p


class nf_tensor_desc(C.Structure):
    _fields_ = [
        ("dtype", C.c_int),
        ("ndim", C.c_uint32),
        ("shape", C.c_uint64 * NF_MAX_DIMS),
        ("strides", C.c_uint64 * NF_MAX_DIMS),
        ("size_bytes", C.c_uint64),
    ]


class nf_buffer_info(C.Structure):
    _fields_ = [
        ("desc", nf_tensor_desc),
        ("domain", C.c_int),
        ("offset_bytes", C.c_uint64),
        ("share_token", C.c_uint64),
        ("refcount", C.c_uint32),
        ("_reserved", C.c_uint32),
    ]


RETAIN_FN = C.CFUNCTYPE(C.c_uint32, nf_buffer)
RELEASE_FN = C.CFUNCTYPE(C.c_uint32, nf_buffer)
MAP_FN = C.CFUNCTYPE(nf_status, nf_buffer, C.POINTER(C.c_void_p))
UNMAP_FN = C.CFUNCTYPE(nf_status, nf_buffer)
CACHE_SYNC_FN = C.CFUNCTYPE(nf_status, nf_buffer, C.c_int, C.c_uint64, C.c_uint64)
GET_INFO_FN = C.CFUNCTYPE(nf_status, nf_buffer, C.POINTER(nf_buffer_info))
EXPORT_FN = C.CFUNCTYPE(nf_status, nf_buffer, C.POINTER(C.c_uint64), C.POINTER(C.c_int))
IMPORT_FN = C.CFUNCTYPE(nf_status, nf_provider, C.c_uint64, C.c_int, C.POINTER(nf_tensor_desc),
                        C.POINTER(nf_buffer))


class nf_buffer_ops(C.Structure):
    _fields_ = [
        ("retain", RETAIN_FN),
        ("release", RELEASE_FN),
        ("map", MAP_FN),
        ("unmap", UNMAP_FN),
        ("cache_sync", CACHE_SYNC_FN),
        ("get_info", GET_INFO_FN),
        ("export_handle", EXPORT_FN),
        ("import_handle", IMPORT_FN),
    ]


GET_NAME_FN = C.CFUNCTYPE(C.c_char_p, nf_provider)
GET_ABI_FN = C.CFUNCTYPE(C.c_uint32, nf_provider)
INIT_FN = C.CFUNCTYPE(nf_status, nf_provider)
SHUTDOWN_FN = C.CFUNCTYPE(None, nf_provider)
BUF_ALLOC_FN = C.CFUNCTYPE(nf_status, nf_provider, C.POINTER(nf_tensor_desc), C.POINTER(nf_buffer))
BUF_FREE_FN = C.CFUNCTYPE(None, nf_provider, nf_buffer)
BUF_MAP_FN = C.CFUNCTYPE(nf_status, nf_provider, nf_buffer, C.POINTER(C.c_void_p))
BUF_UNMAP_FN = C.CFUNCTYPE(nf_status, nf_provider, nf_buffer)
DISPATCH_FN = C.CFUNCTYPE(nf_status, nf_provider, C.c_char_p, C.POINTER(nf_buffer), C.c_uint32,
                          C.POINTER(nf_buffer), C.c_uint32)
SYNC_FN = C.CFUNCTYPE(nf_status, nf_provider)


class nf_provider_vtable(C.Structure):
    _fields_ = [
        ("get_name", GET_NAME_FN),
        ("get_abi_version", GET_ABI_FN),
        ("init", INIT_FN),
        ("shutdown", SHUTDOWN_FN),
        ("buffer_alloc", BUF_ALLOC_FN),
        ("buffer_free", BUF_FREE_FN),
        ("buffer_map", BUF_MAP_FN),
        ("buffer_unmap", BUF_UNMAP_FN),
        ("dispatch", DISPATCH_FN),
        ("synchronize", SYNC_FN),
    ]


class nf_buffer_alloc_request(C.Structure):
    _fields_ = [
        ("desc", nf_tensor_desc),
        ("preferred", C.c_int),
        ("flags", C.c_uint32),
        ("_reserved", C.c_uint32),
    ]


MEM_ALLOC_FN = C.CFUNCTYPE(nf_status, nf_provider, C.POINTER(nf_buffer_alloc_request),
                           C.POINTER(nf_buffer_ops), C.POINTER(nf_buffer))
MEM_IMPORT_FN = C.CFUNCTYPE(nf_status, nf_provider, C.c_uint64, C.c_int, C.POINTER(nf_tensor_desc),
                            C.POINTER(nf_buffer_ops), C.POINTER(nf_buffer))
MEM_CAN_IMPORT_FN = C.CFUNCTYPE(nf_status, nf_provider, C.c_int)


class nf_provider_mem_vtable(C.Structure):
    _fields_ = [
        ("alloc", MEM_ALLOC_FN),
        ("import_buffer", MEM_IMPORT_FN),
        ("can_import", MEM_CAN_IMPORT_FN),
    ]


class nf_task_desc(C.Structure):
    _fields_ = [
        ("op_name", C.c_char * NF_MAX_OP_NAME),
        ("inputs", nf_buffer * NF_MAX_TASK_INPUTS),
        ("input_ops", nf_buffer_ops * NF_MAX_TASK_INPUTS),
        ("n_inputs", C.c_uint32),
        ("outputs", nf_buffer * NF_MAX_TASK_OUTPUTS),
        ("output_ops", nf_buffer_ops * NF_MAX_TASK_OUTPUTS),
        ("n_outputs", C.c_uint32),
        ("output_descs", nf_tensor_desc * NF_MAX_TASK_OUTPUTS),
        ("affinity", C.c_int),
        ("priority", C.c_int),
        ("flags", C.c_uint32),
        ("user_data", C.c_void_p),
        ("push_constants_size", C.c_uint32),
        ("push_constants", C.c_uint8 * NF_MAX_PUSH_CONSTANTS),
    ]


class nf_push_constants(C.Structure):
    """48-byte block at nf_task_desc.push_constants (metal_provider.mm:70-83)."""
    _fields_ = [
        ("seq_len", C.c_uint32), ("n_heads", C.c_uint32), ("head_dim", C.c_uint32),
        ("epsilon", C.c_float), ("theta", C.c_float),
        ("M", C.c_uint32), ("N", C.c_uint32), ("K", C.c_uint32),
        ("step_idx", C.c_uint32), ("max_seq_len", C.c_uint32), ("window_size", C.c_uint32),
        ("_pad1", C.c_uint32),
    ]


class nf_driver_caps(C.Structure):
    _fields_ = [
        ("max_concurrent", C.c_uint32),
        ("memory_bytes", C.c_uint64),
        ("flops", C.c_uint64),
        ("supported_dtypes", C.c_uint32),
        ("flags", C.c_uint32),
    ]


nf_completion_token = C.c_void_p
DDI_DISPATCH_FN = C.CFUNCTYPE(nf_status, nf_provider, C.c_char_p, C.POINTER(nf_buffer), C.c_uint32,
                              C.POINTER(nf_buffer), C.c_uint32, C.POINTER(nf_completion_token))
DDI_WAIT_FN = C.CFUNCTYPE(nf_status, nf_provider, nf_completion_token, C.c_uint64)
DDI_POLL_FN = C.CFUNCTYPE(nf_status, nf_provider, nf_completion_token)
DDI_CAPS_FN = C.CFUNCTYPE(nf_status, nf_provider, C.POINTER(nf_driver_caps))


class nf_ddi_vtable(C.Structure):
    _fields_ = [
        ("dispatch_async", DDI_DISPATCH_FN),
        ("wait_completion", DDI_WAIT_FN),
        ("poll_completion", DDI_POLL_FN),
        ("query_caps", DDI_CAPS_FN),
    ]


class nf_hip_plan(C.Structure):
    _fields_ = [
        ("kernel", C.c_char * 64),
        ("M", C.c_uint32), ("N", C.c_uint32), ("K", C.c_uint32),
        ("count", C.c_uint64),
        ("weight_bytes", C.c_uint64),
        ("act_bytes", C.c_uint64),
        ("out_bytes", C.c_uint64),
        ("flops", C.c_uint64),
    ]


def check_layout() -> None:
    """Assert the byte layout pinned by the reference's static_asserts."""
    assert C.sizeof(nf_tensor_desc) == 144
    assert C.sizeof(nf_buffer_info) == 176
    assert C.sizeof(nf_buffer_alloc_request) == 160
    assert C.sizeof(nf_task_desc) == 3056
    assert C.sizeof(nf_driver_caps) == 32
    assert C.sizeof(nf_push_constants) == 48
    assert nf_task_desc.inputs.offset == 64
    assert nf_task_desc.push_constants_size.offset == 2984
    assert nf_task_desc.push_constants.offset == 2988
    assert nf_push_constants.M.offset == 20
    assert nf_push_constants.N.offset == 24
    assert nf_push_constants.K.offset == 28


def make_desc(dtype: int, size_bytes: int, shape=None) -> nf_tensor_desc:
    """1-D descriptor the way the reference's tests build them
    (dequant_test.cpp:46-53): shape[0] = size_bytes unless a shape is given."""
    d = nf_tensor_desc()
    d.dtype = dtype
    if shape:
        d.ndim = len(shape)
        for i, s in enumerate(shape):
            d.shape[i] = int(s)
    else:
        d.ndim = 1
        d.shape[0] = int(size_bytes)
    d.size_bytes = int(size_bytes)
    return d
