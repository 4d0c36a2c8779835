"""Python host binding of libnf_plugin_hip.so through its C ABI.

Mirrors how the reference's callers drive a provider
(tests/driver/fused_matmul_test.cpp:108-126, llama_dag_builder.hpp:114-178):
register -> init -> mem alloc -> map/memcpy/unmap -> dispatch with a task
descriptor carrying push constants -> synchronize / cache_sync -> map.
Every call goes through the provider's function tables; there is no other
compute path, and a missing library is an error.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

from . import abi
from .abi import (NF_OK, nf_buffer, nf_buffer_alloc_request, nf_buffer_ops, nf_ddi_vtable,
                  nf_driver_caps, nf_hip_plan, nf_provider_mem_vtable, nf_provider_vtable,
                  nf_push_constants, nf_task_desc, nf_tensor_desc)

_PKG = Path(__file__).resolve().parent
DEFAULT_LIB = _PKG / "_lib" / "libnf_plugin_hip.so"

_DTYPE_NP = {
    abi.NF_DTYPE_F32: np.float32,
    abi.NF_DTYPE_F16: np.float16,
    abi.NF_DTYPE_Q4_0: np.uint8,
    abi.NF_DTYPE_Q8_0: np.uint8,
    abi.NF_DTYPE_U8: np.uint8,
    abi.NF_DTYPE_I32: np.int32,
}


class NfError(RuntimeError):
    def __init__(self, status: int, where: str, detail: str = ""):
        self.status = status
        name = abi.STATUS_NAMES.get(status, str(status))
        super().__init__(f"{where}: {name}" + (f" ({detail})" if detail else ""))


def load_library(path: str | os.PathLike | None = None) -> C.CDLL:
    p = Path(path) if path else DEFAULT_LIB
    if not p.exists():
        raise RuntimeError(
            f"HIP provider library not found at {p}; build it with "
            "`python -m neurofabric_amd.build` (gfx950 kernels are required, there is no fallback)")
    lib = C.CDLL(str(p), mode=C.RTLD_LOCAL)
    lib.nf_plugin_register.argtypes = [C.POINTER(nf_provider_vtable), C.POINTER(C.c_void_p)]
    lib.nf_plugin_register.restype = C.c_int
    lib.nf_plugin_register_mem.argtypes = [C.POINTER(nf_provider_mem_vtable)]
    lib.nf_plugin_register_mem.restype = C.c_int
    lib.nf_plugin_register_ddi.argtypes = [C.POINTER(nf_ddi_vtable)]
    lib.nf_plugin_register_ddi.restype = C.c_int
    lib.nf_hip_last_error.argtypes = []
    lib.nf_hip_last_error.restype = C.c_char_p
    lib.nf_hip_plan_dispatch.argtypes = [C.c_char_p, C.POINTER(nf_tensor_desc), C.c_uint32,
                                         C.POINTER(nf_tensor_desc), C.c_uint32, C.c_void_p,
                                         C.c_uint32, C.POINTER(nf_hip_plan)]
    lib.nf_hip_plan_dispatch.restype = C.c_int
    lib.nf_hip_set_gemv_max_m.argtypes = [C.c_uint32, C.c_uint32]
    lib.nf_hip_set_gemv_max_m.restype = None
    lib.nf_hip_set_gemv_row_limits.argtypes = [C.c_uint32, C.c_uint64]
    lib.nf_hip_set_gemv_row_limits.restype = None
    lib.nf_hip_get_gemv_row_limits.argtypes = [C.POINTER(C.c_uint32), C.POINTER(C.c_uint64)]
    lib.nf_hip_get_gemv_row_limits.restype = None
    lib.nf_hip_get_gemv_max_m.argtypes = [C.POINTER(C.c_uint32), C.POINTER(C.c_uint32)]
    lib.nf_hip_get_gemv_max_m.restype = None
    lib.nf_hip_set_skinny_max_m.argtypes = [C.c_uint32]
    lib.nf_hip_set_skinny_max_m.restype = None
    lib.nf_hip_launch_count.argtypes = [C.c_void_p]
    lib.nf_hip_launch_count.restype = C.c_uint64
    lib.nf_hip_set_gemm_tile.argtypes = [C.c_int32]
    lib.nf_hip_set_gemm_tile.restype = None
    lib.nf_hip_get_gemm_tile.argtypes = []
    lib.nf_hip_get_gemm_tile.restype = C.c_int32
    lib.nf_hip_get_skinny_max_m.argtypes = []
    lib.nf_hip_get_skinny_max_m.restype = C.c_uint32
    lib.nf_hip_diag_stream_read.argtypes = [C.c_void_p, C.c_uint64, C.c_void_p]
    lib.nf_hip_diag_stream_read.restype = C.c_int
    lib.nf_hip_set_skinny_f16_max_k.argtypes = [C.c_uint32]
    lib.nf_hip_set_skinny_f16_max_k.restype = None
    lib.nf_hip_get_skinny_f16_max_k.argtypes = []
    lib.nf_hip_get_skinny_f16_max_k.restype = C.c_uint32
    lib.nf_hip_set_skinny_max_m_f32.argtypes = [C.c_uint32]
    lib.nf_hip_set_skinny_max_m_f32.restype = None
    lib.nf_hip_get_skinny_max_m_f32.argtypes = []
    lib.nf_hip_get_skinny_max_m_f32.restype = C.c_uint32
    lib.nf_hip_get_stream.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
    lib.nf_hip_get_stream.restype = C.c_int
    lib.nf_hip_run_tasks.argtypes = [C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32]
    lib.nf_hip_run_tasks.restype = C.c_int
    lib.nf_hip_buffer_device_ptr.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
    lib.nf_hip_buffer_device_ptr.restype = C.c_int
    for fn in ("nf_hip_buffer_write", "nf_hip_buffer_read"):
        getattr(lib, fn).argtypes = [C.c_void_p, C.c_uint64, C.c_void_p, C.c_uint64]
        getattr(lib, fn).restype = C.c_int
    lib.nf_hip_release_staging.argtypes = [C.c_void_p]
    lib.nf_hip_release_staging.restype = None
    lib.nf_hip_enable_timing.argtypes = [C.c_bool]
    lib.nf_hip_enable_timing.restype = None
    lib.nf_hip_get_timing_count.argtypes = []
    lib.nf_hip_get_timing_count.restype = C.c_uint32
    lib.nf_hip_get_timings_ext.argtypes = [C.c_void_p, C.POINTER(C.c_double), C.POINTER(C.c_uint8),
                                           C.POINTER(C.c_uint32), C.c_uint32]
    lib.nf_hip_get_timings_ext.restype = None
    return lib


def push_constants(M: int = 0, N: int = 0, K: int = 0, **extra) -> bytes:
    pc = nf_push_constants()
    pc.M, pc.N, pc.K = M, N, K
    for k, v in extra.items():
        setattr(pc, k, v)
    return bytes(pc)


class Buffer:
    """One provider buffer plus the nf_buffer_ops the allocator returned."""

    def __init__(self, prov: "Provider", handle: int, ops: nf_buffer_ops, dtype: int, nbytes: int):
        self.prov = prov
        self.handle = C.c_void_p(handle)
        self.ops = ops
        self.dtype = dtype
        self.nbytes = nbytes
        self._released = False

    # -- map / unmap ----------------------------------------------------
    def map(self) -> int:
        ptr = C.c_void_p()
        st = self.ops.map(self.handle, C.byref(ptr))
        self.prov.check(st, "map")
        return ptr.value or 0

    def unmap(self) -> None:
        self.prov.check(self.ops.unmap(self.handle), "unmap")

    def upload(self, data) -> None:
        raw = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        if raw.nbytes > self.nbytes:
            raise ValueError(f"upload of {raw.nbytes} B into a {self.nbytes} B buffer")
        ptr = self.map()
        try:
            C.memmove(ptr, raw.ctypes.data, raw.nbytes)
        finally:
            self.unmap()

    def download(self, dtype=None, count: int | None = None) -> np.ndarray:
        self.cache_sync(abi.NF_CACHE_INVALIDATE)
        dt = np.dtype(dtype or _DTYPE_NP.get(self.dtype, np.uint8))
        n = self.nbytes // dt.itemsize if count is None else count
        out = np.empty(n, dtype=dt)
        ptr = self.map()
        try:
            C.memmove(out.ctypes.data, ptr, out.nbytes)
        finally:
            self.unmap()
        return out

    def write(self, data, offset: int = 0) -> None:
        """nf_hip_buffer_write: one copy from host memory into [offset, offset + nbytes)."""
        raw = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        self.prov.check(self.prov.lib.nf_hip_buffer_write(self.handle, offset, raw.ctypes.data, raw.nbytes),
                        "buffer_write")

    def read(self, dtype=np.uint8, count: int | None = None, offset: int = 0) -> np.ndarray:
        """nf_hip_buffer_read of `count` elements of `dtype` from byte `offset`."""
        dt = np.dtype(dtype)
        n = (self.nbytes - offset) // dt.itemsize if count is None else count
        out = np.empty(n, dtype=dt)
        self.prov.check(self.prov.lib.nf_hip_buffer_read(self.handle, offset, out.ctypes.data, out.nbytes),
                        "buffer_read")
        return out

    def cache_sync(self, op: int = abi.NF_CACHE_INVALIDATE) -> None:
        self.prov.check(self.ops.cache_sync(self.handle, op, 0, 0), "cache_sync")

    def info(self) -> abi.nf_buffer_info:
        inf = abi.nf_buffer_info()
        self.prov.check(self.ops.get_info(self.handle, C.byref(inf)), "get_info")
        return inf

    def device_ptr(self) -> int:
        p = C.c_void_p()
        self.prov.check(self.prov.lib.nf_hip_buffer_device_ptr(self.handle, C.byref(p)), "device_ptr")
        return p.value or 0

    def retain(self) -> int:
        return self.ops.retain(self.handle)

    def release(self) -> int:
        if self._released:
            return 0
        n = self.ops.release(self.handle)
        if n == 0:
            self._released = True
        return n

    def __del__(self):  # best effort; tests release explicitly
        pass


class Provider:
    """register -> init -> alloc/dispatch/synchronize through the vtables."""

    def __init__(self, lib_path=None):
        self.lib = load_library(lib_path)
        self.vt = nf_provider_vtable()
        self.mem = nf_provider_mem_vtable()
        self.ddi = nf_ddi_vtable()
        h = C.c_void_p()
        self.check(self.lib.nf_plugin_register(C.byref(self.vt), C.byref(h)), "nf_plugin_register")
        self.handle = h
        self.check(self.lib.nf_plugin_register_mem(C.byref(self.mem)), "nf_plugin_register_mem")
        self.check(self.lib.nf_plugin_register_ddi(C.byref(self.ddi)), "nf_plugin_register_ddi")
        self._keep = []

    # -- errors ---------------------------------------------------------
    def last_error(self) -> str:
        return (self.lib.nf_hip_last_error() or b"").decode(errors="replace")

    def check(self, st: int, where: str) -> None:
        if st != NF_OK:
            raise NfError(st, where, self.last_error())

    # -- lifecycle ------------------------------------------------------
    @property
    def name(self) -> str:
        return self.vt.get_name(self.handle).decode()

    @property
    def abi_version(self) -> int:
        return self.vt.get_abi_version(self.handle)

    def init(self) -> None:
        self.check(self.vt.init(self.handle), "init")

    def shutdown(self) -> None:
        self.vt.shutdown(self.handle)

    def synchronize(self) -> None:
        self.check(self.vt.synchronize(self.handle), "synchronize")

    def stream(self) -> int:
        s = C.c_void_p()
        self.check(self.lib.nf_hip_get_stream(self.handle, C.byref(s)), "get_stream")
        return s.value or 0

    def caps(self) -> nf_driver_caps:
        c = nf_driver_caps()
        self.check(self.ddi.query_caps(self.handle, C.byref(c)), "query_caps")
        return c

    # -- memory ---------------------------------------------------------
    def alloc(self, dtype: int, nbytes: int, shape=None) -> Buffer:
        req = nf_buffer_alloc_request()
        req.desc = abi.make_desc(dtype, nbytes, shape)
        req.preferred = abi.NF_MEM_DOMAIN_DEVICE
        ops = nf_buffer_ops()
        h = C.c_void_p()
        self.check(self.mem.alloc(self.handle, C.byref(req), C.byref(ops), C.byref(h)), "alloc")
        return Buffer(self, h.value, ops, dtype, nbytes)

    def alloc_array(self, arr: np.ndarray, dtype: int) -> Buffer:
        arr = np.ascontiguousarray(arr)
        b = self.alloc(dtype, arr.nbytes)
        b.upload(arr)
        return b

    # -- dispatch -------------------------------------------------------
    def task(self, op: str, inputs, outputs, M=0, N=0, K=0, pc: bytes | None = None) -> nf_task_desc:
        """A task descriptor as the engine builds it (PipelineEngine.hpp:415-429)."""
        td = nf_task_desc()
        td.op_name = op.encode()
        for i, b in enumerate(inputs):
            td.inputs[i] = b.handle.value
            td.input_ops[i] = b.ops
        td.n_inputs = len(inputs)
        for i, b in enumerate(outputs):
            td.outputs[i] = b.handle.value
            td.output_ops[i] = b.ops
        td.n_outputs = len(outputs)
        td.affinity = abi.NF_AFFINITY_GPU
        raw = pc if pc is not None else (push_constants(M, N, K) if (M or N or K) else b"")
        C.memmove(td.push_constants, raw, len(raw))
        td.push_constants_size = len(raw)
        td.user_data = C.addressof(td)
        return td

    @staticmethod
    def _inputs_ptr(td: nf_task_desc):
        return C.cast(C.addressof(td) + nf_task_desc.inputs.offset, C.POINTER(nf_buffer))

    @staticmethod
    def _outputs_ptr(td: nf_task_desc):
        return C.cast(C.addressof(td) + nf_task_desc.outputs.offset, C.POINTER(nf_buffer))

    def dispatch_task(self, td: nf_task_desc) -> int:
        """Raw vtable dispatch of a prepared descriptor; returns the status."""
        return self.vt.dispatch(self.handle, td.op_name, self._inputs_ptr(td), td.n_inputs,
                                self._outputs_ptr(td), td.n_outputs)

    def dispatch(self, op: str, inputs, outputs, M=0, N=0, K=0, pc: bytes | None = None) -> None:
        td = self.task(op, inputs, outputs, M, N, K, pc)
        self.check(self.dispatch_task(td), f"dispatch {op}")

    def dispatch_bare(self, op: str, inputs, outputs) -> int:
        """Dispatch with plain handle arrays (no task descriptor), the way
        fused_matmul_test.cpp:175-177 calls the dequant ops."""
        ins = (nf_buffer * max(1, len(inputs)))(*[b.handle.value for b in inputs])
        outs = (nf_buffer * max(1, len(outputs)))(*[b.handle.value for b in outputs])
        return self.vt.dispatch(self.handle, op.encode(), ins, len(inputs), outs, len(outputs))

    def run_tasks(self, tasks, repeat: int = 1) -> None:
        """Dispatch a ctypes array of nf_task_desc in order, `repeat` times."""
        self.check(self.lib.nf_hip_run_tasks(self.handle, C.addressof(tasks), len(tasks), repeat),
                   "run_tasks")

    # -- planning (no GPU needed) -------------------------------------------
    def plan(self, op: str, in_descs, out_descs, M=0, N=0, K=0, pc: bytes | None = None) -> dict:
        return plan(self.lib, op, in_descs, out_descs, M, N, K, pc)

    # -- per-dispatch GPU timing ring ----------------------------------
    def enable_timing(self, on: bool = True) -> None:
        """Record a HIP-event pair around every dispatch on the provider
        stream (1024-entry ring, cleared when enabled)."""
        self.lib.nf_hip_enable_timing(bool(on))

    def timings(self):
        """[(op_name, gpu_ms, out_dtype, elems)] for the recorded dispatches,
        oldest first (waits for the last recorded dispatch to finish)."""
        n = self.lib.nf_hip_get_timing_count()
        names = (C.c_char * 64 * max(1, n))()
        ms = (C.c_double * max(1, n))()
        dts = (C.c_uint8 * max(1, n))()
        els = (C.c_uint32 * max(1, n))()
        self.lib.nf_hip_get_timings_ext(names, ms, dts, els, n)
        return [(bytes(names[i]).split(b"\0", 1)[0].decode(), ms[i], dts[i], els[i]) for i in range(n)]

    # -- crossover ------------------------------------------------------
    def set_gemv_max_m(self, f32: int, f16: int) -> None:
        self.lib.nf_hip_set_gemv_max_m(f32, f16)

    def set_gemv_row_limits(self, m2_max_stage_bytes: int, m34_max_weight_bytes: int) -> None:
        """The GEMV takes two rows only while their activation stage is at
        most m2_max_stage_bytes, three or four only while the weights are at
        most m34_max_weight_bytes."""
        self.lib.nf_hip_set_gemv_row_limits(m2_max_stage_bytes, m34_max_weight_bytes)

    def get_gemv_row_limits(self) -> tuple:
        a, b = C.c_uint32(), C.c_uint64()
        self.lib.nf_hip_get_gemv_row_limits(C.byref(a), C.byref(b))
        return a.value, b.value

    def set_skinny_max_m(self, f16: int, f32: int | None = None, f16_max_k: int | None = None) -> None:
        """Largest M on the small-batch kernel for f16 (and, if given, f32)
        activations; f16_max_k: longest rows it takes at M > 4 (f16)."""
        self.lib.nf_hip_set_skinny_max_m(f16)
        if f32 is not None:
            self.lib.nf_hip_set_skinny_max_m_f32(f32)
        if f16_max_k is not None:
            self.lib.nf_hip_set_skinny_f16_max_k(f16_max_k)

    def release_staging(self) -> None:
        self.lib.nf_hip_release_staging(self.handle)

    def launch_count(self) -> int:
        """Launches enqueued so far (a merged GEMV group counts once)."""
        return int(self.lib.nf_hip_launch_count(self.handle))

    def set_gemm_tile(self, tile: int) -> None:
        """-1: register-dequantizing GEMM kernels picked by M (default); 0..6:
        LDS-staged tile shapes; 7: the one-wave-per-SIMD register kernel;
        8 / 9 / 10: the two-wave kernel with 128 / 64 / 32-row waves wherever
        it applies (K % 128 == 0; 8: Q4_0 only); 11: its 128-row waves on
        128-column tiles (Q4_0 only); with f32 activations 8 / 9 force the
        bf16-piece kernel's 128- / 64-row waves."""
        self.lib.nf_hip_set_gemm_tile(tile)

    def get_gemm_tile(self) -> int:
        return int(self.lib.nf_hip_get_gemm_tile())

    def get_skinny_max_m(self) -> int:
        return self.lib.nf_hip_get_skinny_max_m()

    def diag_stream_read(self, dev_ptr: int, nbytes: int) -> None:
        """Enqueue the launch-floor calibration read of `nbytes` at device
        address `dev_ptr` on the provider stream (an empty kernel for < 16)."""
        self.check(self.lib.nf_hip_diag_stream_read(C.c_void_p(dev_ptr), nbytes, C.c_void_p(self.stream())),
                   "nf_hip_diag_stream_read")

    def get_skinny_max_m_f32(self) -> int:
        return self.lib.nf_hip_get_skinny_max_m_f32()

    def get_tuning(self) -> tuple:
        """Every switch point and the GEMM kernel choice, for set_tuning."""
        return (self.get_gemv_max_m(), self.get_skinny_max_m(), self.get_skinny_max_m_f32(), self.get_gemm_tile(),
                int(self.lib.nf_hip_get_skinny_f16_max_k()), self.get_gemv_row_limits())

    def set_tuning(self, t: tuple) -> None:
        self.set_gemv_max_m(*t[0])
        self.set_skinny_max_m(t[1], t[2], t[4])
        self.set_gemm_tile(t[3])
        self.set_gemv_row_limits(*t[5])

    def get_gemv_max_m(self):
        a, b = C.c_uint32(), C.c_uint32()
        self.lib.nf_hip_get_gemv_max_m(C.byref(a), C.byref(b))
        return a.value, b.value


def plan(lib: C.CDLL, op: str, in_descs, out_descs, M=0, N=0, K=0, pc: bytes | None = None) -> dict:
    ins = (nf_tensor_desc * max(1, len(in_descs)))(*in_descs)
    outs = (nf_tensor_desc * max(1, len(out_descs)))(*out_descs)
    raw = pc if pc is not None else (push_constants(M, N, K) if (M or N or K) else b"")
    buf = C.create_string_buffer(raw, max(1, len(raw)))
    out = nf_hip_plan()
    st = lib.nf_hip_plan_dispatch(op.encode(), ins, len(in_descs), outs, len(out_descs),
                                  C.cast(buf, C.c_void_p) if raw else None, len(raw), C.byref(out))
    if st != NF_OK:
        raise NfError(st, f"plan {op}", (lib.nf_hip_last_error() or b"").decode())
    return {"kernel": out.kernel.decode(), "M": out.M, "N": out.N, "K": out.K, "count": out.count,
            "weight_bytes": out.weight_bytes, "act_bytes": out.act_bytes,
            "out_bytes": out.out_bytes, "flops": out.flops}
