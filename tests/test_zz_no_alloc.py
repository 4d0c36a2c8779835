"""nf_hip_fused_linear_noalloc against dispatch(), through the C ABI.

The no-allocation entry point runs the fused dequant + linear on raw device
pointers with its split-K scratch in a static device array.  Each case runs
the same inputs through vtable dispatch (provider workspace) and through the
entry point, twice in a row with the second call on a smaller input (the
static array keeps the first call's partials and counters), and checks both
against each other and against the CPU oracle within max relative error
1e-3 (tests/helpers.py).  Shapes cover every kernel family the planner
picks: the decode GEMV, the small-batch MFMA kernel with K split across
workgroups (partials and counters in the scratch), the tiled fp16 GEMM whose
K split would need more partials than the scratch holds (runs with fewer
splits), the f32 tiled GEMM with a K split, and the flat-index kernel for
K % 32 != 0.
"""
import ctypes as C

import numpy as np
import pytest

from helpers import assert_close
from neurofabric_amd import abi
from neurofabric_amd import synthetic as syn

pytestmark = pytest.mark.gpu

QDT = {"q4_0": abi.NF_DTYPE_Q4_0, "q8_0": abi.NF_DTYPE_Q8_0}


def _entry(provider):
    fn = provider.lib.nf_hip_fused_linear_noalloc
    fn.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_bool,
                   C.c_void_p]
    fn.restype = C.c_int
    return fn


def _one(provider, fmt, M, N, K, f16, seed):
    """(noalloc result, dispatch result, oracle) for one shape."""
    adt = abi.NF_DTYPE_F16 if f16 else abi.NF_DTYPE_F32
    npt = np.float16 if f16 else np.float32
    W = syn.weights(fmt, N, K, seed=seed) if K % 32 == 0 else syn.weights(fmt, 1, (N * K + 31) // 32 * 32, seed=seed)
    A = syn.activations(M, K, seed=seed + 1, dtype=npt)
    a = provider.alloc_array(A, adt)
    w = provider.alloc_array(W, QDT[fmt])
    c_disp = provider.alloc(adt, M * N * A.itemsize)
    c_noal = provider.alloc(adt, M * N * A.itemsize)
    try:
        provider.dispatch(f"dequant_{fmt}_linear" + ("_f16" if f16 else ""), [a, w], [c_disp], M, N, K)
        provider.synchronize()
        st = _entry(provider)(QDT[fmt], a.device_ptr(), w.device_ptr(), c_noal.device_ptr(), M, N, K, f16,
                              provider.stream())
        assert st == abi.NF_OK, provider.last_error()
        provider.synchronize()
        got = c_noal.download(npt).reshape(M, N).astype(np.float32)
        disp = c_disp.download(npt).reshape(M, N).astype(np.float32)
    finally:
        for b in (a, w, c_disp, c_noal):
            b.release()
    cols = (0, N) if N <= 1024 else (N - 512, N)
    ref = orc_fused(A, W, fmt, M, N, K, f16, cols)
    return got, disp, ref, cols


def orc_fused(A, W, fmt, M, N, K, f16, cols):
    from oracle import oracle as orc
    ref = orc.fused(A, W, fmt, M, N, K, f16=f16, cols=cols, threads=8)
    return (ref.view(np.float16) if f16 else ref).astype(np.float32)


# (fmt, f16, first shape, second smaller shape): decode GEMV; small-batch MFMA
# with a cross-workgroup K split; tiled fp16 GEMM whose split would need
# 32 MB of partials; the f32 bf16-piece tiled GEMM with its K split (partials
# and counters in the scratch, twice in a row); ragged K on the flat-index
# kernel.
CASES = [
    ("q4_0", False, (1, 5632, 2048), (1, 256, 2048)),
    ("q8_0", True, (16, 4096, 4096), (8, 1024, 4096)),
    ("q4_0", False, (24, 2048, 5632), (5, 300, 1024)),
    ("q4_0", True, (512, 4096, 4096), (256, 1024, 4096)),
    ("q4_0", False, (128, 4096, 4096), (96, 1024, 4096)),
    ("q8_0", False, (3, 70, 96), (2, 33, 48)),
]


@pytest.mark.parametrize("fmt,f16,first,second", CASES, ids=lambda v: str(v))
def test_noalloc_matches_dispatch_twice(provider, fmt, f16, first, second):
    for i, (M, N, K) in enumerate((first, second)):
        print(f"noalloc case {fmt} f16={f16} call {i} shape {M}x{N}x{K}", flush=True)
        got, disp, ref, cols = _one(provider, fmt, M, N, K, f16, seed=M + N + K + i)
        assert_close(got, disp, what=f"noalloc vs dispatch call {i} {M}x{N}x{K}")
        assert_close(got[:, cols[0]:cols[1]], ref[:, cols[0]:cols[1]], what=f"noalloc vs oracle call {i}")


def test_noalloc_rejects_bad_arguments(provider):
    fn = _entry(provider)
    a = provider.alloc(abi.NF_DTYPE_F32, 64 * 4)
    try:
        p = a.device_ptr()
        assert fn(abi.NF_DTYPE_F32, p, p, p, 1, 1, 64, False, None) == abi.NF_ERROR_INVALID_ARG  # dense dtype
        assert fn(abi.NF_DTYPE_Q4_0, None, p, p, 1, 1, 64, False, None) == abi.NF_ERROR_INVALID_ARG
        assert fn(abi.NF_DTYPE_Q4_0, p, p, p, 0, 1, 64, False, None) == abi.NF_ERROR_INVALID_ARG
        assert "noalloc" in provider.last_error()
    finally:
        a.release()
