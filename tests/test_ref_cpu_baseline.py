"""The CPU baseline bench.py times is the reference's own CPU path.

oracle/_ref/libnfref_cpu_{release,v3}.so are built by `make -C oracle ref`
from the reference's tests/driver/dequant_test.cpp (its ref_dequant_q4_0 /
ref_dequant_q8_0 and f16_to_f32, lines 77-128) plus the test's naive fp32
loop (lines 313-319).  Before its time is reported beside the GPU, it must
compute what the oracle computes: the same dequantized weights and the same
sequential-k fp32 sums, so the Release build (no FMA contraction on
x86-64 without -march) matches the oracle bit for bit, and the x86-64-v3
build (g++ may contract a*b+c into one FMA) within the fp32 rounding bound.
Skipped where the reference tree was not present to build them.
"""
import ctypes as C
from pathlib import Path

import numpy as np
import pytest

from neurofabric_amd import synthetic as syn
from oracle import oracle as orc

REF = Path(__file__).resolve().parents[1] / "oracle" / "_ref"


def _lib(variant):
    p = REF / f"libnfref_cpu_{variant}.so"
    if not p.exists():
        pytest.skip(f"{p.name} not built (needs the reference sources)")
    L = C.CDLL(str(p))
    L.nfref_cpu_fused.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p] + [C.c_uint32] * 6
    L.nfref_cpu_fused.restype = C.c_int
    return L


def _run(L, fmt, A, W, M, N, K, threads=1, cols=None):
    n0, n1 = cols or (0, N)
    out = np.zeros((M, N), np.float32)
    assert L.nfref_cpu_fused(0 if fmt == "q4_0" else 1, A.ctypes.data, W.ctypes.data, out.ctypes.data, M, N, K,
                             n0, n1, threads) == 0
    return out


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("M,N,K", [(1, 5632, 2048), (3, 70, 96), (4, 8, 32)])
def test_reference_release_build_matches_oracle_bitwise(fmt, M, N, K):
    L = _lib("release")
    W = syn.weights(fmt, N, K, seed=N + K)
    A = syn.activations(M, K, seed=M)
    got = _run(L, fmt, A, W, M, N, K, threads=3)
    want = orc.fused(A, W, fmt, M, N, K)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
def test_reference_v3_build_within_fp32_rounding(fmt):
    L = _lib("v3")
    if "avx2" not in Path("/proc/cpuinfo").read_text():
        pytest.skip("host CPU lacks AVX2")
    M, N, K = 2, 300, 2048
    W = syn.weights(fmt, N, K, seed=5)
    A = syn.activations(M, K, seed=6)
    got = _run(L, fmt, A, W, M, N, K, threads=4)
    want = orc.fused(A, W, fmt, M, N, K)
    # |fl(sum) - sum| <= K * u * sum |a_k w_k| for either rounding sequence
    deq = orc.dequant(W, fmt, N * K).reshape(N, K).astype(np.float64)
    bound = 2 * K * 2.0 ** -24 * (np.abs(A.astype(np.float64)) @ np.abs(deq).T)
    assert np.all(np.abs(got.astype(np.float64) - want) <= bound)


def test_reference_rows_window_and_rejects_bad_args():
    L = _lib("release")
    M, N, K = 1, 64, 64
    W = syn.weights("q4_0", N, K, seed=1)
    A = syn.activations(M, K, seed=2)
    got = _run(L, "q4_0", A, W, M, N, K, cols=(10, 20))
    want = orc.fused(A, W, "q4_0", M, N, K)
    assert np.array_equal(got[:, 10:20], want[:, 10:20]) and not got[:, :10].any() and not got[:, 20:].any()
    out = np.zeros(N, np.float32)
    assert L.nfref_cpu_fused(0, A.ctypes.data, W.ctypes.data, out.ctypes.data, 1, N, 48, 0, N, 1) == -1  # K % 32
    assert L.nfref_cpu_fused(2, A.ctypes.data, W.ctypes.data, out.ctypes.data, 1, N, K, 0, N, 1) == -1  # format
