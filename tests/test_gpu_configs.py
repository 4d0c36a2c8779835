"""Oracle parity at the full BASELINE.json config shapes, through the C ABI.

configs[1] TinyLlama q/o and gate/up at M = 1, 4 and 16; configs[2]
Llama-2-7B prefill at M = 512 (the K-split grid of the 4096-row outputs) and
M = 2048 (the non-split tiled GEMM grid); configs[3] Llama-3-8B Q8_0 q/o,
FFN shapes and the 128256 x 4096 lm_head at M = 1, 16 and 64 (f32
activations: GEMV, small-batch kernel), and the FFN shapes through the f32
families the switch points do not pick;
configs[4] the Llama-70B FFN pair at every M of the crossover sweep, through
the kernel the switch points select and through each kernel family forced.

The oracle (the restated reference dequant + sequential-k loop,
dequant_test.cpp:112-128, 313-319) computes whole output columns, so a
window of columns is exact for its entries.  Three windows per case: the
first 128 columns, 128 columns straddling the middle at an offset that is
not a multiple of any tile, and the last 256 (the ragged edge of the row and
tile grids).  Every row of A is checked in each window.  Tolerance: max
relative error 1e-3, mixed and normwise (tests/helpers.py).
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import assert_close
from neurofabric_amd import abi
from neurofabric_amd import synthetic as syn

pytestmark = pytest.mark.gpu

QDT = {"q4_0": abi.NF_DTYPE_Q4_0, "q8_0": abi.NF_DTYPE_Q8_0}


def windows(N):
    mid = N // 2 - 61
    wins = [(0, min(128, N)), (mid, mid + 128), (max(0, N - 256), N)]
    return sorted(set(wins))


class Weights:
    """Device copies of config weights, uploaded once per module."""

    def __init__(self, provider):
        self.provider = provider
        self.host, self.dev = {}, {}

    def get(self, fmt, N, K):
        key = (fmt, N, K)
        if key not in self.dev:
            self.host[key] = syn.weights(fmt, N, K, seed=N * 3 + K)
            self.dev[key] = self.provider.alloc_array(self.host[key], QDT[fmt])
        return self.host[key], self.dev[key]

    def release(self):
        for b in self.dev.values():
            b.release()
        self.dev.clear()
        self.host.clear()


@pytest.fixture(scope="module")
def weights(provider):
    w = Weights(provider)
    yield w
    w.release()


def planned_kernel(provider, fmt, M, N, K, f16):
    adt = abi.NF_DTYPE_F16 if f16 else abi.NF_DTYPE_F32
    elt = 2 if f16 else 4
    op = f"dequant_{fmt}_linear" + ("_f16" if f16 else "")
    bb = syn.BLOCK_BYTES[fmt]
    return provider.plan(op, [abi.make_desc(adt, M * K * elt), abi.make_desc(QDT[fmt], N * K // 32 * bb)],
                         [abi.make_desc(adt, M * N * elt)], M, N, K)["kernel"]


def check_config(provider, oracle_mod, weights, fmt, M, N, K, f16, seed):
    Wh, w = weights.get(fmt, N, K)
    adt = abi.NF_DTYPE_F16 if f16 else abi.NF_DTYPE_F32
    A = syn.activations(M, K, seed=seed, dtype=np.float16 if f16 else np.float32)
    a = provider.alloc_array(A, adt)
    c = provider.alloc(adt, M * N * (2 if f16 else 4))
    try:
        provider.dispatch(f"dequant_{fmt}_linear" + ("_f16" if f16 else ""), [a, w], [c], M, N, K)
        provider.synchronize()
        got = c.download(np.float16 if f16 else np.float32).reshape(M, N).astype(np.float32)
    finally:
        a.release()
        c.release()
    kernel = planned_kernel(provider, fmt, M, N, K, f16)
    for n0, n1 in windows(N):
        ref = oracle_mod.fused(A, Wh, fmt, M, N, K, f16=f16, cols=(n0, n1), threads=16)
        ref = (ref.view(np.float16) if f16 else ref)[:, n0:n1].astype(np.float32)
        assert_close(got[:, n0:n1], ref, what=f"{kernel} {fmt} {M}x{N}x{K} cols {n0}:{n1}")
    return kernel


def _force(provider, path):
    if path == "gemv":
        provider.set_gemv_max_m(1 << 30, 1 << 30)
        provider.set_gemv_row_limits((1 << 32) - 1, (1 << 64) - 1)
    elif path == "skinny":
        provider.set_gemv_max_m(0, 0)
        provider.set_skinny_max_m(1 << 30, 1 << 30, 1 << 30)
    else:
        provider.set_gemv_max_m(0, 0)
        provider.set_skinny_max_m(0, 0)


class forced:
    def __init__(self, provider, path):
        self.provider, self.path = provider, path

    def __enter__(self):
        self.old = self.provider.get_tuning()
        if self.path:
            _force(self.provider, self.path)
        return self

    def __exit__(self, *exc):
        self.provider.set_tuning(self.old)


# ---- TinyLlama decode projections not covered elsewhere ----------------

@pytest.mark.parametrize("M", [1, 4, 16])
@pytest.mark.parametrize("NK", [(2048, 2048), (5632, 2048)], ids=["q_o", "gate_up"])
def test_config1_q_o_gate_up(provider, oracle_mod, weights, M, NK):
    check_config(provider, oracle_mod, weights, "q4_0", M, *NK, f16=False, seed=M + NK[0])


# ---- Llama-2-7B prefill at M = 512 and 2048 ----------------------------

@pytest.mark.parametrize("NK", [(4096, 4096), (11008, 4096), (4096, 11008)], ids=["qkvo", "gate_up", "down"])
def test_config2_prefill_m512(provider, oracle_mod, weights, NK):
    k = check_config(provider, oracle_mod, weights, "q4_0", 512, *NK, f16=True, seed=NK[0] + 5)
    assert k.startswith("gemm_mfma"), k


@pytest.mark.parametrize("NK", [(4096, 4096), (11008, 4096), (4096, 11008)], ids=["qkvo", "gate_up", "down"])
def test_config2_prefill_m2048(provider, oracle_mod, weights, NK):
    k = check_config(provider, oracle_mod, weights, "q4_0", 2048, *NK, f16=True, seed=NK[1] + 7)
    assert k.startswith("gemm_mfma"), k


# ---- Llama-3-8B Q8_0 decode ------------------------------------------------

@pytest.mark.parametrize("M", [1, 16, 64])
@pytest.mark.parametrize("NK", [(4096, 4096), (14336, 4096), (4096, 14336), (128256, 4096)],
                         ids=["q_o", "gate_up", "down", "lm_head"])
def test_config3_q8_0_ffn_and_lm_head(provider, oracle_mod, weights, M, NK):
    check_config(provider, oracle_mod, weights, "q8_0", M, *NK, f16=False, seed=M * 5 + NK[0])


@pytest.mark.parametrize("path,M", [("tiled", 1), ("tiled", 16), ("tiled", 40), ("skinny", 64)],
                         ids=lambda v: str(v))
@pytest.mark.parametrize("NK", [(14336, 4096), (4096, 14336)], ids=["gate_up", "down"])
def test_config3_forced_family(provider, oracle_mod, weights, path, M, NK):
    """The f32 families the switch points do not pick at these M: the
    bf16-piece tiled GEMM at small batches, the small-batch kernel at M = 64
    (two launches of 32 rows)."""
    with forced(provider, path):
        kernel = planned_kernel(provider, "q8_0", M, *NK, False)
        want = {"skinny": "skinny_mfma_", "tiled": "gemm_mfma_"}[path]
        assert kernel.startswith(want), f"forced {path} planned {kernel}"
        check_config(provider, oracle_mod, weights, "q8_0", M, *NK, f16=False, seed=7 * M + NK[1])


# ---- Llama-70B FFN crossover sweep ------------------------------------------

C4_SHAPES = [(28672, 8192), (8192, 28672)]
C4_M = [1, 2, 4, 8, 16, 32, 64, 128, 256]


@pytest.mark.parametrize("M", C4_M)
@pytest.mark.parametrize("NK", C4_SHAPES, ids=["gate_up", "down"])
def test_config4_selected_kernel(provider, oracle_mod, weights, M, NK):
    """The kernel the switch points pick at each M of the sweep."""
    check_config(provider, oracle_mod, weights, "q4_0", M, *NK, f16=True, seed=M + NK[1])


# (family, M) pairs where the forced family actually serves the shape: the
# GEMV needs its activation stage (M' x K fp16) within 120 KB of LDS, the
# small-batch kernel takes any M (64 rows per launch), the tiled GEMM any M.
C4_FORCED = [("gemv", 1), ("gemv", 2), ("skinny", 1), ("skinny", 8), ("skinny", 64), ("skinny", 128),
             ("tiled", 1), ("tiled", 16), ("tiled", 64), ("tiled", 256)]


@pytest.mark.parametrize("path,M", C4_FORCED, ids=lambda v: str(v))
@pytest.mark.parametrize("NK", C4_SHAPES, ids=["gate_up", "down"])
def test_config4_forced_family(provider, oracle_mod, weights, path, M, NK):
    with forced(provider, path):
        kernel = planned_kernel(provider, "q4_0", M, *NK, True)
        want = {"gemv": "gemv_", "skinny": "skinny_mfma_", "tiled": "gemm_mfma_"}[path]
        assert kernel.startswith(want), f"forced {path} planned {kernel}"
        check_config(provider, oracle_mod, weights, "q4_0", M, *NK, f16=True, seed=3 * M + NK[0])
