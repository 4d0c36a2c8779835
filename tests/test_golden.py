"""The committed golden fixtures of tests/golden/ (written by
tests/golden/make_golden.py): the reference tests' known-answer blocks, small
fused dequant+linear cases with expected outputs, and SHA-256 of the
synthetic config inputs.

CPU tests: the oracle reproduces every fixture bit for bit, and the
synthetic generator reproduces every hash.  GPU tests: the provider, through
the C ABI, reproduces the dequant fixtures bit for bit and the linear
fixtures within the 1e-3 tolerance.
"""
import json
from pathlib import Path

import numpy as np
import pytest

from helpers import assert_close
from neurofabric_amd import abi
from neurofabric_amd import synthetic as syn

GOLDEN = Path(__file__).resolve().parent / "golden"
KA = ["q4_dt", "q8_dt", "q4_pipe", "q4_f16t"]
FMT = {"q4_dt": "q4_0", "q8_dt": "q8_0", "q4_pipe": "q4_0", "q4_f16t": "q4_0"}
QDT = {"q4_0": abi.NF_DTYPE_Q4_0, "q8_0": abi.NF_DTYPE_Q8_0}


def known():
    return np.load(GOLDEN / "known_answer_blocks.npz")


def small_cases():
    z = np.load(GOLDEN / "small_linear_cases.npz")
    n = len([k for k in z.files if k.endswith("_meta")])
    out = []
    for i in range(n):
        M, N, K, f16, q = (int(v) for v in z[f"c{i}_meta"])
        out.append(("q4_0" if q == 0 else "q8_0", bool(f16), M, N, K, z[f"c{i}_A"], z[f"c{i}_W"], z[f"c{i}_C"]))
    return out


# ---- CPU -------------------------------------------------------------------

@pytest.mark.parametrize("name", KA)
def test_oracle_reproduces_known_answer_blocks(oracle_mod, name):
    z = known()
    blocks, fmt = z[f"{name}_blocks"], FMT[name]
    n = z[f"{name}_f32"].size
    assert np.array_equal(oracle_mod.dequant(blocks, fmt, n).view(np.uint32), z[f"{name}_f32"].view(np.uint32))
    assert np.array_equal(np.asarray(oracle_mod.dequant(blocks, fmt, n, f16=True)).view(np.uint16), z[f"{name}_f16bits"])


def test_known_answer_closed_form():
    """Independent of the oracle: the Q4_0 fixture values are d * (nibble - 8)
    with nibble i < 16 the low half of qs[i] and i >= 16 the high half of
    qs[i - 16] (dequant_test.cpp:112-120)."""
    z = known()
    raw = z["q4_dt_blocks"].reshape(-1, 18)
    d = raw[:, :2].copy().view(np.float16).astype(np.float32).reshape(-1)
    qs = raw[:, 2:]
    nib = np.concatenate([qs & 0xF, qs >> 4], axis=1).astype(np.float32)
    assert np.array_equal(z["q4_dt_f32"].reshape(-1, 32), d[:, None] * (nib - 8))
    raw8 = z["q8_dt_blocks"].reshape(-1, 34)
    d8 = raw8[:, :2].copy().view(np.float16).astype(np.float32).reshape(-1)
    assert np.array_equal(z["q8_dt_f32"].reshape(-1, 32), d8[:, None] * raw8[:, 2:].view(np.int8).astype(np.float32))


def test_oracle_reproduces_pipeline_matmul(oracle_mod):
    z = known()
    A = z["q4_pipe_f32"].reshape(1, 32)
    assert np.array_equal(oracle_mod.linear_f32(A, z["q4_pipe_B"], 1, 4, 32), z["q4_pipe_C"])


@pytest.mark.parametrize("i", range(12))
def test_oracle_reproduces_small_linear_cases(oracle_mod, i):
    fmt, f16, M, N, K, A, W, C = small_cases()[i]
    got = np.asarray(oracle_mod.fused(A, W, fmt, M, N, K, f16=f16))
    assert np.array_equal(got.view(np.uint8), C.view(np.uint8))


def test_synthetic_inputs_reproduce_hashes():
    h = json.loads((GOLDEN / "synthetic_sha256.json").read_text())
    for label, e in h["weights"].items():
        assert syn.sha256(syn.weights(e["fmt"], e["N"], e["K"], seed=e["N"] * 7 + e["K"])) == e["sha256"], label
    for label, e in h["activations"].items():
        dt = np.float16 if e["dtype"] == "float16" else np.float32
        assert syn.sha256(syn.activations(e["M"], e["K"], seed=e["K"], dtype=dt)) == e["sha256"], label


# ---- GPU -------------------------------------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize("name", KA)
@pytest.mark.parametrize("f16", [False, True], ids=["f32", "f16"])
def test_gpu_known_answer_blocks(provider, name, f16):
    z = known()
    fmt = FMT[name]
    n = z[f"{name}_f32"].size
    w = provider.alloc_array(z[f"{name}_blocks"], QDT[fmt])
    out = provider.alloc(abi.NF_DTYPE_F16 if f16 else abi.NF_DTYPE_F32, n * (2 if f16 else 4))
    provider.dispatch(f"dequant_{fmt}" + ("_f16" if f16 else ""), [w], [out])
    provider.synchronize()
    got = out.download(np.uint16 if f16 else np.uint32)
    w.release()
    out.release()
    want = z[f"{name}_f16bits"] if f16 else z[f"{name}_f32"].view(np.uint32)
    assert np.array_equal(got, want)


@pytest.mark.gpu
def test_gpu_pipeline_matmul(provider):
    """dequant_test.cpp:400-460: dequant one block, then `linear` 1x32 @ 32x4."""
    z = known()
    w = provider.alloc_array(z["q4_pipe_blocks"], abi.NF_DTYPE_Q4_0)
    a = provider.alloc(abi.NF_DTYPE_F32, 32 * 4)
    b = provider.alloc_array(z["q4_pipe_B"], abi.NF_DTYPE_F32)
    c = provider.alloc(abi.NF_DTYPE_F32, 4 * 4)
    provider.dispatch("dequant_q4_0", [w], [a])
    provider.dispatch("linear", [a, b], [c], 1, 4, 32)
    provider.synchronize()
    got = c.download(np.float32).reshape(1, 4)
    for x in (w, a, b, c):
        x.release()
    assert_close(got, z["q4_pipe_C"])


@pytest.mark.gpu
@pytest.mark.parametrize("i", range(12))
def test_gpu_small_linear_cases(provider, i):
    fmt, f16, M, N, K, A, W, C = small_cases()[i]
    adt = abi.NF_DTYPE_F16 if f16 else abi.NF_DTYPE_F32
    a = provider.alloc_array(A, adt)
    w = provider.alloc_array(W, QDT[fmt])
    c = provider.alloc(adt, M * N * (2 if f16 else 4))
    provider.dispatch(f"dequant_{fmt}_linear" + ("_f16" if f16 else ""), [a, w], [c], M, N, K)
    provider.synchronize()
    got = c.download(np.float16 if f16 else np.float32).reshape(M, N)
    for x in (a, w, c):
        x.release()
    want = C.view(np.float16) if f16 else C
    assert_close(got.astype(np.float32), want.reshape(M, N).astype(np.float32), what=f"{fmt} f16={f16} {M}x{N}x{K}")
