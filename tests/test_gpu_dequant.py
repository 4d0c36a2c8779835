"""Dequantization parity on the GPU (bit-exact), through the C ABI.

Exhaustive over every fp16 scale pattern: Q4_0 x 16 codes and Q8_0 x 256
codes, to f32 (exact products) and to f16 (round-to-nearest-even of the exact
product, subnormals kept), compared bit for bit with the oracle; NaN scales
compared as a class.  Plus the reference tests' own known-answer blocks,
partial (ragged) element counts and a full config-sized weight.
"""
import numpy as np
import pytest

from helpers import assert_bits_equal_f16, assert_bits_equal_f32
from neurofabric_amd import abi
from neurofabric_amd import synthetic as syn

pytestmark = [pytest.mark.gpu, pytest.mark.filterwarnings("ignore::RuntimeWarning")]

ALL_F16 = np.arange(65536, dtype=np.uint32).astype(np.uint16)
QDT = {"q4_0": abi.NF_DTYPE_Q4_0, "q8_0": abi.NF_DTYPE_Q8_0}


def _exhaustive_blocks(fmt):
    if fmt == "q4_0":
        return syn.pack_q4_0(ALL_F16.view(np.float16), np.tile(np.arange(32) % 16, (65536, 1)))
    d = np.repeat(ALL_F16, 8)
    return syn.pack_q8_0(d.view(np.float16), np.tile(np.arange(-128, 128).reshape(8, 32), (65536, 1)))


def _gpu_dequant(provider, blocks, fmt, count, f16, bare=False):
    w = provider.alloc_array(blocks.reshape(-1), QDT[fmt])
    out_dt = abi.NF_DTYPE_F16 if f16 else abi.NF_DTYPE_F32
    out = provider.alloc(out_dt, count * (2 if f16 else 4))
    op = f"dequant_{fmt}" + ("_f16" if f16 else "")
    if bare:
        provider.check(provider.dispatch_bare(op, [w], [out]), op)
    else:
        provider.dispatch(op, [w], [out])
    provider.synchronize()
    got = out.download(np.uint16 if f16 else np.float32)
    w.release()
    out.release()
    return got


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("f16", [False, True], ids=["f32", "f16"])
def test_dequant_exhaustive_scales_and_codes(provider, oracle_mod, fmt, f16):
    blocks = _exhaustive_blocks(fmt)
    count = blocks.shape[0] * 32
    got = _gpu_dequant(provider, blocks, fmt, count, f16)
    want = oracle_mod.dequant(blocks, fmt, count, f16=f16)
    if f16:
        assert_bits_equal_f16(got, want, f"{fmt} f16")
    else:
        assert_bits_equal_f32(got, want, f"{fmt} f32")


def test_dequant_reference_known_answer_blocks(provider, oracle_mod):
    """dequant_test.cpp:155-168 (Q4_0) and :233-239 (Q8_0), scales built with
    the tests' truncating encoder; the reference asserts |gpu - cpu| < 1e-4,
    we assert bit equality."""
    q4, q8 = [], []
    for b in range(8):
        d = np.array([oracle_mod.f32_to_f16_trunc(0.5 + 0.1 * b)], np.uint16).view(np.float16)
        codes = [(j + b) & 0xF for j in range(16)] + [(15 - j + b) & 0xF for j in range(16)]
        q4.append(syn.pack_q4_0(d, np.array(codes)[None, :]))
        d8 = np.array([oracle_mod.f32_to_f16_trunc(0.25 + 0.05 * b)], np.uint16).view(np.float16)
        q8.append(syn.pack_q8_0(d8, (np.arange(32) - 16 + b)[None, :]))
    for fmt, blocks in (("q4_0", np.concatenate(q4)), ("q8_0", np.concatenate(q8))):
        for f16 in (False, True):
            got = _gpu_dequant(provider, blocks, fmt, 256, f16, bare=True)
            want = oracle_mod.dequant(blocks, fmt, 256, f16=f16)
            (assert_bits_equal_f16 if f16 else assert_bits_equal_f32)(got, want, f"{fmt} known answer")


@pytest.mark.parametrize("count", [1, 7, 8, 31, 33, 77, 1000])
def test_dequant_ragged_counts(provider, oracle_mod, count):
    """count = out.size_bytes / element size (metal_provider.mm:2667); a
    trailing partial block and partial 8-element chunks are handled."""
    for fmt in ("q4_0", "q8_0"):
        blocks = syn.weights(fmt, 1, (count + 31) // 32 * 32, seed=count)
        for f16 in (False, True):
            got = _gpu_dequant(provider, blocks, fmt, count, f16)
            want = oracle_mod.dequant(blocks, fmt, count, f16=f16)
            (assert_bits_equal_f16 if f16 else assert_bits_equal_f32)(got, want, f"{fmt} count={count}")


def test_dequant_config0_weight(provider, oracle_mod):
    """The full C0 weight (Q4_0 5632 x 2048), f32 and f16."""
    w = syn.q4_0_weights(5632, 2048, seed=0)
    n = 5632 * 2048
    assert_bits_equal_f32(_gpu_dequant(provider, w, "q4_0", n, False), oracle_mod.dequant(w, "q4_0", n))
    assert_bits_equal_f16(_gpu_dequant(provider, w, "q4_0", n, True), oracle_mod.dequant(w, "q4_0", n, True))


def test_dequant_rejects_short_input(provider):
    w = provider.alloc(abi.NF_DTYPE_Q4_0, 18)
    out = provider.alloc(abi.NF_DTYPE_F32, 64 * 4)  # needs 2 blocks
    st = provider.dispatch_bare("dequant_q4_0", [w], [out])
    assert st == abi.NF_ERROR_INVALID_ARG
    w.release()
    out.release()
