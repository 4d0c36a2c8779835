"""Dequantization parity of the other block formats on the GPU, bit-exact,
through the C ABI: dequant_{q4_1,q5_0,q5_1,q2_k,q3_k,q4_k,q5_k,q6_k}[_f16]
(metal_provider.mm:534-894, op names :3159-3176).

Against the oracle (itself pinned to the reference's CPU dequantizers,
kquant_dequant_test.cpp:118-224): seeded random blocks at several scales,
the reference test's own input pattern, every fp16 scale pattern, ragged
counts (partial blocks, partial 8-element chunks, partial workgroups),
dequant_q3_k_f16's read past its last block, inputs and outputs at
unaligned addresses, and a full 7B-shape weight.
"""
import ctypes as C

import numpy as np
import pytest

from helpers import assert_bits_equal_f16, assert_bits_equal_f32
from neurofabric_amd import abi
from neurofabric_amd import synthetic as syn
from neurofabric_amd.plugin import Buffer

pytestmark = [pytest.mark.gpu, pytest.mark.filterwarnings("ignore::RuntimeWarning")]

FMTS = ["q4_1", "q5_0", "q5_1", "q2_k", "q3_k", "q4_k", "q5_k", "q6_k"]
QDT = {"q4_1": abi.NF_DTYPE_Q4_1, "q5_0": abi.NF_DTYPE_Q5_0, "q5_1": abi.NF_DTYPE_Q5_1,
       "q2_k": abi.NF_DTYPE_Q2_K, "q3_k": abi.NF_DTYPE_Q3_K, "q4_k": abi.NF_DTYPE_Q4_K,
       "q5_k": abi.NF_DTYPE_Q5_K, "q6_k": abi.NF_DTYPE_Q6_K}


def _gpu_dequant(provider, blocks, fmt, count, f16):
    w = provider.alloc_array(np.ascontiguousarray(blocks, np.uint8).reshape(-1), QDT[fmt])
    out = provider.alloc(abi.NF_DTYPE_F16 if f16 else abi.NF_DTYPE_F32, count * (2 if f16 else 4))
    provider.dispatch(f"dequant_{fmt}" + ("_f16" if f16 else ""), [w], [out])
    provider.synchronize()
    got = out.download(np.uint16 if f16 else np.float32)
    w.release()
    out.release()
    return got


def _check(got, want, f16, what):
    (assert_bits_equal_f16 if f16 else assert_bits_equal_f32)(got, want, what)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("f16", [False, True], ids=["f32", "f16"])
def test_random_blocks(provider, oracle_mod, fmt, f16):
    """Several workgroups of seeded random blocks at three scale magnitudes."""
    _, be = syn.KQ_GEOM[fmt]
    for seed, scale in ((0, 0.01), (1, 30.0), (2, 2e-6)):
        nb = 4 * 2048 // be + 3
        blocks = syn.kquant_blocks(fmt, nb, seed=seed, scale=scale)
        n = nb * be
        _check(_gpu_dequant(provider, blocks, fmt, n, f16), oracle_mod.dequant(blocks, fmt, n, f16=f16), f16,
               f"{fmt} seed={seed}")


@pytest.mark.parametrize("fmt", FMTS)
def test_any_bytes(provider, oracle_mod, fmt):
    """Uniform random bytes everywhere, fp16 fields included (subnormal,
    Inf and NaN scales); NaN compared as a class."""
    bs, be = syn.KQ_GEOM[fmt]
    raw = np.random.default_rng(5).integers(0, 256, (1024, bs), dtype=np.uint8)
    for f16 in (False, True):
        _check(_gpu_dequant(provider, raw, fmt, 1024 * be, f16), oracle_mod.dequant(raw, fmt, 1024 * be, f16=f16),
               f16, f"{fmt} any bytes f16={f16}")


@pytest.mark.parametrize("fmt", FMTS)
def test_every_scale_pattern(provider, oracle_mod, fmt):
    """Each of the 65536 fp16 bit patterns as the block scale d (random
    codes, other fields random finite)."""
    bs, be = syn.KQ_GEOM[fmt]
    blocks = syn.kquant_blocks(fmt, 65536, seed=9)
    d_off = syn.KQ_F16_FIELDS[fmt][0]
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    blocks[:, d_off] = (allh & 0xFF).astype(np.uint8)
    blocks[:, d_off + 1] = (allh >> 8).astype(np.uint8)
    if be == 256:
        blocks = blocks[::4]  # 16384 super-blocks x 256 elements: every fourth pattern
    n = blocks.shape[0] * be
    for f16 in (False, True):
        _check(_gpu_dequant(provider, blocks, fmt, n, f16), oracle_mod.dequant(blocks, fmt, n, f16=f16), f16,
               f"{fmt} scales f16={f16}")


def test_reference_test_pattern(provider, oracle_mod):
    """The inputs of kquant_dequant_test.cpp:240-252 (bytes (i*73+17) & 0xFF,
    bytes 0-1 of block b = the test's fp16 of 0.01*(b+1)) at its block counts."""
    for fmt, nb in (("q4_1", 8), ("q5_0", 8), ("q5_1", 8), ("q2_k", 4), ("q3_k", 4), ("q4_k", 4), ("q5_k", 4),
                    ("q6_k", 4)):
        bs, be = syn.KQ_GEOM[fmt]
        raw = ((np.arange(nb * bs) * 73 + 17) & 0xFF).astype(np.uint8).reshape(nb, bs)
        for b in range(nb):
            h = oracle_mod.f32_to_f16_trunc(np.float32(0.01) * np.float32(b + 1))
            raw[b, 0], raw[b, 1] = h & 0xFF, h >> 8
        for f16 in (False, True):
            _check(_gpu_dequant(provider, raw, fmt, nb * be, f16), oracle_mod.dequant(raw, fmt, nb * be, f16=f16),
                   f16, f"{fmt} reference pattern")


@pytest.mark.parametrize("count", [1, 7, 8, 9, 31, 33, 255, 257, 2047, 2049, 5000])
def test_ragged_counts(provider, oracle_mod, count):
    """count = out.size_bytes / element size (metal_provider.mm:2667): partial
    blocks, partial 8-element chunks and partial workgroups."""
    for fmt in FMTS:
        _, be = syn.KQ_GEOM[fmt]
        blocks = syn.kquant_blocks(fmt, (count + be - 1) // be, seed=count)
        for f16 in (False, True):
            _check(_gpu_dequant(provider, blocks, fmt, count, f16), oracle_mod.dequant(blocks, fmt, count, f16=f16),
                   f16, f"{fmt} count={count}")


def test_q3_k_f16_reads_past_last_block(provider, oracle_mod):
    """dequant_q3_k_f16's scales for sub-blocks 14, 15 come from the next
    block's first two bytes: across workgroup boundaries (8 blocks each), and
    0 past the end of the input buffer, or the buffer's spare bytes when it is
    longer than the blocks the output needs."""
    for nb in (1, 8, 9, 17):
        blocks = syn.kquant_blocks("q3_k", nb, seed=nb)
        got = _gpu_dequant(provider, blocks, "q3_k", nb * 256, True)
        _check(got, oracle_mod.dequant(blocks, "q3_k", nb * 256, f16=True), True, f"q3_k_f16 nb={nb}")
    spare = np.concatenate([syn.kquant_blocks("q3_k", 3, seed=4).reshape(-1), np.array([0x47, 0x9C, 1], np.uint8)])
    got = _gpu_dequant(provider, spare, "q3_k", 3 * 256, True)
    _check(got, oracle_mod.dequant(spare, "q3_k", 3 * 256, f16=True), True, "q3_k_f16 spare bytes")


def _import(provider, parent, offset, dtype, nbytes):
    ops, h = abi.nf_buffer_ops(), C.c_void_p()
    desc = abi.make_desc(dtype, nbytes)
    st = provider.mem.import_buffer(provider.handle, parent.device_ptr() + offset, abi.NF_MEM_DOMAIN_DEVICE,
                                    C.byref(desc), C.byref(ops), C.byref(h))
    assert st == abi.NF_OK
    return Buffer(provider, h.value, ops, dtype, nbytes)


@pytest.mark.parametrize("fmt", ["q5_0", "q3_k", "q6_k"])
def test_unaligned_buffers(provider, oracle_mod, fmt):
    """An input imported at an odd device address (byte-wise staging) and an
    output at a 4-byte (f32) / 2-byte (f16) offset (element-wise stores)."""
    bs, be = syn.KQ_GEOM[fmt]
    nb = 2 * 2048 // be + 1
    blocks = syn.kquant_blocks(fmt, nb, seed=21).reshape(-1)
    n = nb * be - 3
    for f16 in (False, True):
        e = 2 if f16 else 4
        odt = abi.NF_DTYPE_F16 if f16 else abi.NF_DTYPE_F32
        wp = provider.alloc_array(np.concatenate([np.zeros(1, np.uint8), blocks]), abi.NF_DTYPE_U8)
        op_ = provider.alloc(odt, (n + 1) * e)
        wi = _import(provider, wp, 1, QDT[fmt], blocks.size)
        oi = _import(provider, op_, e, odt, n * e)
        provider.dispatch(f"dequant_{fmt}" + ("_f16" if f16 else ""), [wi], [oi])
        provider.synchronize()
        got = op_.download(np.uint16 if f16 else np.float32)[1:]
        _check(got, oracle_mod.dequant(blocks, fmt, n, f16=f16), f16, f"{fmt} unaligned f16={f16}")
        for b in (wi, oi, wp, op_):
            b.release()


@pytest.mark.parametrize("fmt", ["q4_k", "q6_k"])
def test_7b_shape_weight(provider, oracle_mod, fmt):
    """A full Llama-2-7B FFN weight (11008 x 4096 elements), f32 and f16."""
    _, be = syn.KQ_GEOM[fmt]
    n = 11008 * 4096
    blocks = syn.kquant_blocks(fmt, n // be, seed=77)
    for f16 in (False, True):
        _check(_gpu_dequant(provider, blocks, fmt, n, f16), oracle_mod.dequant(blocks, fmt, n, f16=f16), f16,
               f"{fmt} 7B f16={f16}")


def test_rejects_short_input(provider):
    for fmt in FMTS:
        bs, be = syn.KQ_GEOM[fmt]
        w = provider.alloc(QDT[fmt], 2 * bs - 1)
        out = provider.alloc(abi.NF_DTYPE_F32, 2 * be * 4)
        assert provider.dispatch_bare(f"dequant_{fmt}", [w], [out]) == abi.NF_ERROR_INVALID_ARG
        w.release()
        out.release()
