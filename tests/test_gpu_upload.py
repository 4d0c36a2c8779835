"""The weight-upload path on the GPU, through the C ABI.

* map / memcpy / unmap, the reference model layer's load_weight
  (llama_dag_builder.hpp:146-156), on buffers large enough (>= 64 MiB) to
  take their pinned staging from the provider's reuse pool: contents right
  when blocks are reused, when two large buffers are mapped at once and
  after the pool is released.
* nf_hip_buffer_write / nf_hip_buffer_read: byte ranges, bounds and
  mapped-buffer errors, and ordering after dispatches already issued.
* The warm-up flow of llama_dag_builder.hpp:973-1066: upload K-quant
  weights, dequantize them all in one run of tasks, compare bit for bit.
"""
import numpy as np
import pytest

from helpers import assert_bits_equal_f16
from neurofabric_amd import abi
from neurofabric_amd import synthetic as syn
from neurofabric_amd.plugin import NfError

pytestmark = pytest.mark.gpu

MB = 1 << 20


def _pattern(n, seed):
    return np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8)


def test_map_upload_large_buffers_reuse_staging(provider):
    sizes = [80 * MB, 72 * MB, 130 * MB, 80 * MB]
    for i, n in enumerate(sizes):
        data = _pattern(n, i)
        b = provider.alloc(abi.NF_DTYPE_U8, n)
        b.upload(data)  # map (staging from the pool after the first), memcpy, unmap
        assert np.array_equal(b.read(np.uint8), data), f"buffer {i}"
        # a second map of the same buffer sees the device contents
        assert np.array_equal(b.download(np.uint8)[-4096:], data[-4096:])
        b.release()
    provider.release_staging()


def test_two_large_mappings_at_once(provider):
    n = 70 * MB
    a, b = provider.alloc(abi.NF_DTYPE_U8, n), provider.alloc(abi.NF_DTYPE_U8, n)
    da, db = _pattern(n, 10), _pattern(n, 11)
    pa = a.map()
    pb = b.map()
    assert pa != pb
    import ctypes as C
    C.memmove(pa, da.ctypes.data, n)
    C.memmove(pb, db.ctypes.data, n)
    b.unmap()
    a.unmap()
    assert np.array_equal(a.read(np.uint8), da)
    assert np.array_equal(b.read(np.uint8), db)
    # both blocks are back in the pool: map again, the staging mirrors the device
    assert np.array_equal(a.download(np.uint8), da)
    a.release()
    b.release()
    provider.release_staging()


def test_write_read_ranges(provider):
    n = 1 << 16
    b = provider.alloc(abi.NF_DTYPE_U8, n)
    assert not b.read(np.uint8).any()  # alloc zero-fills
    data = _pattern(n, 3)
    b.write(data)
    assert np.array_equal(b.read(np.uint8), data)
    b.write(np.full(100, 7, np.uint8), offset=1001)
    want = data.copy()
    want[1001:1101] = 7
    assert np.array_equal(b.read(np.uint8), want)
    assert np.array_equal(b.read(np.uint8, count=10, offset=1000), want[1000:1010])
    assert np.array_equal(b.download(np.uint8), want)  # the map path agrees
    b.release()


def test_write_read_errors(provider):
    b = provider.alloc(abi.NF_DTYPE_U8, 256)
    for off, cnt in ((0, 257), (200, 57), (257, 0), (2**63, 1)):
        with pytest.raises(NfError) as e:
            provider.check(provider.lib.nf_hip_buffer_write(b.handle, off, np.zeros(max(cnt, 1), np.uint8).ctypes.data, cnt),
                           "write")
        assert e.value.status == abi.NF_ERROR_INVALID_ARG
    b.map()
    with pytest.raises(NfError) as e:
        b.write(np.zeros(16, np.uint8))
    assert e.value.status == abi.NF_ERROR_INVALID_ARG
    b.unmap()
    b.write(np.zeros(0, np.uint8))  # empty copy is a no-op
    b.release()


def test_write_is_ordered_after_issued_dispatches(provider, oracle_mod):
    """A dispatch reading W, then a write replacing W, then the same dispatch:
    the first result uses the old weights, the second the new ones."""
    M, N, K = 1, 512, 1024
    A = syn.activations(M, K, seed=1)
    W0, W1 = syn.q4_0_weights(N, K, seed=2), syn.q4_0_weights(N, K, seed=3)
    a = provider.alloc_array(A, abi.NF_DTYPE_F32)
    w = provider.alloc_array(W0, abi.NF_DTYPE_Q4_0)
    c0, c1 = provider.alloc(abi.NF_DTYPE_F32, M * N * 4), provider.alloc(abi.NF_DTYPE_F32, M * N * 4)
    provider.dispatch("dequant_q4_0_linear", [a, w], [c0], M, N, K)
    w.write(W1)
    provider.dispatch("dequant_q4_0_linear", [a, w], [c1], M, N, K)
    provider.synchronize()
    r0 = oracle_mod.fused(A, W0, "q4_0", M, N, K)
    r1 = oracle_mod.fused(A, W1, "q4_0", M, N, K)
    g0, g1 = c0.read(np.float32).reshape(M, N), c1.read(np.float32).reshape(M, N)
    assert np.max(np.abs(g0 - r0)) <= 1e-3 * np.max(np.abs(r0))
    assert np.max(np.abs(g1 - r1)) <= 1e-3 * np.max(np.abs(r1))
    for x in (a, w, c0, c1):
        x.release()


def test_warmup_flow_upload_then_dequant_all(provider, oracle_mod):
    """Upload one weight per K-quant format with nf_hip_buffer_write, then
    dequantize all of them to f16 in one nf_hip_run_tasks call (the warm-up
    graph of llama_dag_builder.hpp:973-1066)."""
    fmts = ["q2_k", "q3_k", "q4_k", "q5_k", "q6_k", "q4_1", "q5_0", "q5_1"]
    n = 4096 * 1024
    ins, outs, blocks, tasks = [], [], [], []
    for i, fmt in enumerate(fmts):
        bs, be = syn.KQ_GEOM[fmt]
        blk = syn.kquant_blocks(fmt, n // be, seed=40 + i)
        w = provider.alloc(getattr(abi, f"NF_DTYPE_{fmt.upper()}"), blk.size)
        w.write(blk)
        o = provider.alloc(abi.NF_DTYPE_F16, n * 2)
        ins.append(w)
        outs.append(o)
        blocks.append(blk)
        tasks.append(provider.task(f"dequant_{fmt}_f16", [w], [o]))
    import ctypes as C
    arr = (abi.nf_task_desc * len(tasks))()
    for i, td in enumerate(tasks):
        C.memmove(C.addressof(arr[i]), C.addressof(td), C.sizeof(abi.nf_task_desc))
        arr[i].user_data = C.addressof(arr[i])
    provider.run_tasks(arr)
    provider.synchronize()
    for fmt, blk, o in zip(fmts, blocks, outs):
        assert_bits_equal_f16(o.read(np.uint16), oracle_mod.dequant(blk, fmt, n, f16=True), fmt)
    for x in ins + outs:
        x.release()
