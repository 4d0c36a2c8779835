"""Boundary semantics of the HIP provider on the GPU (the reference's buffer,
dispatch and threading contract, SURVEY-level summary in DESIGN.md):

* alloc zero-fills (metal_provider.mm:2277-2278); map/unmap round-trips;
  double map is NF_ERROR_INVALID_ARG (metal_provider.mm:2031-2037);
* refcounts (retain/release) and get_info/export report DEVICE memory;
* dispatch returns once enqueued; cache_sync(INVALIDATE) and map observe the
  finished result; dependent ops dispatched from different threads run in
  submission order (PipelineEngine.hpp:609-650);
* error codes for bad sizes, missing push constants and unknown ops;
* the async DDI (dispatch_async / wait / poll / query_caps) and the timing ring.
"""
import ctypes as C
import threading

import numpy as np
import pytest

from helpers import assert_close
from neurofabric_amd import abi
from neurofabric_amd import synthetic as syn
from neurofabric_amd.plugin import NfError

pytestmark = pytest.mark.gpu


def test_alloc_zero_fills_and_roundtrips(provider):
    b = provider.alloc(abi.NF_DTYPE_U8, 1 << 20)
    assert not b.download(np.uint8).any()
    data = np.random.default_rng(0).integers(0, 256, 1 << 20, dtype=np.uint8)
    b.upload(data)
    assert np.array_equal(b.download(np.uint8), data)
    b.release()


def test_double_map_is_invalid(provider):
    b = provider.alloc(abi.NF_DTYPE_F32, 64)
    b.map()
    ptr = C.c_void_p()
    assert b.ops.map(b.handle, C.byref(ptr)) == abi.NF_ERROR_INVALID_ARG
    b.unmap()
    b.release()


def test_refcount_info_and_export(provider):
    b = provider.alloc(abi.NF_DTYPE_F16, 4096)
    assert b.retain() == 2
    info = b.info()
    assert info.domain == abi.NF_MEM_DOMAIN_DEVICE and info.refcount == 2 and info.desc.size_bytes == 4096
    tok, dom = C.c_uint64(), C.c_int()
    assert b.ops.export_handle(b.handle, C.byref(tok), C.byref(dom)) == abi.NF_OK
    assert dom.value == abi.NF_MEM_DOMAIN_DEVICE and tok.value == b.device_ptr() != 0
    assert b.release() == 1
    assert b.release() == 0


def test_import_device_token_zero_copy(provider, oracle_mod):
    """A DEVICE token from export_handle imports as a non-owning buffer that
    dispatch can read (neuro_buffer_abi.h:165-183)."""
    M, N, K = 2, 64, 128
    A = syn.activations(M, K, seed=1)
    W = syn.q4_0_weights(N, K, seed=2)
    a = provider.alloc_array(A, abi.NF_DTYPE_F32)
    w = provider.alloc_array(W, abi.NF_DTYPE_Q4_0)
    c = provider.alloc(abi.NF_DTYPE_F32, M * N * 4)
    assert provider.mem.can_import(provider.handle, abi.NF_MEM_DOMAIN_DEVICE) == abi.NF_OK
    assert provider.mem.can_import(provider.handle, abi.NF_MEM_DOMAIN_DMA_BUF) == abi.NF_ERROR_UNSUPPORTED_OP
    ops, h = abi.nf_buffer_ops(), C.c_void_p()
    desc = abi.make_desc(abi.NF_DTYPE_Q4_0, W.nbytes)
    st = provider.mem.import_buffer(provider.handle, w.device_ptr(), abi.NF_MEM_DOMAIN_DEVICE, C.byref(desc),
                                    C.byref(ops), C.byref(h))
    assert st == abi.NF_OK
    from neurofabric_amd.plugin import Buffer
    wi = Buffer(provider, h.value, ops, abi.NF_DTYPE_Q4_0, W.nbytes)
    provider.dispatch("dequant_q4_0_linear", [a, wi], [c], M, N, K)
    assert_close(c.download(np.float32).reshape(M, N), oracle_mod.fused(A, W, "q4_0", M, N, K))
    wi.release()  # non-owning: the exporter's memory stays valid
    assert np.array_equal(w.download(np.uint8), W)
    for b in (a, w, c):
        b.release()


def test_cache_sync_and_live_mapping(provider, oracle_mod):
    """A buffer mapped while a dispatch writes it sees the result after
    cache_sync(INVALIDATE), and unmap does not clobber the device result."""
    M, N, K = 1, 256, 256
    A = syn.activations(M, K, seed=3)
    W = syn.q4_0_weights(N, K, seed=4)
    a, w = provider.alloc_array(A, abi.NF_DTYPE_F32), provider.alloc_array(W, abi.NF_DTYPE_Q4_0)
    c = provider.alloc(abi.NF_DTYPE_F32, M * N * 4)
    ptr = c.map()
    provider.dispatch("dequant_q4_0_linear", [a, w], [c], M, N, K)
    c.cache_sync(abi.NF_CACHE_INVALIDATE)
    view = np.ctypeslib.as_array((C.c_float * (M * N)).from_address(ptr)).copy()
    c.unmap()
    ref = oracle_mod.fused(A, W, "q4_0", M, N, K)
    assert_close(view.reshape(M, N), ref)
    assert_close(c.download(np.float32).reshape(M, N), ref)
    for b in (a, w, c):
        b.release()


def test_error_codes(provider):
    a = provider.alloc(abi.NF_DTYPE_F32, 4 * 64 * 4)
    w = provider.alloc(abi.NF_DTYPE_Q4_0, 8 * 2 * 18)
    c = provider.alloc(abi.NF_DTYPE_F32, 4 * 8 * 4)
    td = provider.task("dequant_q4_0_linear", [a, w], [c], 4, 8, 64)
    assert provider.dispatch_task(td) == abi.NF_OK
    assert provider.dispatch_task(provider.task("dequant_q4_0_linear", [a, w], [c], 4, 9, 64)) == abi.NF_ERROR_INVALID_ARG
    assert provider.dispatch_task(provider.task("dequant_q4_0_linear", [a, w], [c], 5, 8, 64)) == abi.NF_ERROR_INVALID_ARG
    no_pc = provider.task("dequant_q4_0_linear", [a, w], [c])
    assert provider.dispatch_task(no_pc) == abi.NF_ERROR_INVALID_ARG
    assert provider.dispatch_task(provider.task("dequant_q4_0_linear", [a], [c], 4, 8, 64)) == abi.NF_ERROR_INVALID_ARG
    assert provider.dispatch_task(provider.task("sparse_moe_router", [a], [c])) == abi.NF_ERROR_UNSUPPORTED_OP
    assert provider.dispatch_task(provider.task("flash_attention_gqa", [a], [c])) == abi.NF_ERROR_INVALID_ARG
    provider.synchronize()
    for b in (a, w, c):
        b.release()


def test_dependent_dispatch_from_different_threads(provider, oracle_mod):
    """dequant (thread 1) then linear over its output (thread 2): ordered by
    submission on the provider's in-order stream, no explicit sync between."""
    M, N, K = 3, 512, 1024
    A = syn.activations(M, K, seed=5)
    W = syn.q4_0_weights(N, K, seed=6)
    a, w = provider.alloc_array(A, abi.NF_DTYPE_F32), provider.alloc_array(W, abi.NF_DTYPE_Q4_0)
    for _ in range(5):
        dq = provider.alloc(abi.NF_DTYPE_F32, N * K * 4)
        c = provider.alloc(abi.NF_DTYPE_F32, M * N * 4)
        t1 = threading.Thread(target=lambda: provider.check(provider.dispatch_bare("dequant_q4_0", [w], [dq]), "dq"))
        t1.start()
        t1.join()
        t2 = threading.Thread(target=lambda: provider.dispatch("linear", [a, dq], [c], M, N, K))
        t2.start()
        t2.join()
        assert_close(c.download(np.float32).reshape(M, N), oracle_mod.fused(A, W, "q4_0", M, N, K))
        dq.release()
        c.release()
    a.release()
    w.release()


def test_concurrent_dispatch_from_pool_threads(provider, oracle_mod):
    """8 threads dispatch independent projections at once (the engine runs
    q/k/v and gate/up concurrently); every output is correct."""
    K = 2048
    shapes = [(1, 256 + 64 * i, K) for i in range(8)]
    A = syn.activations(1, K, seed=7)
    a = provider.alloc_array(A, abi.NF_DTYPE_F32)
    ws, cs, refs = [], [], []
    for i, (M, N, _) in enumerate(shapes):
        W = syn.q4_0_weights(N, K, seed=100 + i)
        ws.append(provider.alloc_array(W, abi.NF_DTYPE_Q4_0))
        cs.append(provider.alloc(abi.NF_DTYPE_F32, N * 4))
        refs.append(oracle_mod.fused(A, W, "q4_0", 1, N, K))
    errs = []

    def work(i):
        try:
            for _ in range(20):
                provider.dispatch("dequant_q4_0_linear", [a, ws[i]], [cs[i]], 1, shapes[i][1], K)
        except Exception as e:  # pragma: no cover - reported below
            errs.append(e)

    ts = [threading.Thread(target=work, args=(i,)) for i in range(8)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errs
    provider.synchronize()
    for i in range(8):
        assert_close(cs[i].download(np.float32).reshape(1, -1), refs[i])
    for b in ws + cs + [a]:
        b.release()


def test_async_ddi_and_caps(provider, oracle_mod):
    caps = provider.caps()
    assert caps.memory_bytes > 200 * 2 ** 30  # 288 GB HBM3E
    assert caps.flags & abi.NF_CAP_ASYNC and caps.flags & abi.NF_CAP_FP16
    for dt in (abi.NF_DTYPE_F32, abi.NF_DTYPE_F16, abi.NF_DTYPE_Q4_0, abi.NF_DTYPE_Q8_0, abi.NF_DTYPE_Q4_1,
               abi.NF_DTYPE_Q5_0, abi.NF_DTYPE_Q5_1, abi.NF_DTYPE_Q2_K, abi.NF_DTYPE_Q3_K, abi.NF_DTYPE_Q4_K,
               abi.NF_DTYPE_Q5_K, abi.NF_DTYPE_Q6_K):
        assert caps.supported_dtypes & (1 << dt), dt
    assert not caps.supported_dtypes & (1 << abi.NF_DTYPE_BF16)
    M, N, K = 1, 1024, 2048
    A = syn.activations(M, K, seed=8)
    W = syn.q4_0_weights(N, K, seed=9)
    a, w = provider.alloc_array(A, abi.NF_DTYPE_F32), provider.alloc_array(W, abi.NF_DTYPE_Q4_0)
    c = provider.alloc(abi.NF_DTYPE_F32, M * N * 4)
    td = provider.task("dequant_q4_0_linear", [a, w], [c], M, N, K)
    tok = C.c_void_p()
    st = provider.ddi.dispatch_async(provider.handle, td.op_name, provider._inputs_ptr(td), 2,
                                     provider._outputs_ptr(td), 1, C.byref(tok))
    assert st == abi.NF_OK
    assert provider.ddi.wait_completion(provider.handle, tok, 10_000) == abi.NF_OK
    td2 = provider.task("dequant_q4_0_linear", [a, w], [c], M, N, K)
    tok2 = C.c_void_p()
    assert provider.ddi.dispatch_async(provider.handle, td2.op_name, provider._inputs_ptr(td2), 2,
                                       provider._outputs_ptr(td2), 1, C.byref(tok2)) == abi.NF_OK
    provider.synchronize()
    assert provider.ddi.poll_completion(provider.handle, tok2) == abi.NF_OK
    assert_close(c.download(np.float32).reshape(M, N), oracle_mod.fused(A, W, "q4_0", M, N, K))
    for b in (a, w, c):
        b.release()


def test_timing_ring(provider):
    lib = provider.lib
    M, N, K = 1, 2048, 2048
    a = provider.alloc(abi.NF_DTYPE_F32, M * K * 4)
    w = provider.alloc_array(syn.q4_0_weights(N, K, seed=10), abi.NF_DTYPE_Q4_0)
    c = provider.alloc(abi.NF_DTYPE_F32, M * N * 4)
    lib.nf_hip_enable_timing(True)
    try:
        for _ in range(3):
            provider.dispatch("dequant_q4_0_linear", [a, w], [c], M, N, K)
        provider.synchronize()
        n = lib.nf_hip_get_timing_count()
        assert n == 3
        names = (C.c_char * 64 * n)()
        ms = (C.c_double * n)()
        dts = (C.c_uint8 * n)()
        els = (C.c_uint32 * n)()
        lib.nf_hip_get_timings_ext(names, ms, dts, els, n)
        assert all(bytes(names[i]).split(b"\0")[0] == b"dequant_q4_0_linear" for i in range(n))
        assert all(0 < ms[i] < 100 for i in range(n))
        assert all(els[i] == M * N for i in range(n)) and all(dts[i] == abi.NF_DTYPE_F32 for i in range(n))
    finally:
        lib.nf_hip_enable_timing(False)
    for b in (a, w, c):
        b.release()


def test_get_stream(provider):
    assert provider.stream() != 0


def test_diag_stream_read(provider):
    """The launch-floor calibration read: an empty launch, reads of aligned
    buffers of several sizes (every per-thread chunk count), and a misaligned
    source rejected without a launch."""
    for nbytes in (16, 4096, 1 << 21, (1 << 21) + 48, 40 << 20):
        b = provider.alloc(abi.NF_DTYPE_U8, nbytes)
        provider.diag_stream_read(b.device_ptr(), nbytes)
        provider.synchronize()
        b.release()
    provider.diag_stream_read(0, 0)
    provider.synchronize()
    b = provider.alloc(abi.NF_DTYPE_U8, 4096)
    with pytest.raises(NfError) as e:
        provider.diag_stream_read(b.device_ptr() + 4, 1024)
    assert e.value.status == abi.NF_ERROR_INVALID_ARG
    b.release()


@pytest.mark.parametrize("M,N,K", [(1, 256, 256), (16, 1024, 4096)], ids=["gemv", "skinny_splitk"])
def test_graph_replay_then_read(provider, oracle_mod, M, N, K):
    """Dispatches captured into a HIP graph on the provider stream
    (nf_hip_get_stream) and replayed there by the caller: a download or
    nf_hip_buffer_read right after each replay, with no synchronize in
    between, sees that replay's result.  The activations change between
    replays (an upload, eager work of the provider's own), and every replay
    is checked against an eager dispatch of the same inputs and the oracle."""
    from neurofabric_amd import hiprt
    W = syn.q4_0_weights(N, K, seed=5)
    a = provider.alloc(abi.NF_DTYPE_F32, M * K * 4)
    w = provider.alloc_array(W, abi.NF_DTYPE_Q4_0)
    c = provider.alloc(abi.NF_DTYPE_F32, M * N * 4)
    c_eager = provider.alloc(abi.NF_DTYPE_F32, M * N * 4)
    try:
        a.upload(syn.activations(M, K, seed=100))
        provider.dispatch("dequant_q4_0_linear", [a, w], [c], M, N, K)  # warm (any one-time set-up)
        provider.synchronize()
        g = hiprt.Graph(provider.stream(), lambda: provider.dispatch("dequant_q4_0_linear", [a, w], [c], M, N, K))
        for i in range(4):
            A = syn.activations(M, K, seed=200 + i)
            a.upload(A)
            print(f"graph replay {i} M={M} N={N} K={K}", flush=True)
            g.launch()
            got = c.download(np.float32) if i % 2 == 0 else c.read(np.float32)
            provider.dispatch("dequant_q4_0_linear", [a, w], [c_eager], M, N, K)
            eager = c_eager.download(np.float32)
            assert np.array_equal(got, eager), f"replay {i}: graph result differs from eager dispatch"
            assert_close(got.reshape(M, N), oracle_mod.fused(A, W, "q4_0", M, N, K), what=f"replay {i}")
        del g
    finally:
        provider.synchronize()
        for b in (a, w, c, c_eager):
            b.release()
