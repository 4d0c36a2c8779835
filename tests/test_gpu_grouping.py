"""nf_hip_run_tasks merges adjacent decode GEMVs and small-batch linears
that read the same activation buffer (q/k/v, gate/up) into one launch.  Each
result must be bit-identical to dispatching the tasks one by one, the launch
count must show the merge, and a hazard between two tasks (here: both write
the same output; a weight buffer written mid-list; each task reading the
previous one's output) must keep the order."""
import ctypes as C

import numpy as np
import pytest

from helpers import assert_close
from neurofabric_amd import abi
from neurofabric_amd import synthetic as syn
from neurofabric_amd.abi import nf_task_desc

pytestmark = pytest.mark.gpu

QDT = {"q4_0": abi.NF_DTYPE_Q4_0, "q8_0": abi.NF_DTYPE_Q8_0}


def _array(tasks):
    arr = (nf_task_desc * len(tasks))()
    for i, td in enumerate(tasks):
        C.memmove(C.addressof(arr[i]), C.addressof(td), C.sizeof(nf_task_desc))
        arr[i].user_data = C.addressof(arr[i])
    return arr


def _block(provider, fmt, f16, M, hidden, kv, ffn, seed):
    """One Llama block's projections with the model's dataflow."""
    adt = abi.NF_DTYPE_F16 if f16 else abi.NF_DTYPE_F32
    npdt = np.float16 if f16 else np.float32
    elt = 2 if f16 else 4
    acts = {r: provider.alloc_array(syn.activations(M, k, seed=seed + i, dtype=npdt), adt)
            for i, (r, k) in enumerate((("attn_norm", hidden), ("attn_out", hidden), ("ffn_norm", hidden),
                                       ("ffn_act", ffn)))}
    projs = [("q", "attn_norm", hidden, hidden), ("k", "attn_norm", kv, hidden), ("v", "attn_norm", kv, hidden),
             ("o", "attn_out", hidden, hidden), ("gate", "ffn_norm", ffn, hidden), ("up", "ffn_norm", ffn, hidden),
             ("down", "ffn_act", hidden, ffn)]
    host_w, bufs, outs, specs = {}, [], {}, []
    op = f"dequant_{fmt}_linear" + ("_f16" if f16 else "")
    for j, (name, role, N, K) in enumerate(projs):
        host_w[name] = syn.weights(fmt, N, K, seed=seed + 10 + j)
        w = provider.alloc_array(host_w[name], QDT[fmt])
        outs[name] = provider.alloc(adt, M * N * elt)
        bufs.append(w)
        specs.append((name, role, w, N, K))
    tasks = [provider.task(op, [acts[role], w], [outs[name]], M, N, K) for (name, role, w, N, K) in specs]
    return op, acts, outs, specs, tasks, bufs + list(acts.values()) + list(outs.values()), host_w


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("f16", [False, True], ids=["f32", "f16"])
@pytest.mark.parametrize("M", [1, 3, 8, 16])
def test_run_tasks_merges_same_input_gemvs(provider, oracle_mod, fmt, f16, M):
    """M <= 4: decode GEMV groups; M = 8, 16: small-batch MFMA groups."""
    hidden, kv, ffn = 1024, 128, 2816
    op, acts, outs, specs, tasks, bufs, host_w = _block(provider, fmt, f16, M, hidden, kv, ffn, seed=M * 7)
    npdt = np.float16 if f16 else np.float32
    try:
        arr = _array(tasks)
        before = provider.launch_count()
        provider.run_tasks(arr, 1)
        provider.synchronize()
        assert provider.launch_count() - before == 4  # q+k+v, o, gate+up, down
        grouped = {name: outs[name].download(npdt).copy() for (name, *_r) in specs}
        # the same tasks one dispatch each
        for (name, role, w, N, K) in specs:
            provider.dispatch(op, [acts[role], w], [outs[name]], M, N, K)
        provider.synchronize()
        for (name, *_r) in specs:
            single = outs[name].download(npdt)
            assert np.array_equal(grouped[name].view(np.uint8), single.view(np.uint8)), name
        # and one merged member against the oracle
        A = acts["attn_norm"].download(npdt).reshape(M, hidden)
        ref = oracle_mod.fused(A, host_w["k"], fmt, M, kv, hidden, f16=f16, threads=8)
        if f16:
            ref = ref.view(np.float16)
        assert_close(grouped["k"].reshape(M, kv).astype(np.float32), ref.astype(np.float32), what=f"{fmt} k")
    finally:
        for b in bufs:
            b.release()


def test_run_tasks_keeps_hazards_apart(provider, oracle_mod):
    """Two GEMVs over the same activations that write the same output are
    not merged; the output is the second one's, as in dispatch order."""
    M, N, K = 1, 300, 512
    A = syn.activations(M, K, seed=1)
    W1, W2 = syn.q4_0_weights(N, K, seed=2), syn.q4_0_weights(N, K, seed=3)
    a = provider.alloc_array(A, abi.NF_DTYPE_F32)
    w1 = provider.alloc_array(W1, abi.NF_DTYPE_Q4_0)
    w2 = provider.alloc_array(W2, abi.NF_DTYPE_Q4_0)
    c = provider.alloc(abi.NF_DTYPE_F32, M * N * 4)
    try:
        arr = _array([provider.task("dequant_q4_0_linear", [a, w], [c], M, N, K) for w in (w1, w2)])
        before = provider.launch_count()
        provider.run_tasks(arr, 1)
        provider.synchronize()
        assert provider.launch_count() - before == 2
        assert_close(c.download(np.float32).reshape(M, N), oracle_mod.fused(A, W2, "q4_0", M, N, K))
    finally:
        for b in (a, w1, w2, c):
            b.release()


def test_run_tasks_weight_written_mid_list(provider, oracle_mod):
    """A task in the middle of a batch overwrites the weight buffer a later
    GEMV reads (embedding_lookup copying new Q4_0 bytes into it, bit for
    bit); the later GEMV must use the new bytes, also when the list is run
    twice in one call (repeat=2)."""
    from neurofabric_amd.plugin import push_constants
    M, N, K = 1, 300, 512
    A = syn.activations(M, K, seed=5)
    W1, W2_old, W2_new = (syn.q4_0_weights(N, K, seed=s) for s in (6, 7, 8))
    assert W2_new.nbytes % 4 == 0
    dim = W2_new.nbytes // 4
    a = provider.alloc_array(A, abi.NF_DTYPE_F32)
    w1 = provider.alloc_array(W1, abi.NF_DTYPE_Q4_0)
    w2 = provider.alloc_array(W2_old.view(np.float32), abi.NF_DTYPE_F32)
    table = provider.alloc_array(W2_new.view(np.float32), abi.NF_DTYPE_F32)
    ids = provider.alloc_array(np.zeros(1, np.int32), abi.NF_DTYPE_I32)
    c1 = provider.alloc(abi.NF_DTYPE_F32, M * N * 4)
    c2 = provider.alloc(abi.NF_DTYPE_F32, M * N * 4)
    try:
        arr = _array([provider.task("dequant_q4_0_linear", [a, w1], [c1], M, N, K),
                      provider.task("embedding_lookup", [table, ids], [w2], pc=push_constants(seq_len=1, head_dim=dim)),
                      provider.task("dequant_q4_0_linear", [a, w2], [c2], M, N, K)])
        provider.run_tasks(arr, 2)
        provider.synchronize()
        assert np.array_equal(w2.download(np.uint8), W2_new)
        assert_close(c1.download(np.float32).reshape(M, N), oracle_mod.fused(A, W1, "q4_0", M, N, K), what="first")
        assert_close(c2.download(np.float32).reshape(M, N), oracle_mod.fused(A, W2_new, "q4_0", M, N, K),
                     what="after the write")
    finally:
        for b in (a, w1, w2, table, ids, c1, c2):
            b.release()


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
def test_run_tasks_chain_bit_identical(provider, fmt):
    """Twelve decode GEMVs with distinct weights and shapes, the adjacent
    same-input ones merged, through nf_hip_run_tasks three times in one
    call, then one dispatch each: bit-identical outputs."""
    M, K = 1, 2048
    A = syn.activations(M, K, seed=9)
    a = provider.alloc_array(A, abi.NF_DTYPE_F32)
    shapes = [2048, 256, 256, 2048, 5632, 5632, 2048, 1024, 4096, 300, 64, 8192]
    bufs, tasks, outs = [a], [], []
    op = f"dequant_{fmt}_linear"
    for i, N in enumerate(shapes):
        w = provider.alloc_array(syn.weights(fmt, N, K, seed=20 + i), QDT[fmt])
        c = provider.alloc(abi.NF_DTYPE_F32, M * N * 4)
        bufs += [w, c]
        outs.append((w, c, N))
        tasks.append(provider.task(op, [a, w], [c], M, N, K))
    try:
        provider.run_tasks(_array(tasks), 3)
        provider.synchronize()
        got = [c.download(np.float32).copy() for (_, c, _) in outs]
        for (w, c, N) in outs:
            provider.dispatch(op, [a, w], [c], M, N, K)
        provider.synchronize()
        for i, (_, c, _) in enumerate(outs):
            assert np.array_equal(got[i].view(np.uint32), c.download(np.float32).view(np.uint32)), i
    finally:
        for b in bufs:
            b.release()


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("f16", [False, True], ids=["f32", "f16"])
@pytest.mark.parametrize("dims", [(2048, 1024, 64, 5632, 2048, 128, 4096), (512, 256, 64, 256, 1024)],
                         ids=["mixed", "small"])
def test_run_tasks_dependent_sequence(provider, oracle_mod, fmt, f16, dims):
    """Decode GEMVs where each reads the previous one's output (layer i:
    K = dims[i], N = dims[i+1]), some with few rows: one launch each (no
    two share an input), bit-identical to one dispatch each, in order; the
    first layer against the oracle."""
    M = 1
    adt = abi.NF_DTYPE_F16 if f16 else abi.NF_DTYPE_F32
    npdt = np.float16 if f16 else np.float32
    op = f"dequant_{fmt}_linear" + ("_f16" if f16 else "")
    x0 = syn.activations(M, dims[0], seed=31, dtype=npdt)
    acts = [provider.alloc_array(x0, adt)] + [provider.alloc(adt, M * n * x0.itemsize) for n in dims[1:]]
    host_w, ws, tasks = [], [], []
    for i in range(len(dims) - 1):
        K, N = dims[i], dims[i + 1]
        host_w.append(syn.weights(fmt, N, K, seed=40 + i))
        ws.append(provider.alloc_array(host_w[-1], QDT[fmt]))
        tasks.append(provider.task(op, [acts[i], ws[-1]], [acts[i + 1]], M, N, K))
    try:
        before = provider.launch_count()
        provider.run_tasks(_array(tasks), 1)
        provider.synchronize()
        assert provider.launch_count() - before == len(tasks)
        chained = [a.download(npdt).copy() for a in acts[1:]]
        for t_i in range(len(tasks)):
            K, N = dims[t_i], dims[t_i + 1]
            provider.dispatch(op, [acts[t_i], ws[t_i]], [acts[t_i + 1]], M, N, K)
        provider.synchronize()
        for i, a in enumerate(acts[1:]):
            assert np.array_equal(chained[i].view(np.uint8), a.download(npdt).view(np.uint8)), f"layer {i}"
        ref = oracle_mod.fused(x0, host_w[0], fmt, M, dims[1], dims[0], f16=f16, threads=8)
        if f16:
            ref = ref.view(np.float16)
        assert_close(chained[0].reshape(M, dims[1]).astype(np.float32), ref.astype(np.float32), what=f"{fmt} layer 0")
    finally:
        for b in acts + ws:
            b.release()
