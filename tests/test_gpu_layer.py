"""The layer ops around the linears on the GPU, through the C ABI, against
the oracle (pinned in test_oracle_layer.py).

Bars: metal_vector_add / elementwise_mul / mock_relu / attention_prefill /
embedding_lookup / argmax bit-exact (single IEEE operations, copies and
indices); silu / gelu within 3e-7 relative plus the fp32 cancellation term;
rms_norm and softmax within 2e-6 (tree sums against the sequential loop);
rope within the fp32 angle-error bound (3e-7 rad per position);
attention within 2e-5 of the
max output (a 64-key online softmax against the reference variants'
arithmetic) and the appended cache rows bit-exact; every f16 output within
one fp16 unit in the last place of the oracle's.
"""
import numpy as np
import pytest

from neurofabric_amd import abi
from neurofabric_amd.plugin import NfError, push_constants
from oracle import oracle as orc

pytestmark = [pytest.mark.gpu, pytest.mark.filterwarnings("ignore::RuntimeWarning")]

F32, F16, I32 = abi.NF_DTYPE_F32, abi.NF_DTYPE_F16, abi.NF_DTYPE_I32


def _rng(s):
    return np.random.default_rng(s)


def _run(provider, op, ins, out_specs, pc=None):
    """ins: numpy arrays (dtype picks the buffer dtype) or Buffers; out_specs:
    (dtype, nbytes) or Buffers.  Returns the output Buffers (caller releases)."""
    bufs, own = [], []
    for a in ins:
        if isinstance(a, np.ndarray):
            dt = {np.float32: F32, np.uint16: F16, np.int32: I32, np.uint32: abi.NF_DTYPE_U8}[a.dtype.type]
            b = provider.alloc_array(a, dt)
            own.append(b)
        else:
            b = a
        bufs.append(b)
    outs = []
    for spec in out_specs:
        if isinstance(spec, tuple):
            outs.append(provider.alloc(*spec))
        else:
            outs.append(spec)
    provider.dispatch(op, bufs, outs, pc=pc)
    provider.synchronize()
    for b in own:
        b.release()
    return outs


def _ulp16_ok(got_bits, want_bits, ulps=1, abs_frac=0.0):
    """Every element within `ulps` fp16 spacings of the reference, or within
    abs_frac * max|reference| (for sums whose fp32 evaluation order differs
    from the reference's: near-zero results then carry the cancellation
    error of the sum, a few 1e-7 of its scale, which is many fp16 spacings
    of a tiny value)."""
    g = np.asarray(got_bits, np.uint16).view(np.float16).astype(np.float64)
    w = np.asarray(want_bits, np.uint16).view(np.float16).astype(np.float64)
    spacing = np.abs(np.spacing(w.astype(np.float16)).astype(np.float64))
    floor = abs_frac * float(np.max(np.abs(w[np.isfinite(w)]))) if abs_frac and np.isfinite(w).any() else 0.0
    return bool(np.all(np.abs(g - w) <= np.maximum(ulps * spacing, floor) + 1e-12))


def _read(buf, dt):
    return buf.read(dt)


# ---- element-wise ------------------------------------------------------------------

@pytest.mark.parametrize("n", [1, 7, 4096 + 3, 1 << 20])
def test_binary_ops_bit_exact(provider, n):
    a, b = _rng(n).standard_normal((2, n)).astype(np.float32)
    for op, f in (("metal_vector_add", "add"), ("elementwise_mul", "mul")):
        (o,) = _run(provider, op, [a, b], [(F32, n * 4)])
        assert np.array_equal(_read(o, np.float32), orc.binary(f, a, b)), op
        o.release()
        ha, hb = a.astype(np.float16).view(np.uint16), b.astype(np.float16).view(np.uint16)
        (o,) = _run(provider, op, [ha, hb], [(F16, n * 2)])
        assert np.array_equal(_read(o, np.uint16), orc.binary(f, ha, hb, f16=True)), op + " f16"
        o.release()


@pytest.mark.parametrize("n", [5, 4096 + 1, 1 << 20])
def test_unary_ops(provider, n):
    x = (_rng(n + 1).standard_normal(n) * 4).astype(np.float32)
    x64 = x.astype(np.float64)
    for op, f in (("silu", "silu"), ("gelu", "gelu")):
        (o,) = _run(provider, op, [x], [(F32, n * 4)])
        got, want = _read(o, np.float32), orc.unary(f, x)
        o.release()
        assert np.all(np.abs(got - want) <= 3e-7 * np.abs(want) + 3e-7 * np.abs(x64) + 1e-30), op
        h = x.astype(np.float16).view(np.uint16)
        (o,) = _run(provider, op, [h], [(F16, n * 2)])
        assert _ulp16_ok(_read(o, np.uint16), orc.unary(f, h, f16=True)), op + " f16"
        o.release()
    (o,) = _run(provider, "mock_relu", [x], [(F32, n * 4)])
    assert np.array_equal(_read(o, np.float32), np.maximum(x, 0))
    o.release()
    # mock_relu without an output works in place (metal_provider.mm:2435-2444)
    b = provider.alloc_array(x, F32)
    provider.dispatch("mock_relu", [b], [])
    provider.synchronize()
    assert np.array_equal(b.read(np.float32), np.maximum(x, 0))
    b.release()


def test_attention_prefill_mock(provider):
    x = _rng(3).standard_normal(1000).astype(np.float32)
    k, v = _run(provider, "attention_prefill", [x], [(F32, 1000 * 4), (F32, 600 * 4)])
    assert np.array_equal(_read(k, np.float32), x * np.float32(0.5))
    assert np.array_equal(_read(v, np.float32), x[:600] * np.float32(-0.25))
    k.release()
    v.release()


# ---- norms, softmax, argmax, embedding, rope ------------------------------------------

# rows held in registers (16-byte chunks: 1, 2, 4 or 8 per thread, partial
# last chunks), and the element-wise kernel for widths that do not split
@pytest.mark.parametrize("rows,dim", [(1, 2048), (7, 64), (16, 4096), (3, 5000), (2, 8192), (5, 12), (4, 30),
                                      (2, 16384)])
def test_rms_norm(provider, rows, dim):
    x = _rng(dim).standard_normal(rows * dim).astype(np.float32)
    w = _rng(dim + 1).standard_normal(dim).astype(np.float32)
    pc = push_constants(head_dim=dim, epsilon=1e-5)
    (o,) = _run(provider, "rms_norm", [x, w], [(F32, rows * dim * 4)], pc)
    want = orc.rms_norm(x, w, dim, 1e-5)
    assert np.max(np.abs(_read(o, np.float32) - want)) <= 2e-6 * np.max(np.abs(want))
    o.release()
    h = x.astype(np.float16).view(np.uint16)
    (o,) = _run(provider, "rms_norm", [h, w], [(F16, rows * dim * 2)], pc)
    assert _ulp16_ok(_read(o, np.uint16), orc.rms_norm(h, w, dim, 1e-5, f16=True))
    o.release()


@pytest.mark.parametrize("rows,dim", [(1, 32000), (9, 100), (4, 1)])
def test_softmax(provider, rows, dim):
    x = (_rng(dim).standard_normal(rows * dim) * 6).astype(np.float32)
    pc = push_constants(seq_len=rows, head_dim=dim)
    (o,) = _run(provider, "softmax", [x], [(F32, rows * dim * 4)], pc)
    got = _read(o, np.float32)
    o.release()
    # Against the oracle's sequential sum: within its worst-case summation
    # error, (dim - 1) * 2^-24 relative; against float64 within 4e-6 (the
    # tree sum is the more accurate of the two).
    want = orc.softmax(x, rows, dim)
    assert np.all(np.abs(got - want) <= (dim * 2.0 ** -24 + 4e-7) * want + 1e-30)
    x64 = x.reshape(rows, dim).astype(np.float64)
    e = np.exp(x64 - x64.max(axis=1, keepdims=True))
    ref = (e / e.sum(axis=1, keepdims=True)).reshape(-1)
    assert np.all(np.abs(got - ref) <= 4e-6 * ref + 1e-30)


@pytest.mark.parametrize("rows,dim", [(1, 32000), (5, 128256), (8, 3)])
def test_argmax(provider, rows, dim):
    x = _rng(dim).integers(-1000, 1000, rows * dim).astype(np.float32) / 8  # ties
    x[dim // 2] = np.nan
    if rows > 1:
        x[dim] = np.nan  # row 1 starts with NaN -> 0
    pc = push_constants(seq_len=rows, N=dim)
    (o,) = _run(provider, "argmax", [x], [(I32, rows * 4)], pc)
    assert np.array_equal(_read(o, np.int32), orc.argmax(x, rows, dim))
    o.release()


def test_argmax_width_zero_and_softmax_width_zero(provider):
    """transformer_test.cpp:446-447 passes the row width in head_dim, leaving
    N = 0: the reference's argmax then returns 0 for every row; a softmax of
    width 0 writes nothing."""
    x = provider.alloc_array(np.arange(16, dtype=np.float32), F32)
    o = provider.alloc_array(np.full(2, 9, np.int32), I32)
    provider.dispatch("argmax", [x], [o], pc=push_constants(seq_len=2, head_dim=16))
    provider.synchronize()
    assert np.array_equal(o.read(np.int32), [0, 0])
    y = provider.alloc_array(np.full(16, 3.0, np.float32), F32)
    provider.dispatch("softmax", [x], [y], pc=push_constants(seq_len=2, head_dim=0))
    provider.synchronize()
    assert np.all(y.read(np.float32) == 3.0)
    for b in (x, o, y):
        b.release()


@pytest.mark.parametrize("dim", [256, 12, 7])  # 16-byte chunks (both types), f32 only, neither
def test_embedding_lookup(provider, dim):
    vocab, seq = 1000, 12
    w = _rng(5).standard_normal(vocab * dim).astype(np.float32)
    ids = np.array([0, 999, 5, 5, 17, -3, 1000, 123, 456, 789, 1, 2], np.int32)
    pc = push_constants(seq_len=seq, head_dim=dim)
    (o,) = _run(provider, "embedding_lookup", [w, ids], [(F32, seq * dim * 4)], pc)
    assert np.array_equal(_read(o, np.float32), orc.embedding(w, ids, seq * dim, dim, seq))
    o.release()
    wh = w.astype(np.float16).view(np.uint16)
    (o,) = _run(provider, "embedding_lookup", [wh, ids], [(F16, seq * dim * 2)], pc)
    assert np.array_equal(_read(o, np.uint16), orc.embedding(wh, ids, seq * dim, dim, seq, f16=True))
    o.release()


@pytest.mark.parametrize("seq,heads,dim,step,cut", [(5, 4, 64, 0, 0), (3, 8, 128, 100, 0), (1, 32, 64, 17, 0),
                                                   (4, 6, 64, 3, 0), (3, 12, 128, 9, 0), (5, 7, 32, 1, 0),
                                                   (3, 12, 64, 2, 5 * 64), (4, 14, 32, 0, 3 * 32)])
def test_rope_batch_and_rope(provider, seq, heads, dim, step, cut):
    """Head counts with and without a divisor <= 8 (the kernel applies one
    angle to a group of heads of a token), and outputs whose length ends
    inside a token (`cut` elements, whole heads, short of the last one)."""
    x = _rng(seq).standard_normal(seq * heads * dim - cut).astype(np.float32)
    pc = push_constants(n_heads=heads, head_dim=dim, theta=10000.0, step_idx=step)
    # The angle pos * theta^(-2p/d) is formed in fp32 by both sides with powf
    # implementations that may differ by an ulp, so the rotation can differ
    # by ~3e-7 * pos radians: the bound scales with the largest position.
    tol = (3e-7 * (seq + step) + 1e-6) * 2 * float(np.max(np.abs(x)))
    (o,) = _run(provider, "rope_batch", [x], [(F32, x.size * 4)], pc)
    assert np.max(np.abs(_read(o, np.float32) - orc.rope(x, heads, dim, step, 10000.0))) < tol
    o.release()
    h = x.astype(np.float16).view(np.uint16)
    (o,) = _run(provider, "rope_batch", [h], [(F16, x.size * 2)], pc)
    got16 = _read(o, np.uint16)
    assert _ulp16_ok(got16, orc.rope(h, heads, dim, step, 10000.0, f16=True), ulps=1 + tol * 1024)
    o.release()
    # the name the model layer emits in fp16 mode runs the same kernel
    (o,) = _run(provider, "rope_batch_f16", [h], [(F16, x.size * 2)], pc)
    assert np.array_equal(_read(o, np.uint16), got16)
    o.release()
    (o,) = _run(provider, "rope", [x], [(F32, x.size * 4)], pc)
    assert np.max(np.abs(_read(o, np.float32) - orc.rope(x, heads, dim, step, 10000.0, batch=False))) < tol
    o.release()


def test_layer_ops_reject_bad_shapes(provider):
    x = provider.alloc(F32, 100 * 4)
    w = provider.alloc(F32, 64 * 4)
    o = provider.alloc(F32, 100 * 4)
    with pytest.raises(NfError):  # 100 elements are not rows of 64
        provider.dispatch("rms_norm", [x, w], [o], pc=push_constants(head_dim=64, epsilon=1e-5))
    with pytest.raises(NfError):  # no push constants
        provider.dispatch("rms_norm", [x, w], [o])
    with pytest.raises(NfError):  # odd head_dim
        provider.dispatch("rope_batch", [x], [o], pc=push_constants(n_heads=1, head_dim=5, theta=1e4))
    with pytest.raises(NfError):  # softmax rows beyond the buffers
        provider.dispatch("softmax", [x], [o], pc=push_constants(seq_len=2, head_dim=64))
    for b in (x, w, o):
        b.release()


# ---- attention -------------------------------------------------------------------------

def _attn_case(provider, op, f16, H, KV, D, S, step, max_seq, window=0, bs=16, n_blocks=0, q_offset=0, seed=0):
    r = _rng(seed)
    mode = orc.ATTN_VARIANT[op][0]
    decode = mode != 0 and step > 0
    nq = 1 if decode else S
    et = np.uint16 if f16 else np.float32
    edt = F16 if f16 else F32

    def rnd(n):
        x = r.standard_normal(n).astype(np.float32)
        return x.astype(np.float16).view(np.uint16) if f16 else x

    prm = dict(n_heads=H, n_kv=KV, head_dim=D, seq_len=S, step=step, max_seq=max_seq, window=window,
               block_size=bs, n_blocks=n_blocks, q_offset=q_offset)
    pc = push_constants(seq_len=S, n_heads=H, head_dim=D, M=KV if KV != H else 0, N=n_blocks, K=q_offset,
                        step_idx=step, max_seq_len=max_seq, window_size=window if mode != 3 else bs)
    if mode == 0:
        q, k, v = rnd(H * S * D), rnd(H * S * D), rnd(H * S * D)
        want = orc.attention(op, prm, q, k=k.copy(), v=v.copy(), out=np.zeros(q.size, et), f16=f16)
        (o,) = _run(provider, op, [q, k, v], [(edt, q.size * q.itemsize)], pc)
        got = _read(o, et)
        o.release()
        return got, want, None
    if mode == 3:
        pool_blocks = max(n_blocks, 1) + 3
        kp, vp = rnd(pool_blocks * KV * bs * D), rnd(pool_blocks * KV * bs * D)
        table = r.permutation(pool_blocks)[:max(n_blocks, 1)].astype(np.uint32)
        q = rnd((q_offset + nq) * H * D)
        prm["pool_blocks"] = pool_blocks
        want = orc.attention(op, prm, q, k=kp.copy(), v=vp.copy(), table=table, out=np.zeros(q.size, et), f16=f16)
        tb = provider.alloc_array(table.view(np.uint8), abi.NF_DTYPE_U8)
        (o,) = _run(provider, op, [q, kp, vp, tb], [(edt, q.size * q.itemsize)], pc)
        tb.release()
        got = _read(o, et)
        o.release()
        sl = slice(q_offset * H * D, None)
        return got[sl], want[sl], None
    ck, cv = rnd(KV * max_seq * D), rnd(KV * max_seq * D)
    kn, vn, q = rnd(nq * KV * D), rnd(nq * KV * D), rnd(nq * H * D)
    ck_o, cv_o = ck.copy(), cv.copy()
    want = orc.attention(op, prm, q, kn, vn, ck_o, cv_o, out=np.zeros(q.size, et), f16=f16)
    bk, bv = provider.alloc_array(ck, edt), provider.alloc_array(cv, edt)
    (o,) = _run(provider, op, [q, kn, vn, bk, bv], [(edt, q.size * q.itemsize)], pc)
    got = _read(o, et)
    caches = (bk.read(et), bv.read(et), ck_o, cv_o)
    for b in (o, bk, bv):
        b.release()
    return got, want, caches


GPU_ATTN = [
    ("causal_attention", False, dict(H=4, KV=4, D=64, S=50, step=0, max_seq=0)),
    # prefill shapes of the many-queries-per-workgroup kernel: a partial last
    # query block, head_dim below 128, and head_dim 256 (the per-query kernel)
    ("flash_attention_gqa", True, dict(H=16, KV=4, D=128, S=100, step=0, max_seq=128)),
    ("causal_attention_cached", False, dict(H=4, KV=2, D=96, S=33, step=0, max_seq=40)),
    ("flash_attention_cached", False, dict(H=2, KV=1, D=256, S=20, step=0, max_seq=32)),
    ("causal_attention_cached", False, dict(H=8, KV=2, D=64, S=70, step=0, max_seq=80)),
    ("causal_attention_cached", False, dict(H=8, KV=2, D=128, S=1, step=300, max_seq=512, window=100)),
    ("flash_attention_cached", False, dict(H=4, KV=4, D=128, S=130, step=0, max_seq=160, window=40)),
    ("flash_attention_cached", False, dict(H=32, KV=8, D=128, S=1, step=2000, max_seq=2048)),
    ("flash_attention_cached", True, dict(H=8, KV=2, D=64, S=40, step=0, max_seq=64)),
    ("flash_attention_cached", True, dict(H=8, KV=2, D=64, S=1, step=63, max_seq=64)),
    ("flash_attention_gqa", False, dict(H=8, KV=2, D=64, S=65, step=0, max_seq=80)),
    ("flash_attention_gqa", False, dict(H=32, KV=8, D=128, S=1, step=777, max_seq=1024)),
    ("flash_attention_gqa", True, dict(H=8, KV=2, D=96, S=1, step=200, max_seq=256)),
    ("flash_attention_paged", False, dict(H=4, KV=4, D=64, S=1, step=37, max_seq=0, bs=16, n_blocks=3)),
    ("flash_attention_paged", False, dict(H=8, KV=2, D=128, S=24, step=0, max_seq=0, bs=8, n_blocks=3, q_offset=2)),
    ("flash_attention_paged", False, dict(H=2, KV=1, D=64, S=1, step=500, max_seq=0, bs=16, n_blocks=20)),
    # f16 prefill on MFMA (head_dim 64 / 128): a sliding window, ragged last
    # query and key blocks, 32 heads over 8 KV heads
    ("flash_attention_cached", True, dict(H=4, KV=4, D=128, S=130, step=0, max_seq=160, window=40)),
    ("flash_attention_gqa", True, dict(H=8, KV=2, D=64, S=257, step=0, max_seq=300)),
    ("flash_attention_cached", True, dict(H=32, KV=8, D=128, S=200, step=0, max_seq=256)),
    # f32 prefill on fp32 MFMA (head_dim 64 / 128; the cases above with those
    # head_dims take it too): 32 heads over 8 KV heads, ragged last blocks
    ("flash_attention_cached", False, dict(H=32, KV=8, D=128, S=200, step=0, max_seq=256)),
    ("flash_attention_gqa", False, dict(H=8, KV=2, D=128, S=97, step=0, max_seq=128)),
    # f16 decode with the scores on MFMA (head_dim 64 / 128): partial last
    # tiles, groups of 1 / 3 / 4 / 8 query heads, a sliding window, a 6-key
    # cache (the paged op is f32-only, as in the reference)
    ("flash_attention_cached", True, dict(H=32, KV=8, D=128, S=1, step=2000, max_seq=2048)),
    ("flash_attention_cached", True, dict(H=8, KV=2, D=128, S=1, step=300, max_seq=512, window=100)),
    ("flash_attention_gqa", True, dict(H=32, KV=8, D=128, S=1, step=777, max_seq=1024)),
    ("flash_attention_gqa", True, dict(H=8, KV=1, D=64, S=1, step=100, max_seq=128)),
    ("flash_attention_gqa", True, dict(H=6, KV=2, D=64, S=1, step=70, max_seq=128)),
    ("flash_attention_gqa", True, dict(H=4, KV=4, D=128, S=1, step=5, max_seq=16)),
]


@pytest.mark.parametrize("op,f16,kw", GPU_ATTN, ids=[f"{o}-{'f16' if h else 'f32'}-{i}" for i, (o, h, _) in enumerate(GPU_ATTN)])
def test_attention(provider, op, f16, kw):
    got, want, caches = _attn_case(provider, op, f16, seed=len(kw) + kw["S"], **kw)
    if f16:
        # MFMA sums keys and head_dim in another fp32 order than the
        # reference's sequential loops (bound: 1e-5 of the output scale)
        assert _ulp16_ok(got, want, ulps=2, abs_frac=1e-5), op
    else:
        assert np.max(np.abs(got - want)) <= 2e-5 * np.max(np.abs(want)), op
    if caches is not None:
        gk, gv, wk, wv = caches
        assert np.array_equal(gk, wk) and np.array_equal(gv, wv), "cache append"


@pytest.mark.parametrize("op,kw,bad,f16", [
    ("causal_attention", dict(H=4, KV=4, D=64, S=50, step=0, max_seq=0), 40, False),
    ("flash_attention_cached", dict(H=4, KV=4, D=128, S=130, step=0, max_seq=160, window=40), 10, False),
    ("flash_attention_cached", dict(H=4, KV=4, D=128, S=130, step=0, max_seq=160, window=40), 10, True),
    ("flash_attention_gqa", dict(H=8, KV=2, D=64, S=70, step=0, max_seq=80), 33, False),
    ("flash_attention_gqa", dict(H=8, KV=2, D=64, S=70, step=0, max_seq=80), 33, True)],
    ids=["causal-f32", "cached-window-f32", "cached-window-f16", "gqa-f32", "gqa-f16"])
def test_attention_prefill_nonfinite_value_row(provider, op, kw, bad, f16):
    """An infinite value in the V row of token `bad` reaches only the queries
    whose key range holds that token (the per-query reference kernel never
    reads a row outside the range): every query the oracle keeps finite is
    finite on the GPU too and matches it."""
    H, KV, D, S, max_seq, window = kw["H"], kw["KV"], kw["D"], kw["S"], kw["max_seq"], kw.get("window", 0)
    r = _rng(bad)
    et, edt = (np.uint16, F16) if f16 else (np.float32, F32)
    inf = np.array([np.inf], np.float16).view(np.uint16)[0] if f16 else np.float32(np.inf)

    def rnd(n):
        x = r.standard_normal(n).astype(np.float32)
        return x.astype(np.float16).view(np.uint16) if f16 else x

    mode = orc.ATTN_VARIANT[op][0]
    prm = dict(n_heads=H, n_kv=KV, head_dim=D, seq_len=S, step=0, max_seq=max_seq, window=window)
    pc = push_constants(seq_len=S, n_heads=H, head_dim=D, M=KV if KV != H else 0, step_idx=0,
                        max_seq_len=max_seq, window_size=window)
    if mode == 0:  # Q, K, V, out [n_heads, seq, dim]
        q, k, v = rnd(H * S * D), rnd(H * S * D), rnd(H * S * D)
        v.reshape(H, S, D)[:, bad, 3] = inf
        want = orc.attention(op, prm, q, k=k.copy(), v=v.copy(), out=np.zeros(q.size, et), f16=f16)
        (o,) = _run(provider, op, [q, k, v], [(edt, q.size * q.itemsize)], pc)
        got = _read(o, et)
        o.release()
        qrows = lambda a: a.reshape(H, S, D).transpose(1, 0, 2)  # noqa: E731
    else:
        ck, cv = rnd(KV * max_seq * D), rnd(KV * max_seq * D)
        kn, vn, q = rnd(S * KV * D), rnd(S * KV * D), rnd(S * H * D)
        if mode == 1:  # K_new / V_new [seq, n_kv, dim], Q / out [seq, n_heads, dim]
            vn.reshape(S, KV, D)[bad, :, 3] = inf
            qrows = lambda a: a.reshape(S, H, D)  # noqa: E731
        else:  # [n_kv, seq, dim], Q / out [n_heads, seq, dim]
            vn.reshape(KV, S, D)[:, bad, 3] = inf
            qrows = lambda a: a.reshape(H, S, D).transpose(1, 0, 2)  # noqa: E731
        want = orc.attention(op, prm, q, kn, vn, ck.copy(), cv.copy(), out=np.zeros(q.size, et), f16=f16)
        bk, bv = provider.alloc_array(ck, edt), provider.alloc_array(cv, edt)
        (o,) = _run(provider, op, [q, kn, vn, bk, bv], [(edt, q.size * q.itemsize)], pc)
        got = _read(o, et)
        for b in (o, bk, bv):
            b.release()
    gf = qrows(got.view(np.float16).astype(np.float32) if f16 else got)
    wf = qrows(want.view(np.float16).astype(np.float32) if f16 else want)
    clean = np.isfinite(wf).all(axis=(1, 2))
    assert clean[:bad].all() and not clean.all(), "the case must have clean and affected queries"
    assert np.isfinite(gf[clean]).all(), f"non-finite output in queries {np.flatnonzero(~np.isfinite(gf).all(axis=(1, 2)) & clean)}"
    if f16:
        assert _ulp16_ok(qrows(got)[clean], qrows(want)[clean], ulps=2, abs_frac=1e-5)
    else:
        assert np.max(np.abs(gf[clean] - wf[clean])) <= 2e-5 * np.max(np.abs(wf[clean]))


def test_attention_decode_past_cache_is_noop(provider):
    H, KV, D, max_seq = 4, 2, 32, 8
    out = provider.alloc_array(np.full(H * D, 5.0, np.float32), F32)
    ck = provider.alloc(F32, KV * max_seq * D * 4)
    cv = provider.alloc(F32, KV * max_seq * D * 4)
    q, kn, vn = (np.ones(n, np.float32) for n in (H * D, KV * D, KV * D))
    pc = push_constants(seq_len=1, n_heads=H, head_dim=D, M=KV, step_idx=max_seq, max_seq_len=max_seq)
    _run(provider, "flash_attention_cached", [q, kn, vn, ck, cv], [out], pc)
    assert np.all(out.read(np.float32) == 5.0) and not ck.read(np.float32).any()
    for b in (out, ck, cv):
        b.release()


def test_attention_rejects_prefill_longer_than_cache(provider):
    H, D = 2, 16
    q = provider.alloc(F32, 10 * H * D * 4)
    c = provider.alloc(F32, H * 8 * D * 4)
    o = provider.alloc(F32, 10 * H * D * 4)
    pc = push_constants(seq_len=10, n_heads=H, head_dim=D, step_idx=0, max_seq_len=8)
    with pytest.raises(NfError):
        provider.dispatch("flash_attention_cached", [q, q, q, c, c], [o], pc=pc)
    for b in (q, c, o):
        b.release()


# ---- MoE (metal_provider.mm:1907-1997) -------------------------------------------

@pytest.mark.parametrize("batch,n,top_k", [(1, 8, 2), (37, 64, 8), (300, 100, 4), (5, 3, 12), (4, 6, 4)])
def test_moe_top_k_gating(provider, batch, n, top_k):
    rng = _rng(batch + n)
    if n == 6:   # ties everywhere: the lowest expert ids win
        logits = np.zeros((batch, n), np.float32)
    else:        # a 1/16 grid: selections are decided, not rounding accidents
        logits = (rng.integers(-64, 64, size=(batch, n)) / 16.0).astype(np.float32)
    k = min(top_k, 8)
    pc = push_constants(seq_len=batch, M=n, N=top_k)
    ids_o, w_o = _run(provider, "moe_top_k_gating", [logits], [(I32, batch * k * 4), (F32, batch * k * 4)], pc)
    ids, w = orc.moe_gate(logits, batch, n, top_k)
    assert np.array_equal(_read(ids_o, np.int32).reshape(batch, k), ids)
    # expf of the device and of libm may differ by an ulp: weights to a few ulps
    assert np.allclose(_read(w_o, np.float32).reshape(batch, k), w, rtol=1e-6, atol=1e-7)
    ids_o.release()
    w_o.release()


def test_moe_scatter_gather(provider):
    rng = _rng(77)
    n_exp, dim, batch, top_k = 8, 4096 + 3, 33, 2
    E = rng.standard_normal((n_exp, dim)).astype(np.float32)
    ids = rng.integers(-1, n_exp + 2, size=(batch, top_k)).astype(np.int32)   # includes -1 and ids past the rows
    w = rng.random((batch, top_k)).astype(np.float32)
    pc = push_constants(seq_len=batch, M=n_exp, N=top_k, K=dim)
    (o,) = _run(provider, "moe_scatter_gather", [E, ids, w], [(F32, batch * dim * 4)], pc)
    assert np.array_equal(_read(o, np.float32).reshape(batch, dim), orc.moe_scatter(E, ids, w, batch, top_k, dim))
    o.release()


def test_moe_gating_then_scatter_chain(provider):
    """Gate logits -> top-2 ids and weights -> weighted sum of expert rows,
    buffers passed from one op to the next on the device."""
    rng = _rng(3)
    batch, n_exp, dim = 16, 8, 256
    logits = (rng.integers(-64, 64, size=(batch, n_exp)) / 16.0).astype(np.float32)
    E = rng.standard_normal((n_exp, dim)).astype(np.float32)
    ids_o, w_o = _run(provider, "moe_top_k_gating", [logits], [(I32, batch * 8), (F32, batch * 8)],
                      push_constants(seq_len=batch, M=n_exp, N=2))
    (o,) = _run(provider, "moe_scatter_gather", [E, ids_o, w_o], [(F32, batch * dim * 4)],
                push_constants(seq_len=batch, M=n_exp, N=2, K=dim))
    ids, w = orc.moe_gate(logits, batch, n_exp, 2)
    want = orc.moe_scatter(E, ids, _read(w_o, np.float32).reshape(batch, 2), batch, 2, dim)
    assert np.array_equal(_read(o, np.float32).reshape(batch, dim), want)
    for b in (ids_o, w_o, o):
        b.release()
