"""Pins the oracle's restatement of the layer ops (silu, gelu, relu, add,
mul, rms_norm, rope / rope_batch, softmax, argmax, embedding_lookup and the
five attention ops) before the GPU is checked against it.

Each is checked against an independent float64 (or exact) evaluation of the
op's mathematics in numpy, written from the kernel text's layouts
(metal_provider.mm), and against closed forms and invariants: silu(0) = 0,
rope at position 0 is the identity and preserves pair norms, softmax rows
sum to 1, a constant row normalises to w / sqrt(1 + eps / c^2), one key
returns its value row, the attention variants (two-pass, 32-key tiles,
per-key and per-block online softmax) agree with each other and with the
float64 attention for every layout, GQA head mapping, sliding window and
paged block table.  The last test plants plausible mistakes (a wrong KV
head map, a missing scale, an off-by-one window, swapped rope halves, a
paged table ignored) and checks that the same pins reject them.
"""
import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.filterwarnings("ignore::RuntimeWarning")


def _rng(seed):
    return np.random.default_rng(seed)


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


# ---- element-wise ------------------------------------------------------------------

def test_unary_against_float64():
    x = np.concatenate([np.linspace(-20, 20, 4001), _rng(1).standard_normal(5000) * 3]).astype(np.float32)
    x64 = x.astype(np.float64)
    silu = x64 / (1 + np.exp(-x64))
    gelu = 0.5 * x64 * (1 + np.tanh(0.7978845608 * (x64 + 0.044715 * x64 ** 3)))
    assert np.all(np.abs(orc.unary("silu", x) - silu) <= 4e-7 * np.maximum(np.abs(silu), 1e-3))
    # 1 + tanh(.) cancels for negative x: its fp32 rounding (2^-24 absolute)
    # is scaled by 0.5|x|, so the bound carries that term
    assert np.all(np.abs(orc.unary("gelu", x) - gelu) <= 4e-7 * np.abs(gelu) + 3e-7 * np.abs(x64) + 1e-30)
    assert np.array_equal(orc.unary("relu", x), np.maximum(x, 0))
    assert orc.unary("silu", np.zeros(1, np.float32))[0] == 0.0


def test_unary_f16_is_rne_of_f32():
    h = _rng(2).standard_normal(4096).astype(np.float16)
    f32 = orc.unary("silu", h.astype(np.float32))
    assert np.array_equal(orc.unary("silu", h.view(np.uint16), f16=True), f32.astype(np.float16).view(np.uint16))


def test_binary_exact():
    a, b = _rng(3).standard_normal((2, 10000)).astype(np.float32)
    assert np.array_equal(orc.binary("add", a, b), a + b)
    assert np.array_equal(orc.binary("mul", a, b), a * b)
    # f16: every pair of a grid of halves, against numpy's half arithmetic
    ha = _rng(4).standard_normal(20000).astype(np.float16) * np.float16(100)
    hb = (_rng(5).standard_normal(20000) * np.exp2(_rng(6).integers(-20, 10, 20000))).astype(np.float16)
    assert np.array_equal(orc.binary("add", ha.view(np.uint16), hb.view(np.uint16), f16=True), (ha + hb).view(np.uint16))
    assert np.array_equal(orc.binary("mul", ha.view(np.uint16), hb.view(np.uint16), f16=True), (ha * hb).view(np.uint16))


# ---- rms_norm, softmax, argmax, embedding ------------------------------------------

def test_rms_norm():
    dim, rows, eps = 256, 7, 1e-5
    x = _rng(7).standard_normal(rows * dim).astype(np.float32)
    w = _rng(8).standard_normal(dim).astype(np.float32)
    x64 = x.reshape(rows, dim).astype(np.float64)
    want = x64 / np.sqrt(np.mean(x64 ** 2, axis=1, keepdims=True) + eps) * w
    assert _rel(orc.rms_norm(x, w, dim, eps).reshape(rows, dim), want) < 2e-6
    c = np.full(dim, 3.0, np.float32)
    got = orc.rms_norm(c, np.ones(dim, np.float32), dim, 0.0)
    assert np.allclose(got, 1.0, rtol=2e-7)


def test_softmax():
    rows, dim = 5, 1000
    x = (_rng(9).standard_normal(rows * dim) * 5).astype(np.float32)
    got = orc.softmax(x, rows, dim).reshape(rows, dim)
    x64 = x.reshape(rows, dim).astype(np.float64)
    e = np.exp(x64 - x64.max(axis=1, keepdims=True))
    assert _rel(got, e / e.sum(axis=1, keepdims=True)) < 2e-6
    assert np.allclose(got.sum(axis=1), 1.0, atol=1e-5)
    assert np.array_equal(orc.softmax(x + np.float32(0.0), rows, dim), orc.softmax(x, rows, dim))


def test_argmax():
    rows, dim = 50, 1000
    x = _rng(10).integers(-50, 50, (rows, dim)).astype(np.float32)  # many ties
    assert np.array_equal(orc.argmax(x, rows, dim), np.argmax(x, axis=1).astype(np.int32))
    y = x.copy()
    y[0, 0] = np.nan  # a NaN first element: the strict > scan never moves
    y[1, 5] = np.nan  # a NaN later on is never taken
    got = orc.argmax(y, rows, dim)
    assert got[0] == 0 and got[1] == np.nanargmax(y[1])


def test_embedding():
    vocab, dim, seq = 100, 64, 9
    w = _rng(11).standard_normal((vocab, dim)).astype(np.float32)
    ids = np.array([3, 0, 99, 42, 42, -1, 100, 7, 5], np.int32)
    got = orc.embedding(w, ids, seq * dim, dim, seq).reshape(seq, dim)
    for t, tok in enumerate(ids):
        assert np.array_equal(got[t], w[tok] if 0 <= tok < vocab else np.zeros(dim, np.float32))
    # elements past seq_len rows are untouched
    out = np.full((seq + 2) * dim, 7.0, np.float32)
    orc.embedding(w, ids, out.size, dim, seq, out=out)
    assert np.all(out[seq * dim:] == 7.0)


# ---- rope ----------------------------------------------------------------------------

def _rope64(x, n_heads, dim, step, theta, batch=True):
    x = x.astype(np.float64).reshape(-1, dim)
    half = dim // 2
    rows = np.arange(x.shape[0])
    pos = (rows // n_heads + step) if batch else np.full(x.shape[0], step)
    p = np.arange(half)
    freq = 1.0 / np.power(np.float64(np.float32(theta)), (2.0 * p) / dim)
    ang = pos[:, None] * freq[None, :]
    c, s = np.cos(ang), np.sin(ang)
    x0, x1 = x[:, :half], x[:, half:]
    return np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], axis=1).reshape(-1)


def test_rope_batch_and_rope():
    seq, heads, dim, theta = 6, 4, 64, 10000.0
    x = _rng(12).standard_normal(seq * heads * dim).astype(np.float32)
    got = orc.rope(x, heads, dim, 3, theta)
    assert np.max(np.abs(got - _rope64(x, heads, dim, 3, theta))) < 3e-5
    assert np.array_equal(orc.rope(x, heads, dim, 0, theta)[: heads * dim], x[: heads * dim])  # position 0
    g = got.reshape(-1, dim).astype(np.float64)
    xx = x.reshape(-1, dim).astype(np.float64)
    assert np.allclose(g[:, :32] ** 2 + g[:, 32:] ** 2, xx[:, :32] ** 2 + xx[:, 32:] ** 2, rtol=1e-5)
    single = orc.rope(x, heads, dim, 5, theta, batch=False)
    assert np.max(np.abs(single - _rope64(x, heads, dim, 5, theta, batch=False))) < 3e-5


# ---- attention -----------------------------------------------------------------------

def _attn64(q, k, v, lo_hi):
    """Softmax attention of one query row against key rows [lo, hi]."""
    lo, hi = lo_hi
    if hi < lo:
        return np.zeros(q.shape[-1])
    s = k[lo:hi + 1] @ q / np.sqrt(q.shape[-1])
    p = np.exp(s - s.max())
    return (p / p.sum()) @ v[lo:hi + 1]


def _case(op, H, KV, D, S, step, max_seq, window=0, seed=0, bs=16, n_blocks=0, q_offset=0, kv_map=None,
          scale_fix=True):
    """Build inputs, run the oracle and a float64 evaluation from the layouts."""
    r = _rng(seed)
    mode = orc.ATTN_VARIANT[op][0]
    decode = mode != 0 and step > 0
    nq = 1 if decode else S
    kvmap = kv_map or (lambda h: h * KV // H)
    prm = dict(n_heads=H, n_kv=KV, head_dim=D, seq_len=S, step=step, max_seq=max_seq, window=window)
    out = np.zeros((q_offset + nq) * H * D if mode == 3 else nq * H * D, np.float32)
    if mode == 0:
        q, k, v = (r.standard_normal(H * S * D).astype(np.float32) for _ in range(3))
        orc.attention(op, prm, q, k=k, v=v, out=out)
        q3, k3, v3 = (a.reshape(H, S, D).astype(np.float64) for a in (q, k, v))
        want = np.stack([[_attn64(q3[h, i], k3[h], v3[h], (0, i)) for i in range(S)] for h in range(H)])
        return out.reshape(H, S, D), want
    if mode == 3:
        pool_blocks = max(n_blocks, 1) + 2
        kp = r.standard_normal(pool_blocks * KV * bs * D).astype(np.float32)
        vp = r.standard_normal(pool_blocks * KV * bs * D).astype(np.float32)
        table = r.permutation(pool_blocks)[:max(n_blocks, 1)].astype(np.uint32)
        q = r.standard_normal((q_offset + nq) * H * D).astype(np.float32)
        prm.update(block_size=bs, n_blocks=n_blocks, q_offset=q_offset, pool_blocks=pool_blocks)
        orc.attention(op, prm, q, k=kp, v=vp, table=table, out=out)
        k5 = kp.reshape(pool_blocks, KV, bs, D).astype(np.float64)
        v5 = vp.reshape(pool_blocks, KV, bs, D).astype(np.float64)
        ntok = n_blocks * bs
        kl = np.concatenate([k5[table[b]] for b in range(n_blocks)], axis=1) if n_blocks else np.zeros((KV, 0, D))
        vl = np.concatenate([v5[table[b]] for b in range(n_blocks)], axis=1) if n_blocks else np.zeros((KV, 0, D))
        q3 = q.reshape(q_offset + nq, H, D).astype(np.float64)
        want = np.zeros((q_offset + nq, H, D))
        for i in range(nq):
            pos = step if decode else i
            for h in range(H):
                want[q_offset + i, h] = _attn64(q3[q_offset + i, h], kl[kvmap(h)], vl[kvmap(h)], (0, min(pos, ntok - 1)))
        return out.reshape(q_offset + nq, H, D)[q_offset:], want[q_offset:]
    # cached / gqa: the cache holds earlier positions, the op appends the new rows
    ck = r.standard_normal(KV * max_seq * D).astype(np.float32)
    cv = r.standard_normal(KV * max_seq * D).astype(np.float32)
    ntok = nq
    kn = r.standard_normal(ntok * KV * D).astype(np.float32)
    vn = r.standard_normal(ntok * KV * D).astype(np.float32)
    q = r.standard_normal(nq * H * D).astype(np.float32)
    ck0, cv0 = ck.copy(), cv.copy()
    orc.attention(op, prm, q, kn, vn, ck, cv, out=out)
    c4 = ck0.reshape(KV, max_seq, D).astype(np.float64)
    v4 = cv0.reshape(KV, max_seq, D).astype(np.float64)
    if mode == 1:
        kn3, vn3 = kn.reshape(ntok, KV, D).transpose(1, 0, 2), vn.reshape(ntok, KV, D).transpose(1, 0, 2)
        q3 = q.reshape(nq, H, D).astype(np.float64)
    else:
        kn3, vn3 = kn.reshape(KV, ntok, D), vn.reshape(KV, ntok, D)
        q3 = q.reshape(H, nq, D).transpose(1, 0, 2).astype(np.float64)
    first = step if decode else 0
    c4[:, first:first + ntok], v4[:, first:first + ntok] = kn3, vn3
    assert np.array_equal(ck.reshape(KV, max_seq, D), c4.astype(np.float32))  # the append
    want = np.zeros((nq, H, D))
    for i in range(nq):
        pos = step if decode else i
        lo = pos - window + 1 if (mode == 1 and window > 0 and pos >= window) else 0
        for h in range(H):
            want[i, h] = _attn64(q3[i, h], c4[kvmap(h)], v4[kvmap(h)], (lo, pos))
    got = out.reshape(nq, H, D) if mode == 1 else out.reshape(H, nq, D).transpose(1, 0, 2)
    return got, want


ATTN_CASES = [
    ("causal_attention", dict(H=3, KV=3, D=32, S=20, step=0, max_seq=0)),
    ("causal_attention_cached", dict(H=4, KV=4, D=64, S=40, step=0, max_seq=64)),
    ("causal_attention_cached", dict(H=8, KV=2, D=64, S=1, step=37, max_seq=64)),
    ("causal_attention_cached", dict(H=4, KV=2, D=32, S=30, step=0, max_seq=40, window=8)),
    ("flash_attention_cached", dict(H=4, KV=4, D=128, S=70, step=0, max_seq=80)),
    ("flash_attention_cached", dict(H=8, KV=2, D=64, S=1, step=100, max_seq=128, window=33)),
    ("flash_attention_gqa", dict(H=8, KV=2, D=64, S=33, step=0, max_seq=40)),
    ("flash_attention_gqa", dict(H=8, KV=2, D=64, S=1, step=90, max_seq=128)),
    ("flash_attention_paged", dict(H=4, KV=4, D=64, S=1, step=37, max_seq=0, bs=16, n_blocks=3)),
    ("flash_attention_paged", dict(H=4, KV=2, D=32, S=20, step=0, max_seq=0, bs=8, n_blocks=3, q_offset=2)),
    ("flash_attention_paged", dict(H=2, KV=1, D=32, S=1, step=50, max_seq=0, bs=16, n_blocks=2)),
]


@pytest.mark.parametrize("op,kw", ATTN_CASES, ids=[f"{o}-{i}" for i, (o, _) in enumerate(ATTN_CASES)])
def test_attention_against_float64(op, kw):
    got, want = _case(op, **kw)
    assert _rel(got, want) < 2e-5, (op, kw)


def test_attention_variants_agree_and_one_key():
    # two-pass (causal_attention_cached) vs 32-key tiles (flash_attention_cached)
    a, _ = _case("causal_attention_cached", H=4, KV=2, D=64, S=50, step=0, max_seq=64, seed=3)
    b, _ = _case("flash_attention_cached", H=4, KV=2, D=64, S=50, step=0, max_seq=64, seed=3)
    assert _rel(a, b) < 2e-6
    # the first query sees one key: its value row
    got, want = _case("causal_attention", H=2, KV=2, D=16, S=4, step=0, max_seq=0, seed=4)
    assert _rel(got[:, 0], want[:, 0]) < 1e-6


def test_attention_decode_past_cache_is_a_noop():
    out = np.full(4 * 32, 5.0, np.float32)
    ck = np.zeros(2 * 8 * 32, np.float32)
    cv = ck.copy()
    prm = dict(n_heads=4, n_kv=2, head_dim=32, seq_len=1, step=8, max_seq=8)
    orc.attention("flash_attention_cached", prm, np.ones(4 * 32, np.float32), np.ones(64, np.float32),
                  np.ones(64, np.float32), ck, cv, out=out)
    assert np.all(out == 5.0) and not ck.any()


# ---- planted mistakes -----------------------------------------------------------------

def test_planted_mistakes_are_caught():
    # the KV head map h % n_kv instead of h * n_kv / n_heads
    got, _ = _case("flash_attention_gqa", H=8, KV=2, D=32, S=1, step=20, max_seq=32, seed=5)
    _, wrong = _case("flash_attention_gqa", H=8, KV=2, D=32, S=1, step=20, max_seq=32, seed=5, kv_map=lambda h: h % 2)
    assert _rel(got, wrong) > 1e-3
    # an off-by-one sliding window
    got, _ = _case("causal_attention_cached", H=2, KV=2, D=32, S=30, step=0, max_seq=32, window=8, seed=6)
    _, w9 = _case("causal_attention_cached", H=2, KV=2, D=32, S=30, step=0, max_seq=32, window=9, seed=6)
    assert _rel(got, w9) > 1e-3
    # a missing 1/sqrt(head_dim) scale
    q = _rng(7).standard_normal(32).astype(np.float32)
    k = _rng(8).standard_normal((5, 32))
    v = _rng(9).standard_normal((5, 32))
    s = k @ q
    p = np.exp(s - s.max())
    assert _rel(_attn64(q.astype(np.float64), k, v, (0, 4)), (p / p.sum()) @ v) > 1e-3
    # rope with its two halves swapped
    x = _rng(10).standard_normal(4 * 64).astype(np.float32)
    sw = x.reshape(-1, 64)[:, ::-1].reshape(-1).copy()
    assert np.max(np.abs(orc.rope(sw, 1, 64, 3, 10000.0) - _rope64(x, 1, 64, 3, 10000.0))) > 1e-2
    # a paged lookup that ignores the block table (identity mapping)
    got, want = _case("flash_attention_paged", H=2, KV=1, D=32, S=1, step=40, max_seq=0, bs=16, n_blocks=3, seed=11)
    assert _rel(got, want) < 2e-5
    r = _rng(11)
    pool_blocks = 5
    kp = r.standard_normal(pool_blocks * 16 * 32)
    vp = r.standard_normal(pool_blocks * 16 * 32)
    table = r.permutation(pool_blocks)[:3]
    if not np.array_equal(table, np.arange(3)):
        q3 = r.standard_normal(2 * 32)
        ident = _attn64(q3[:32], kp.reshape(pool_blocks, 16, 32)[:3].reshape(-1, 32),
                        vp.reshape(pool_blocks, 16, 32)[:3].reshape(-1, 32), (0, 40))
        mapped = _attn64(q3[:32], kp.reshape(pool_blocks, 16, 32)[table].reshape(-1, 32),
                         vp.reshape(pool_blocks, 16, 32)[table].reshape(-1, 32), (0, 40))
        assert _rel(ident, mapped) > 1e-3


# ---- MoE gating / scatter-gather (metal_provider.mm:1907-1997) ------------------

def _gate64(logits, n, top_k):
    """float64 restatement from the definition: softmax over the first
    min(n, 64) experts (the max taken over all n), the top_k (<= 8) largest,
    earlier expert first on ties, zero probabilities never selected,
    renormalized."""
    k = min(top_k, 8)
    ne = min(n, 64)
    ids = np.full((logits.shape[0], k), -1, np.int64)
    w = np.zeros((logits.shape[0], k))
    for b, row in enumerate(logits.astype(np.float64)):
        p = np.exp(row[:ne] - row.max())
        p /= p.sum()
        order = sorted(range(ne), key=lambda i: (-p[i], i))
        sel = [i for i in order[:k] if p[i] > 0]
        ids[b, :len(sel)] = sel
        s = sum(p[i] for i in sel)
        w[b, :len(sel)] = [p[i] / s for i in sel]
    return ids, w


@pytest.mark.parametrize("n,top_k", [(1, 1), (5, 2), (8, 2), (8, 8), (64, 4), (100, 8), (40, 12)])
def test_oracle_moe_gate_against_float64(n, top_k):
    rng = _rng(n * 31 + top_k)
    # logits on a 1/16 grid: distinct probabilities are >= 6 % apart, so the
    # selection is decided, not a rounding accident
    logits = (rng.integers(-64, 64, size=(37, n)) / 16.0).astype(np.float32)
    ids, w = orc.moe_gate(logits, 37, n, top_k)
    ids64, w64 = _gate64(logits, n, top_k)
    assert np.array_equal(ids, ids64)
    assert np.max(np.abs(w - w64)) < 2e-6
    assert np.all(ids < 64)                       # experts past the 64th never selected
    sel = ids >= 0
    assert np.allclose(np.where(sel, w, 0).sum(1), 1.0, atol=2e-6)


def test_oracle_moe_gate_ties_underflow_and_empty():
    ids, w = orc.moe_gate(np.zeros((2, 6), np.float32), 2, 6, 4)      # all tied: lowest ids, equal weights
    assert ids.tolist() == [[0, 1, 2, 3]] * 2 and np.allclose(w, 0.25)
    lg = np.zeros((1, 5), np.float32)
    lg[0, 3] = 1000.0                                                 # exp(-1000) = 0: never selected
    ids, w = orc.moe_gate(lg, 1, 5, 3)
    assert ids.tolist() == [[3, -1, -1]] and w.tolist() == [[1.0, 0.0, 0.0]]
    ids, w = orc.moe_gate(np.zeros(0, np.float32), 2, 0, 2)            # no experts
    assert ids.tolist() == [[-1, -1]] * 2 and not w.any()
    # a planted mistake: '>=' in the insertion would put the LAST tied expert first
    lg = np.array([[1.0, 1.0, 0.0]], np.float32)
    assert orc.moe_gate(lg, 1, 3, 1)[0].tolist() == [[0]]


def test_oracle_moe_scatter_against_float64():
    rng = _rng(5)
    E = rng.standard_normal((6, 40)).astype(np.float32)
    ids = np.array([[0, 5], [-1, 2], [7, 1], [3, -1]], np.int32)     # -1 and 7 (past the 6 rows) skipped
    w = rng.random((4, 2)).astype(np.float32)
    out = orc.moe_scatter(E, ids, w, 4, 2, 40)
    want = np.zeros((4, 40))
    for b in range(4):
        for k in range(2):
            if 0 <= ids[b, k] < 6:
                want[b] += float(w[b, k]) * E[ids[b, k]].astype(np.float64)
    assert np.max(np.abs(out - want)) < 1e-6
