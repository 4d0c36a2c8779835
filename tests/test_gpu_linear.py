"""Fused dequant+linear and dense linear parity on the GPU, through the C ABI.

Every case compares the HIP result with the CPU oracle (the restated
reference dequant + sequential-k loop) on identical seeded inputs, within
max relative error 1e-3 (mixed and normwise, tests/helpers.py).  Shapes:
the reference's own fused cases (fused_matmul_test.cpp:294-297), its
linear_tiled case (dequant_test.cpp:300-394), decode edge cases (M=1,
N not a multiple of any tile, ragged K), config shapes, and both sides of the
GEMV/MFMA switch.  Config-sized prefill shapes are checked on a sample of
output columns (the oracle computes only those), which is exact for the
sampled entries.
"""
import numpy as np
import pytest

from helpers import assert_close
from neurofabric_amd import abi
from neurofabric_amd import synthetic as syn

pytestmark = pytest.mark.gpu

QDT = {"q4_0": abi.NF_DTYPE_Q4_0, "q8_0": abi.NF_DTYPE_Q8_0}


def run_fused(provider, fmt, A, W, M, N, K, f16):
    op = f"dequant_{fmt}_linear" + ("_f16" if f16 else "")
    a = provider.alloc_array(A, abi.NF_DTYPE_F16 if f16 else abi.NF_DTYPE_F32)
    w = provider.alloc_array(W, QDT[fmt])
    c = provider.alloc(abi.NF_DTYPE_F16 if f16 else abi.NF_DTYPE_F32, M * N * (2 if f16 else 4))
    provider.dispatch(op, [a, w], [c], M, N, K)
    provider.synchronize()
    got = c.download(np.float16 if f16 else np.float32).reshape(M, N)
    for b in (a, w, c):
        b.release()
    return got


def check_fused(provider, oracle_mod, fmt, M, N, K, f16, seed=0, cols=None, threads=8):
    W = syn.weights(fmt, N, K, seed=seed)
    A = syn.activations(M, K, seed=seed + 1, dtype=np.float16 if f16 else np.float32)
    got = run_fused(provider, fmt, A, W, M, N, K, f16)
    ref = oracle_mod.fused(A, W, fmt, M, N, K, f16=f16, cols=cols, threads=threads)
    if f16:
        ref = ref.view(np.float16)
    if cols:
        got, ref = got[:, cols[0]:cols[1]], ref[:, cols[0]:cols[1]]
    return assert_close(got.astype(np.float32), ref.astype(np.float32), what=f"{fmt} f16={f16} {M}x{N}x{K}")


SMALL = [(4, 8, 32), (5, 7, 64), (64, 128, 256), (1, 1, 32), (1, 3, 64), (2, 100, 96), (3, 257, 128),
         (9, 33, 160), (16, 64, 512), (17, 31, 64), (1, 4096, 64)]


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("f16", [False, True], ids=["f32", "f16"])
@pytest.mark.parametrize("shape", SMALL, ids=lambda s: "x".join(map(str, s)))
def test_fused_small_shapes(provider, oracle_mod, fmt, f16, shape):
    check_fused(provider, oracle_mod, fmt, *shape, f16=f16, seed=sum(shape))


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("f16", [False, True], ids=["f32", "f16"])
@pytest.mark.parametrize("shape", [(2, 5, 48), (3, 9, 80), (1, 7, 33)], ids=lambda s: "x".join(map(str, s)))
def test_fused_ragged_k_flat_indexing(provider, oracle_mod, fmt, f16, shape):
    M, N, K = shape
    nblk = (N * K + 31) // 32
    W = syn.weights(fmt, 1, nblk * 32, seed=K)
    A = syn.activations(M, K, seed=N, dtype=np.float16 if f16 else np.float32)
    got = run_fused(provider, fmt, A, W, M, N, K, f16)
    ref = oracle_mod.fused(A, W, fmt, M, N, K, f16=f16)
    ref = ref.view(np.float16) if f16 else ref
    assert_close(got.astype(np.float32), ref.astype(np.float32), what=f"ragged {shape}")


def test_config0_gemv_full(provider, oracle_mod):
    """C0: x[1,2048] f32, W Q4_0 [5632,2048] -> y[1,5632], whole output."""
    check_fused(provider, oracle_mod, "q4_0", 1, 5632, 2048, f16=False, seed=0)


@pytest.mark.parametrize("M", [1, 4, 16])
@pytest.mark.parametrize("NK", [(256, 2048), (2048, 5632), (32000, 2048)], ids=["kv", "down", "lm_head"])
def test_config1_tinyllama_shapes(provider, oracle_mod, M, NK):
    N, K = NK
    cols = None if N * M <= 64 * 2048 else (N // 2 - 512, N // 2 + 512)
    check_fused(provider, oracle_mod, "q4_0", M, N, K, f16=False, seed=N + M, cols=cols)


@pytest.mark.parametrize("M", [1, 8, 64])
def test_config3_q8_0_decode(provider, oracle_mod, M):
    check_fused(provider, oracle_mod, "q8_0", M, 1024, 4096, f16=False, seed=M)


@pytest.mark.parametrize("M,N,K", [(512, 4096, 4096), (512, 11008, 4096), (512, 4096, 11008)])
def test_config2_prefill_sampled_columns(provider, oracle_mod, M, N, K):
    check_fused(provider, oracle_mod, "q4_0", M, N, K, f16=True, seed=K, cols=(N - 256, N), threads=8)


def _force_path(provider, path, f16):
    """Pin the switch points so `path` ('gemv', 'skinny', 'tiled') serves every M."""
    if path == "gemv":
        provider.set_gemv_max_m(1 << 30, 1 << 30)
    elif path == "skinny":
        provider.set_gemv_max_m(0, 0)
        provider.set_skinny_max_m(1 << 30, 1 << 30, 1 << 30)
    else:
        provider.set_gemv_max_m(0, 0)
        provider.set_skinny_max_m(0, 0)


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("f16", [False, True], ids=["f32", "f16"])
@pytest.mark.parametrize("M", [3, 24, 64, 100])
def test_kernel_paths_agree(provider, oracle_mod, fmt, f16, M):
    """The same inputs through every kernel family that serves the op (GEMV,
    small-batch MFMA, tiled MFMA GEMM: fp16 MFMA for f16 activations, bf16
    pieces for f32) each match the oracle within the tolerance; N and M are
    not multiples of any tile."""
    N, K = 392, 1024
    old = provider.get_tuning()
    W = syn.weights(fmt, N, K, seed=3 + M)
    A = syn.activations(M, K, seed=4 + M, dtype=np.float16 if f16 else np.float32)
    ref = oracle_mod.fused(A, W, fmt, M, N, K, f16=f16)
    ref = (ref.view(np.float16) if f16 else ref).astype(np.float32)
    try:
        for path in ("gemv", "skinny", "tiled"):
            _force_path(provider, path, f16)
            got = run_fused(provider, fmt, A, W, M, N, K, f16).astype(np.float32)
            assert_close(got, ref, what=f"{path} {fmt} f16={f16} M={M}")
    finally:
        provider.set_tuning(old)


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("f16", [False, True], ids=["f32", "f16"])
@pytest.mark.parametrize("shape", [(2, 200, 256), (8, 1000, 768), (16, 64, 4096), (17, 257, 2048),
                                   (33, 130, 512), (64, 96, 1024), (130, 72, 256), (5, 40, 192)],
                         ids=lambda s: "x".join(map(str, s)))
def test_skinny_mfma_shapes(provider, oracle_mod, fmt, f16, shape):
    """Small-batch MFMA kernel at ragged M/N, short and long K (the per-wave
    K split and the LDS combine), rows beyond one launch (32 for f32, 64 for
    f16); K % 256 != 0 falls back to the GEMV."""
    M, N, K = shape
    old = provider.get_tuning()
    try:
        _force_path(provider, "skinny", f16)
        check_fused(provider, oracle_mod, fmt, M, N, K, f16=f16, seed=M * 7 + N)
    finally:
        provider.set_tuning(old)


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("shape", [(5, 300, 256), (16, 1000, 4096), (17, 257, 2048), (31, 130, 768),
                                   (33, 520, 1024), (64, 4096, 512), (48, 33000, 256), (64, 66000, 256)],
                         ids=lambda s: "x".join(map(str, s)))
def test_skinny_ring_f32_edges(provider, oracle_mod, fmt, shape):
    """The f32 small-batch kernel (weights through an LDS ring, activations
    split once per workgroup): one, two and four 16-row activation tiles with
    ragged M and N, a single chunk per workgroup and K split over
    workgroups, and the 32- and 64-row waves of tall matrices (N >= 32768,
    65536); up to 64 rows in one pass.  Each shape twice in a row (the
    split-K arrival counters must be back at zero)."""
    M, N, K = shape
    old = provider.get_tuning()
    try:
        _force_path(provider, "skinny", False)
        for rep in range(2):
            check_fused(provider, oracle_mod, fmt, M, N, K, f16=False, seed=M * 5 + N + rep)
    finally:
        provider.set_tuning(old)


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("f16", [False, True], ids=["f32", "f16"])
@pytest.mark.parametrize("shape", [(4, 300, 4096), (3, 130, 5632), (4, 64, 7168)], ids=lambda s: "x".join(map(str, s)))
def test_gemv_large_activation_staging(provider, oracle_mod, fmt, f16, shape):
    """GEMV with the activations' LDS stage above 64 KB (opt-in dynamic LDS):
    M = 3..4 rows of long K."""
    M, N, K = shape
    old = provider.get_tuning()
    try:
        _force_path(provider, "gemv", f16)
        check_fused(provider, oracle_mod, fmt, M, N, K, f16=f16, seed=M + N + K)
    finally:
        provider.set_tuning(old)


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("tile", [-1, 8, 9, 10, 11], ids=["default", "wq2", "wq2m64", "wq2m32", "wq2n128"])
@pytest.mark.parametrize("shape", [(200, 520, 8192), (130, 300, 16384), (512, 4096, 11008)],
                         ids=lambda s: "x".join(map(str, s)))
def test_tiled_gemm_split_k(provider, oracle_mod, fmt, tile, shape):
    """Tiled MFMA GEMM with fewer tiles than CUs and long K: K is split over
    2-4 workgroups per tile and the last one adds the partial tiles.  Two
    calls in a row: the per-tile counters must be back at zero after each.
    Tiles 8 / 9 / 10 force the two-waves-per-SIMD kernel with 128 / 64 /
    32-row waves, tile 11 its 128-row waves on 128-column tiles (8 and 11:
    Q4_0 only; Q8_0 falls back to the one-wave kernel)."""
    M, N, K = shape
    W = syn.weights(fmt, N, K, seed=N + 1)
    old = provider.get_tuning()
    try:
        _force_path(provider, "tiled", True)
        provider.set_gemm_tile(tile)
        for rep in range(2):
            A = syn.activations(M, K, seed=K + rep, dtype=np.float16)
            cols = (0, N) if N <= 520 else (N - 256, N)
            ref = oracle_mod.fused(A, W, fmt, M, N, K, f16=True, cols=cols, threads=8).view(np.float16)
            got = run_fused(provider, fmt, A, W, M, N, K, True)
            assert_close(got[:, cols[0]:cols[1]].astype(np.float32), ref[:, cols[0]:cols[1]].astype(np.float32),
                         what=f"{fmt} {M}x{N}x{K} call {rep}")
    finally:
        provider.set_tuning(old)


@pytest.mark.parametrize("path,f16,shape", [("skinny", False, (16, 4096, 4096)), ("skinny", True, (8, 8192, 28672)),
                                             ("tiled", True, (512, 4096, 4096)), ("tiled", False, (128, 4096, 4096))],
                         ids=["skinny-f32", "skinny-f16", "tiled-f16", "tiled-f32"])
def test_split_k_back_to_back(provider, oracle_mod, path, f16, shape):
    """Split-K launches enqueued back to back with no synchronisation between
    them: every launch parks its partial tiles in the same workspace slots
    and reuses the same tile counters, so a partial read before the previous
    launch's was replaced, or a counter not back at zero, shows as a wrong
    output.  Six launches on distinct activations, each checked against the
    oracle on a column window."""
    M, N, K = shape
    fmt = "q8_0"
    W = syn.weights(fmt, N, K, seed=N + K)
    dt = abi.NF_DTYPE_F16 if f16 else abi.NF_DTYPE_F32
    old = provider.get_tuning()
    bufs = []
    try:
        _force_path(provider, path, f16)
        w = provider.alloc_array(W, QDT[fmt])
        bufs.append(w)
        runs = []
        for rep in range(6):
            A = syn.activations(M, K, seed=100 + rep, dtype=np.float16 if f16 else np.float32)
            a = provider.alloc_array(A, dt)
            c = provider.alloc(dt, M * N * (2 if f16 else 4))
            bufs += [a, c]
            provider.dispatch(f"dequant_{fmt}_linear" + ("_f16" if f16 else ""), [a, w], [c], M, N, K)
            runs.append((A, c))
        provider.synchronize()
        cols = (N - 192, N)
        for rep, (A, c) in enumerate(runs):
            got = c.download(np.float16 if f16 else np.float32).reshape(M, N)[:, cols[0]:cols[1]]
            ref = oracle_mod.fused(A, W, fmt, M, N, K, f16=f16, cols=cols, threads=8)
            ref = (ref.view(np.float16) if f16 else ref)[:, cols[0]:cols[1]]
            assert_close(got.astype(np.float32), ref.astype(np.float32), what=f"{path} {M}x{N}x{K} launch {rep}")
    finally:
        for b in bufs:
            b.release()
        provider.set_tuning(old)


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("tile", [-1, 0, 1, 2, 5, 7, 8, 9, 10, 11],
                         ids=lambda t: "regdq" if t < 0 else f"lds{t}" if t < 7 else f"wq{t - 6}")
@pytest.mark.parametrize("shape", [(129, 260, 64), (257, 514, 192), (130, 302, 320), (200, 777, 448),
                                   (129, 260, 128), (257, 514, 384), (130, 302, 640), (200, 777, 896)],
                         ids=lambda s: "x".join(map(str, s)))
def test_gemm_kernels_edges(provider, oracle_mod, fmt, tile, shape):
    """Every f16 GEMM kernel (weights dequantized in registers: tile -1 the
    default pick, tile 7 the one-wave kernel, tiles 8 / 9 / 10 the
    two-waves-per-SIMD kernel with 128 / 64 / 32-row waves where K % 128 ==
    0, tile 11 its 128-row waves on 128-column tiles; into LDS: tiles 0..6) against the oracle on ragged
    shapes: M and N past a tile edge, N % 4 != 0 (element-wise stores), and
    1, 3, 5, 7 K steps, or 1, 3, 5, 7 step pairs per K-group (K = 128 ..
    896), i.e. fewer steps than the prefetch depth and every loop
    remainder."""
    M, N, K = shape
    W = syn.weights(fmt, N, K, seed=N + K)
    A = syn.activations(M, K, seed=M + K, dtype=np.float16)
    old = provider.get_tuning()
    try:
        _force_path(provider, "tiled", True)
        provider.set_gemm_tile(tile)
        got = run_fused(provider, fmt, A, W, M, N, K, True)
    finally:
        provider.set_tuning(old)
    ref = oracle_mod.fused(A, W, fmt, M, N, K, f16=True, threads=8).view(np.float16)
    assert_close(got.astype(np.float32), ref.astype(np.float32), what=f"{fmt} tile {tile} {M}x{N}x{K}")


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("shape", [(33, 130, 512), (64, 96, 1024), (100, 777, 448), (129, 260, 64),
                                   (257, 514, 192), (200, 520, 8192), (65, 300, 16384), (512, 4096, 4096)],
                         ids=lambda s: "x".join(map(str, s)))
def test_f32_tiled_gemm(provider, oracle_mod, fmt, shape):
    """The f32-activation tiled GEMM (exact bf16 pieces on bf16 MFMA) against
    the oracle: M and N past tile edges (64- and 128-row tiles), N % 4 != 0,
    1..7 K steps and long K split over workgroups (two calls in a row: the
    per-tile counters must be back at zero)."""
    M, N, K = shape
    W = syn.weights(fmt, N, K, seed=N + 2 * K)
    old = provider.get_tuning()
    try:
        _force_path(provider, "tiled", False)
        for rep in range(2 if K >= 8192 else 1):
            A = syn.activations(M, K, seed=M + K + rep, dtype=np.float32)
            cols = (0, N) if N <= 1024 else (N - 256, N)
            got = run_fused(provider, fmt, A, W, M, N, K, False)
            ref = oracle_mod.fused(A, W, fmt, M, N, K, cols=cols, threads=8)
            assert_close(got[:, cols[0]:cols[1]], ref[:, cols[0]:cols[1]], what=f"{fmt} {M}x{N}x{K} call {rep}")
    finally:
        provider.set_tuning(old)


@pytest.mark.parametrize("path", ["skinny", "tiled"])
def test_f32_large_activations(provider, oracle_mod, path):
    """The two bf16 pieces keep f32 activations far outside the fp16 range
    (|x| ~ 1e6 and 1e-6) within 2^-16 of their value before accumulation,
    on both bf16-piece kernels.  With such data most outputs are sums that
    cancel to far below their terms, where any two fp32 summation orders (the
    oracle's sequential one included) differ by more than 1e-3 of the
    result; so each output is held to the fp32 summation bound
    |got - exact| <= 4 K 2^-24 sum_k |x_k w_k| against the float64 result
    (at K = 512, 1.2e-4 of sum_k |x_k w_k|, above the tiled kernel's 4.6e-5
    for its dropped piece products), and to 1e-3 normwise against the
    oracle.  A lost piece (fp16 overflow at 1e6, underflow at 1e-6, or a
    dropped leading term) breaks the bound by orders of magnitude."""
    M, N, K = 40, 128, 512
    W = syn.q4_0_weights(N, K, seed=11)
    rng = np.random.default_rng(5)
    A = (rng.standard_normal((M, K)) * np.where(rng.random((M, K)) < 0.5, 1e6, 1e-6)).astype(np.float32)
    old = provider.get_tuning()
    try:
        _force_path(provider, path, False)
        got = run_fused(provider, "q4_0", A, W, M, N, K, False).astype(np.float64)
    finally:
        provider.set_tuning(old)
    Wd = oracle_mod.dequant(W, "q4_0", N * K).astype(np.float64).reshape(N, K)
    exact = A.astype(np.float64) @ Wd.T
    bound = 4 * K * 2.0 ** -24 * (np.abs(A.astype(np.float64)) @ np.abs(Wd).T)
    worst = float(np.max(np.abs(got - exact) / bound))
    assert worst <= 1.0, f"{path}: error {worst:.3g} x the fp32 summation bound"
    ref = oracle_mod.fused(A, W, "q4_0", M, N, K)
    assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) <= 1e-3


# ---- the reference's fused-vs-separate test (fused_matmul_test.cpp:134-285) ----------

def _quantize_like_reference_test(src, oracle_mod):
    """Test-only quantizer of fused_matmul_test.cpp:87-104: d = amax/7 encoded
    with the truncating encoder, codes round(x/d)+8 clamped to 0..15."""
    blocks = src.reshape(-1, 32)
    out = []
    for b in blocks:
        amax = float(np.max(np.abs(b)))
        d = np.float32(amax / 7.0)
        dh = oracle_mod.f32_to_f16_trunc(float(d))
        df = float(np.array([dh], np.uint16).view(np.float16)[0])
        inv = 1.0 / df if df != 0.0 else 0.0
        codes = np.clip(np.round(b.astype(np.float32) * np.float32(inv)).astype(np.int64) + 8, 0, 15)
        out.append(syn.pack_q4_0(np.array([dh], np.uint16).view(np.float16), codes[None, :]))
    return np.concatenate(out).reshape(-1)


@pytest.mark.parametrize("M,N,K", [(4, 8, 32), (5, 7, 64), (64, 128, 256)])
def test_reference_fused_vs_separate_f32(provider, oracle_mod, M, N, K):
    rng = np.random.default_rng(42)
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    kn = K * N
    kn_pad = (kn + 31) // 32 * 32
    bsrc = np.zeros(kn_pad, np.float32)
    bsrc[:kn] = rng.uniform(-1, 1, kn)
    Wq = _quantize_like_reference_test(bsrc, oracle_mod)
    a = provider.alloc_array(A, abi.NF_DTYPE_F32)
    w = provider.alloc_array(Wq, abi.NF_DTYPE_Q4_0)
    dq = provider.alloc(abi.NF_DTYPE_F32, kn_pad * 4)
    sep = provider.alloc(abi.NF_DTYPE_F32, M * N * 4)
    fused = provider.alloc(abi.NF_DTYPE_F32, M * N * 4)
    provider.check(provider.dispatch_bare("dequant_q4_0", [w], [dq]), "dequant")
    provider.synchronize()
    provider.dispatch("linear_tiled", [a, dq], [sep], M, N, K)
    provider.dispatch("dequant_q4_0_linear", [a, w], [fused], M, N, K)
    provider.synchronize()
    s, f = sep.download(np.float32), fused.download(np.float32)
    assert np.max(np.abs(s - f)) < 1e-3  # the reference's own criterion
    ref = oracle_mod.fused(A, Wq, "q4_0", M, N, K)
    assert_close(f.reshape(M, N), ref)
    for b in (a, w, dq, sep, fused):
        b.release()


def test_reference_fused_vs_separate_f16(provider, oracle_mod):
    M, N, K = 64, 128, 256
    rng = np.random.default_rng(99)
    A32 = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    A16 = np.array([oracle_mod.f32_to_f16_trunc(float(v)) for v in A32.reshape(-1)], np.uint16)
    bsrc = rng.uniform(-1, 1, K * N).astype(np.float32)
    Wq = _quantize_like_reference_test(bsrc, oracle_mod)
    a = provider.alloc_array(A16, abi.NF_DTYPE_F16)
    w = provider.alloc_array(Wq, abi.NF_DTYPE_Q4_0)
    dq = provider.alloc(abi.NF_DTYPE_F16, K * N * 2)
    sep = provider.alloc(abi.NF_DTYPE_F16, M * N * 2)
    fused = provider.alloc(abi.NF_DTYPE_F16, M * N * 2)
    provider.check(provider.dispatch_bare("dequant_q4_0_f16", [w], [dq]), "dequant_f16")
    provider.synchronize()
    provider.dispatch("linear", [a, dq], [sep], M, N, K)
    provider.dispatch("dequant_q4_0_linear_f16", [a, w], [fused], M, N, K)
    provider.synchronize()
    s = sep.download(np.float16).astype(np.float32)
    f = fused.download(np.float16).astype(np.float32)
    assert np.max(np.abs(s - f)) < 0.1  # the reference's own criterion
    ref = oracle_mod.fused(A16, Wq, "q4_0", M, N, K, f16=True).view(np.float16).astype(np.float32)
    assert_close(f.reshape(M, N), ref)
    for b in (a, w, dq, sep, fused):
        b.release()


# ---- dense linear ---------------------------------------------------------------------

def test_dense_linear_tiled_reference_case(provider, oracle_mod):
    """dequant_test.cpp:300-394: A 64x32, B 48x32 (transposed), f32."""
    M, N, K = 64, 48, 32
    A = ((np.arange(M * K) % 17) * np.float32(0.1) - np.float32(0.8)).astype(np.float32).reshape(M, K)
    Bl = ((np.arange(K * N) % 13) * np.float32(0.15) - np.float32(0.9)).astype(np.float32).reshape(K, N)
    B = np.ascontiguousarray(Bl.T)
    a, b = provider.alloc_array(A, abi.NF_DTYPE_F32), provider.alloc_array(B, abi.NF_DTYPE_F32)
    c = provider.alloc(abi.NF_DTYPE_F32, M * N * 4)
    provider.dispatch("linear_tiled", [a, b], [c], M, N, K)
    got = c.download(np.float32).reshape(M, N)
    assert_close(got, oracle_mod.linear_f32(A, B, M, N, K))
    for x in (a, b, c):
        x.release()


@pytest.mark.parametrize("shape", [(32, 136, 128), (300, 1000, 4096), (1024, 256, 640)],
                         ids=lambda s: "x".join(map(str, s)))
def test_dense_linear_f16_mfma(provider, oracle_mod, shape):
    """f16 x f16 -> f16 dense linear on the tiled MFMA kernel (B rows streamed
    into LDS like A), ragged M/N."""
    M, N, K = shape
    rng = np.random.default_rng(M + N)
    A = rng.standard_normal((M, K)).astype(np.float16)
    B = rng.standard_normal((N, K)).astype(np.float16)
    a, b = provider.alloc_array(A, abi.NF_DTYPE_F16), provider.alloc_array(B, abi.NF_DTYPE_F16)
    c = provider.alloc(abi.NF_DTYPE_F16, M * N * 2)
    provider.dispatch("linear", [a, b], [c], M, N, K)
    got = c.download(np.float16).reshape(M, N).astype(np.float32)
    ref = oracle_mod.linear_f16(A.view(np.uint16), B.view(np.uint16), M, N, K).view(np.float16).astype(np.float32)
    assert_close(got, ref)
    for x in (a, b, c):
        x.release()


@pytest.mark.parametrize("adt,bdt,cdt", [("f16", "f16", "f16"), ("f16", "f16", "f32"), ("f32", "f32", "f32"),
                                         ("f32", "f16", "f32")])
def test_dense_linear_dtype_mixes(provider, oracle_mod, adt, bdt, cdt):
    M, N, K = 33, 70, 96
    rng = np.random.default_rng(7)
    np_t = {"f16": np.float16, "f32": np.float32}
    nf_t = {"f16": abi.NF_DTYPE_F16, "f32": abi.NF_DTYPE_F32}
    A = rng.standard_normal((M, K)).astype(np_t[adt])
    B = rng.standard_normal((N, K)).astype(np_t[bdt])
    a, b = provider.alloc_array(A, nf_t[adt]), provider.alloc_array(B, nf_t[bdt])
    c = provider.alloc(nf_t[cdt], M * N * (2 if cdt == "f16" else 4))
    provider.dispatch("linear", [a, b], [c], M, N, K)
    got = c.download(np_t[cdt]).reshape(M, N).astype(np.float32)
    ref = oracle_mod.linear_f32(A.astype(np.float32), B.astype(np.float32), M, N, K)
    if cdt == "f16":
        ref = ref.astype(np.float16).astype(np.float32)
    assert_close(got, ref)
    for x in (a, b, c):
        x.release()


@pytest.mark.parametrize("adt,bdt,cdt", [("f32", "f32", "f32"), ("f32", "f16", "f32"), ("f16", "f32", "f16"),
                                         ("f16", "f16", "f32")])
@pytest.mark.parametrize("shape", [(300, 1000, 1024), (129, 257, 96), (1024, 256, 640), (9, 130, 32), (40, 50, 100)],
                         ids=lambda s: "x".join(map(str, s)))
def test_dense_linear_f32_mfma(provider, oracle_mod, adt, bdt, cdt, shape):
    """`linear` with an fp32 operand or output above decode batch sizes: the
    fp32 MFMA kernel (fp16 operands widened exactly), ragged M/N, a single K
    step; K % 32 != 0 (the last shape) falls back to the VALU tile kernel."""
    M, N, K = shape
    rng = np.random.default_rng(M + N + K)
    np_t = {"f16": np.float16, "f32": np.float32}
    nf_t = {"f16": abi.NF_DTYPE_F16, "f32": abi.NF_DTYPE_F32}
    A = rng.standard_normal((M, K)).astype(np_t[adt])
    B = rng.standard_normal((N, K)).astype(np_t[bdt])
    a, b = provider.alloc_array(A, nf_t[adt]), provider.alloc_array(B, nf_t[bdt])
    c = provider.alloc(nf_t[cdt], M * N * (2 if cdt == "f16" else 4))
    provider.dispatch("linear", [a, b], [c], M, N, K)
    got = c.download(np_t[cdt]).reshape(M, N).astype(np.float32)
    ref = oracle_mod.linear_f32(A.astype(np.float32), B.astype(np.float32), M, N, K)
    if cdt == "f16":
        ref = ref.astype(np.float16).astype(np.float32)
    assert_close(got, ref, what=f"{adt}{bdt}->{cdt} {M}x{N}x{K}")
    for x in (a, b, c):
        x.release()


@pytest.mark.parametrize("adt,bdt", [("f32", "f32"), ("f16", "f32")])
@pytest.mark.parametrize("shape", [(16, 4096, 4096), (64, 1000, 2048), (33, 300, 8192)],
                         ids=lambda s: "x".join(map(str, s)))
def test_dense_linear_f32_split_k(provider, oracle_mod, adt, bdt, shape):
    """fp32 dense linear at small batches: 32-row tiles with K split over
    workgroups (partial tiles added by the last arrival).  Two calls in a row
    with different activations: the per-tile counters must be back at zero."""
    M, N, K = shape
    rng = np.random.default_rng(M * 3 + N)
    np_t = {"f16": np.float16, "f32": np.float32}
    nf_t = {"f16": abi.NF_DTYPE_F16, "f32": abi.NF_DTYPE_F32}
    B = rng.standard_normal((N, K)).astype(np_t[bdt])
    b = provider.alloc_array(B, nf_t[bdt])
    c = provider.alloc(abi.NF_DTYPE_F32, M * N * 4)
    try:
        for rep in range(2):
            A = rng.standard_normal((M, K)).astype(np_t[adt])
            a = provider.alloc_array(A, nf_t[adt])
            provider.dispatch("linear", [a, b], [c], M, N, K)
            got = c.download(np.float32).reshape(M, N)
            a.release()
            ref = oracle_mod.linear_f32(A.astype(np.float32), B.astype(np.float32), M, N, K)
            assert_close(got, ref, what=f"{adt}{bdt} {M}x{N}x{K} call {rep}")
    finally:
        b.release()
        c.release()


@pytest.mark.parametrize("adt,bdt,cdt,M,N,K", [
    ("f32", "f32", "f32", 1, 1000, 4096), ("f32", "f32", "f32", 2, 64, 100), ("f16", "f16", "f16", 3, 333, 2048),
    ("f32", "f16", "f32", 8, 130, 1024), ("f16", "f16", "f32", 4, 257, 512), ("f16", "f32", "f16", 5, 96, 256),
    ("f32", "f32", "f32", 1, 32000, 2048)],
    ids=lambda v: str(v))
def test_dense_linear_decode_gemv(provider, oracle_mod, adt, bdt, cdt, M, N, K):
    """`linear` at decode batch sizes (M <= 8) runs the HBM-bound dense GEMV:
    dtype mixes, ragged N and K, an lm_head-sized f32 case."""
    rng = np.random.default_rng(M * 7 + N)
    np_t = {"f16": np.float16, "f32": np.float32}
    nf_t = {"f16": abi.NF_DTYPE_F16, "f32": abi.NF_DTYPE_F32}
    A = rng.standard_normal((M, K)).astype(np_t[adt])
    B = rng.standard_normal((N, K)).astype(np_t[bdt])
    a, b = provider.alloc_array(A, nf_t[adt]), provider.alloc_array(B, nf_t[bdt])
    c = provider.alloc(nf_t[cdt], M * N * (2 if cdt == "f16" else 4))
    provider.dispatch("linear", [a, b], [c], M, N, K)
    got = c.download(np_t[cdt]).reshape(M, N).astype(np.float32)
    ref = oracle_mod.linear_f32(A.astype(np.float32), B.astype(np.float32), M, N, K)
    if cdt == "f16":
        ref = ref.astype(np.float16).astype(np.float32)
    assert_close(got, ref)
    for x in (a, b, c):
        x.release()


def _import_at(provider, base, offset, dtype, nbytes):
    """A non-owning buffer over `nbytes` of `base`'s memory from byte
    `offset` on (an imported DEVICE token, neuro_buffer_abi.h:165-183)."""
    import ctypes as C
    from neurofabric_amd.plugin import Buffer
    ops, h = abi.nf_buffer_ops(), C.c_void_p()
    desc = abi.make_desc(dtype, nbytes)
    st = provider.mem.import_buffer(provider.handle, base.device_ptr() + offset, abi.NF_MEM_DOMAIN_DEVICE,
                                    C.byref(desc), C.byref(ops), C.byref(h))
    assert st == abi.NF_OK, provider.last_error()
    return Buffer(provider, h.value, ops, dtype, nbytes)


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("M", [128, 24, 2])
@pytest.mark.parametrize("a_off,w_off", [(4, 0), (0, 2)], ids=["A+4", "W+2"])
def test_fused_f32_misaligned_operands(provider, oracle_mod, fmt, M, a_off, w_off):
    """f32 activations 4 bytes past a 16-byte boundary, or weights 2 bytes
    past a dword, as imported buffers at odd offsets give them: every batch
    size (the MFMA kernels need aligned operands, so these run on the GEMV's
    block kernel) matches the oracle, through dispatch and through the
    no-allocation entry point on the same raw pointers."""
    import ctypes as C
    N, K = 512, 4096
    W = syn.weights(fmt, N, K, seed=M + a_off)
    A = syn.activations(M, K, seed=M + 1)
    a_raw = provider.alloc_array(np.concatenate([np.zeros(a_off, np.uint8), A.reshape(-1).view(np.uint8)]),
                                 abi.NF_DTYPE_U8)
    w_raw = provider.alloc_array(np.concatenate([np.zeros(w_off, np.uint8), W.reshape(-1).view(np.uint8)]),
                                 abi.NF_DTYPE_U8)
    a = _import_at(provider, a_raw, a_off, abi.NF_DTYPE_F32, A.nbytes)
    w = _import_at(provider, w_raw, w_off, QDT[fmt], W.nbytes)
    c = provider.alloc(abi.NF_DTYPE_F32, M * N * 4)
    c2 = provider.alloc(abi.NF_DTYPE_F32, M * N * 4)
    try:
        print(f"misaligned f32 {fmt} M={M} A+{a_off} W+{w_off}", flush=True)
        provider.dispatch(f"dequant_{fmt}_linear", [a, w], [c], M, N, K)
        fn = provider.lib.nf_hip_fused_linear_noalloc
        fn.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_bool,
                       C.c_void_p]
        fn.restype = C.c_int
        st = fn(QDT[fmt], a_raw.device_ptr() + a_off, w_raw.device_ptr() + w_off, c2.device_ptr(), M, N, K, False,
                provider.stream())
        assert st == abi.NF_OK, provider.last_error()
        provider.synchronize()
        ref = oracle_mod.fused(A, W, fmt, M, N, K, threads=8)
        assert_close(c.download(np.float32).reshape(M, N), ref, what=f"dispatch {fmt} M={M}")
        assert_close(c2.download(np.float32).reshape(M, N), ref, what=f"noalloc {fmt} M={M}")
    finally:
        for b in (a, w, a_raw, w_raw, c, c2):
            b.release()
