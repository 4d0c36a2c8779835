"""Pins the CPU oracle (oracle/nf_oracle.c) before anything is checked against it.

Each restated reference function is checked against something independent
of it: numpy's own IEEE-754 binary16 implementation (decode and
round-to-nearest-even encode), closed forms (d*q is exact in fp32), hand-
written known answers for the nibble order, and rigorous error bounds for
the sequential-k fp32 loop.  The last group plants plausible mistakes
(swapped nibbles, wrong offset, transposed operand, truncating encoder) and
asserts the same checks reject them.
"""
import numpy as np
import pytest

from neurofabric_amd import synthetic as syn
from oracle import oracle as orc

pytestmark = pytest.mark.filterwarnings("ignore::RuntimeWarning")

ALL_F16 = np.arange(65536, dtype=np.uint32).astype(np.uint16)


def _is_nan16(bits):
    return ((bits & 0x7C00) == 0x7C00) & ((bits & 0x03FF) != 0)


# ---- fp16 decode / encode ------------------------------------------------

def test_f16_decode_exhaustive_matches_numpy():
    got = orc.f16_to_f32(ALL_F16)
    want = ALL_F16.view(np.float16).astype(np.float32)
    nan = _is_nan16(ALL_F16)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    assert np.isnan(got[nan]).all()


def test_f16_encode_roundtrips_every_half():
    vals = ALL_F16.view(np.float16).astype(np.float32)
    back = orc.f32_to_f16_rne(vals)
    nan = _is_nan16(ALL_F16)
    assert np.array_equal(back[~nan], ALL_F16[~nan])
    assert _is_nan16(back[nan]).all()


def _check_encoder(encode):
    """RNE encoder pins: ties, near-ties, overflow and subnormal edges vs numpy."""
    pos = np.arange(0, 0x7BFF, dtype=np.uint16)             # finite positive halves
    lo = pos.view(np.float16).astype(np.float64)
    hi = (pos + 1).view(np.float16).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)                 # exact ties (fit in fp32)
    xs = [mid, np.nextafter(mid, np.float32(np.inf)), np.nextafter(mid, np.float32(0)),
          np.float32([65504.0, 65519.996, 65520.0, 65536.0, 1e30, 2.0 ** -24, 2.0 ** -25,
                      2.0 ** -25 * 1.0000001, 2.0 ** -26, 6.0e-8, 1e-30, 0.0])]
    rng = np.random.default_rng(1)
    xs.append(rng.integers(0x30000000, 0x48000000, 2_000_000, dtype=np.uint32).view(np.float32))
    x = np.concatenate(xs).astype(np.float32)
    x = np.concatenate([x, -x])
    got = encode(x)
    want = x.astype(np.float16).view(np.uint16)
    return np.array_equal(got, want)


def test_f16_encode_rne_matches_numpy():
    assert _check_encoder(orc.f32_to_f16_rne)


def test_trunc_encoder_matches_closed_form():
    """The reference tests' encoder (dequant_test.cpp:100-109) truncates toward
    zero and flushes below 2^-14: it returns the largest-magnitude normal half
    not exceeding |x| (or signed zero)."""
    rng = np.random.default_rng(2)
    x = rng.uniform(-70000, 70000, 20000).astype(np.float32)
    x = np.concatenate([x, np.float32([0.5, 0.6, 0.7, 1e-5, 6.2e-5, -3.3, 65504, 65535])])
    for v in x:
        got = orc.f32_to_f16_trunc(float(v))
        a = abs(float(v))
        if a < 2.0 ** -14:
            want = 0x8000 if np.signbit(v) else 0
        elif a >= 65536.0:
            want = 0x7C00 | (0x8000 if v < 0 else 0)
        else:
            h = np.float16(a)
            if float(h) > a:
                h = np.float16(np.nextafter(h, np.float16(0)))
            want = int(np.array([h]).view(np.uint16)[0]) | (0x8000 if v < 0 else 0)
        assert got == want, (v, hex(got), hex(want))


# ---- dequant ------------------------------------------------------------------

def _all_scale_blocks(fmt):
    """One block per fp16 scale pattern; Q4_0 codes 0..15 twice, Q8_0 codes in
    8 blocks per scale covering -128..127."""
    if fmt == "q4_0":
        codes = np.tile(np.arange(32) % 16, (65536, 1))
        return syn.pack_q4_0(ALL_F16.view(np.float16), codes), ALL_F16, codes - 8
    d = np.repeat(ALL_F16, 8)
    codes = np.tile(np.arange(-128, 128).reshape(8, 32), (65536, 1))
    return syn.pack_q8_0(d.view(np.float16), codes), d, codes


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
def test_dequant_f32_exhaustive_closed_form(fmt):
    blocks, d_bits, q = _all_scale_blocks(fmt)
    got = orc.dequant(blocks, fmt, q.size)
    want = (d_bits.view(np.float16).astype(np.float32)[:, None] * q.astype(np.float32)).reshape(-1)
    nan = np.isnan(want)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    assert np.isnan(got[nan]).all()


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
def test_dequant_f16_exhaustive_rne_of_exact_product(fmt):
    blocks, d_bits, q = _all_scale_blocks(fmt)
    got = orc.dequant(blocks, fmt, q.size, f16=True)
    exact = d_bits.view(np.float16).astype(np.float64)[:, None] * q.astype(np.float64)
    want = exact.astype(np.float32).astype(np.float16).view(np.uint16).reshape(-1)
    nan = _is_nan16(want)
    assert np.array_equal(got[~nan], want[~nan])
    assert _is_nan16(got[nan]).all()
    # Same bits as an IEEE fp16 multiply of the two exactly representable factors.
    prod16 = (d_bits.view(np.float16)[:, None] * q.astype(np.float16)).view(np.uint16).reshape(-1)
    assert np.array_equal(got[~nan], prod16[~nan])


def _known_answer_q4(dequant_fn):
    """qs[i] = i | (15-i) << 4 with d = 1: elements 0..15 are i-8 (low nibbles),
    elements 16..31 are 7-i (high nibbles), per dequant_test.cpp:112-120."""
    codes = np.concatenate([np.arange(16), 15 - np.arange(16)])
    blk = syn.pack_q4_0(np.float16([1.0]), codes[None, :])
    want = np.concatenate([np.arange(16) - 8, 7 - np.arange(16)]).astype(np.float32)
    return np.array_equal(dequant_fn(blk, "q4_0", 32), want)


def test_dequant_q4_0_known_answer_nibble_order():
    assert _known_answer_q4(orc.dequant)


def test_reference_known_answer_inputs():
    """The input patterns of dequant_test.cpp:155-168 / 233-239 and
    fp16_kernel_test.cpp:292-307, with scales encoded by the tests' own
    truncating encoder, dequantize to d*(code-8) / d*code."""
    for b in range(8):
        d = orc.f32_to_f16_trunc(0.5 + 0.1 * b)
        codes = np.array([(j + b) & 0xF for j in range(16)] + [(15 - j + b) & 0xF for j in range(16)])
        blk = syn.pack_q4_0(np.array([d], np.uint16).view(np.float16), codes[None, :])
        dv = np.float32(np.array([d], np.uint16).view(np.float16)[0])
        assert np.array_equal(orc.dequant(blk, "q4_0", 32), dv * (codes - 8).astype(np.float32))
        d8 = orc.f32_to_f16_trunc(0.25 + 0.05 * b)
        c8 = np.arange(32) - 16 + b
        blk8 = syn.pack_q8_0(np.array([d8], np.uint16).view(np.float16), c8[None, :])
        dv8 = np.float32(np.array([d8], np.uint16).view(np.float16)[0])
        assert np.array_equal(orc.dequant(blk8, "q8_0", 32), dv8 * c8.astype(np.float32))


def test_dequant_partial_block_count():
    w = syn.q4_0_weights(2, 64, seed=5)
    full = orc.dequant(w, "q4_0", 128)
    part = orc.dequant(w, "q4_0", 77)
    assert np.array_equal(full[:77], part)


# ---- sequential-k linear -------------------------------------------------------

def _bound_ok(got, A64, B64, K):
    """|fl(sum) - sum| <= gamma_K * sum|a||b| for recursive summation."""
    exact = A64 @ B64.T
    gamma = K * 2.0 ** -24 / (1 - K * 2.0 ** -24)
    return np.all(np.abs(got.astype(np.float64) - exact) <= gamma * (np.abs(A64) @ np.abs(B64).T) + 1e-30)


def test_linear_f32_reference_linear_tiled_case():
    """Inputs of dequant_test.cpp:303-325 (64x48x32, B transposed to [N,K])."""
    M, N, K = 64, 48, 32
    A = ((np.arange(M * K) % 17) * np.float32(0.1) - np.float32(0.8)).astype(np.float32).reshape(M, K)
    Bl = ((np.arange(K * N) % 13) * np.float32(0.15) - np.float32(0.9)).astype(np.float32).reshape(K, N)
    B = np.ascontiguousarray(Bl.T)
    got = orc.linear_f32(A, B, M, N, K)
    assert _bound_ok(got, A.astype(np.float64), B.astype(np.float64), K)


def test_linear_f32_exact_cases():
    rng = np.random.default_rng(3)
    M, N, K = 5, 7, 33
    B = rng.standard_normal((N, K)).astype(np.float32)
    eye = np.eye(K, dtype=np.float32)[:M]
    assert np.array_equal(orc.linear_f32(eye, B, M, N, K), B[:, :M].T)  # picks columns of B
    Ai = rng.integers(-4, 5, (M, K)).astype(np.float32)
    Bi = rng.integers(-4, 5, (N, K)).astype(np.float32)
    assert np.array_equal(orc.linear_f32(Ai, Bi, M, N, K), (Ai.astype(np.int64) @ Bi.T.astype(np.int64)).astype(np.float32))


def test_linear_f32_is_sequential_k():
    """Order matters in fp32: 1e8 + 1 - 1e8 in k order gives 0 (not 1)."""
    A = np.float32([[1e8, 1.0, -1e8]])
    B = np.float32([[1.0, 1.0, 1.0]])
    assert orc.linear_f32(A, B, 1, 1, 3)[0, 0] == 0.0


def test_linear_f16_semantics():
    rng = np.random.default_rng(4)
    M, N, K = 8, 9, 64
    A = rng.standard_normal((M, K)).astype(np.float16)
    B = rng.standard_normal((N, K)).astype(np.float16)
    got = orc.linear_f16(A.view(np.uint16), B.view(np.uint16), M, N, K).view(np.float16)
    exact = A.astype(np.float64) @ B.astype(np.float64).T
    gamma = K * 2.0 ** -24 / (1 - K * 2.0 ** -24)
    acc_err = gamma * (np.abs(A.astype(np.float64)) @ np.abs(B.astype(np.float64)).T)
    ulp_half = np.abs(exact) * 2.0 ** -11 + 2.0 ** -25
    assert np.all(np.abs(got.astype(np.float64) - exact) <= acc_err + ulp_half)


# ---- fused ------------------------------------------------------------------------

@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("shape", [(4, 8, 32), (5, 7, 64), (3, 40, 256)])
def test_fused_f32_equals_dequant_then_linear(fmt, shape):
    M, N, K = shape
    W = syn.weights(fmt, N, K, seed=11)
    A = syn.activations(M, K, seed=12)
    fused = orc.fused(A, W, fmt, M, N, K)
    sep = orc.linear_f32(A, orc.dequant(W, fmt, N * K).reshape(N, K), M, N, K)
    assert np.array_equal(fused.view(np.uint32), sep.view(np.uint32))
    Wd = orc.dequant(W, fmt, N * K).reshape(N, K).astype(np.float64)
    assert _bound_ok(fused, A.astype(np.float64), Wd, K)


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
def test_fused_f16_semantics(fmt):
    M, N, K = 6, 10, 128
    W = syn.weights(fmt, N, K, seed=13)
    A = syn.activations(M, K, seed=14, dtype=np.float16)
    got = orc.fused(A, W, fmt, M, N, K, f16=True)
    w16 = orc.dequant(W, fmt, N * K, f16=True).reshape(N, K)
    assert np.array_equal(got, orc.linear_f16(A.view(np.uint16), w16, M, N, K))


def test_fused_closed_forms():
    M, N, K = 3, 4, 64
    A = syn.activations(M, K, seed=15)
    zero_codes = np.full((N * K // 32, 32), 8)
    W0 = syn.pack_q4_0(np.ones(N * K // 32, np.float16), zero_codes).reshape(-1)
    assert np.array_equal(orc.fused(A, W0, "q4_0", M, N, K), np.zeros((M, N), np.float32))
    # A single code 9 (value +d) at (n=2, k=37) with d = 0.5 picks 0.5*A[:, 37].
    codes = zero_codes.copy()
    codes[(2 * K + 37) // 32, (2 * K + 37) % 32] = 9
    W1 = syn.pack_q4_0(np.full(N * K // 32, 0.5, np.float16), codes).reshape(-1)
    want = np.zeros((M, N), np.float32)
    want[:, 2] = 0.5 * A[:, 37]
    assert np.array_equal(orc.fused(A, W1, "q4_0", M, N, K), want)


def test_fused_flat_index_for_ragged_k():
    """K % 32 != 0: element (n,k) is flat element n*K+k of the block stream
    (metal_provider.mm:1413-1420)."""
    M, N, K = 2, 5, 48
    W = syn.q4_0_weights(1, (N * K + 31) // 32 * 32, seed=16)
    A = syn.activations(M, K, seed=17)
    Wd = orc.dequant(W, "q4_0", N * K).reshape(N, K)
    assert np.array_equal(orc.fused(A, W, "q4_0", M, N, K), orc.linear_f32(A, Wd, M, N, K))


def test_fused_column_window_and_threads():
    M, N, K = 4, 64, 256
    W = syn.q4_0_weights(N, K, seed=18)
    A = syn.activations(M, K, seed=19)
    full = orc.fused(A, W, "q4_0", M, N, K)
    win = orc.fused(A, W, "q4_0", M, N, K, cols=(10, 30), threads=3)
    assert np.array_equal(win[:, 10:30], full[:, 10:30])
    assert not win[:, :10].any() and not win[:, 30:].any()


# ---- planted mistakes: the pins above must reject each of these ---------------

def _mutant_swapped_nibbles(blocks, fmt, count, f16=False):
    out = orc.dequant(blocks, fmt, count, f16).reshape(-1, 32)
    return np.concatenate([out[:, 16:], out[:, :16]], axis=1).reshape(-1)


def _mutant_offset7(blocks, fmt, count, f16=False):
    d, q = syn.unpack_codes(blocks, fmt)
    return (d.astype(np.float32)[:, None] * (q + 1).astype(np.float32)).reshape(-1)[:count]


def test_planted_mistakes_are_caught():
    assert not _known_answer_q4(_mutant_swapped_nibbles)
    assert not _known_answer_q4(_mutant_offset7)
    # An encoder that truncates instead of rounding fails the RNE pin.
    assert not _check_encoder(lambda x: np.array([orc.f32_to_f16_trunc(float(v)) for v in x[:5000]] +
                                                 list(orc.f32_to_f16_rne(x[5000:])), np.uint16))
    # A transposed weight operand fails the reference linear_tiled bound check.
    M, N, K = 64, 48, 32
    A = ((np.arange(M * K) % 17) * np.float32(0.1) - np.float32(0.8)).astype(np.float32).reshape(M, K)
    Bl = ((np.arange(K * N) % 13) * np.float32(0.15) - np.float32(0.9)).astype(np.float32).reshape(K, N)
    wrong = orc.linear_f32(A, Bl.reshape(-1)[: N * K].reshape(N, K), M, N, K)  # forgot the transpose
    assert not _bound_ok(wrong, A.astype(np.float64), np.ascontiguousarray(Bl.T).astype(np.float64), K)
