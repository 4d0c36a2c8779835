"""Pins the oracle's restatement of the other dequant ops (Q4_1, Q5_0, Q5_1,
Q2_K, Q3_K, Q4_K, Q5_K, Q6_K; f32 and f16 outputs) before the GPU is checked
against it.

* Seven f32 formats against the reference's own CPU dequantizers
  (kquant_dequant_test.cpp:118-224): bit for bit on the committed vectors
  those functions produced (tests/golden/kquant_reference_vectors.npz), and
  live on fresh seeds where oracle/_ref/libnfref_kquant.so is built.
* Q6_K has no CPU reference (only the kernel, metal_provider.mm:534-573): a
  hand-packed known-answer block (layout of ql / qh / int8 scales) and the
  rounding closed form fp32(exact product).
* f16 outputs: numpy's float32 -> float16 round-to-nearest-even of the pinned
  f32 values; dequant_q3_k_f16's raw-byte scales (metal_provider.mm:833-848)
  by a hand-packed known answer that includes the read past the last block.
* The 6-bit scale/min packing of Q4_K/Q5_K by a hand-packed known answer.
The last test plants plausible mistakes in copies of the oracle and checks the
same pins reject them.
"""
from pathlib import Path

import numpy as np
import pytest

from neurofabric_amd import synthetic as syn
from oracle import oracle as orc

pytestmark = pytest.mark.filterwarnings("ignore::RuntimeWarning")

GOLDEN = Path(__file__).resolve().parent / "golden" / "kquant_reference_vectors.npz"
REF_FMTS = ["q4_1", "q5_0", "q5_1", "q2_k", "q3_k", "q4_k", "q5_k"]
ALL_FMTS = REF_FMTS + ["q6_k"]


def _bits_equal(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


def _f16(x):
    return np.float16(x).view(np.uint16)


# ---- the reference's CPU dequantizers ----------------------------------------------

def _golden_ok(dequant_fn) -> bool:
    g = np.load(GOLDEN)
    for fmt in REF_FMTS:
        for tag in ("reftest", "rand"):
            blocks, want = g[f"{fmt}_{tag}_blocks"], g[f"{fmt}_{tag}_f32"]
            if not _bits_equal(dequant_fn(blocks, fmt, want.size), want):
                return False
    return True


def test_golden_reference_vectors():
    assert _golden_ok(lambda b, f, n: orc.dequant(b, f, n))


@pytest.mark.skipif(not orc.ref_kquant_available(), reason="oracle/_ref/libnfref_kquant.so not built (needs the reference tree)")
@pytest.mark.parametrize("fmt", REF_FMTS)
def test_matches_reference_cpu_functions_live(fmt):
    bs, be = syn.KQ_GEOM[fmt]
    for seed in range(4):
        nb = 37
        blocks = syn.kquant_blocks(fmt, nb, seed=seed, scale=[0.01, 1.0, 3e-5, 100.0][seed])
        want = orc.ref_kquant_dequant(blocks, fmt, nb)
        assert _bits_equal(orc.dequant(blocks, fmt, nb * be), want)
        # a partial last block: the oracle's prefix
        assert _bits_equal(orc.dequant(blocks, fmt, nb * be - 13), want[: nb * be - 13])
    # every byte value in every position (random bytes, fp16 fields included:
    # Inf / NaN scales propagate as the reference's arithmetic does)
    raw = np.random.default_rng(7).integers(0, 256, (512, bs), dtype=np.uint8)
    assert _bits_equal(orc.dequant(raw, fmt, 512 * be), orc.ref_kquant_dequant(raw, fmt, 512))


# ---- f16 outputs ---------------------------------------------------------------------

@pytest.mark.parametrize("fmt", [f for f in ALL_FMTS if f != "q3_k"])
def test_f16_is_rne_of_f32(fmt):
    _, be = syn.KQ_GEOM[fmt]
    blocks = syn.kquant_blocks(fmt, 64, seed=3, scale=[0.01, 40.0][fmt in ("q4_k", "q5_k")])
    f32 = orc.dequant(blocks, fmt, 64 * be)
    f16 = orc.dequant(blocks, fmt, 64 * be, f16=True)
    assert np.array_equal(f16, f32.astype(np.float16).view(np.uint16))


def _q3_pack(d_bits, codes, scale_bytes):
    """One Q3_K block {hmask[32], qs[64], scales[12], d} from 3-bit codes."""
    blk = np.zeros(110, np.uint8)
    for i, q in enumerate(codes):
        blk[32 + i // 4] |= (q & 3) << (2 * (i % 4))
        blk[i // 8] |= (q >> 2) << (i % 8)
    blk[96:108] = scale_bytes
    blk[108], blk[109] = d_bits & 0xFF, d_bits >> 8
    return blk


def _q3_known():
    codes = [(i * 5 + 1) % 8 for i in range(256)]
    b0 = _q3_pack(int(_f16(0.5)), codes, [32 + k for k in range(12)])
    b1 = _q3_pack(int(_f16(0.25)), codes[::-1], [40 - k for k in range(12)])
    return np.concatenate([b0, b1]), codes


def _q3_f16_ok(dequant_fn) -> bool:
    """dequant_q3_k_f16: scale = byte 96 + sub of the block - 32 for sub =
    0..15; sub 12, 13 are d's bytes, sub 14, 15 the next block's first two
    bytes, 0 past the end of the buffer."""
    blocks, codes = _q3_known()
    got = np.asarray(dequant_fn(blocks, "q3_k", 512, True))
    want = []
    for b in range(2):
        d = np.frombuffer(blocks[b * 110 + 108: b * 110 + 110].tobytes(), np.float16)[0].astype(np.float64)
        cb = codes if b == 0 else codes[::-1]
        for i in range(256):
            off = b * 110 + 96 + i // 16
            raw = int(blocks[off]) if off < blocks.size else 0
            want.append(d * (raw - 32) * (cb[i] - 4))
    return np.array_equal(got, np.array(want).astype(np.float16).view(np.uint16))


def _q3_f32_ok(dequant_fn) -> bool:
    """dequant_q3_k: 6-bit scales, low/high nibble of bytes 0..7, two bits
    from bytes 8..11 (kquant_dequant_test.cpp:165-174)."""
    six = [(5 * s + 3) % 64 for s in range(16)]
    sb = np.zeros(12, np.uint8)
    for s in range(16):
        j = s % 8
        sb[j] |= (six[s] & 0xF) << (0 if s < 8 else 4)
        sb[8 + j // 2] |= (six[s] >> 4) << (4 * (j % 2) + (0 if s < 8 else 2))
    codes = [(i * 3) % 8 for i in range(256)]
    blk = _q3_pack(int(_f16(0.375)), codes, sb)
    want = np.array([0.375 * (six[i // 16] - 32) * (codes[i] - 4) for i in range(256)], np.float32)
    return _bits_equal(dequant_fn(blk, "q3_k", 256, False), want)


def test_q3_k_known_answers():
    assert _q3_f32_ok(lambda b, f, n, h: orc.dequant(b, f, n, f16=h))
    assert _q3_f16_ok(lambda b, f, n, h: orc.dequant(b, f, n, f16=h))


# ---- Q4_K / Q5_K scale-min packing ---------------------------------------------------

def _k_scales_pack(sc, mn):
    """12 bytes holding eight 6-bit scales and mins (kquant_dequant_test.cpp:190-198)."""
    b = np.zeros(12, np.uint8)
    for j in range(4):
        b[j] = sc[j] | ((sc[j + 4] & 3) << 6)
        b[j + 4] = mn[j] | ((mn[j + 4] & 3) << 6)
        b[j + 8] = (sc[j + 4] >> 2) | ((mn[j + 4] >> 2) << 4)
    return b


def _qk_known(fmt):
    sc = [7, 63, 1, 32, 45, 2, 60, 17]
    mn = [0, 5, 63, 31, 12, 48, 3, 58]
    codes = [(i * 11 + 5) % (32 if fmt == "q5_k" else 16) for i in range(256)]
    blk = np.zeros(176 if fmt == "q5_k" else 144, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(0.125).tobytes(), np.uint8)
    blk[2:4] = np.frombuffer(np.float16(0.0625).tobytes(), np.uint8)
    blk[4:16] = _k_scales_pack(sc, mn)
    for i, q in enumerate(codes):
        blk[16 + i // 2] |= (q & 0xF) << (4 * (i & 1))
        if fmt == "q5_k":
            blk[144 + i // 8] |= (q >> 4) << (i % 8)
    want = np.array([0.125 * sc[i // 32] * codes[i] - 0.0625 * mn[i // 32] for i in range(256)], np.float64)
    return blk, want.astype(np.float32)


def _qk_ok(dequant_fn) -> bool:
    return all(_bits_equal(dequant_fn(*_qk_known(f)[:1], f, 256), _qk_known(f)[1]) for f in ("q4_k", "q5_k"))


def test_q4_k_q5_k_scale_min_packing():
    assert _qk_ok(lambda b, f, n: orc.dequant(b, f, n))


# ---- Q6_K (no CPU reference) ---------------------------------------------------------

def _q6_pack(d, scales, codes):
    blk = np.zeros(210, np.uint8)
    for i, q in enumerate(codes):
        blk[i // 2] |= (q & 0xF) << (4 * (i & 1))
        blk[128 + i // 4] |= (q >> 4) << (2 * (i % 4))
    blk[192:208] = np.array(scales, np.int8).view(np.uint8)
    blk[208:210] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    return blk


def _q6_ok(dequant_fn) -> bool:
    """metal_provider.mm:541-573: 6-bit code = (2-bit field i%4 of qh[i/4]) << 4
    | nibble (i odd: high) of ql[i/2]; value (int8 scales[i/16] * d) * (code - 32)."""
    codes = [(i * 7 + 3) % 64 for i in range(256)]
    scales = [s - 8 for s in range(16)]
    blk = _q6_pack(0.5, scales, codes)
    want = np.array([0.5 * scales[i // 16] * (codes[i] - 32) for i in range(256)], np.float32)
    if not _bits_equal(dequant_fn(blk, "q6_k", 256), want):
        return False
    # Rounding: full-significand d and scales up to +-128 make d*s*q need
    # up to 25 bits; the value is the exact product rounded once.
    r = np.random.default_rng(11)
    blks, want = [], []
    for _ in range(64):
        d = np.float16(r.uniform(0.5, 1.0))
        sc = r.integers(-128, 128, 16)
        cd = r.integers(0, 64, 256)
        blks.append(_q6_pack(d, sc, cd))
        want.append(np.float64(d) * sc[np.arange(256) // 16].astype(np.float64) * (cd - 32))
    want = np.concatenate(want)
    return _bits_equal(dequant_fn(np.concatenate(blks), "q6_k", want.size), want.astype(np.float32))


def test_q6_k_known_answer_and_rounding():
    assert _q6_ok(lambda b, f, n: orc.dequant(b, f, n))


def test_partial_counts_and_short_input():
    for fmt in ALL_FMTS:
        bs, be = syn.KQ_GEOM[fmt]
        blocks = syn.kquant_blocks(fmt, 3, seed=1)
        full = orc.dequant(blocks, fmt, 3 * be)
        assert _bits_equal(orc.dequant(blocks, fmt, 2 * be + 1), full[: 2 * be + 1])
        with pytest.raises(ValueError):
            orc.dequant(blocks.reshape(-1)[:-1], fmt, 3 * be)


# ---- planted mistakes ------------------------------------------------------------------

def _mutant(fmt_bad, transform):
    """A copy of the oracle whose `fmt_bad` output passes through `transform`."""
    def fn(blocks, fmt, n, f16=False):
        if fmt != fmt_bad:
            return orc.dequant(blocks, fmt, n, f16=f16)
        return transform(np.ascontiguousarray(blocks, np.uint8).reshape(-1), fmt, n, f16)
    return fn


def _swap_nibbles(b, fmt, n, f16, lo, hi):
    b = b.copy()
    bs, _ = syn.KQ_GEOM[fmt]
    v = b.reshape(-1, bs)
    v[:, lo:hi] = ((v[:, lo:hi] & 0xF) << 4) | (v[:, lo:hi] >> 4)
    return orc.dequant(v, fmt, n, f16=f16)


def test_planted_mistakes_are_caught():
    # Q4_K read with the (scale, min) nibble pairs of bytes 8..11 swapped
    def q4k_swapped(b, fmt, n, f16):
        return _swap_nibbles(b, fmt, n, f16, 12, 16)
    assert not _golden_ok(lambda b, f, n: _mutant("q4_k", q4k_swapped)(b, f, n))
    assert not _qk_ok(lambda b, f, n: _mutant("q4_k", q4k_swapped)(b, f, n))
    # Q5_0 with its high-bit mask ignored
    def q5_no_high(b, fmt, n, f16):
        v = b.reshape(-1, 22).copy()
        v[:, 2:6] = 0
        return orc.dequant(v, fmt, n, f16=f16)
    assert not _golden_ok(lambda b, f, n: _mutant("q5_0", q5_no_high)(b, f, n))
    # Q6_K with the ql nibble order reversed (odd elements from the low nibble)
    def q6_swapped(b, fmt, n, f16):
        return _swap_nibbles(b, fmt, n, f16, 0, 128)
    assert not _q6_ok(lambda b, f, n: _mutant("q6_k", q6_swapped)(b, f, n))
    # Q6_K with the scales read unsigned
    def q6_unsigned(b, fmt, n, f16):
        v = b.reshape(-1, 210)
        out = orc.dequant(v, fmt, n, f16=f16).astype(np.float64)
        sc = v[:, 192:208].view(np.int8).astype(np.float64)
        fix = np.where(sc < 0, (sc + 256) / np.where(sc == 0, 1, sc), 1.0)
        return (out * np.repeat(fix, 16, axis=1).reshape(-1)[:n]).astype(np.float32)
    assert not _q6_ok(lambda b, f, n: _mutant("q6_k", q6_unsigned)(b, f, n))
    # dequant_q3_k_f16 computed with the f32 op's 6-bit scales
    def q3_f16_as_f32(b, fmt, n, f16):
        return orc.dequant(b, fmt, n, f16=False).astype(np.float16).view(np.uint16) if f16 else orc.dequant(b, fmt, n)
    assert not _q3_f16_ok(lambda b, f, n, h: _mutant("q3_k", q3_f16_as_f32)(b, f, n, h))
    # the overrun bytes taken from the wrong block (the block's own hmask)
    def q3_own_block(b, fmt, n, f16):
        if not f16:
            return orc.dequant(b, fmt, n)
        v = np.concatenate([b, np.zeros(2, np.uint8)])
        out = []
        for k in range(v.size // 110):
            blk = v[k * 110:(k + 1) * 110]
            padded = np.concatenate([blk, blk[:2]])
            out.append(orc.dequant(padded, fmt, 256, f16=True))
        return np.concatenate(out)[:n]
    assert not _q3_f16_ok(lambda b, f, n, h: _mutant("q3_k", q3_own_block)(b, f, n, h))
