"""Shared numerics checks for the GPU parity tests.

Tolerance: matmul outputs within max relative
error 1e-3 of the CPU oracle.  Two forms are reported and both must hold:
  mixed    : max |got - ref| / max(1, |ref|)       (dequant_test.cpp:376-379)
  normwise : max |got - ref| / max |ref|
Dequantized weights must be bit-exact.
"""
import numpy as np

REL_TOL = 1e-3


def rel_errors(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    d = np.abs(got - ref)
    mixed = float(np.max(d / np.maximum(1.0, np.abs(ref)))) if d.size else 0.0
    scale = float(np.max(np.abs(ref))) if ref.size else 0.0
    normwise = float(np.max(d)) / scale if scale > 0 else float(np.max(d, initial=0.0))
    return mixed, normwise


def assert_close(got, ref, tol=REL_TOL, what=""):
    mixed, normwise = rel_errors(got, ref)
    assert mixed <= tol and normwise <= tol, f"{what}: mixed={mixed:.3e} normwise={normwise:.3e} tol={tol}"
    return mixed, normwise


def is_nan16(bits):
    bits = np.asarray(bits, np.uint16)
    return ((bits & 0x7C00) == 0x7C00) & ((bits & 0x03FF) != 0)


def assert_bits_equal_f16(got_bits, want_bits, what=""):
    got_bits = np.asarray(got_bits, np.uint16)
    want_bits = np.asarray(want_bits, np.uint16)
    nan = is_nan16(want_bits)
    bad = np.flatnonzero((got_bits != want_bits) & ~nan)
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first at {bad[:5]} got {got_bits[bad[:5]]} want {want_bits[bad[:5]]}"
    assert is_nan16(got_bits[nan]).all(), f"{what}: NaN class mismatch"


def assert_bits_equal_f32(got, want, what=""):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    nan = np.isnan(want)
    bad = np.flatnonzero((got.view(np.uint32) != want.view(np.uint32)) & ~nan)
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first at {bad[:5]} got {got[bad[:5]]} want {want[bad[:5]]}"
    assert np.isnan(got[nan]).all(), f"{what}: NaN class mismatch"
