"""ctypes wrapper of oracle/lib/libnf_oracle.so.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker / timed CPU reference.  The
product (neurofabric_amd, libnf_plugin_hip.so) never imports it.

Every function restates the reference's CPU algorithm; see nf_oracle.h for
the file:line each one follows.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "lib" / "libnf_oracle.so"
Q4_0, Q8_0 = 0, 1
FMT = {"q4_0": Q4_0, "q8_0": Q8_0}

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = C.CDLL(str(LIB_PATH))
        u8p, f32p, u16p = (np.ctypeslib.ndpointer(np.uint8, flags="C"),
                           np.ctypeslib.ndpointer(np.float32, flags="C"),
                           np.ctypeslib.ndpointer(np.uint16, flags="C"))
        L.nf_oracle_f16_to_f32.argtypes = [C.c_uint16]
        L.nf_oracle_f16_to_f32.restype = C.c_float
        L.nf_oracle_f32_to_f16_rne.argtypes = [C.c_float]
        L.nf_oracle_f32_to_f16_rne.restype = C.c_uint16
        L.nf_oracle_f32_to_f16_trunc.argtypes = [C.c_float]
        L.nf_oracle_f32_to_f16_trunc.restype = C.c_uint16
        L.nf_oracle_f16_to_f32_n.argtypes = [u16p, f32p, C.c_uint64]
        L.nf_oracle_f32_to_f16_rne_n.argtypes = [f32p, u16p, C.c_uint64]
        for name in ("q4_0", "q8_0"):
            getattr(L, f"nf_oracle_dequant_{name}_f32").argtypes = [u8p, C.c_uint64, f32p]
            getattr(L, f"nf_oracle_dequant_{name}_f16").argtypes = [u8p, C.c_uint64, u16p]
        L.nf_oracle_linear_f32.argtypes = [f32p, f32p, f32p, C.c_uint32, C.c_uint32, C.c_uint32]
        L.nf_oracle_linear_f16.argtypes = [u16p, u16p, u16p, C.c_uint32, C.c_uint32, C.c_uint32]
        L.nf_oracle_fused_f32.argtypes = [f32p, u8p, C.c_int, f32p] + [C.c_uint32] * 6
        L.nf_oracle_fused_f16.argtypes = [u16p, u8p, C.c_int, u16p] + [C.c_uint32] * 6
        _lib = L
    return _lib


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16).reshape(-1)
    out = np.empty(h.size, np.float32)
    lib().nf_oracle_f16_to_f32_n(h, out, h.size)
    return out


def f32_to_f16_rne(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.empty(x.size, np.uint16)
    lib().nf_oracle_f32_to_f16_rne_n(x, out, x.size)
    return out


def f32_to_f16_trunc(x: float) -> int:
    return lib().nf_oracle_f32_to_f16_trunc(float(x))


def dequant(blocks: np.ndarray, fmt: str, count: int, f16: bool = False) -> np.ndarray:
    """f32 values, or fp16 BITS (uint16) when f16=True."""
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    bs = 18 if fmt == "q4_0" else 34
    if b.size < (count + 31) // 32 * bs:
        raise ValueError("not enough blocks")
    if f16:
        out = np.empty(count, np.uint16)
        getattr(lib(), f"nf_oracle_dequant_{fmt}_f16")(b, count, out)
    else:
        out = np.empty(count, np.float32)
        getattr(lib(), f"nf_oracle_dequant_{fmt}_f32")(b, count, out)
    return out


def linear_f32(A, B, M, N, K) -> np.ndarray:
    A = np.ascontiguousarray(A, np.float32).reshape(-1)
    B = np.ascontiguousarray(B, np.float32).reshape(-1)
    C_ = np.empty(M * N, np.float32)
    lib().nf_oracle_linear_f32(A, B, C_, M, N, K)
    return C_.reshape(M, N)


def linear_f16(A_bits, B_bits, M, N, K) -> np.ndarray:
    A = np.ascontiguousarray(A_bits, np.uint16).reshape(-1)
    B = np.ascontiguousarray(B_bits, np.uint16).reshape(-1)
    C_ = np.empty(M * N, np.uint16)
    lib().nf_oracle_linear_f16(A, B, C_, M, N, K)
    return C_.reshape(M, N)


def fused(A, W, fmt: str, M, N, K, f16: bool = False, cols=None, threads: int = 1) -> np.ndarray:
    """Fused dequant+linear.  f32 path: A float32, returns float32 [M,N].
    f16 path: A fp16 bits (uint16) or float16, returns fp16 bits [M,N].
    `cols=(n0, n1)` computes only those output columns (others are 0)."""
    n0, n1 = cols if cols else (0, N)
    W = np.ascontiguousarray(W, np.uint8).reshape(-1)
    if f16:
        A = np.ascontiguousarray(np.asarray(A).view(np.uint16) if np.asarray(A).dtype == np.float16
                                 else A, np.uint16).reshape(-1)
        out = np.zeros(M * N, np.uint16)
        lib().nf_oracle_fused_f16(A, W, FMT[fmt], out, M, N, K, n0, n1, threads)
    else:
        A = np.ascontiguousarray(A, np.float32).reshape(-1)
        out = np.zeros(M * N, np.float32)
        lib().nf_oracle_fused_f32(A, W, FMT[fmt], out, M, N, K, n0, n1, threads)
    return out.reshape(M, N)


def available() -> bool:
    try:
        lib()
        return True
    except OSError:
        return False


__all__ = ["build", "lib", "f16_to_f32", "f32_to_f16_rne", "f32_to_f16_trunc", "dequant",
           "linear_f32", "linear_f16", "fused", "Q4_0", "Q8_0", "available"]
