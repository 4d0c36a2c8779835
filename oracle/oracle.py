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
FMT = {"q4_0": 0, "q8_0": 1, "q4_1": 2, "q5_0": 3, "q5_1": 4,
       "q2_k": 5, "q3_k": 6, "q4_k": 7, "q5_k": 8, "q6_k": 9}
# (block bytes, elements per block) of each format (gguf_loader.hpp:64-74).
GEOM = {"q4_0": (18, 32), "q8_0": (34, 32), "q4_1": (20, 32), "q5_0": (22, 32),
        "q5_1": (24, 32), "q2_k": (84, 256), "q3_k": (110, 256), "q4_k": (144, 256),
        "q5_k": (176, 256), "q6_k": (210, 256)}
REF_KQUANT = HERE / "_ref" / "libnfref_kquant.so"

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
        L.nf_oracle_dequant.argtypes = [C.c_int, u8p, C.c_uint64, C.c_uint64, C.c_int, C.c_void_p]
        L.nf_oracle_dequant.restype = C.c_int
        L.nf_oracle_block_bytes.argtypes = [C.c_int]
        L.nf_oracle_block_bytes.restype = C.c_uint32
        L.nf_oracle_block_elems.argtypes = [C.c_int]
        L.nf_oracle_block_elems.restype = C.c_uint32
        L.nf_oracle_linear_f32.argtypes = [f32p, f32p, f32p, C.c_uint32, C.c_uint32, C.c_uint32]
        L.nf_oracle_linear_f16.argtypes = [u16p, u16p, u16p, C.c_uint32, C.c_uint32, C.c_uint32]
        L.nf_oracle_fused_f32.argtypes = [f32p, u8p, C.c_int, f32p] + [C.c_uint32] * 6
        L.nf_oracle_fused_f32.restype = C.c_int
        L.nf_oracle_fused_f16.argtypes = [u16p, u8p, C.c_int, u16p] + [C.c_uint32] * 6
        L.nf_oracle_fused_f16.restype = C.c_int
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
    """f32 values, or fp16 BITS (uint16) when f16=True.  `blocks` is the whole
    input buffer (dequant_q3_k_f16 reads two bytes past its last block)."""
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    bs, be = GEOM[fmt]
    if b.size < (count + be - 1) // be * bs:
        raise ValueError("not enough blocks")
    if fmt not in ("q4_0", "q8_0"):
        out = np.empty(count, np.uint16 if f16 else np.float32)
        if lib().nf_oracle_dequant(FMT[fmt], b, b.size, count, int(f16), out.ctypes.data) != 0:
            raise ValueError("nf_oracle_dequant rejected the input")
        return out
    if f16:
        out = np.empty(count, np.uint16)
        getattr(lib(), f"nf_oracle_dequant_{fmt}_f16")(b, count, out)
    else:
        out = np.empty(count, np.float32)
        getattr(lib(), f"nf_oracle_dequant_{fmt}_f32")(b, count, out)
    return out


def ref_kquant_available() -> bool:
    return REF_KQUANT.exists()


def ref_kquant_dequant(blocks: np.ndarray, fmt: str, n_blocks: int) -> np.ndarray:
    """The reference's own CPU dequantizer for `fmt` (q4_1, q5_0, q5_1, q2_k,
    q3_k, q4_k, q5_k), compiled from kquant_dequant_test.cpp by
    `make -C oracle ref` into oracle/_ref/libnfref_kquant.so."""
    L = C.CDLL(str(REF_KQUANT))
    L.nfref_kquant_dequant.argtypes = [C.c_int, C.c_void_p, C.c_int, C.c_void_p]
    L.nfref_kquant_dequant.restype = C.c_int
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    bs, be = GEOM[fmt]
    assert b.size >= n_blocks * bs
    out = np.empty(n_blocks * be, np.float32)
    if L.nfref_kquant_dequant(FMT[fmt], b.ctypes.data, n_blocks, out.ctypes.data) != 0:
        raise ValueError(f"no reference CPU dequantizer for {fmt}")
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
        rc = lib().nf_oracle_fused_f16(A, W, FMT[fmt], out, M, N, K, n0, n1, threads)
    else:
        A = np.ascontiguousarray(A, np.float32).reshape(-1)
        out = np.zeros(M * N, np.float32)
        rc = lib().nf_oracle_fused_f32(A, W, FMT[fmt], out, M, N, K, n0, n1, threads)
    if rc != 0:
        raise MemoryError(f"oracle fused {fmt} {M}x{N}x{K}: working buffer or thread allocation failed")
    return out.reshape(M, N)


def available() -> bool:
    try:
        lib()
        return True
    except OSError:
        return False


__all__ = ["build", "lib", "f16_to_f32", "f32_to_f16_rne", "f32_to_f16_trunc", "dequant",
           "linear_f32", "linear_f16", "fused", "Q4_0", "Q8_0", "available"]


# ---- layer ops --------------------------------------------------------------

UNARY = {"silu": 0, "gelu": 1, "relu": 2}
BINARY = {"add": 0, "mul": 1}
ATTN_MODE = {"plain": 0, "cached": 1, "gqa": 2, "paged": 3}
# softmax arithmetic of each reference attention op
ATTN_VARIANT = {"causal_attention": (0, 0), "causal_attention_cached": (1, 0), "flash_attention_cached": (1, 1),
                "flash_attention_gqa": (2, 2), "flash_attention_paged": (3, 3)}


def _layer_lib():
    L = lib()
    if not getattr(L, "_layer_ready", False):
        vp, u32, u64, f32, i = C.c_void_p, C.c_uint32, C.c_uint64, C.c_float, C.c_int
        L.nf_oracle_unary.argtypes = [i, vp, vp, u64, i]
        L.nf_oracle_binary.argtypes = [i, vp, vp, vp, u64, i]
        L.nf_oracle_rms_norm.argtypes = [vp, vp, vp, u32, u32, f32, i]
        L.nf_oracle_rope.argtypes = [vp, vp, u64, u32, u32, u32, f32, i, i]
        L.nf_oracle_softmax.argtypes = [vp, vp, u32, u32]
        L.nf_oracle_argmax.argtypes = [vp, vp, u32, u32]
        L.nf_oracle_moe_gate.argtypes = [vp, vp, vp, u32, u32, u32]
        L.nf_oracle_moe_scatter.argtypes = [vp, u32, vp, vp, vp, u32, u32, u32]
        L.nf_oracle_embedding.argtypes = [vp, u32, vp, vp, u64, u32, u32, i]
        L.nf_oracle_attention.argtypes = [vp, i, vp, vp, vp, vp, vp, vp, vp]
        L.nf_oracle_attention.restype = C.c_int
        L._layer_ready = True
    return L


def _arr(x, f16):
    """float32 array, or fp16 bits (uint16) when f16."""
    return np.ascontiguousarray(x, np.uint16 if f16 else np.float32).reshape(-1)


def unary(fn: str, x, f16: bool = False) -> np.ndarray:
    a = _arr(x, f16)
    out = np.empty_like(a)
    _layer_lib().nf_oracle_unary(UNARY[fn], a.ctypes.data, out.ctypes.data, a.size, int(f16))
    return out


def binary(fn: str, a, b, f16: bool = False) -> np.ndarray:
    a, b = _arr(a, f16), _arr(b, f16)
    out = np.empty_like(a)
    _layer_lib().nf_oracle_binary(BINARY[fn], a.ctypes.data, b.ctypes.data, out.ctypes.data, a.size, int(f16))
    return out


def rms_norm(x, w, dim: int, eps: float, f16: bool = False) -> np.ndarray:
    a = _arr(x, f16)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(a)
    _layer_lib().nf_oracle_rms_norm(a.ctypes.data, w.ctypes.data, out.ctypes.data, a.size // dim, dim, eps, int(f16))
    return out


def rope(x, n_heads: int, head_dim: int, step: int, theta: float, batch: bool = True, f16: bool = False):
    a = _arr(x, f16)
    out = np.empty_like(a)
    _layer_lib().nf_oracle_rope(a.ctypes.data, out.ctypes.data, a.size, n_heads, head_dim, step, theta, int(batch),
                                int(f16))
    return out


def softmax(x, rows: int, dim: int) -> np.ndarray:
    a = _arr(x, False)
    out = np.empty(rows * dim, np.float32)
    _layer_lib().nf_oracle_softmax(a.ctypes.data, out.ctypes.data, rows, dim)
    return out


def argmax(x, rows: int, dim: int) -> np.ndarray:
    a = _arr(x, False)
    out = np.empty(rows, np.int32)
    _layer_lib().nf_oracle_argmax(a.ctypes.data, out.ctypes.data, rows, dim)
    return out


def moe_gate(logits, batch: int, n_experts: int, top_k: int):
    """(ids int32 [batch, min(top_k, 8)], weights float32 [batch, min(top_k, 8)])."""
    a = np.ascontiguousarray(logits, np.float32).reshape(-1)
    k = min(top_k, 8)
    ids = np.zeros(batch * k, np.int32)
    w = np.zeros(batch * k, np.float32)
    _layer_lib().nf_oracle_moe_gate(a.ctypes.data, ids.ctypes.data, w.ctypes.data, batch, n_experts, top_k)
    return ids.reshape(batch, k), w.reshape(batch, k)


def moe_scatter(experts, ids, w, batch: int, top_k: int, dim: int) -> np.ndarray:
    e = np.ascontiguousarray(experts, np.float32).reshape(-1)
    ids = np.ascontiguousarray(ids, np.int32).reshape(-1)
    w = np.ascontiguousarray(w, np.float32).reshape(-1)
    out = np.zeros(batch * dim, np.float32)
    _layer_lib().nf_oracle_moe_scatter(e.ctypes.data, e.size // dim if dim else 0, ids.ctypes.data, w.ctypes.data,
                                       out.ctypes.data, batch, top_k, dim)
    return out.reshape(batch, dim)


def embedding(w, ids, n: int, dim: int, seq_len: int, f16: bool = False, out=None) -> np.ndarray:
    wa = _arr(w, f16)
    ids = np.ascontiguousarray(ids, np.int32)
    if out is None:
        out = np.zeros(n, np.uint16 if f16 else np.float32)
    _layer_lib().nf_oracle_embedding(wa.ctypes.data, wa.size // dim, ids.ctypes.data, out.ctypes.data, n, dim,
                                     seq_len, int(f16))
    return out


def attention(op: str, prm: dict, q, k_new=None, v_new=None, k=None, v=None, table=None, out=None,
              f16: bool = False):
    """The attention op `op` with the reference's softmax arithmetic.  prm
    keys: n_heads, n_kv, head_dim, seq_len, step, max_seq, window,
    block_size, n_blocks, q_offset, pool_blocks.  k / v are the caches
    (modified in place for the cached ops), K / V for causal_attention, the
    pools for paged.  Returns `out`."""
    mode, variant = ATTN_VARIANT[op]
    P = np.array([mode, variant] + [int(prm.get(key, 0)) for key in
                 ("n_heads", "n_kv", "head_dim", "seq_len", "step", "max_seq", "window", "block_size",
                  "n_blocks", "q_offset", "pool_blocks")], np.uint32)
    q = _arr(q, f16)
    bufs = [None if b is None else _arr(b, f16) for b in (k_new, v_new)]
    assert k.dtype == (np.uint16 if f16 else np.float32) and v.dtype == k.dtype and k.flags.c_contiguous
    tb = None if table is None else np.ascontiguousarray(table, np.uint32)
    assert out is not None and out.flags.c_contiguous
    ptr = lambda a: None if a is None else a.ctypes.data  # noqa: E731
    rc = _layer_lib().nf_oracle_attention(P.ctypes.data, int(f16), q.ctypes.data, ptr(bufs[0]), ptr(bufs[1]),
                                          k.ctypes.data, v.ctypes.data, ptr(tb), out.ctypes.data)
    if rc != 0:
        raise MemoryError(f"oracle attention {op}: working buffer allocation failed")
    return out
