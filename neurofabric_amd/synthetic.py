"""Seeded synthetic inputs for the quantized linear path.

Block packing follows ggml/GGUF (dequant_test.cpp:61-74, gguf_loader.hpp:64,68):
  Q4_0 block (18 B) = fp16 scale d (little endian) + qs[16], where
      qs[i] = code[i] | (code[i + 16] << 4), codes in 0..15, value d*(code-8)
  Q8_0 block (34 B) = fp16 scale d + 32 int8 codes, value d*code
Weights W[N, K] are stored row-major as N*K/32 blocks along K.

Statistics are the ones BASELINE.json's configs name: Q4_0 scales
|N(0,1)|*0.01 and codes uniform 0..15; Q8_0 scales |N(0,1)|*0.002 and codes
uniform -127..127; activations N(0,1).  The scale is computed in float64 and
rounded once to fp16 (round to nearest even).  numpy's PCG64 stream makes the
bytes reproducible for a given seed on any host with the same numpy.
"""
from __future__ import annotations

import hashlib

import numpy as np

Q4_0_BYTES = 18
Q8_0_BYTES = 34
BLOCK_BYTES = {"q4_0": Q4_0_BYTES, "q8_0": Q8_0_BYTES}


def pack_q4_0(d_f16: np.ndarray, codes: np.ndarray) -> np.ndarray:
    """d_f16: (nb,) float16 scales; codes: (nb, 32) ints in 0..15 -> (nb, 18) uint8."""
    d_f16 = np.ascontiguousarray(d_f16, dtype=np.float16).reshape(-1)
    codes = np.asarray(codes, dtype=np.uint8).reshape(-1, 32)
    if codes.max(initial=0) > 15:
        raise ValueError("Q4_0 codes must be in 0..15")
    out = np.empty((codes.shape[0], Q4_0_BYTES), dtype=np.uint8)
    out[:, 0:2] = d_f16.view(np.uint8).reshape(-1, 2)
    out[:, 2:18] = codes[:, :16] | (codes[:, 16:] << 4)
    return out


def pack_q8_0(d_f16: np.ndarray, codes: np.ndarray) -> np.ndarray:
    """d_f16: (nb,) float16 scales; codes: (nb, 32) ints in -128..127 -> (nb, 34) uint8."""
    d_f16 = np.ascontiguousarray(d_f16, dtype=np.float16).reshape(-1)
    codes = np.asarray(codes, dtype=np.int8).reshape(-1, 32)
    out = np.empty((codes.shape[0], Q8_0_BYTES), dtype=np.uint8)
    out[:, 0:2] = d_f16.view(np.uint8).reshape(-1, 2)
    out[:, 2:34] = codes.view(np.uint8)
    return out


def unpack_codes(blocks: np.ndarray, fmt: str):
    """Inverse of pack_*: returns (d_f16 (nb,), signed values q' (nb, 32) int16)
    where q' = code - 8 for Q4_0 and the int8 code for Q8_0."""
    b = np.asarray(blocks, dtype=np.uint8).reshape(-1, BLOCK_BYTES[fmt])
    d = b[:, 0:2].copy().view(np.float16).reshape(-1)
    if fmt == "q4_0":
        qs = b[:, 2:18]
        q = np.concatenate([qs & 0xF, qs >> 4], axis=1).astype(np.int16) - 8
    else:
        q = b[:, 2:34].copy().view(np.int8).astype(np.int16)
    return d, q


def rng_for(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def q4_0_weights(n: int, k: int, seed: int, scale: float = 0.01) -> np.ndarray:
    """Q4_0 W[n, k] (k % 32 == 0) as a flat uint8 array of n*k/32 blocks."""
    if k % 32:
        raise ValueError("K must be a multiple of 32")
    rng = rng_for(seed)
    nb = n * k // 32
    d = (np.abs(rng.standard_normal(nb)) * scale).astype(np.float16)
    codes = rng.integers(0, 16, size=(nb, 32), dtype=np.uint8)
    return pack_q4_0(d, codes).reshape(-1)


def q8_0_weights(n: int, k: int, seed: int, scale: float = 0.002) -> np.ndarray:
    """Q8_0 W[n, k] (k % 32 == 0): codes uniform in -127..127."""
    if k % 32:
        raise ValueError("K must be a multiple of 32")
    rng = rng_for(seed)
    nb = n * k // 32
    d = (np.abs(rng.standard_normal(nb)) * scale).astype(np.float16)
    codes = rng.integers(-127, 128, size=(nb, 32), dtype=np.int16).astype(np.int8)
    return pack_q8_0(d, codes).reshape(-1)


def weights(fmt: str, n: int, k: int, seed: int) -> np.ndarray:
    return q4_0_weights(n, k, seed) if fmt == "q4_0" else q8_0_weights(n, k, seed)


# Geometry (block bytes, elements per block) and the byte offsets of the fp16
# fields (scale d, min m / dmin) of every block format the dequant ops take
# (gguf_loader.hpp:64-74, metal_provider.mm:500-736).
KQ_GEOM = {"q4_0": (18, 32), "q8_0": (34, 32), "q4_1": (20, 32), "q5_0": (22, 32),
           "q5_1": (24, 32), "q2_k": (84, 256), "q3_k": (110, 256), "q4_k": (144, 256),
           "q5_k": (176, 256), "q6_k": (210, 256)}
KQ_F16_FIELDS = {"q4_0": (0,), "q8_0": (0,), "q4_1": (0, 2), "q5_0": (0,), "q5_1": (0, 2),
                 "q2_k": (80, 82), "q3_k": (108,), "q4_k": (0, 2), "q5_k": (0, 2), "q6_k": (208,)}


def kquant_blocks(fmt: str, n_blocks: int, seed: int, scale: float = 0.01) -> np.ndarray:
    """n_blocks random blocks of `fmt` as uint8 [n_blocks, block_bytes]: every
    code / scale byte uniform, every fp16 field |N(0,1)| * scale rounded to
    nearest even (finite, so no NaN reaches the outputs)."""
    bs, _ = KQ_GEOM[fmt]
    r = rng_for(seed)
    raw = r.integers(0, 256, (n_blocks, bs), dtype=np.uint8)
    for off in KQ_F16_FIELDS[fmt]:
        h = (np.abs(r.standard_normal(n_blocks)) * scale).astype(np.float16).view(np.uint16)
        raw[:, off] = (h & 0xFF).astype(np.uint8)
        raw[:, off + 1] = (h >> 8).astype(np.uint8)
    return raw


def activations(m: int, k: int, seed: int, dtype=np.float32) -> np.ndarray:
    """A[m, k] ~ N(0, 1); f16 activations are rounded to nearest even."""
    x = rng_for(seed).standard_normal((m, k)).astype(np.float32)
    return x.astype(dtype) if dtype != np.float32 else x


def sha256(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).view(np.uint8).tobytes()).hexdigest()


# ---- model shapes ---------------------------------
# (name, N, K) of every projection; all Q4_0 unless noted.
TINYLLAMA_LAYER = [("q_proj", 2048, 2048), ("k_proj", 256, 2048), ("v_proj", 256, 2048),
                   ("o_proj", 2048, 2048), ("gate_proj", 5632, 2048), ("up_proj", 5632, 2048),
                   ("down_proj", 2048, 5632)]
TINYLLAMA_LAYERS = 22
TINYLLAMA_LM_HEAD = ("lm_head", 32000, 2048)

LLAMA2_7B_PREFILL = [("qkvo_proj", 4096, 4096), ("gate_up_proj", 11008, 4096),
                     ("down_proj", 4096, 11008)]

# Llama-2-7B decode projections (north_star's "Llama-7B shapes"): 32 layers.
LLAMA2_7B_LAYER = [("q_proj", 4096, 4096), ("k_proj", 4096, 4096), ("v_proj", 4096, 4096),
                   ("o_proj", 4096, 4096), ("gate_proj", 11008, 4096), ("up_proj", 11008, 4096),
                   ("down_proj", 4096, 11008)]
LLAMA2_7B_LAYERS = 32
LLAMA2_7B_LM_HEAD = ("lm_head", 32000, 4096)

LLAMA3_8B_Q8 = [("q_proj", 4096, 4096), ("k_proj", 1024, 4096), ("v_proj", 1024, 4096),
                ("o_proj", 4096, 4096), ("gate_proj", 14336, 4096), ("up_proj", 14336, 4096),
                ("down_proj", 4096, 14336), ("lm_head", 128256, 4096)]

LLAMA70B_FFN = [("gate_up_proj", 28672, 8192), ("down_proj", 8192, 28672)]


def tinyllama_step_shapes():
    """The 155 projections of one TinyLlama-1.1B decode step, in order."""
    out = []
    for layer in range(TINYLLAMA_LAYERS):
        for name, n, k in TINYLLAMA_LAYER:
            out.append((f"l{layer}.{name}", n, k))
    out.append(TINYLLAMA_LM_HEAD)
    return out


def llama2_7b_step_shapes():
    """The 225 projections of one Llama-2-7B decode step, in order."""
    out = []
    for layer in range(LLAMA2_7B_LAYERS):
        for name, n, k in LLAMA2_7B_LAYER:
            out.append((f"l{layer}.{name}", n, k))
    out.append(LLAMA2_7B_LM_HEAD)
    return out
