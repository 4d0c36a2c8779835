"""Writes the committed golden fixtures of this directory (test data only).

    python tests/golden/make_golden.py

known_answer_blocks.npz
    The block patterns of the reference's own tests, with their expected
    dequantized values:
      q4_dt   tests/driver/dequant_test.cpp:155-168   8 Q4_0 blocks, d = 0.5 + 0.1 b
      q8_dt   tests/driver/dequant_test.cpp:233-239   8 Q8_0 blocks, d = 0.25 + 0.05 b
      q4_pipe tests/driver/dequant_test.cpp:408-411   1 Q4_0 block, d = 1, and the
              1x32 @ 32x4 matmul of :418-429 (B[k, n] = (k*4 + n) % 5 * 0.2)
      q4_f16t tests/driver/fp16_kernel_test.cpp:292-302  4 Q4_0 blocks for
              dequant_q4_0_f16
    Scales are encoded with the tests' own truncating fp16 encoder
    (dequant_test.cpp:100-109, fp16_kernel_test.cpp:45-53).  Expected f32
    values are d * (code - 8) (Q4_0) / d * code (Q8_0), computed here in
    float64 from the decoded scale (exact in f32); expected f16 bits are the
    round-to-nearest-even of that exact product.  The oracle must reproduce
    both; the script asserts it before writing.

small_linear_cases.npz
    Fused dequant+linear cases (inputs and expected outputs), including the
    reference's own shapes (4,8,32), (5,7,64), (64,128,256)
    (fused_matmul_test.cpp:294-297), computed by the oracle's sequential-k
    restatement and checked here against a float64 evaluation of the same
    dequantized values (relative error <= 1e-5 normwise).

kquant_reference_vectors.npz
    Inputs and outputs of the reference's own CPU dequantizers
    ref_dequant_q4_1 .. ref_dequant_q5_k (kquant_dequant_test.cpp:118-224),
    compiled from that file by `make -C oracle ref` into
    oracle/_ref/libnfref_kquant.so (only where the reference tree is
    present).  Per format: `<fmt>_reftest_*` is the test's own input pattern
    (bytes (i*73+17) & 0xFF, bytes 0-1 of block b = its truncating fp16
    encoding of 0.01*(b+1); kquant_dequant_test.cpp:240-252) over the test's
    block count, `<fmt>_rand_*` is synthetic.kquant_blocks(fmt, .., seed=900+i)
    over 2048 elements.  The oracle must reproduce every output bit (NaN as a
    class); the script asserts it before writing.

synthetic_sha256.json
    SHA-256 of the deterministic synthetic inputs of the BASELINE configs
    (weights seeded N*7 + K, activations seeded K), so any host can check it
    regenerates identical bytes.  Q8_0 lm_head 128256x4096 (558 MB) is
    omitted to keep generation short.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
sys.path.insert(0, str(REPO))

from neurofabric_amd import synthetic as syn  # noqa: E402
from oracle import oracle as orc  # noqa: E402


def trunc_f16(x: float) -> int:
    """The reference tests' encoder: truncate the mantissa, flush subnormals."""
    fb = int(np.array([x], np.float32).view(np.uint32)[0])
    sign = (fb >> 16) & 0x8000
    exp = ((fb >> 23) & 0xFF) - 127 + 15
    mant = (fb >> 13) & 0x3FF
    if exp <= 0:
        return sign
    if exp >= 31:
        return sign | 0x7C00
    return sign | (exp << 10) | mant


def rne_f16_bits(x64: np.ndarray) -> np.ndarray:
    """float64 values that are exact products -> RNE fp16 bits (numpy's
    float64 -> float16 cast rounds to nearest even)."""
    return x64.astype(np.float16).view(np.uint16)


def q4_blocks(ds, codes):
    return syn.pack_q4_0(np.array(ds, np.uint16).view(np.float16), np.array(codes)).reshape(-1)


def q8_blocks(ds, codes):
    return syn.pack_q8_0(np.array(ds, np.uint16).view(np.float16), np.array(codes)).reshape(-1)


def known_answers() -> dict:
    out = {}
    # dequant_test.cpp:155-168
    ds, codes = [], []
    for b in range(8):
        ds.append(trunc_f16(0.5 + 0.1 * b))
        codes.append([(j + b) & 0xF for j in range(16)] + [(15 - j + b) & 0xF for j in range(16)])
    out["q4_dt"] = (q4_blocks(ds, codes), "q4_0", ds, codes)
    # dequant_test.cpp:233-239
    ds, codes = [], []
    for b in range(8):
        ds.append(trunc_f16(0.25 + 0.05 * b))
        codes.append([j - 16 + b for j in range(32)])
    out["q8_dt"] = (q8_blocks(ds, codes), "q8_0", ds, codes)
    # dequant_test.cpp:408-411
    ds = [trunc_f16(1.0)]
    codes = [[j & 0xF for j in range(16)] + [(j + 1) & 0xF for j in range(16)]]
    out["q4_pipe"] = (q4_blocks(ds, codes), "q4_0", ds, codes)
    # fp16_kernel_test.cpp:292-302
    ds, codes = [], []
    for b in range(4):
        ds.append(trunc_f16(0.5 + b * 0.1))
        codes.append([(i + 1) & 0xF for i in range(16)] + [(i + 2) & 0xF for i in range(16)])
    out["q4_f16t"] = (q4_blocks(ds, codes), "q4_0", ds, codes)
    return out


def write_known_answers(path: Path):
    arrays = {}
    for name, (blocks, fmt, ds, codes) in known_answers().items():
        d64 = np.array(ds, np.uint16).view(np.float16).astype(np.float64)
        q = np.array(codes, np.float64) - (8.0 if fmt == "q4_0" else 0.0)
        want = (d64[:, None] * q).reshape(-1)
        want32 = want.astype(np.float32)
        assert np.array_equal(want32.astype(np.float64), want), "products must be exact in f32"
        want16 = rne_f16_bits(want)
        n = want.size
        got32 = orc.dequant(blocks, fmt, n)
        got16 = orc.dequant(blocks, fmt, n, f16=True)
        assert np.array_equal(got32.view(np.uint32), want32.view(np.uint32)), name
        assert np.array_equal(np.asarray(got16).view(np.uint16), want16), name
        arrays[f"{name}_blocks"] = blocks
        arrays[f"{name}_f32"] = want32
        arrays[f"{name}_f16bits"] = want16
    # the pipeline matmul of dequant_test.cpp:418-429: A = dequant [1, 32],
    # B_logical[k, n] = (k*N + n) % 5 * 0.2 for N = 4, stored [N, K]
    K, N = 32, 4
    bl = ((np.arange(K * N) % 5).astype(np.float32) * np.float32(0.2)).reshape(K, N)
    B = np.ascontiguousarray(bl.T)
    A = arrays["q4_pipe_f32"].reshape(1, K)
    C = orc.linear_f32(A, B, 1, N, K)
    ref64 = A.astype(np.float64) @ B.T.astype(np.float64)
    assert np.max(np.abs(C - ref64)) <= 1e-5 * np.max(np.abs(ref64))
    arrays["q4_pipe_B"] = B
    arrays["q4_pipe_C"] = C
    np.savez_compressed(path, **arrays)


SMALL = [("q4_0", False, 4, 8, 32), ("q4_0", False, 5, 7, 64), ("q4_0", False, 64, 128, 256),
         ("q4_0", True, 4, 8, 32), ("q4_0", True, 5, 7, 64), ("q8_0", False, 4, 8, 32),
         ("q8_0", False, 5, 7, 64), ("q8_0", True, 5, 7, 64), ("q4_0", False, 1, 40, 512),
         ("q4_0", False, 3, 33, 96), ("q8_0", False, 17, 9, 320), ("q4_0", True, 6, 20, 256)]


def write_small_cases(path: Path):
    arrays = {}
    for i, (fmt, f16, M, N, K) in enumerate(SMALL):
        W = syn.weights(fmt, N, K, seed=100 + i)
        A = syn.activations(M, K, seed=200 + i, dtype=np.float16 if f16 else np.float32)
        C = orc.fused(A, W, fmt, M, N, K, f16=f16)
        # float64 evaluation of the same dequantized values
        Wd = orc.dequant(W, fmt, N * K, f16=f16)
        Wd = (np.asarray(Wd).view(np.float16) if f16 else Wd).astype(np.float64).reshape(N, K)
        ref = A.astype(np.float64) @ Wd.T
        got = (np.asarray(C).view(np.float16) if f16 else C).astype(np.float64)
        tol = 1e-3 if f16 else 1e-5
        assert np.max(np.abs(got - ref)) <= tol * max(np.max(np.abs(ref)), 1e-30), (fmt, f16, M, N, K)
        key = f"c{i}"
        arrays[f"{key}_meta"] = np.array([M, N, K, int(f16), 0 if fmt == "q4_0" else 1], np.int64)
        arrays[f"{key}_A"] = A
        arrays[f"{key}_W"] = W
        arrays[f"{key}_C"] = np.asarray(C)
    np.savez_compressed(path, **arrays)


KQ_REF_FORMATS = [("q4_1", 8), ("q5_0", 8), ("q5_1", 8), ("q2_k", 4), ("q3_k", 4), ("q4_k", 4), ("q5_k", 4)]


def reftest_pattern(fmt: str, n_blocks: int) -> np.ndarray:
    """kquant_dequant_test.cpp:240-252: pseudo-random bytes, then bytes 0-1 of
    every block set to the test's fp16 encoding of 0.01 * (b + 1)."""
    bs, _ = syn.KQ_GEOM[fmt]
    raw = ((np.arange(n_blocks * bs, dtype=np.int64) * 73 + 17) & 0xFF).astype(np.uint8).reshape(n_blocks, bs)
    for b in range(n_blocks):
        h = trunc_f16(np.float32(0.01) * np.float32(b + 1))
        raw[b, 0], raw[b, 1] = h & 0xFF, h >> 8
    return raw


def _same_bits_nan_class(a: np.ndarray, b: np.ndarray) -> bool:
    na, nb = np.isnan(a), np.isnan(b)
    return np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


def write_kquant_vectors(path: Path):
    if not orc.ref_kquant_available():
        print("oracle/_ref/libnfref_kquant.so not built (needs the reference tree):", path.name, "kept as is")
        return
    arrays = {}
    for i, (fmt, n_ref) in enumerate(KQ_REF_FORMATS):
        _, be = syn.KQ_GEOM[fmt]
        for tag, blocks in (("reftest", reftest_pattern(fmt, n_ref)),
                            ("rand", syn.kquant_blocks(fmt, 2048 // be, seed=900 + i))):
            n = blocks.shape[0]
            want = orc.ref_kquant_dequant(blocks, fmt, n)
            got = orc.dequant(blocks, fmt, n * be)
            assert _same_bits_nan_class(got, want), (fmt, tag)
            arrays[f"{fmt}_{tag}_blocks"] = blocks
            arrays[f"{fmt}_{tag}_f32"] = want
    np.savez_compressed(path, **arrays)


def config_inputs():
    """(label, fmt, N, K) of every distinct weight shape of the configs, plus
    activation shapes (label, M, K)."""
    w = [("c0_tinyllama_gate", "q4_0", 5632, 2048)]
    w += [(f"c1_{n}", "q4_0", N, K) for (n, N, K) in syn.TINYLLAMA_LAYER[:2] + syn.TINYLLAMA_LAYER[4:5]
          + syn.TINYLLAMA_LAYER[6:7] + [syn.TINYLLAMA_LM_HEAD]]
    w += [(f"c2_{n}", "q4_0", N, K) for (n, N, K) in syn.LLAMA2_7B_PREFILL]
    w += [(f"c3_{n}", "q8_0", N, K) for (n, N, K) in syn.LLAMA3_8B_Q8 if n in ("q_proj", "k_proj", "gate_proj", "down_proj")]
    w += [(f"c4_{n}", "q4_0", N, K) for (n, N, K) in syn.LLAMA70B_FFN]
    a = [("x_f32_1x2048", 1, 2048, np.float32), ("x_f32_16x5632", 16, 5632, np.float32),
         ("x_f16_512x4096", 512, 4096, np.float16), ("x_f32_64x14336", 64, 14336, np.float32)]
    return w, a


def write_hashes(path: Path):
    w, a = config_inputs()
    out = {"weights_seed": "N*7 + K", "activations_seed": "K", "weights": {}, "activations": {}}
    for (label, fmt, N, K) in w:
        out["weights"][label] = {"fmt": fmt, "N": N, "K": K, "sha256": syn.sha256(syn.weights(fmt, N, K, seed=N * 7 + K))}
    for (label, M, K, dt) in a:
        out["activations"][label] = {"M": M, "K": K, "dtype": np.dtype(dt).name,
                                     "sha256": syn.sha256(syn.activations(M, K, seed=K, dtype=dt))}
    path.write_text(json.dumps(out, indent=1) + "\n")


def main():
    write_known_answers(HERE / "known_answer_blocks.npz")
    write_small_cases(HERE / "small_linear_cases.npz")
    write_kquant_vectors(HERE / "kquant_reference_vectors.npz")
    write_hashes(HERE / "synthetic_sha256.json")
    print("wrote", *(p.name for p in sorted(HERE.glob("*.npz"))), "synthetic_sha256.json")


if __name__ == "__main__":
    main()
