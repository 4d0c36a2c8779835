"""Random-weight GGUF files of a llama-family shape.

No real checkpoint is available offline, so the end-to-end runs of the
reference's own application (`apps/nf_generate.cpp`) load a GGUF written
here: the llama metadata keys and tensor names that
`model/model/gguf_loader.hpp:222-361` parses and
`model/model/llama_dag_builder.hpp:848-960` looks up, a SentencePiece-style
vocabulary (`<unk>`, `<s>`, `</s>`, the 256 byte tokens `<0xNN>`, then word
pieces) that `model/model/tokenizer.hpp:41-80` accepts, and seeded weights
with the block statistics of the benchmark configurations (Q4_0: fp16 scale
|N(0,1)|*0.01, codes uniform 0..15; Q8_0: |N(0,1)|*0.002, codes -127..127;
norm weights 1 + 0.1*N(0,1) in f32).

    python -m neurofabric_amd.gguf_synth out.gguf --shape tinyllama --quant q4_0

GGUF v3 layout: magic, version, tensor count, key/value count, the key/value
pairs, the tensor infos (name, dims innermost first, ggml type, data offset),
padding to `general.alignment`, then each tensor's data at its offset.
"""
from __future__ import annotations

import argparse
import struct

import numpy as np

from . import synthetic as syn

GGUF_MAGIC = 0x46554747
T_UINT32, T_INT32, T_FLOAT32, T_BOOL, T_STRING, T_ARRAY = 4, 5, 6, 7, 8, 9
GGML_F32, GGML_Q4_0, GGML_Q8_0 = 0, 2, 8
ALIGN = 32

# dim, layers, heads, kv heads, ffn, vocab, context
SHAPES = {
    "tinyllama": (2048, 22, 32, 4, 5632, 32000, 2048),
    "tiny": (256, 2, 4, 2, 512, 512, 512),
}


def _str(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _kv(key: str, vtype: int, payload: bytes) -> bytes:
    return _str(key) + struct.pack("<I", vtype) + payload


def _u32(key, v):
    return _kv(key, T_UINT32, struct.pack("<I", v))


def _f32(key, v):
    return _kv(key, T_FLOAT32, struct.pack("<f", v))


def _array(key: str, etype: int, items: list[bytes]) -> bytes:
    return _kv(key, T_ARRAY, struct.pack("<IQ", etype, len(items)) + b"".join(items))


def vocabulary(n: int) -> list[str]:
    """`<unk>`, `<s>`, `</s>`, the byte tokens, then word pieces up to n."""
    words = ["▁Hello", "▁world", "▁the", "▁a", "▁of", "▁and",
             "▁to", "▁is", "▁in", "▁it"]
    toks = ["<unk>", "<s>", "</s>"] + [f"<0x{i:02X}>" for i in range(256)] + words
    if n < len(toks):
        raise ValueError(f"vocabulary needs at least {len(toks)} entries")
    toks += [f"▁t{i}" for i in range(n - len(toks))]
    return toks


def tensors(shape: str, quant: str, seed: int):
    """Yields (name, dims innermost first, ggml type, bytes) in file order."""
    D, L, H, KVH, F, V, _ = SHAPES[shape]
    kvd = KVH * (D // H)
    qtype = {"q4_0": GGML_Q4_0, "q8_0": GGML_Q8_0}[quant]
    rng = syn.rng_for(seed)

    def quant_w(n, k, s):
        return syn.weights(quant, n, k, seed * 1000 + s).tobytes()

    def norm_w(n):
        return (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32).tobytes()

    yield "token_embd.weight", (D, V), qtype, quant_w(V, D, 0)
    for l in range(L):
        base = 10 + 10 * l
        yield f"blk.{l}.attn_norm.weight", (D,), GGML_F32, norm_w(D)
        yield f"blk.{l}.ffn_norm.weight", (D,), GGML_F32, norm_w(D)
        for j, (nm, n, k) in enumerate([("attn_q", D, D), ("attn_k", kvd, D), ("attn_v", kvd, D),
                                        ("attn_output", D, D), ("ffn_gate", F, D),
                                        ("ffn_up", F, D), ("ffn_down", D, F)]):
            yield f"blk.{l}.{nm}.weight", (k, n), qtype, quant_w(n, k, base + j)
    yield "output_norm.weight", (D,), GGML_F32, norm_w(D)
    yield "output.weight", (D, V), qtype, quant_w(V, D, 1)


def write(path: str, shape: str = "tiny", quant: str = "q4_0", seed: int = 7) -> None:
    D, L, H, KVH, F, V, ctx = SHAPES[shape]
    toks = vocabulary(V)
    kvs = [
        _kv("general.architecture", T_STRING, _str("llama")),
        _u32("general.alignment", ALIGN),
        _u32("llama.embedding_length", D),
        _u32("llama.block_count", L),
        _u32("llama.attention.head_count", H),
        _u32("llama.attention.head_count_kv", KVH),
        _u32("llama.feed_forward_length", F),
        _u32("llama.context_length", ctx),
        _f32("llama.rope.freq_base", 10000.0),
        _f32("llama.attention.layer_norm_rms_epsilon", 1e-5),
        _kv("tokenizer.ggml.model", T_STRING, _str("llama")),
        _array("tokenizer.ggml.tokens", T_STRING, [_str(t) for t in toks]),
        _array("tokenizer.ggml.scores", T_FLOAT32,
               [struct.pack("<f", -float(i)) for i in range(V)]),
        _array("tokenizer.ggml.token_type", T_INT32,
               [struct.pack("<i", 3 if i < 3 else (6 if i < 259 else 1)) for i in range(V)]),
        _u32("tokenizer.ggml.bos_token_id", 1),
        _u32("tokenizer.ggml.eos_token_id", 2),
        _u32("tokenizer.ggml.unknown_token_id", 0),
        _kv("tokenizer.ggml.add_bos_token", T_BOOL, b"\x01"),
    ]
    ts = list(tensors(shape, quant, seed))
    infos, offset = [], 0
    for name, dims, gtype, data in ts:
        infos.append(_str(name) + struct.pack("<I", len(dims))
                     + b"".join(struct.pack("<Q", d) for d in dims)
                     + struct.pack("<IQ", gtype, offset))
        offset += -(-len(data) // ALIGN) * ALIGN
    head = (struct.pack("<IIQQ", GGUF_MAGIC, 3, len(ts), len(kvs))
            + b"".join(kvs) + b"".join(infos))
    with open(path, "wb") as f:
        f.write(head + b"\0" * (-len(head) % ALIGN))
        for _, _, _, data in ts:
            f.write(data + b"\0" * (-len(data) % ALIGN))


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("path")
    ap.add_argument("--shape", choices=sorted(SHAPES), default="tiny")
    ap.add_argument("--quant", choices=["q4_0", "q8_0"], default="q4_0")
    ap.add_argument("--seed", type=int, default=7)
    a = ap.parse_args()
    write(a.path, a.shape, a.quant, a.seed)


if __name__ == "__main__":
    main()
