"""This repository's model layer (neurofabric_amd/model/llama_step.hpp) on the
reference's PipelineEngine: fused Q8_0 projections and a fused quantized
output projection, end to end.

The reference's model layer fuses Q4_0 only and dequantizes every other
projection, and always the output projection, to dense fp32 at load
(quant_registry.hpp:84-88; llama_dag_builder.hpp:1025-1056, 1411-1422,
1520-1523).  Here oracle/_ref/model_run (built by `make -C oracle ref` from
oracle/model_run.cpp, the reference's engine and GGUF loader headers, and
this provider) loads a random-weight GGUF, runs a prefill step and one decode
step through PipelineEngine sessions, and prints the logits and the ops it
dispatched.  Checks:
  * every projection and the output projection run the fused op of their
    format in the decode step, with no `linear` and no dequantization there,
    and the only load-time dequantization is the embedding table's (which
    embedding_lookup reads dense in the reference as well);
  * prefill and decode logits match the oracle's forward pass of the same
    model (the oracle's restatements of each op, with the KV caches carried
    from prefill to decode), over every logit: within 2e-3 absolute on
    logits of magnitude ~3 for f32; for the f16 chain, where both sides
    round every activation of both layers to fp16 but sum in different
    orders, within 4e-2 (about 20 fp16 ulps at |logit| ~3).
"""
import subprocess
from pathlib import Path

import numpy as np
import pytest

from neurofabric_amd import gguf_synth

pytestmark = pytest.mark.gpu

REPO = Path(__file__).resolve().parents[1]
MODEL_RUN = REPO / "oracle" / "_ref" / "model_run"
MAX_SEQ = 64  # KV-cache positions model_run allocates


def oracle_forward(quant, seed, ids, next_id, f16=False):
    """(prefill logits of the last position, decode-step logits)."""
    from oracle import oracle as orc

    D, L, H, KVH, F, V, _ = gguf_synth.SHAPES["tiny"]
    hd, kvd = D // H, KVH * (D // H)
    W = {n: np.frombuffer(b, np.uint8) for n, _, _, b in gguf_synth.tensors("tiny", quant, seed)}
    f32 = lambda n: W[n].view(np.float32)  # noqa: E731
    act = np.uint16 if f16 else np.float32
    table = orc.dequant(W["token_embd.weight"], quant, V * D, f16=f16).reshape(V, D)
    caches = [(np.zeros(kvd * MAX_SEQ, act), np.zeros(kvd * MAX_SEQ, act)) for _ in range(L)]

    def step(toks, pos):
        S = len(toks)

        def lin(a, name, n, k):
            return orc.fused(a, W[name], quant, S, n, k, f16=f16)

        x = table[toks].astype(act).reshape(-1)
        for l in range(L):
            b = f"blk.{l}."
            h = orc.rms_norm(x, f32(b + "attn_norm.weight"), D, 1e-5, f16=f16)
            q, k, v = lin(h, b + "attn_q.weight", D, D), lin(h, b + "attn_k.weight", kvd, D), lin(h, b + "attn_v.weight", kvd, D)
            q = orc.rope(q, H, hd, pos, 10000.0, f16=f16)
            k = orc.rope(k, KVH, hd, pos, 10000.0, f16=f16)
            att = np.zeros(S * D, act)
            kc, vc = caches[l]
            orc.attention("flash_attention_cached", dict(n_heads=H, n_kv=KVH, head_dim=hd, seq_len=S, step=pos,
                                                         max_seq=MAX_SEQ), q, k, v, k=kc, v=vc, out=att, f16=f16)
            x = orc.binary("add", x, lin(att, b + "attn_output.weight", D, D), f16=f16)
            h2 = orc.rms_norm(x, f32(b + "ffn_norm.weight"), D, 1e-5, f16=f16)
            g = orc.unary("silu", lin(h2, b + "ffn_gate.weight", F, D), f16=f16)
            m = orc.binary("mul", g, lin(h2, b + "ffn_up.weight", F, D), f16=f16)
            x = orc.binary("add", x, orc.fused(m, W[b + "ffn_down.weight"], quant, S, D, F, f16=f16), f16=f16)
        hf = orc.rms_norm(x, f32("output_norm.weight"), D, 1e-5, f16=f16)
        logits = orc.fused(hf, W["output.weight"], quant, S, V, D, f16=f16)[S - 1]
        return orc.f16_to_f32(logits) if f16 else logits

    return step(list(ids), 0), step([next_id], len(ids))


def _parse(stdout, f16):
    lines = {l.split(" ", 1)[0]: l.split()[1:] for l in stdout.splitlines() if l.strip()}
    conv = (lambda xs: np.array([int(t) for t in xs], np.uint16).view(np.float16).astype(np.float32)) if f16 else \
        (lambda xs: np.array([float(t) for t in xs], np.float32))
    return lines["load_ops"], conv(lines["prefill"]), conv(lines["decode"]), lines["step_ops"]


@pytest.mark.skipif(not MODEL_RUN.exists(), reason="model_run not built (needs the reference's engine headers)")
@pytest.mark.parametrize("quant,f16,tol", [("q8_0", False, 2e-3), ("q4_0", False, 2e-3), ("q8_0", True, 4e-2)],
                         ids=["q8_0-f32", "q4_0-f32", "q8_0-f16"])
def test_model_layer_fused_projections_end_to_end(tmp_path, quant, f16, tol):
    seed = 13
    path = tmp_path / "tiny.gguf"
    gguf_synth.write(str(path), "tiny", quant, seed=seed)
    ids, nxt = [1, 300, 301, 5, 77, 260], 290
    print("case", quant, "f16" if f16 else "f32", flush=True)
    r = subprocess.run([str(MODEL_RUN), str(path), str(int(f16)), ",".join(map(str, ids)), str(nxt)],
                       capture_output=True, text=True, timeout=120)
    print(r.stderr[-3000:])
    assert r.returncode == 0
    load_ops, prefill, decode, step_ops = _parse(r.stdout, f16)
    fused = f"dequant_{quant}_linear" + ("_f16" if f16 else "")
    deq = f"dequant_{quant}" + ("_f16" if f16 else "")
    D, L, H, KVH, F, V, _ = gguf_synth.SHAPES["tiny"]
    # load: only the embedding table is dequantized (no projection, no lm_head)
    assert load_ops == [deq], load_ops
    # decode step: 7 projections per layer + the output projection, all fused
    assert step_ops.count(fused) == 7 * L + 1, step_ops
    assert "linear" not in step_ops and deq not in step_ops, step_ops
    assert step_ops[-2:] == [fused, "argmax"] if not f16 else step_ops[-1] == fused, step_ops[-4:]
    ref_p, ref_d = oracle_forward(quant, seed, ids, nxt, f16=f16)
    assert np.isfinite(ref_p).all() and np.abs(ref_p).max() > 0.1
    assert np.max(np.abs(prefill - ref_p)) <= tol, np.max(np.abs(prefill - ref_p))
    assert np.max(np.abs(decode - ref_d)) <= tol, np.max(np.abs(decode - ref_d))
