"""The reference's own driver test, compiled from its source by
oracle/Makefile (`make -C oracle ref`) and linked against this provider,
plus the register -> init -> shutdown lifecycle repeated in one process
(cuda_stub_test.cpp:33-140 pattern).  Both run in child processes so the
session provider of the other GPU tests is untouched."""
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu
REPO = Path(__file__).resolve().parents[1]
REF_DEQUANT = REPO / "oracle" / "_ref" / "dequant_test"
REF_KQUANT = REPO / "oracle" / "_ref" / "kquant_dequant_test"


@pytest.mark.skipif(not REF_DEQUANT.exists(), reason="reference test binary not built (needs the reference sources)")
def test_reference_dequant_test_binary_passes():
    """tests/driver/dequant_test.cpp: Q4_0/Q8_0 dequant vs its CPU reference,
    linear_tiled 64x48x32 and dequant->linear through PipelineEngine."""
    r = subprocess.run([str(REF_DEQUANT)], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0
    assert "OK: all Phase 17 dequant tests passed" in r.stdout


@pytest.mark.skipif(not REF_KQUANT.exists(), reason="reference test binary not built (needs the reference sources)")
def test_reference_kquant_dequant_test_binary_passes():
    """tests/driver/kquant_dequant_test.cpp: dequant_q4_1 .. dequant_q5_k on
    the GPU against the test's own CPU dequantizers (tolerance 1e-3)."""
    r = subprocess.run([str(REF_KQUANT)], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0
    assert "OK: all Phase 25 K-quant dequant tests passed" in r.stdout


REF_FUSED = REPO / "oracle" / "_ref" / "fused_matmul_test"


@pytest.mark.skipif(not REF_FUSED.exists(), reason="reference test binary not built (needs the reference sources)")
def test_reference_fused_matmul_test_binary_passes():
    """tests/driver/fused_matmul_test.cpp, unedited (oracle/ref_fused.cpp
    renames its `sync` around the #include): the fused ops against the
    separate dequant -> linear_tiled / linear pipeline at (4, 8, 32),
    (5, 7, 64), (64, 128, 256) f32 and (64, 128, 256) f16, dispatched with its
    FakeTaskDesc push constants (fused_matmul_test.cpp:108-126, 287-300)."""
    r = subprocess.run([str(REF_FUSED)], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0
    assert r.stdout.count("PASS") == 4 and "FAIL" not in r.stdout
    assert "=== 4/4 tests passed ===" in r.stdout


# The reference's other driver tests this provider serves, with the line each
# prints when every check passed (tests/driver/<name>.cpp).
REF_LAYER_TESTS = {
    "transformer_test": "=== ALL PASSED ===",          # softmax, silu, mul, embedding, argmax,
                                                        # causal_attention[_cached], single layer
    "gqa_attention_test": "=== All GQA attention tests passed ===",
    "paged_attn_test": "All 3 paged_attn tests passed.",
    "fp16_kernel_test": "All 7 tests PASSED",
    "dag_inference_test": "=== ALL PASSED ===",         # 2-layer model through PipelineEngine
    "multi_layer_test": "=== ALL PASSED ===",
    "benchmark_kernels": "=== Benchmark complete ===",  # f16 vs f32 element-wise ops timed
                                                        # through the nf_metal_* timing ring
}


@pytest.mark.parametrize("name", sorted(REF_LAYER_TESTS))
def test_reference_layer_test_binaries_pass(name):
    exe = REPO / "oracle" / "_ref" / name
    if not exe.exists():
        pytest.skip("reference test binary not built (needs the reference sources)")
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    print(r.stdout[-4000:], r.stderr[-2000:])
    assert r.returncode == 0
    assert REF_LAYER_TESTS[name] in r.stdout


def test_reference_trace_export_over_timing_ring(tmp_path):
    """model/model/trace_export.hpp (the reference's Chrome-trace exporter,
    compiled from where it lies by oracle/Makefile into trace_export_run)
    reads this provider's GPU timing ring through the nf_metal_* names."""
    import json
    exe = REPO / "oracle" / "_ref" / "trace_export_run"
    if not exe.exists():
        pytest.skip("trace_export_run not built (needs the reference sources)")
    out = tmp_path / "trace.json"
    r = subprocess.run([str(exe), str(out)], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0 and "trace_export_run ok 3" in r.stdout
    ev = json.loads(out.read_text())["traceEvents"]
    assert [e["name"] for e in ev] == ["dequant_q4_0_linear", "dequant_q4_0", "silu"]
    assert all(e["ph"] == "X" and e["dur"] > 0 for e in ev)
    assert ev[1]["args"]["elements"] == 4096 * 4096 and ev[2]["args"]["dtype"] == "F32"


def test_reference_nf_bench_runs():
    """tools/nf_bench.cpp (buffer allocation, dispatch round trip,
    linear / linear_tiled at 256..1024) linked against this provider."""
    exe = REPO / "oracle" / "_ref" / "nf_bench"
    if not exe.exists():
        pytest.skip("nf_bench not built (needs the reference sources)")
    r = subprocess.run([str(exe), "--iterations", "5"], capture_output=True, text=True, timeout=300)
    print(r.stdout[-3000:], r.stderr[-1000:])
    assert r.returncode == 0 and "=== Benchmark complete ===" in r.stdout


LIFECYCLE = r"""
import sys
sys.path.insert(0, %r)
from neurofabric_amd.plugin import Provider
from neurofabric_amd import abi
import numpy as np
for i in range(3):
    p = Provider()
    p.init()
    assert p.name == "amd_hip" and p.abi_version == abi.NF_ABI_VERSION
    b = p.alloc(abi.NF_DTYPE_U8, 256)
    b.upload(np.full(256, 0x42, np.uint8))
    assert (b.download(np.uint8) == 0x42).all()
    b.release()
    p.shutdown()
    p.shutdown()  # idempotent
print("lifecycle ok")
"""


def test_register_init_shutdown_repeated():
    r = subprocess.run([sys.executable, "-c", LIFECYCLE % str(REPO)], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0 and "lifecycle ok" in r.stdout


NF_GENERATE = REPO / "oracle" / "_ref" / "nf_generate"
REF_GGUF = REPO / "oracle" / "_ref" / "ref_gguf"


def _llama_prefill_logits(quant, ids, seed, zero_attention=False, f16=False):
    """Last-position logits of the tiny synthetic model for prompt `ids`,
    composed from the oracle's restatements of the ops the reference's step
    graph emits (llama_dag_builder.hpp:1386-1530): embedding, rms_norm, fused
    Q4_0 / warm-up-dequantized linears, rope_batch, flash_attention_cached,
    residual adds, silu * up, final norm, lm_head `linear`.  With f16 every
    activation and dequantized weight is fp16 and each op is its `_f16`
    variant, as the app's --fp16 mode runs them.

    zero_attention: the paged path of the reference's step graph reads K/V
    pools that nothing writes (llama_dag_builder.hpp:1185-1194 zero them,
    :1444-1450 gives flash_attention_paged no new K/V), so its attention
    output is the weighted sum of zero value rows."""
    import numpy as np

    from neurofabric_amd import gguf_synth
    from oracle import oracle as orc

    D, L, H, KVH, F, V, _ = gguf_synth.SHAPES["tiny"]
    hd, kvd, S, MS = D // H, KVH * (D // H), len(ids), 512
    W = {n: np.frombuffer(b, np.uint8) for n, _, _, b in gguf_synth.tensors("tiny", quant, seed)}
    f32 = lambda n: W[n].view(np.float32)  # noqa: E731
    act = np.uint16 if f16 else np.float32

    def lin(a, name, n, k):
        return orc.fused(a, W[name], quant, S, n, k, f16=f16)

    x = orc.dequant(W["token_embd.weight"], quant, V * D, f16=f16).reshape(V, D)[ids].astype(act)
    for l in range(L):
        b = f"blk.{l}."
        h = orc.rms_norm(x, f32(b + "attn_norm.weight"), D, 1e-5, f16=f16)
        q, k, v = lin(h, b + "attn_q.weight", D, D), lin(h, b + "attn_k.weight", kvd, D), lin(h, b + "attn_v.weight", kvd, D)
        q = orc.rope(q, H, hd, 0, 10000.0, f16=f16)
        k = orc.rope(k, KVH, hd, 0, 10000.0, f16=f16)
        kc, vc = np.zeros(KVH * MS * hd, act), np.zeros(KVH * MS * hd, act)
        att = np.zeros(S * D, act)
        orc.attention("flash_attention_cached", dict(n_heads=H, n_kv=KVH, head_dim=hd, seq_len=S, step=0,
                                                     max_seq=MS), q, k, v, k=kc, v=vc, out=att, f16=f16)
        if zero_attention:
            att[:] = 0
        x = orc.binary("add", x, lin(att, b + "attn_output.weight", D, D), f16=f16)
        h2 = orc.rms_norm(x, f32(b + "ffn_norm.weight"), D, 1e-5, f16=f16)
        g = orc.unary("silu", lin(h2, b + "ffn_gate.weight", F, D), f16=f16)
        m = orc.binary("mul", g, lin(h2, b + "ffn_up.weight", F, D), f16=f16)
        x = orc.binary("add", x, orc.fused(m, W[b + "ffn_down.weight"], quant, S, D, F, f16=f16), f16=f16)
    hf = orc.rms_norm(x, f32("output_norm.weight"), D, 1e-5, f16=f16)
    lm = orc.dequant(W["output.weight"], quant, V * D, f16=f16)
    if f16:
        return orc.f16_to_f32(orc.linear_f16(hf, lm, S, V, D)[S - 1])
    return orc.linear_f32(hf, lm, S, V, D)[S - 1]


@pytest.mark.skipif(not (NF_GENERATE.exists() and REF_GGUF.exists()),
                    reason="reference app not built (needs the reference sources)")
@pytest.mark.parametrize("quant,flags,tol", [
    ("q4_0", [], 2e-3),            # fused dequant_q4_0_linear + flash_attention_cached
    ("q8_0", [], 2e-3),            # warm-up dequant_q8_0 + dense linear
    ("q4_0", ["--paged"], 2e-3),   # flash_attention_paged through the NeuralOS runtime
    ("q4_0", ["--fp16"], 2e-2),    # f16 activations and f16 layer ops (~10 fp16 ulps at |logit| ~3)
])
def test_reference_nf_generate_end_to_end(tmp_path, quant, flags, tol):
    """apps/nf_generate.cpp, the reference's text-generation app, compiled
    from its source and linked against this provider: loads a random-weight
    GGUF through the reference's loader, warms up, prefills, and decodes
    greedily.  The five largest prefill logits it prints are checked against
    the oracle's forward pass of the same model (tolerance 2e-3 absolute on
    logits of magnitude ~3; the fp16 run against the oracle's f16 chain,
    2e-2).  The printed values carry 4 decimals."""
    import re

    import numpy as np

    from neurofabric_amd import gguf_synth

    seed = 11
    path = tmp_path / "tiny.gguf"
    gguf_synth.write(str(path), "tiny", quant, seed=seed)
    prompt = "Hello world"
    tk = subprocess.run([str(REF_GGUF), str(path), prompt], capture_output=True, text=True, timeout=60)
    assert tk.returncode == 0
    ids = [int(x) for x in tk.stdout.splitlines()[-2].split()[1:]]
    print("case", quant, flags, "prompt ids", len(ids), flush=True)
    r = subprocess.run([str(NF_GENERATE), str(path), prompt, "--max-tokens", "6", "--temperature", "0",
                        "--seed", "1", *flags], capture_output=True, text=True, errors="replace",
                       timeout=120)
    print(r.stdout[-2000:], r.stderr[-4000:])
    assert r.returncode == 0
    m = re.search(r"decode: [\d.]+ ms \((\d+) tokens", r.stderr)
    assert m and int(m.group(1)) >= 1
    top = [(int(i), float(v)) for i, v in re.findall(r"top\d: id=(\d+) val=(-?[\d.]+)", r.stderr)]
    assert len(top) == 5
    ref = _llama_prefill_logits(quant, ids, seed, zero_attention="--paged" in flags, f16="--fp16" in flags)
    assert np.isfinite(ref).all() and np.abs(ref).max() > 0.1
    fifth = np.sort(ref)[-5]
    print("printed top-5 vs oracle:", [(tid, val, round(float(ref[tid]), 4)) for tid, val in top])
    for tid, val in top:
        assert abs(ref[tid] - val) <= tol + 1e-4, (tid, val, ref[tid])
        assert val >= fifth - tol - 1e-4
