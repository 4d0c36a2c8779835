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
