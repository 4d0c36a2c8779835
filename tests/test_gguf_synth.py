"""The synthetic GGUF writer (neurofabric_amd/gguf_synth.py) against the
reference's own GGUF loader and tokenizer (model/model/gguf_loader.hpp,
model/model/tokenizer.hpp), compiled by oracle/Makefile into
oracle/_ref/ref_gguf.  CPU only."""
import subprocess
from pathlib import Path

import pytest

from neurofabric_amd import gguf_synth

REPO = Path(__file__).resolve().parents[1]
REF_GGUF = REPO / "oracle" / "_ref" / "ref_gguf"


@pytest.mark.skipif(not REF_GGUF.exists(), reason="reference GGUF loader not built (needs the reference sources)")
@pytest.mark.parametrize("quant", ["q4_0", "q8_0"])
def test_reference_loader_reads_synthetic_model(tmp_path, quant):
    path = tmp_path / "m.gguf"
    gguf_synth.write(str(path), "tiny", quant, seed=3)
    r = subprocess.run([str(REF_GGUF), str(path), "Hello world"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    lines = r.stdout.splitlines()
    D, L, H, KVH, F, V, ctx = gguf_synth.SHAPES["tiny"]
    assert lines[0] == (f"arch=llama dim={D} layers={L} heads={H} kv_heads={KVH} ff={F} vocab={V} "
                        f"ctx={ctx} theta=10000 eps=1e-05 tensors={3 + 9 * L}")
    parsed = {}
    for ln in lines:
        if ln.startswith("tensor "):
            name, *kv = ln.split()[1:]
            parsed[name] = dict(x.split("=") for x in kv)
    gtype = {"q4_0": 2, "q8_0": 8}[quant]
    for name, dims, t, data in gguf_synth.tensors("tiny", quant, 3):
        p = parsed[name]
        n = 1
        for d in dims:
            n *= d
        assert int(p["type"]) == t and t in (0, gtype)
        assert int(p["elems"]) == n and int(p["bytes"]) == len(data)
        assert int(p["first"], 16) == data[0]          # tensor data found at its offset
    # the tokenizer: BOS, then the UTF-8 bytes of "▁Hello▁world" as byte tokens
    ids = [int(x) for x in lines[-2].split()[1:]]
    text = "▁Hello▁world".encode()
    assert ids == [1] + [3 + b for b in text]
