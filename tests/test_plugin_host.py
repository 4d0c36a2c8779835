"""Host-side boundary tests that need no GPU.

The provider library loads, exports exactly the entry points its headers
declare, fills the vtables, reports the ABI version the loader gates on
(plugin_loader.cpp:48-54), and its planner (shared with dispatch) applies the
reference's selection rules and this provider's size/dtype validation.
"""
import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

from neurofabric_amd import abi
from neurofabric_amd.plugin import NfError, Provider, load_library, plan, push_constants

REPO = Path(__file__).resolve().parents[1]
LIB = REPO / "neurofabric_amd" / "_lib" / "libnf_plugin_hip.so"


def _declared_symbols():
    names = set()
    for h in (REPO / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        text = "\n".join(l for l in text.splitlines() if not l.lstrip().startswith("#"))
        for m in re.finditer(r"NF_API\s+[\w\s\*]*?\b(\w+)\s*\(", text):
            names.add(m.group(1))
    return names


@pytest.fixture(scope="module")
def lib():
    return load_library()


def test_exports_match_headers():
    declared = _declared_symbols()
    assert {"nf_plugin_register", "nf_plugin_register_mem", "nf_plugin_register_ddi"} <= declared
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB)], check=True, capture_output=True,
                         text=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    assert exported == declared


def test_every_declared_symbol_resolves(lib):
    for name in _declared_symbols():
        assert getattr(lib, name) is not None


def test_register_fills_vtables():
    prov = Provider()
    for f, _ in abi.nf_provider_vtable._fields_:
        assert C.cast(getattr(prov.vt, f), C.c_void_p).value, f
    for f, _ in abi.nf_provider_mem_vtable._fields_:
        assert C.cast(getattr(prov.mem, f), C.c_void_p).value, f
    for f, _ in abi.nf_ddi_vtable._fields_:
        assert C.cast(getattr(prov.ddi, f), C.c_void_p).value, f
    assert prov.name == "amd_hip"
    assert prov.abi_version == abi.NF_ABI_VERSION
    assert Provider().handle.value == prov.handle.value  # process-wide singleton


def test_unknown_op_is_unsupported_before_any_device_work():
    prov = Provider()
    st = prov.vt.dispatch(prov.handle, b"no_such_op", None, 0, None, 0)
    assert st == abi.NF_ERROR_UNSUPPORTED_OP
    assert "no_such_op" in prov.last_error()


def _gpu_count():
    try:
        import torch
        return torch.cuda.device_count()
    except Exception:
        return 0


@pytest.mark.skipif(_gpu_count() > 0, reason="checks the no-device error path")
def test_init_without_device_reports_device_lost():
    prov = Provider()
    with pytest.raises(NfError) as e:
        prov.init()
    assert e.value.status == abi.NF_ERROR_DEVICE_LOST
    with pytest.raises(NfError) as e2:
        prov.alloc(abi.NF_DTYPE_F32, 64)
    assert e2.value.status == abi.NF_ERROR_INVALID_ARG


# ---- planner: selection and validation ------------------------------------------------

D = abi.make_desc


def _fused(lib, M, N, K, a=abi.NF_DTYPE_F32, c=abi.NF_DTYPE_F32, w_bytes=None, op="dequant_q4_0_linear",
           pc=None, bs=18):
    w = w_bytes if w_bytes is not None else N * K // 32 * bs
    ea = 2 if a == abi.NF_DTYPE_F16 else 4
    ec = 2 if c == abi.NF_DTYPE_F16 else 4
    return plan(lib, op, [D(a, M * K * ea), D(abi.NF_DTYPE_Q4_0, w)], [D(c, M * N * ec)], M, N, K, pc)


def test_plan_decode_gemv_c0(lib):
    p = _fused(lib, 1, 5632, 2048)
    assert p["kernel"] == "gemv_q4_0_f32"
    assert (p["weight_bytes"], p["act_bytes"], p["out_bytes"]) == (6488064, 8192, 22528)
    assert p["flops"] == 2 * 5632 * 2048


def test_plan_prefill_uses_mfma(lib):
    p = _fused(lib, 512, 4096, 4096, a=abi.NF_DTYPE_F16, c=abi.NF_DTYPE_F16, op="dequant_q4_0_linear_f16")
    assert p["kernel"] == "gemm_mfma_q4_0_f16"
    assert p["flops"] == 2 * 512 * 4096 * 4096


def test_plan_path_follows_output_dtype(lib):
    # metal_provider.mm:2997 — the op-name suffix does not pick the path.
    assert _fused(lib, 2, 64, 64, op="dequant_q4_0_linear_f16")["kernel"] == "gemv_q4_0_f32"
    assert _fused(lib, 2, 64, 64, a=abi.NF_DTYPE_F16, c=abi.NF_DTYPE_F16)["kernel"] == "gemv_q4_0_f16"


def test_plan_q8_0_and_ragged_k(lib):
    p = plan(lib, "dequant_q8_0_linear", [D(abi.NF_DTYPE_F32, 5 * 256 * 4), D(abi.NF_DTYPE_Q8_0, 7 * 8 * 34)],
             [D(abi.NF_DTYPE_F32, 5 * 7 * 4)], 5, 7, 256)
    assert p["kernel"] == "skinny_mfma_q8_0_f32" and p["weight_bytes"] == 7 * 8 * 34
    # K % 256 != 0: the small-batch MFMA kernel stages four block pairs at a time
    p = plan(lib, "dequant_q8_0_linear", [D(abi.NF_DTYPE_F32, 4 * 64 * 4), D(abi.NF_DTYPE_Q8_0, 7 * 2 * 34)],
             [D(abi.NF_DTYPE_F32, 4 * 7 * 4)], 4, 7, 64)
    assert p["kernel"] == "gemv_q8_0_f32"
    # K % 64 == 32: the block-granular GEMV kernel for f32 at any M
    p = plan(lib, "dequant_q8_0_linear", [D(abi.NF_DTYPE_F32, 4 * 96 * 4), D(abi.NF_DTYPE_Q8_0, 7 * 3 * 34)],
             [D(abi.NF_DTYPE_F32, 4 * 7 * 4)], 4, 7, 96)
    assert p["kernel"] == "gemv_q8_0_f32"
    p = _fused(lib, 2, 5, 48, w_bytes=(5 * 48 + 31) // 32 * 18)
    assert p["kernel"] == "generic_q4_0_f32"


@pytest.mark.parametrize("case", ["no_pc", "zero_m", "short_w", "short_a", "short_c", "a_dtype", "c_dtype"])
def test_plan_rejects_bad_arguments(lib, case):
    M, N, K = 4, 8, 64
    kw = {}
    if case == "no_pc":
        with pytest.raises(NfError) as e:
            plan(lib, "dequant_q4_0_linear", [D(0, M * K * 4), D(6, N * K // 32 * 18)], [D(0, M * N * 4)])
        assert e.value.status == abi.NF_ERROR_INVALID_ARG
        return
    if case == "zero_m":
        kw["pc"] = push_constants(0, N, K)
    if case == "short_w":
        kw["w_bytes"] = N * K // 32 * 18 - 1
    with pytest.raises(NfError) as e:
        if case == "short_a":
            plan(lib, "dequant_q4_0_linear", [D(0, M * K * 4 - 4), D(6, N * K // 32 * 18)], [D(0, M * N * 4)], M, N, K)
        elif case == "short_c":
            plan(lib, "dequant_q4_0_linear", [D(0, M * K * 4), D(6, N * K // 32 * 18)], [D(0, M * N * 4 - 1)], M, N, K)
        elif case == "a_dtype":
            _fused(lib, M, N, K, a=abi.NF_DTYPE_F16, c=abi.NF_DTYPE_F32)
        elif case == "c_dtype":
            plan(lib, "dequant_q4_0_linear", [D(0, M * K * 4), D(6, N * K // 32 * 18)], [D(abi.NF_DTYPE_I32, M * N * 4)], M, N, K)
        else:
            _fused(lib, M, N, K, **kw)
    assert e.value.status == abi.NF_ERROR_INVALID_ARG


def test_plan_dequant_count_from_output_size(lib):
    # metal_provider.mm:2667 — count = out.size_bytes / element size
    p = plan(lib, "dequant_q4_0", [D(abi.NF_DTYPE_Q4_0, 8 * 18)], [D(abi.NF_DTYPE_F32, 256 * 4)])
    assert (p["kernel"], p["count"]) == ("dequant_q4_0_f32", 256)
    p = plan(lib, "dequant_q8_0_f16", [D(abi.NF_DTYPE_Q8_0, 3 * 34)], [D(abi.NF_DTYPE_F16, 70 * 2)])
    assert (p["kernel"], p["count"], p["weight_bytes"]) == ("dequant_q8_0_f16", 70, 3 * 34)
    with pytest.raises(NfError):
        plan(lib, "dequant_q4_0", [D(abi.NF_DTYPE_Q4_0, 7 * 18)], [D(abi.NF_DTYPE_F32, 256 * 4)])


KQ_OPS = {"q4_1": (abi.NF_DTYPE_Q4_1, 20, 32), "q5_0": (abi.NF_DTYPE_Q5_0, 22, 32),
          "q5_1": (abi.NF_DTYPE_Q5_1, 24, 32), "q2_k": (abi.NF_DTYPE_Q2_K, 84, 256),
          "q3_k": (abi.NF_DTYPE_Q3_K, 110, 256), "q4_k": (abi.NF_DTYPE_Q4_K, 144, 256),
          "q5_k": (abi.NF_DTYPE_Q5_K, 176, 256), "q6_k": (abi.NF_DTYPE_Q6_K, 210, 256)}


@pytest.mark.parametrize("fmt", sorted(KQ_OPS))
@pytest.mark.parametrize("f16", [False, True], ids=["f32", "f16"])
def test_plan_kquant_dequant_ops(lib, fmt, f16):
    """The dequant ops of metal_provider.mm:3159-3176: count from the output
    size, ceil(count / block elements) blocks of input required."""
    dt, bs, be = KQ_OPS[fmt]
    e = 2 if f16 else 4
    odt = abi.NF_DTYPE_F16 if f16 else abi.NF_DTYPE_F32
    op = f"dequant_{fmt}" + ("_f16" if f16 else "")
    count = 3 * be - 5  # ragged: the last block is partial
    p = plan(lib, op, [D(dt, 3 * bs)], [D(odt, count * e)])
    assert (p["kernel"], p["count"], p["weight_bytes"], p["out_bytes"]) == (
        f"dequant_{fmt}_{'f16' if f16 else 'f32'}", count, 3 * bs, count * e)
    with pytest.raises(NfError) as err:
        plan(lib, op, [D(dt, 3 * bs - 1)], [D(odt, count * e)])
    assert err.value.status == abi.NF_ERROR_INVALID_ARG


def test_plan_layer_ops(lib):
    """The layer ops of metal_provider.mm:3180-3204: f16 variant from the
    output dtype, counts from the output size or the push constants."""
    F32, F16 = abi.NF_DTYPE_F32, abi.NF_DTYPE_F16
    p = plan(lib, "silu", [D(F16, 64)], [D(F16, 64)])
    assert (p["kernel"], p["count"]) == ("silu_f16", 32)
    p = plan(lib, "metal_vector_add", [D(F32, 400), D(F32, 400)], [D(F32, 400)])
    assert (p["kernel"], p["count"]) == ("vector_add_f32", 100)
    pc = push_constants(head_dim=64, epsilon=1e-5)
    p = plan(lib, "rms_norm", [D(F32, 3 * 64 * 4), D(F32, 64 * 4)], [D(F32, 3 * 64 * 4)], pc=pc)
    assert (p["kernel"], p["count"]) == ("rms_norm_f32", 192)
    p = plan(lib, "argmax", [D(F32, 2 * 10 * 4)], [D(abi.NF_DTYPE_I32, 8)], pc=push_constants(seq_len=2, N=10))
    assert (p["kernel"], p["count"]) == ("argmax_f32", 2)
    pc = push_constants(seq_len=1, n_heads=8, head_dim=64, M=2, step_idx=5, max_seq_len=16)
    ins = [D(F16, 8 * 64 * 2), D(F16, 2 * 64 * 2), D(F16, 2 * 64 * 2), D(F16, 2 * 16 * 64 * 2), D(F16, 2 * 16 * 64 * 2)]
    p = plan(lib, "flash_attention_gqa", ins, [D(F16, 8 * 64 * 2)], pc=pc)
    assert (p["kernel"], p["count"]) == ("attention_gqa_decode_f16", 8)
    with pytest.raises(NfError):  # caches too small for n_kv * max_seq * head_dim
        plan(lib, "flash_attention_gqa", ins[:3] + [D(F16, 100), D(F16, 100)], [D(F16, 8 * 64 * 2)], pc=pc)
    with pytest.raises(NfError):  # attention without push constants
        plan(lib, "flash_attention_gqa", ins, [D(F16, 8 * 64 * 2)])
    # MoE: gating writes ids and weights, [seq_len, min(N, 8)] each
    pc = push_constants(seq_len=3, M=16, N=12)
    p = plan(lib, "moe_top_k_gating", [D(F32, 3 * 16 * 4)], [D(abi.NF_DTYPE_I32, 3 * 8 * 4), D(F32, 3 * 8 * 4)], pc=pc)
    assert (p["kernel"], p["count"]) == ("moe_top_k_gating_f32", 24)
    with pytest.raises(NfError):  # one output only
        plan(lib, "moe_top_k_gating", [D(F32, 3 * 16 * 4)], [D(abi.NF_DTYPE_I32, 3 * 8 * 4)], pc=pc)
    pc = push_constants(seq_len=3, M=16, N=2, K=64)
    ins = [D(F32, 16 * 64 * 4), D(abi.NF_DTYPE_I32, 3 * 2 * 4), D(F32, 3 * 2 * 4)]
    p = plan(lib, "moe_scatter_gather", ins, [D(F32, 3 * 64 * 4)], pc=pc)
    assert (p["kernel"], p["count"]) == ("moe_scatter_gather_f32", 192)
    with pytest.raises(NfError):  # output smaller than seq_len * K
        plan(lib, "moe_scatter_gather", ins, [D(F32, 64 * 4)], pc=pc)
    # rope_batch_f16, the model layer's fp16 rope name: f16 buffers only
    pc = push_constants(seq_len=2, n_heads=4, head_dim=64, theta=10000.0)
    p = plan(lib, "rope_batch_f16", [D(F16, 2 * 4 * 64 * 2)], [D(F16, 2 * 4 * 64 * 2)], pc=pc)
    assert p["kernel"] == "rope_batch_f16"
    with pytest.raises(NfError):
        plan(lib, "rope_batch_f16", [D(F32, 2 * 4 * 64 * 4)], [D(F32, 2 * 4 * 64 * 4)], pc=pc)


def test_plan_dense_linear_dtypes(lib):
    M, N, K = 3, 5, 16
    p = plan(lib, "linear", [D(abi.NF_DTYPE_F16, M * K * 2), D(abi.NF_DTYPE_F16, N * K * 2)],
             [D(abi.NF_DTYPE_F32, M * N * 4)], M, N, K)
    assert p["kernel"] == "linear_f16f16_f32"
    p = plan(lib, "linear_tiled", [D(abi.NF_DTYPE_F32, M * K * 4), D(abi.NF_DTYPE_U8, N * K * 4)],
             [D(abi.NF_DTYPE_F32, M * N * 4)], M, N, K)
    assert p["kernel"] == "linear_f32f32_f32"  # untyped B takes A's element type


def test_plan_unknown_op(lib):
    with pytest.raises(NfError) as e:
        plan(lib, "sparse_moe_router", [D(0, 4)], [D(0, 4)])
    assert e.value.status == abi.NF_ERROR_UNSUPPORTED_OP


def test_crossover_setter_roundtrip():
    prov = Provider()
    old = prov.get_gemv_max_m()
    try:
        prov.set_gemv_max_m(3, 5)
        assert prov.get_gemv_max_m() == (3, 5)
        p = _fused(prov.lib, 4, 64, 256, a=abi.NF_DTYPE_F16, c=abi.NF_DTYPE_F16)
        assert p["kernel"] == "gemv_q4_0_f16"
        p = _fused(prov.lib, 6, 64, 256, a=abi.NF_DTYPE_F16, c=abi.NF_DTYPE_F16)
        assert p["kernel"] == "skinny_mfma_q4_0_f16"
        p = _fused(prov.lib, 6, 64, 256)
        assert p["kernel"] == "skinny_mfma_q4_0_f32"
    finally:
        prov.set_gemv_max_m(*old)
    old_s = (prov.get_skinny_max_m(), prov.get_skinny_max_m_f32())
    try:
        prov.set_skinny_max_m(5, 7)
        assert (prov.get_skinny_max_m(), prov.get_skinny_max_m_f32()) == (5, 7)
        p = _fused(prov.lib, 6, 64, 256, a=abi.NF_DTYPE_F16, c=abi.NF_DTYPE_F16)
        assert p["kernel"] == "gemm_mfma_q4_0_f16"
        assert _fused(prov.lib, 7, 64, 256)["kernel"] == "skinny_mfma_q4_0_f32"
        assert _fused(prov.lib, 8, 64, 256)["kernel"] == "gemm_mfma_q4_0_f32"
        assert _fused(prov.lib, 600, 64, 256)["kernel"] == "gemm_mfma_q4_0_f32"
    finally:
        prov.set_skinny_max_m(*old_s)


def test_default_switch_points(lib):
    """Defaults from the measured sweeps: GEMV for M <= 4 while its
    activation stage fits in 120 KB of LDS (M = 3..4 only for weights up to
    16 MB), the small-batch MFMA kernel up to 16 rows, the tiled GEMM beyond
    (f16); for f32 activations the small-batch kernel up to 64 rows."""
    f16 = dict(a=abi.NF_DTYPE_F16, c=abi.NF_DTYPE_F16, op="dequant_q4_0_linear_f16")
    assert _fused(lib, 2, 28672, 8192, **f16)["kernel"] == "gemv_q4_0_f16"   # 2 x 8192 x 2 B = 32 KB
    # M = 2: the GEMV while two of its workgroups fit a CU (stage <= 80 KB)
    assert _fused(lib, 2, 8192, 28672, **f16)["kernel"] == "skinny_mfma_q4_0_f16"  # 112 KB stage
    assert _fused(lib, 1, 8192, 28672, **f16)["kernel"] == "gemv_q4_0_f16"
    # M = 3..4: the GEMV only for weights up to 16 MB (132 MB here)
    assert _fused(lib, 4, 28672, 8192, **f16)["kernel"] == "skinny_mfma_q4_0_f16"
    assert _fused(lib, 4, 11008, 4096, **f16)["kernel"] == "skinny_mfma_q4_0_f16"  # 25 MB
    assert _fused(lib, 4, 4096, 4096, **f16)["kernel"] == "gemv_q4_0_f16"  # 9.4 MB
    assert _fused(lib, 4, 14336, 4096, op="dequant_q8_0_linear", bs=34)["kernel"] == "skinny_mfma_q8_0_f32"
    assert _fused(lib, 4, 32000, 2048)["kernel"] == "skinny_mfma_q4_0_f32"  # TinyLlama lm_head, 37 MB
    assert _fused(lib, 3, 5632, 2048)["kernel"] == "gemv_q4_0_f32"  # 6.5 MB
    assert _fused(lib, 4, 8192, 28672, **f16)["kernel"] == "skinny_mfma_q4_0_f16"  # 4 x 28672 x 2 B > 120 KB
    assert _fused(lib, 5, 28672, 8192, **f16)["kernel"] == "skinny_mfma_q4_0_f16"
    assert _fused(lib, 16, 28672, 8192, **f16)["kernel"] == "skinny_mfma_q4_0_f16"
    # f16, long rows: the small-batch kernel too (no K cap by default)
    assert _fused(lib, 8, 8192, 28672, **f16)["kernel"] == "skinny_mfma_q4_0_f16"
    assert _fused(lib, 16, 8192, 28672, **f16)["kernel"] == "skinny_mfma_q4_0_f16"
    assert _fused(lib, 17, 28672, 8192, **f16)["kernel"] == "gemm_mfma_q4_0_f16"
    assert _fused(lib, 32, 8192, 28672, **f16)["kernel"] == "gemm_mfma_q4_0_f16"
    assert _fused(lib, 4, 4096, 4096)["kernel"] == "gemv_q4_0_f32"
    assert _fused(lib, 2, 28672, 8192)["kernel"] == "gemv_q4_0_f32"           # 2 x 8192 x 4 B + sums
    assert _fused(lib, 3, 28672, 8192)["kernel"] == "skinny_mfma_q4_0_f32"    # 4 x 8192 x 4 B > 120 KB
    assert _fused(lib, 16, 4096, 4096)["kernel"] == "skinny_mfma_q4_0_f32"
    # f32 activations: small-batch kernel up to 64 rows, then the bf16-piece
    # tiled GEMM (K % 64 == 0), else the GEMV
    assert _fused(lib, 64, 14336, 4096, op="dequant_q8_0_linear", bs=34)["kernel"] == "skinny_mfma_q8_0_f32"
    assert _fused(lib, 65, 14336, 4096, op="dequant_q8_0_linear", bs=34)["kernel"] == "gemm_mfma_q8_0_f32"
    assert _fused(lib, 512, 4096, 11008)["kernel"] == "gemm_mfma_q4_0_f32"
    assert _fused(lib, 100, 64, 96)["kernel"] == "gemv_q4_0_f32"  # K % 64 != 0


def test_gemv_row_limits(lib):
    """The GEMV's two-row stage limit and three/four-row weight limit are
    settable through the C-ABI; the defaults come back unchanged."""
    f16 = dict(a=abi.NF_DTYPE_F16, c=abi.NF_DTYPE_F16, op="dequant_q4_0_linear_f16")
    st, wb = C.c_uint32(), C.c_uint64()
    lib.nf_hip_get_gemv_row_limits(C.byref(st), C.byref(wb))
    assert (st.value, wb.value) == (80 * 1024, 16 << 20)
    try:
        lib.nf_hip_set_gemv_row_limits(C.c_uint32(130 * 1024), C.c_uint64(200 << 20))
        # 2 x 28672 f16 activations staged with one padding chunk per pair: 129 KB
        assert _fused(lib, 2, 8192, 28672, **f16)["kernel"] == "gemv_q4_0_f16"
        assert _fused(lib, 4, 28672, 8192, **f16)["kernel"] == "gemv_q4_0_f16"   # 132 MB
        lib.nf_hip_set_gemv_row_limits(C.c_uint32(0), C.c_uint64(0))
        assert _fused(lib, 2, 28672, 8192, **f16)["kernel"] == "skinny_mfma_q4_0_f16"
        assert _fused(lib, 4, 4096, 4096)["kernel"] == "skinny_mfma_q4_0_f32"
        assert _fused(lib, 1, 28672, 8192, **f16)["kernel"] == "gemv_q4_0_f16"
    finally:
        lib.nf_hip_set_gemv_row_limits(C.c_uint32(st.value), C.c_uint64(wb.value))


# Every op name of the Metal provider's dispatch map (metal_provider.mm:3180-3209,
# the dequant names registered from s_dequant_map) plus the model layer's fp16
# rope name (arch_registry.hpp:140).
REFERENCE_OP_NAMES = (
    "argmax attention_prefill causal_attention causal_attention_cached elementwise_mul embedding_lookup "
    "flash_attention_cached flash_attention_gqa flash_attention_paged gelu linear linear_tiled "
    "metal_vector_add mock_relu moe_scatter_gather moe_top_k_gating rms_norm rope rope_batch rope_batch_f16 "
    "silu softmax dequant_q4_0_linear dequant_q4_0_linear_f16 "
    + " ".join(f"dequant_{f}{s}" for f in ("q4_0", "q8_0", "q4_1", "q5_0", "q5_1", "q2_k", "q3_k", "q4_k",
                                           "q5_k", "q6_k") for s in ("", "_f16"))).split()


@pytest.mark.parametrize("op", REFERENCE_OP_NAMES)
def test_every_reference_op_name_is_served(lib, op):
    """No name the reference's engine or model layer dispatches comes back
    NF_ERROR_UNSUPPORTED_OP: with no buffers the planner answers
    NF_ERROR_INVALID_ARG (arity) instead."""
    with pytest.raises(NfError) as e:
        plan(lib, op, [], [])
    assert e.value.status == abi.NF_ERROR_INVALID_ARG, op


def test_model_layer_op_selection(lib):
    """nf_hip_model.h: the op a model layer emits per projection weight dtype.
    Q4_0 and Q8_0 (and so a Q4_0 / Q8_0 output projection) run fused; dense
    weights run `linear`; the other block formats need a warm-up dequant and
    then run `linear` (quant_registry.hpp:50-88; llama_dag_builder.hpp:
    1025-1039, 1411-1422).  Every name it returns is one the provider serves."""
    import ctypes as C
    for fn in ("nf_hip_fused_linear_op_name", "nf_hip_projection_op_name", "nf_hip_dequant_op_name"):
        getattr(lib, fn).argtypes = [C.c_uint32, C.c_bool]
        getattr(lib, fn).restype = C.c_char_p
    lib.nf_hip_projection_needs_dequant.argtypes = [C.c_uint32]
    lib.nf_hip_projection_needs_dequant.restype = C.c_bool
    fused, proj, deq = lib.nf_hip_fused_linear_op_name, lib.nf_hip_projection_op_name, lib.nf_hip_dequant_op_name
    assert fused(abi.NF_DTYPE_Q4_0, False) == b"dequant_q4_0_linear"
    assert fused(abi.NF_DTYPE_Q4_0, True) == b"dequant_q4_0_linear_f16"
    assert fused(abi.NF_DTYPE_Q8_0, False) == b"dequant_q8_0_linear"
    assert fused(abi.NF_DTYPE_Q8_0, True) == b"dequant_q8_0_linear_f16"
    names = ["q4_0", "q8_0", "q4_1", "q5_0", "q5_1", "q2_k", "q3_k", "q4_k", "q5_k", "q6_k"]
    for f16 in (False, True):
        for dt in (abi.NF_DTYPE_F32, abi.NF_DTYPE_F16):
            assert fused(dt, f16) is None and proj(dt, f16) == b"linear" and deq(dt, f16) is None
            assert not lib.nf_hip_projection_needs_dequant(dt)
        for name in names:
            dt = getattr(abi, f"NF_DTYPE_{name.upper()}")
            want_deq = f"dequant_{name}" + ("_f16" if f16 else "")
            assert deq(dt, f16) == want_deq.encode()
            if name in ("q4_0", "q8_0"):
                assert proj(dt, f16) == fused(dt, f16) and not lib.nf_hip_projection_needs_dequant(dt)
            else:
                assert fused(dt, f16) is None and proj(dt, f16) == b"linear"
                assert lib.nf_hip_projection_needs_dequant(dt)
            for op in {proj(dt, f16), deq(dt, f16)}:
                with pytest.raises(NfError) as e:  # served: the planner answers arity, not unsupported
                    plan(lib, op.decode(), [], [])
                assert e.value.status == abi.NF_ERROR_INVALID_ARG, op
