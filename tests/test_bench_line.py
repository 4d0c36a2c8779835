"""bench.py's stdout line: the driver keeps only the last 8000 bytes of
stdout, so the one JSON line must stay well under that with every extra
section a default run produces, and must keep the headline keys, roofline
and cpu_baseline whatever the extras hold.  CPU only (no GPU calls)."""
import json
import random

import pytest

import bench

REQUIRED = ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
            "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline")


def _f(rng):
    # full-precision floats, as the timers produce them
    return rng.uniform(0.1, 9999.0) + rng.random() * 1e-9


def _full_extra(rng):
    """An extra dict with every section a default run writes, shaped as the
    producers in bench.py shape them."""
    step = lambda: {"GB_s": _f(rng), "us_per_step": _f(rng), "frac_of_hbm_peak": rng.random(),  # noqa: E731
                    "tokens_per_s": _f(rng), "dispatches": 155, "launches": 89, "weight_GB_per_step": _f(rng),
                    "kernels": ["gemv_q4_0_f32", "skinny_mfma_q4_0_f32"]}
    ms = (1, 2, 4, 8, 16, 32, 64, 128, 256)
    c4 = {}
    for shape in ("28672x8192", "8192x28672"):
        rows = []
        for m in ms:
            row = {"M": m}
            for fam in ("gemv", "skinny", "tiled"):
                row[fam] = {"us": _f(rng), "GB_s": _f(rng), "TFLOP_s": _f(rng), "kernel": f"{fam}_q4_0_f16"}
            row["selected_by_default"] = "tiled"
            row["fastest"] = rng.choice(["gemv", "skinny", "tiled"])
            rows.append(row)
        c4[shape] = {"rows": rows, "fastest_by_M": {r["M"]: r["fastest"] for r in rows}}
    c4["switch_points"] = {"measured": {"gemv_max_m_f16": 1, "skinny_max_m_f16": 16},
                           "defaults": {"gemv_max_m_f16": 4, "skinny_max_m_f16": 16},
                           "default_not_fastest": [("28672x8192", 2, "gemv", "skinny")] * 5}
    cpu = {"value": _f(rng), "unit": "GB/s", "cores": 16, "kind": "reference", "seconds": 5.0, "steps": 3,
           "tokens_per_s": _f(rng), "build": "release", "sample": "x" * 400}
    fmts = ["q4_0", "q8_0", "q4_1", "q5_0", "q5_1", "q2_k", "q3_k", "q4_k", "q5_k", "q6_k"]
    return {
        "headline_step": {"median_us_per_step": _f(rng), "mean_us_per_step": _f(rng), "min_us_per_step": _f(rng),
                          "wall_us_per_step": _f(rng), "repetitions": 50, "dispatches": 155, "launches": 89,
                          "bytes_per_step": _f(rng), "tokens_per_s": _f(rng)},
        "c1_decode_m4": step(), "c1_decode_m16": step(),
        "c0_gemv_5632x2048": {"GB_s_step": _f(rng), "us_per_launch_step": _f(rng), "us_per_launch_kernel": _f(rng),
                              "GB_s_kernel": _f(rng), "kernels": ["gemv_q4_0_f32"]},
        "llama2_7b_q4_0_decode_m1": step(),
        "c3_llama3_8b_q8_0_decode": {f"m{m}": step() for m in (1, 16, 64)},
        "c2_prefill_f16": {f"{n}_m{m}": {"TFLOP_s": _f(rng), "frac_of_mfma_peak": rng.random(),
                                         "us_per_launch": _f(rng), "kernels": ["gemm_mfma_q4_0_f16"],
                                         "weight_copies": 57, "rotated_MB": _f(rng), "repetitions": 20,
                                         "dense_f16_library_TFLOP_s": _f(rng)}
                           for n in ("qkvo_4096x4096", "gate_up_11008x4096", "down_4096x11008") for m in (512, 2048)},
        "c4_crossover": c4,
        "dequant_7b_ffn_weight": {f"{f}_{o}": {"GB_s": _f(rng), "frac_of_hbm_peak": rng.random(),
                                               "us_per_launch": _f(rng), "bytes_per_launch": _f(rng),
                                               "rotated_MB": _f(rng), "kernel": "dequant_direct"}
                                  for f in fmts for o in ("f16", "f32")},
        "weight_upload_512MiB": {k: {"GB_s": _f(rng), "seconds": _f(rng), "bytes": 1 << 29, "tail_check": True}
                                 for k in ("map_memcpy_unmap_cold", "map_memcpy_unmap_warm", "buffer_write")},
        "layer_ops": {f"layer_op_with_a_long_name_{i}": {"us_per_launch": _f(rng), "GB_s": _f(rng),
                                                         "kernel": "some_kernel", "frac_of_hbm_peak": rng.random()}
                      for i in range(15)},
        "gemv_launch_floor": dict({"empty_kernel_us": _f(rng)},
                                  **{f"shape{i} q/o {i}x{i}": {"weight_bytes": 1, "read_us": _f(rng),
                                                               "read_GB_s": _f(rng), "gemv_us": _f(rng),
                                                               "gemv_GB_s": _f(rng), "gemv_over_read_us": _f(rng)}
                                     for i in range(7)}),
        "cpu_all_cores": cpu, "cpu_x86_64_v3_1_thread": cpu,
    }, cpu


def _line(extra, cpu):
    args = bench.parse([])
    return bench.build_line(gbs=1327.123456789, med_ms=0.4408123456, args=args, dispatches=155, launches=89,
                            kernels=["gemv_q4_0_f32"], achieved=1327.123456789, bytes_per_launch=6574736.123,
                            avg_launch_us=4.9512345, ring_us=6.1234567, traffic=6800298.0, cpu=cpu,
                            extra_full=extra, full_path="gpurun_out/bench_full.json", mode="graph", m=1)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_line_small_and_complete(seed):
    extra, cpu = _full_extra(random.Random(seed))
    line = _line(extra, cpu)
    text = json.dumps(line)
    assert len(text) < 7000, len(text)
    assert "\n" not in text
    back = json.loads(text)
    for k in REQUIRED:
        assert k in back, k
    assert back["roofline"]["bound"] == "hbm" and 0 < back["roofline"]["frac"] < 1
    assert back["cpu_baseline"]["kind"] in ("reference", "port") and back["cpu_baseline"]["cores"] >= 1
    # the short extra carries the key figures of each section
    for k in ("headline", "c1_m4", "c1_m16", "c0", "llama2_7b_q4_0_m1", "c3_q8_0", "c2_TFLOP_s", "c4",
              "dequant_GB_s", "layer_us", "floor", "full_tables"):
        assert k in back["extra"], k


def test_oversized_extra_keeps_headline():
    extra, cpu = _full_extra(random.Random(3))
    extra["layer_ops"] = {f"op{i}" * 20: {"us_per_launch": 1.0} for i in range(400)}
    line = _line(extra, cpu)
    text = json.dumps(line)
    assert len(text) < 7000
    back = json.loads(text)
    for k in REQUIRED:
        assert k in back, k
    assert back["extra"]["dropped"]


def test_rounding():
    assert bench._r(1234.56789) == 1235.0
    assert bench._r(0.000123456) == 0.0001235
    assert bench._r(7) == 7 and bench._r(None) is None and bench._r("x") == "x" and bench._r(True) is True
