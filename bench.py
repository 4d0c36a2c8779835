#!/usr/bin/env python3
"""bench.py — throughput of the Q4_0/Q8_0 fused dequant+matmul path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--mode graph|eager] [--m M]
                    [--no-extra] [--no-cpu]

Headline workload: one TinyLlama-1.1B decode step
= the 155 Q4_0 projections of 22 layers + lm_head, f32 activations, batch M
(default 1), every projection dispatched through the provider's C ABI
(nf_provider_vtable.dispatch semantics, via nf_hip_run_tasks).  A step is one
pass over those 155 linears; W warm-up steps, then K steps timed with HIP
events on the provider's stream, one event between consecutive steps.
Weights, activations and outputs are resident in HBM before timing starts;
the 582 MB of weights per step exceed 2x the 256 MB Infinity Cache, so steps
do not hit in cache.

  value      = algorithmic bytes per step (Q4_0 blocks 18 B/32 weights +
               activations + outputs, each counted once per linear) / median
               step time over the K timed steps (ms_per_step is that median;
               the mean is in extra.headline)
  roofline   = the dominant kernel (the Q4_0 f32 decode GEMV, every launch of
               the step): achieved = algorithmic bytes per launch / launch
               duration (median step time / launches; graph replay: kernels
               run back to back); traffic = measured HBM bytes per launch
               from the rocprofv3 FETCH_SIZE/WRITE_SIZE summary in profiles/
               (scaled by a copy-kernel calibration), when present
  cpu_baseline = the reference's own CPU dequant + naive loop built from its
               source (oracle/_ref), else the oracle's restatement, on this
               host, 1 thread, on whole decode steps repeated for >= 10 s

Also measured (key figures in the line's short `extra`, full tables in the
--full-out file and on stderr): decode steps at M=4 and 16, configs[0] (one
5632x2048 GEMV over 80 rotated weight copies), a Llama-3-8B Q8_0 decode step
(configs[3], 32 layers + lm_head) at M=1/16/64, a Llama-2-7B Q4_0 decode step
at M=1 (north_star's "Llama-7B shapes"), Llama-2-7B Q4_0 prefill GEMMs
(configs[2]) in TFLOP/s over >= 512 MB of rotated weights, and the configs[4]
GEMV / small-batch / tiled-GEMM crossover sweep over M = 1..256 on both 70B
FFN shapes.  The stdout line stays under LINE_MAX_BYTES.

Modes: `graph` captures the step's dispatches (one nf_hip_run_tasks call)
into a HIP graph and replays it; `eager` calls nf_hip_run_tasks every step.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0            # MI355X HBM3E, GB/s
MFMA_F16_PEAK_TFLOPS = 2516.6    # MI355X dense fp16 MFMA
METRIC = "Q4_0 GEMV achieved GB/s (% HBM peak); prefill dequant-GEMM TFLOP/s"
PMC_SUMMARY = REPO / "profiles" / "gemv_q4_0_f32_tinyllama_decode_pmc.json"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--mode", choices=["graph", "eager"], default="graph")
    ap.add_argument("--m", type=int, default=1, help="decode batch of the headline step")
    ap.add_argument("--roof-steps", type=int, default=5, help="eager steps timed per dispatch (<= 6)")
    ap.add_argument("--no-extra", action="store_true", help="only the headline decode step")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline sample length")
    ap.add_argument("--only", choices=["c0", "c2", "c3", "c4", "c7b", "dq", "up", "layer", "floor"], default=None,
                    help="run one configs[i] section alone and print its JSON (profiling aid)")
    ap.add_argument("--full-out", default=str(REPO / "gpurun_out" / "bench_full.json"), metavar="PATH",
                    help="file for the full tables behind the line's short extra ('' = none)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="BYTES",
                    help="only run 4 device-to-device copies of BYTES (reference for HBM byte counters)")
    return ap.parse_args(argv)


def calibrate_copy(nbytes: int) -> int:
    """Device-to-device copies of a known size on the provider stream, so the
    rocprofv3 FETCH_SIZE / WRITE_SIZE counters can be scaled to bytes."""
    from neurofabric_amd import abi, hiprt
    from neurofabric_amd.plugin import Provider
    prov = Provider()
    prov.init()
    src = prov.alloc(abi.NF_DTYPE_U8, nbytes)
    dst = prov.alloc(abi.NF_DTYPE_U8, nbytes)
    hip = hiprt.lib()
    hip.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
    hip.hipMemcpyAsync.restype = C.c_int
    stream = prov.stream()
    for _ in range(4):
        hiprt.check(hip.hipMemcpyAsync(C.c_void_p(dst.device_ptr()), C.c_void_p(src.device_ptr()), nbytes, 3,
                                       C.c_void_p(stream)), "hipMemcpyAsync")
    prov.synchronize()
    src.release()
    dst.release()
    print(json.dumps({"calibrate_copy_bytes": nbytes, "copies": 4}), flush=True)
    return 0


# ---------------------------------------------------------------------------
# workloads

class Step:
    """A list of prepared task descriptors plus the buffers they reference."""

    def __init__(self, prov):
        self.prov = prov
        self.buffers = []
        self.descs = []
        self.weight_bytes = self.act_bytes = self.out_bytes = self.flops = 0
        self.kernels = set()

    def add(self, op, inputs, outputs, M, N, K):
        td = self.prov.task(op, inputs, outputs, M, N, K)
        p = self.prov.plan(op, [self._desc(b) for b in inputs], [self._desc(b) for b in outputs], M, N, K)
        self.kernels.add(p["kernel"])
        self.weight_bytes += p["weight_bytes"]
        self.act_bytes += p["act_bytes"]
        self.out_bytes += p["out_bytes"]
        self.flops += p["flops"]
        self.descs.append(td)

    @staticmethod
    def _desc(b):
        from neurofabric_amd import abi
        return abi.make_desc(b.dtype, b.nbytes)

    def finish(self):
        from neurofabric_amd.abi import nf_task_desc
        arr = (nf_task_desc * len(self.descs))()
        for i, td in enumerate(self.descs):
            C.memmove(C.addressof(arr[i]), C.addressof(td), C.sizeof(nf_task_desc))
            arr[i].user_data = C.addressof(arr[i])
        self.tasks = arr
        return self

    @property
    def bytes(self):
        return self.weight_bytes + self.act_bytes + self.out_bytes

    def release(self):
        for b in self.buffers:
            b.release()
        self.buffers.clear()


class WeightSet:
    """Distinct weight buffers for a list of projections (same bytes per
    shape), uploaded once and reused by steps at different batch sizes."""

    def __init__(self, prov, shapes, fmt: str, seed_base: int = 0):
        from neurofabric_amd import abi, synthetic as syn
        self.fmt, self.shapes = fmt, list(shapes)
        qdt = abi.NF_DTYPE_Q4_0 if fmt == "q4_0" else abi.NF_DTYPE_Q8_0
        cache = {}
        self.bufs = []
        for (_, N, K) in self.shapes:
            if (N, K) not in cache:
                cache[(N, K)] = syn.weights(fmt, N, K, seed=seed_base + N * 7 + K)
            self.bufs.append(prov.alloc_array(cache[(N, K)], qdt))

    def release(self):
        for b in self.bufs:
            b.release()
        self.bufs = []


# Activation buffer each projection reads in a Llama block: q/k/v the
# attention norm's output, o the attention output, gate/up the FFN norm's
# output, down the SiLU(gate)*up product, lm_head the final norm's output.
PROJ_INPUT = {"q_proj": "attn_norm", "k_proj": "attn_norm", "v_proj": "attn_norm", "o_proj": "attn_out",
              "gate_proj": "ffn_norm", "up_proj": "ffn_norm", "down_proj": "ffn_act", "lm_head": "final_norm"}


def model_step(prov, ws: WeightSet, M: int, f16: bool = False) -> Step:
    """One decode step over a weight set, one dispatch per projection, with
    the model's dataflow: each projection reads the activation buffer its
    role reads in a Llama block and writes an output buffer of its own (the
    buffers are reused from layer to layer).  The ops between the linears
    (norms, attention, SiLU) are not part of this path and not run."""
    from neurofabric_amd import abi, synthetic as syn
    st = Step(prov)
    adt = abi.NF_DTYPE_F16 if f16 else abi.NF_DTYPE_F32
    elt = 2 if f16 else 4
    acts, outs = {}, {}
    for (name, N, K), w in zip(ws.shapes, ws.bufs):
        proj = name.split(".")[-1]
        role = PROJ_INPUT[proj]
        if role not in acts:
            acts[role] = prov.alloc_array(syn.activations(M, K, seed=K + len(acts), dtype=np.float16 if f16 else np.float32), adt)
            st.buffers.append(acts[role])
        if proj not in outs:
            outs[proj] = prov.alloc(adt, M * N * elt)
            st.buffers.append(outs[proj])
        st.add(f"dequant_{ws.fmt}_linear" + ("_f16" if f16 else ""), [acts[role], w], [outs[proj]], M, N, K)
    return st.finish()


def rotated_linear(prov, fmt, M, N, K, f16: bool, copies: int) -> Step:
    """One projection shape over `copies` distinct weight buffers."""
    from neurofabric_amd import abi, synthetic as syn
    st = Step(prov)
    qdt = abi.NF_DTYPE_Q4_0 if fmt == "q4_0" else abi.NF_DTYPE_Q8_0
    W = syn.weights(fmt, N, K, seed=N + K)
    adt = abi.NF_DTYPE_F16 if f16 else abi.NF_DTYPE_F32
    a = prov.alloc_array(syn.activations(M, K, seed=M, dtype=np.float16 if f16 else np.float32), adt)
    c = prov.alloc(adt, M * N * (2 if f16 else 4))
    st.buffers += [a, c]
    op = f"dequant_{fmt}_linear" + ("_f16" if f16 else "")
    for _ in range(copies):
        w = prov.alloc_array(W, qdt)
        st.buffers.append(w)
        st.add(op, [a, w], [c], M, N, K)
    return st.finish()


FLOOR_SHAPES = ((2048, 2048, "tinyllama q/o 2048x2048"), (5632, 2048, "tinyllama gate/up 5632x2048"),
                (2048, 5632, "tinyllama down 2048x5632"), (32000, 2048, "tinyllama lm_head 32000x2048"),
                (4096, 4096, "llama-7b q/k/v/o 4096x4096"), (11008, 4096, "llama-7b gate/up 11008x4096"),
                (4096, 11008, "llama-7b down 4096x11008"))


def launch_floor(prov, shapes=FLOOR_SHAPES, copies: int = 64) -> dict:
    """Per-launch cost of the decode GEMV beside the floors under it, each as
    graph-replay launch-to-launch time over `copies` distinct weight buffers
    (HIP events on the provider stream): an empty kernel; a kernel that only
    streams the same weight bytes (nf_hip_diag_stream_read: every 16-byte
    chunk loaded once, all loads of a thread in flight, nothing stored); and
    the fused Q4_0 GEMV (M = 1, f32 activations) over those bytes."""
    from neurofabric_amd import hiprt
    stream = prov.stream()

    def replay(fn, steps=10):
        g = hiprt.Graph(stream, fn)
        for _ in range(3):
            g.launch()
        hiprt.device_synchronize()
        e0, e1 = hiprt.Event(), hiprt.Event()
        e0.record(stream)
        for _ in range(steps):
            g.launch()
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_ms(e1) * 1e3 / steps

    out = {"empty_kernel_us": replay(lambda: [prov.diag_stream_read(0, 0) for _ in range(copies)]) / copies}
    log(f"[bench] floor: empty kernel {out['empty_kernel_us']:.2f} us/launch")
    for N, K, name in shapes:
        st = rotated_linear(prov, "q4_0", 1, N, K, False, copies)
        wbytes = N * (K // 32) * 18
        ptrs = [b.device_ptr() for b in st.buffers[2:]]
        read_us = replay(lambda: [prov.diag_stream_read(p, wbytes) for p in ptrs]) / copies
        r = time_step(prov, st, 10, 2, "graph")
        gemv_us = r["us_per_launch"]
        st.release()
        out[name] = {"weight_bytes": wbytes, "read_us": read_us, "read_GB_s": wbytes / read_us / 1e3,
                     "gemv_us": gemv_us, "gemv_GB_s": wbytes / gemv_us / 1e3,
                     "gemv_over_read_us": gemv_us - read_us}
        log(f"[bench] floor {name}: read {read_us:.2f} us ({wbytes / read_us / 1e3:.0f} GB/s), "
            f"fused GEMV {gemv_us:.2f} us ({wbytes / gemv_us / 1e3:.0f} GB/s)")
    return out


def time_step(prov, st: Step, steps: int, warmup: int, mode: str) -> dict:
    from neurofabric_amd import hiprt
    stream = prov.stream()
    graph = None
    if mode == "graph":
        graph = hiprt.Graph(stream, lambda: prov.run_tasks(st.tasks, 1))
        run = graph.launch
    else:
        def run():
            prov.run_tasks(st.tasks, 1)
    for _ in range(warmup):
        run()
    prov.synchronize()
    hiprt.device_synchronize()
    # Kernel launches per step (nf_hip_run_tasks merges adjacent GEMVs that
    # read the same activations, so this can be below the dispatch count).
    c0 = prov.launch_count()
    prov.run_tasks(st.tasks, 1)
    prov.synchronize()
    launches = prov.launch_count() - c0
    # One HIP event between consecutive steps: the step times give the
    # median; first-to-last event over the step count gives the mean.
    ev = [hiprt.Event() for _ in range(steps + 1)]
    t0 = time.perf_counter()
    ev[0].record(stream)
    for i in range(steps):
        run()
        ev[i + 1].record(stream)
    ev[-1].synchronize()
    prov.synchronize()
    hiprt.device_synchronize()
    wall = time.perf_counter() - t0
    per = np.array([ev[i].elapsed_ms(ev[i + 1]) for i in range(steps)], np.float64)
    mean = ev[0].elapsed_ms(ev[-1]) / steps
    med = float(np.median(per))
    return {"ms_per_step": med, "mean_ms_per_step": mean, "min_ms_per_step": float(per.min()),
            "wall_ms_per_step": wall * 1e3 / steps, "dispatches": len(st.tasks), "repetitions": steps,
            "launches": launches, "us_per_launch": med * 1e3 / launches}


def time_dispatches(prov, st: Step, steps: int) -> dict:
    """Per-dispatch GPU durations of `steps` eager passes (timing ring)."""
    steps = max(1, min(steps, 1024 // len(st.tasks)))
    prov.run_tasks(st.tasks, 1)  # warm
    prov.synchronize()
    prov.enable_timing(True)
    prov.run_tasks(st.tasks, steps)
    prov.synchronize()
    rec = prov.timings()
    prov.enable_timing(False)
    ms = np.array([r[1] for r in rec], np.float64)
    return {"launches": len(ms), "mean_launch_us": float(ms.mean() * 1e3),
            "median_launch_us": float(np.median(ms) * 1e3), "sum_ms": float(ms.sum()),
            "steps": steps}


# ---------------------------------------------------------------------------
# CPU baseline: the reference's own CPU dequant + naive loop
# (dequant_test.cpp:112-128, 313-319), compiled from the reference's source by
# oracle/Makefile into oracle/_ref/libnfref_cpu_*.so; the oracle's restatement
# of the same path when that library was not built.

REF_CPU_LIBS = {"v3": REPO / "oracle" / "_ref" / "libnfref_cpu_v3.so",
                "release": REPO / "oracle" / "_ref" / "libnfref_cpu_release.so"}
REF_CPU_FLAGS = {"v3": "g++ -O3 -DNDEBUG -march=x86-64-v3 -std=c++20",
                 "release": "g++ -O3 -DNDEBUG -std=c++20 (the reference's Release flags)"}


def _host_has(*flags) -> bool:
    try:
        text = Path("/proc/cpuinfo").read_text()
    except OSError:
        return False
    line = next((l for l in text.splitlines() if l.startswith("flags")), "")
    have = set(line.split(":", 1)[-1].split())
    return all(f in have for f in flags)


def _ref_cpu(variant: str):
    path = REF_CPU_LIBS[variant]
    if not path.exists() or (variant == "v3" and not _host_has("avx2", "fma", "bmi2")):
        return None
    L = C.CDLL(str(path))
    L.nfref_cpu_fused.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p] + [C.c_uint32] * 6
    L.nfref_cpu_fused.restype = C.c_int
    return L


def cpu_baseline(threads: int, seconds: float, variant: str = "release") -> dict:
    """configs[1] decode steps (155 Q4_0 linears at M=1) on the host cores,
    repeated for about `seconds`; GB/s of algorithmic bytes."""
    from neurofabric_amd import synthetic as syn
    ref = _ref_cpu(variant)
    shapes = syn.tinyllama_step_shapes()
    cache = {}
    for _, N, K in shapes:
        if (N, K) not in cache:
            cache[(N, K)] = (syn.q4_0_weights(N, K, seed=N * 7 + K), syn.activations(1, K, seed=K),
                             np.zeros(N, np.float32))
    step_bytes = sum(cache[(N, K)][0].nbytes + K * 4 + N * 4 for _, N, K in shapes)
    if ref is not None:
        def linear(W, A, out, N, K):
            if ref.nfref_cpu_fused(0, A.ctypes.data, W.ctypes.data, out.ctypes.data, 1, N, K, 0, N, threads) != 0:
                raise RuntimeError("nfref_cpu_fused rejected its arguments")
        kind, what = "reference", (f"the reference's own ref_dequant_q4_0 and naive fp32 loop "
                                   f"(dequant_test.cpp:112-128, 313-319) built from its source with "
                                   f"{REF_CPU_FLAGS[variant]}")
    else:
        from oracle import oracle as orc

        def linear(W, A, out, N, K):
            orc.fused(A, W, "q4_0", 1, N, K, threads=threads)
        kind, what = "port", "the oracle's restatement of the reference CPU path (dequant + sequential-k fp32 loop)"
    reps = 0
    t0 = time.perf_counter()
    while True:
        for _, N, K in shapes:
            W, A, out = cache[(N, K)]
            linear(W, A, out, N, K)
        reps += 1
        if time.perf_counter() - t0 >= seconds:
            break
    dt = time.perf_counter() - t0
    return {"value": step_bytes * reps / dt / 1e9, "unit": "GB/s", "cores": threads, "kind": kind,
            "seconds": dt, "steps": reps, "tokens_per_s": reps / dt, "build": variant if ref else "oracle",
            "sample": f"{reps} whole configs[1] decode steps (155 Q4_0 linears, M=1, f32 activations, "
                      f"{step_bytes / 1e6:.1f} MB of algorithmic bytes each) through {what}, "
                      f"{threads} thread(s), rows of N split across threads, {dt:.1f} s"}


# ---------------------------------------------------------------------------
# extras

def llama3_q8_step_shapes(layers: int = 32):
    from neurofabric_amd import synthetic as syn
    out = []
    for layer in range(layers):
        for name, n, k in syn.LLAMA3_8B_Q8[:-1]:
            out.append((f"l{layer}.{name}", n, k))
    out.append(syn.LLAMA3_8B_Q8[-1])
    return out


def crossover_sweep(prov, shapes=((28672, 8192), (8192, 28672)), Ms=(1, 2, 4, 8, 16, 32, 64, 128, 256),
                    copies: int = 4) -> dict:
    """the Llama-70B FFN gate/up (28672x8192) and down
    (8192x28672) Q4_0 projections, f16 activations, through every kernel
    family that serves each M (switch points pinned): the VALU GEMV (while
    its activation stage fits in LDS), the small-batch MFMA kernel (M <= 64,
    one launch) and the tiled MFMA GEMM.  Each measurement replays (graph)
    `copies` launches over distinct copies of the weights (4 x 132 MB, twice
    the Infinity Cache), 5 times; the weights are uploaded once per shape."""
    from neurofabric_amd import abi, synthetic as syn
    g32, g16 = prov.get_gemv_max_m()
    sk16 = prov.get_skinny_max_m()
    tuning = prov.get_tuning()
    pins = {"gemv": (1 << 30, 1 << 30), "skinny": (0, 1 << 30), "tiled": (0, 0)}
    family = {"gemv": "gemv_", "skinny": "skinny_mfma_", "tiled": "gemm_mfma_"}
    out = {}
    try:
        for (N, K) in shapes:
            W = syn.weights("q4_0", N, K, seed=N + K)
            ws = [prov.alloc_array(W, abi.NF_DTYPE_Q4_0) for _ in range(copies)]
            rows = []
            for M in Ms:
                a = prov.alloc_array(syn.activations(M, K, seed=M, dtype=np.float16), abi.NF_DTYPE_F16)
                c = prov.alloc(abi.NF_DTYPE_F16, M * N * 2)
                row = {"M": M}
                for path, (gmax, smax) in pins.items():
                    prov.set_gemv_max_m(g32, gmax)
                    prov.set_skinny_max_m(smax, None, 1 << 30 if path == "skinny" else tuning[4])
                    # the GEMV at two rows also past its default stage limit
                    prov.set_gemv_row_limits((1 << 32) - 1 if path == "gemv" else tuning[5][0], tuning[5][1])
                    st = Step(prov)
                    for w in ws:
                        st.add("dequant_q4_0_linear_f16", [a, w], [c], M, N, K)
                    st.finish()
                    kern = sorted(st.kernels)[0]
                    if not kern.startswith(family[path]) or (path == "skinny" and M > 64):
                        continue  # this family does not serve M here
                    r = time_step(prov, st, 5, 2, "graph")
                    us = r["us_per_launch"]
                    row[path] = {"us": us, "GB_s": st.bytes / copies / (us * 1e-6) / 1e9,
                                 "TFLOP_s": st.flops / copies / (us * 1e-6) / 1e12, "kernel": kern}
                # the family the default switch points pick for this M
                prov.set_tuning(tuning)
                sel = Step(prov)
                sel.add("dequant_q4_0_linear_f16", [a, ws[0]], [c], M, N, K)
                sel_kern = sorted(sel.kernels)[0]
                row["selected_by_default"] = next((f for f, pre in family.items() if sel_kern.startswith(pre)), sel_kern)
                a.release()
                c.release()
                fams = [k for k in pins if k in row]
                row["fastest"] = min(fams, key=lambda k: row[k]["us"])
                rows.append(row)
                log(f"[bench] C4 {N}x{K} M={M}: " + ", ".join(f"{k} {row[k]['us']:.1f} us" for k in fams))
            for w in ws:
                w.release()
            out[f"{N}x{K}"] = {"rows": rows, "fastest_by_M": {r["M"]: r["fastest"] for r in rows}}
    finally:
        prov.set_tuning(tuning)
    # The switch points these measurements imply beside the provider's
    # defaults: the largest M at which the family is the fastest on every
    # shape it serves (the GEMV does not serve the 28672-long rows beyond
    # M = 2: its activation stage would not fit in LDS).
    shp = [k for k in out]

    def last_m(fam):
        ms = [m for m in Ms if any(fam in r for k in out for r in out[k]["rows"] if r["M"] == m) and
              all(r["fastest"] == fam for k in out for r in out[k]["rows"] if r["M"] == m and fam in r)]
        return max(ms) if ms else 0
    out["switch_points"] = {"measured": {"gemv_max_m_f16": last_m("gemv"), "skinny_max_m_f16": last_m("skinny")},
                            "defaults": {"gemv_max_m_f16": g16, "skinny_max_m_f16": sk16,
                                         "gemv_m2_only_up_to_stage_KB": tuning[5][0] // 1024,
                                         "gemv_m3_m4_only_up_to_weight_MB": tuning[5][1] >> 20,
                                         "skinny_f16_above_m4_only_up_to_k": tuning[4]},
                            "default_not_fastest": [(k, r["M"], r["selected_by_default"], r["fastest"])
                                                    for k in shp for r in out[k]["rows"]
                                                    if r["selected_by_default"] != r["fastest"]]}
    out["activations"] = "f16 N(0,1); weights Q4_0 per configs[0] statistics"
    return out


def run_step(prov, shapes, fmt, M, steps, warmup, mode) -> dict:
    """A whole decode step over a model's projections (model_step dataflow)."""
    ws = WeightSet(prov, shapes, fmt)
    st = model_step(prov, ws, M)
    r = time_step(prov, st, steps, warmup, mode)
    res = {"GB_s": st.bytes / (r["ms_per_step"] * 1e-3) / 1e9, "us_per_step": r["ms_per_step"] * 1e3,
           "frac_of_hbm_peak": st.bytes / (r["ms_per_step"] * 1e-3) / 1e9 / HBM_PEAK_GBS,
           "tokens_per_s": M / (r["ms_per_step"] * 1e-3), "dispatches": len(st.tasks), "launches": r["launches"],
           "weight_GB_per_step": st.weight_bytes / 1e9, "kernels": sorted(st.kernels)}
    st.release()
    ws.release()
    return res


def run_c0(prov, mode: str) -> dict:
    """one 5632x2048 Q4_0 GEMV over 80 rotated weight copies
    (519 MB > 2x the Infinity Cache)."""
    s0 = rotated_linear(prov, "q4_0", 1, 5632, 2048, False, 80)
    r0 = time_step(prov, s0, 20, 3, mode)
    d0 = time_dispatches(prov, s0, 6)
    out = {"GB_s_step": s0.bytes / (r0["ms_per_step"] * 1e-3) / 1e9,
           "us_per_launch_step": r0["us_per_launch"],
           "us_per_launch_kernel": d0["mean_launch_us"],
           "GB_s_kernel": s0.bytes / len(s0.tasks) / (d0["mean_launch_us"] * 1e-6) / 1e9,
           "kernels": sorted(s0.kernels)}
    log(f"[bench] C0: {out}")
    s0.release()
    return out


def run_c3(prov, mode: str) -> dict:
    """Llama-3-8B Q8_0 decode step (32 layers + lm_head) at M=1/16/64."""
    c3 = {}
    llama3 = WeightSet(prov, llama3_q8_step_shapes(), "q8_0")
    for M in (1, 16, 64):
        s3 = model_step(prov, llama3, M)
        r3 = time_step(prov, s3, 20, 2, mode)
        c3[f"m{M}"] = {"GB_s": s3.bytes / (r3["ms_per_step"] * 1e-3) / 1e9,
                       "us_per_step": r3["ms_per_step"] * 1e3,
                       "tokens_per_s": M / (r3["ms_per_step"] * 1e-3),
                       "weight_GB_per_step": s3.weight_bytes / 1e9, "kernels": sorted(s3.kernels)}
        log(f"[bench] C3 Q8_0 decode M={M}: {c3[f'm{M}']}")
        s3.release()
    llama3.release()
    return c3


_LIB_GEMM_CODE = r"""
import json, sys, torch
shapes, reps = json.loads(sys.argv[1]), int(sys.argv[2])
out = []
for M, N, K in shapes:
    if not torch.cuda.is_available():
        out.append(None)
        continue
    a = torch.randn(M, K, device="cuda", dtype=torch.float16)
    b = torch.randn(N, K, device="cuda", dtype=torch.float16)
    for _ in range(3):
        c = a @ b.t()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        c = a @ b.t()
    e1.record()
    torch.cuda.synchronize()
    out.append(2.0 * M * N * K / (e0.elapsed_time(e1) / reps * 1e-3) / 1e12)
    del a, b, c
print(json.dumps(out))
"""


def dense_f16_library_tflops(shapes, reps: int = 20) -> dict:
    """Calibration: each (M, N, K) contraction as a plain dense fp16 GEMM in the
    vendor library (torch.matmul, which runs hipBLASLt on ROCm), operands
    already fp16, timed with CUDA events, in one child process (torch ships
    its own HIP runtime, which must not share a process with this
    library's).  The ceiling a fused kernel that also dequantizes is compared
    against; not part of the product path.  {shape: TFLOP/s or None}."""
    import subprocess
    shapes = [tuple(x) for x in shapes]
    try:
        r = subprocess.run([sys.executable, "-c", _LIB_GEMM_CODE, json.dumps(shapes), str(reps)],
                           capture_output=True, text=True, timeout=600)
        vals = json.loads(r.stdout.strip().splitlines()[-1]) if r.returncode == 0 else [None] * len(shapes)
    except Exception:
        vals = [None] * len(shapes)
    return dict(zip(shapes, vals))


def run_c2(prov, reps: int = 20) -> dict:
    """Llama-2-7B Q4_0 prefill GEMMs, f16 activations.  Each shape
    runs over as many distinct weight copies as make >= 512 MB (twice the
    Infinity Cache), one pass over all copies per repetition; the figure is
    the median of `reps` repetitions.  Beside each, the vendor library's
    dense fp16 GEMM of the same shape (dense_f16_library_tflops)."""
    pre = {}
    shapes = [("qkvo_4096x4096", 4096, 4096), ("gate_up_11008x4096", 11008, 4096), ("down_4096x11008", 4096, 11008)]
    lib = dense_f16_library_tflops([(M, N, K) for (_, N, K) in shapes for M in (512, 2048)])
    for (name, N, K) in shapes:
        wbytes = N * (K // 32) * 18
        copies = -(-ROTATE_BYTES // wbytes)
        for M in (512, 2048):
            sp = rotated_linear(prov, "q4_0", M, N, K, True, copies)
            rp = time_step(prov, sp, reps, 2, "eager")
            tf = sp.flops / (rp["ms_per_step"] * 1e-3) / 1e12
            lib_tf = lib.get((M, N, K))
            pre[f"{name}_m{M}"] = {"TFLOP_s": tf, "frac_of_mfma_peak": tf / MFMA_F16_PEAK_TFLOPS,
                                   "us_per_launch": rp["us_per_launch"], "kernels": sorted(sp.kernels),
                                   "weight_copies": copies, "rotated_MB": copies * wbytes / 1e6,
                                   "repetitions": reps, "dense_f16_library_TFLOP_s": lib_tf}
            log(f"[bench] prefill {name} M={M}: {tf:.1f} TFLOP/s, {rp['us_per_launch']:.1f} us/launch "
                f"(median of {reps} passes over {copies} weight copies; library dense fp16 GEMM, no dequant: "
                f"{lib_tf if lib_tf is None else round(lib_tf, 1)} TFLOP/s)")
            sp.release()
    return pre


DQ_FORMATS = ["q4_0", "q8_0", "q4_1", "q5_0", "q5_1", "q2_k", "q3_k", "q4_k", "q5_k", "q6_k"]


ROTATE_BYTES = 512 << 20  # 2x the 256 MB Infinity Cache


def run_dq(prov, n_elems: int = 11008 * 4096) -> dict:
    """Standalone dequantization (the weight-upload warm-up path) of one
    Llama-2-7B FFN weight (11008 x 4096 elements) in every block format, to
    f16 and f32, over as many distinct input/output buffer pairs per format
    as make >= 512 MB together (each pair 115..205 MB), so no launch finds
    its bytes in the Infinity Cache.  Achieved bandwidth counts the
    algorithmic bytes: blocks read + output written."""
    from neurofabric_amd import abi, synthetic as syn
    res = {}
    for fmt in DQ_FORMATS:
        bs, be = syn.KQ_GEOM[fmt]
        blocks = syn.kquant_blocks(fmt, n_elems // be, seed=len(res))
        qdt = getattr(abi, f"NF_DTYPE_{fmt.upper()}")
        for f16 in (True, False):
            st = Step(prov)
            odt = abi.NF_DTYPE_F16 if f16 else abi.NF_DTYPE_F32
            pair = blocks.nbytes + n_elems * (2 if f16 else 4)
            copies = max(2, -(-ROTATE_BYTES // pair))
            for _ in range(copies):
                w = prov.alloc_array(blocks, qdt)
                o = prov.alloc(odt, n_elems * (2 if f16 else 4))
                st.buffers += [w, o]
                st.add(f"dequant_{fmt}" + ("_f16" if f16 else ""), [w], [o], 0, 0, 0)
            st.finish()
            r = time_step(prov, st, 10, 2, "eager")
            gbs = st.bytes / (r["ms_per_step"] * 1e-3) / 1e9
            res[f"{fmt}_{'f16' if f16 else 'f32'}"] = {"GB_s": gbs, "frac_of_hbm_peak": gbs / HBM_PEAK_GBS,
                                                       "us_per_launch": r["us_per_launch"],
                                                       "bytes_per_launch": st.bytes / copies,
                                                       "rotated_MB": copies * pair / 1e6,
                                                       "kernel": sorted(st.kernels)[0]}
            log(f"[bench] dequant {fmt} {'f16' if f16 else 'f32'}: {gbs:.0f} GB/s, {r['us_per_launch']:.1f} us")
            st.release()
    return res


def run_layer(prov) -> dict:
    """The layer ops around the linears at Llama-class shapes: decode
    attention over a 4096-token KV cache (GB/s of cache + q/out bytes),
    causal prefill attention over 2048 tokens (TFLOP/s, the causal half:
    2 * S^2 * head_dim * n_heads), rms_norm / rope_batch / silu / add /
    embedding over 2048 x 4096 tokens (GB/s), softmax and argmax over
    32 x 128256 logits.  Graph replay of 2 rotated buffer sets."""
    from neurofabric_amd import abi
    from neurofabric_amd.plugin import push_constants
    r = np.random.default_rng(0)
    F32, F16, I32 = abi.NF_DTYPE_F32, abi.NF_DTYPE_F16, abi.NF_DTYPE_I32
    res = {}

    def buf(n, dt, fill=True):
        e = 2 if dt == F16 else 4
        if not fill:
            return prov.alloc(dt, n * e)
        x = r.standard_normal(n).astype(np.float32)
        arr = x.astype(np.float16) if dt == F16 else (x.astype(np.int32) if dt == I32 else x)
        return prov.alloc_array(arr, dt)

    def measure(name, op, make, pc, flops=0, copies=2, steps=10):
        st = Step(prov)
        for _ in range(copies):
            ins, outs = make()
            st.buffers += ins + outs
            td = prov.task(op, ins, outs, pc=pc)
            p = prov.plan(op, [Step._desc(b) for b in ins], [Step._desc(b) for b in outs], pc=pc)
            st.kernels.add(p["kernel"])
            st.weight_bytes += p["weight_bytes"]
            st.act_bytes += p["act_bytes"]
            st.out_bytes += p["out_bytes"]
            st.descs.append(td)
        st.finish()
        # graph replay: these kernels run for microseconds, less than the
        # host needs to enqueue a dispatch, so eager timing would measure the host
        t = time_step(prov, st, steps, 2, "graph")
        us = t["ms_per_step"] * 1e3 / copies
        d = {"us_per_launch": us, "GB_s": st.bytes / copies / (us * 1e-6) / 1e9, "kernel": sorted(st.kernels)[0]}
        d["frac_of_hbm_peak"] = d["GB_s"] / HBM_PEAK_GBS
        if flops:
            d["TFLOP_s"] = flops / (us * 1e-6) / 1e12
        res[name] = d
        log(f"[bench] {name}: {us:.1f} us, {d['GB_s']:.0f} GB/s" + (f", {d['TFLOP_s']:.1f} TFLOP/s" if flops else ""))
        st.release()

    H, KV, D, ctx = 32, 8, 128, 4096
    for f16 in (True, False):
        dt = F16 if f16 else F32
        pc = push_constants(seq_len=1, n_heads=H, head_dim=D, M=KV, step_idx=ctx - 1, max_seq_len=ctx)
        measure(f"decode_attention_gqa_{'f16' if f16 else 'f32'}_h32kv8d128_ctx4096", "flash_attention_gqa",
                lambda: ([buf(H * D, dt), buf(KV * D, dt), buf(KV * D, dt), buf(KV * ctx * D, dt),
                          buf(KV * ctx * D, dt)], [buf(H * D, dt, False)]), pc, copies=8, steps=40)
    S = 2048
    pc = push_constants(seq_len=S, n_heads=H, head_dim=D, M=KV, step_idx=0, max_seq_len=S)
    for dt, tag in ((F16, "f16"), (F32, "f32")):
        measure(f"prefill_attention_{tag}_h32kv8d128_s2048", "flash_attention_cached",
                lambda: ([buf(S * H * D, dt), buf(S * KV * D, dt), buf(S * KV * D, dt), buf(KV * S * D, dt, False),
                          buf(KV * S * D, dt, False)], [buf(S * H * D, dt, False)]), pc,
                flops=2 * S * S * D * H, steps=3)
    T, E = 2048, 4096
    for f16 in (True, False):
        dt, tag = (F16, "f16") if f16 else (F32, "f32")
        measure(f"rms_norm_{tag}_2048x4096", "rms_norm", lambda: ([buf(T * E, dt), buf(E, F32)], [buf(T * E, dt, False)]),
                push_constants(head_dim=E, epsilon=1e-5))
        measure(f"rope_batch_{tag}_2048x32x128", "rope_batch", lambda: ([buf(T * H * D, dt)], [buf(T * H * D, dt, False)]),
                push_constants(n_heads=H, head_dim=D, theta=10000.0, step_idx=0))
        measure(f"silu_{tag}_2048x11008", "silu", lambda: ([buf(T * 11008, dt)], [buf(T * 11008, dt, False)]), None)
        measure(f"vector_add_{tag}_2048x4096", "metal_vector_add",
                lambda: ([buf(T * E, dt), buf(T * E, dt)], [buf(T * E, dt, False)]), None)
    V = 128256
    measure("softmax_f32_32x128256", "softmax", lambda: ([buf(32 * V, F32)], [buf(32 * V, F32, False)]),
            push_constants(seq_len=32, head_dim=V))
    measure("argmax_f32_32x128256", "argmax", lambda: ([buf(32 * V, F32)], [buf(32, I32, False)]),
            push_constants(seq_len=32, N=V))
    ids = lambda: prov.alloc_array(r.integers(0, 32000, T).astype(np.int32), I32)  # noqa: E731
    measure("embedding_lookup_f16_2048x4096", "embedding_lookup",
            lambda: ([buf(32000 * E, F16), ids()], [buf(T * E, F16, False)]), push_constants(seq_len=T, head_dim=E))
    return res


def run_upload(prov, mb: int = 512) -> dict:
    """Weight upload of one `mb` MiB tensor from pageable host memory (as
    from an mmap of a GGUF file): the reference model layer's map / memcpy /
    unmap (llama_dag_builder.hpp:146-156) on a fresh buffer, cold (pinned
    staging newly allocated) and warm (staging reused from the provider's
    pool), and the one-copy nf_hip_buffer_write.  Host wall time, GB/s."""
    from neurofabric_amd import abi
    n = mb << 20
    src = np.random.default_rng(0).integers(0, 256, n, dtype=np.uint8)
    res = {}
    prov.release_staging()
    for label in ("map_memcpy_unmap_cold", "map_memcpy_unmap_warm", "buffer_write"):
        b = prov.alloc(abi.NF_DTYPE_U8, n)
        t0 = time.perf_counter()
        if label == "buffer_write":
            b.write(src)
        else:
            ptr = b.map()
            C.memmove(ptr, src.ctypes.data, n)
            b.unmap()
        dt = time.perf_counter() - t0
        ok = bool(np.array_equal(b.read(np.uint8, count=1 << 20, offset=n - (1 << 20)), src[-(1 << 20):]))
        b.release()
        res[label] = {"GB_s": n / dt / 1e9, "seconds": dt, "bytes": n, "tail_check": ok}
        log(f"[bench] upload {mb} MiB {label}: {n / dt / 1e9:.1f} GB/s")
    prov.release_staging()
    return res


# ---------------------------------------------------------------------------
# the stdout line: headline keys, roofline, cpu_baseline and a short extra
# (the full tables go to a side file and to stderr)

LINE_MAX_BYTES = 6000  # the driver keeps the last 8000 bytes of stdout


def _r(x, sig: int = 4):
    """Round a number to `sig` significant digits (other values unchanged)."""
    if isinstance(x, bool) or not isinstance(x, (int, float)):
        return x
    if isinstance(x, int) or x == 0 or x != x:
        return x
    return float(f"{x:.{sig}g}")


def summarize_extra(full: dict) -> dict:
    """Key figures of the full extra tables, a few hundred bytes each."""
    s = {}
    h = full.get("headline_step")
    if h:
        s["headline"] = {k: _r(h[k]) for k in ("median_us_per_step", "mean_us_per_step", "min_us_per_step",
                                               "launches", "dispatches", "tokens_per_s", "repetitions") if k in h}
    for M in (1, 4, 16):
        d = full.get(f"c1_decode_m{M}")
        if d:
            s[f"c1_m{M}"] = {"us": _r(d["us_per_step"]), "GB_s": _r(d["GB_s"]), "tok_s": _r(d["tokens_per_s"])}
    d = full.get("c0_gemv_5632x2048")
    if d:
        s["c0"] = {"us_per_launch": _r(d["us_per_launch_step"]), "GB_s": _r(d["GB_s_step"])}
    d = full.get("llama2_7b_q4_0_decode_m1")
    if d:
        s["llama2_7b_q4_0_m1"] = {"us": _r(d["us_per_step"]), "GB_s": _r(d["GB_s"]),
                                  "frac": _r(d["frac_of_hbm_peak"], 3), "tok_s": _r(d["tokens_per_s"])}
    d = full.get("c3_llama3_8b_q8_0_decode")
    if d:
        s["c3_q8_0"] = {k: {"us": _r(v["us_per_step"]), "GB_s": _r(v["GB_s"])} for k, v in d.items()}
    d = full.get("c2_prefill_f16")
    if d:
        s["c2_TFLOP_s"] = {k: _r(v["TFLOP_s"]) for k, v in d.items()}
        s["c2_library_dense_f16_TFLOP_s"] = {k: _r(v.get("dense_f16_library_TFLOP_s")) for k, v in d.items()}
    d = full.get("c4_crossover")
    if d:
        c4 = {"switch_points": d.get("switch_points", {}).get("measured"),
              "default_not_fastest": len(d.get("switch_points", {}).get("default_not_fastest", []))}
        for shape, v in d.items():
            if isinstance(v, dict) and "rows" in v:
                c4[shape] = {r["M"]: [r["fastest"], _r(r[r["fastest"]]["us"], 3)] for r in v["rows"]}
        s["c4"] = c4
    d = full.get("dequant_7b_ffn_weight")
    if d:
        g = [v["GB_s"] for v in d.values()]
        s["dequant_GB_s"] = {"min": _r(min(g)), "max": _r(max(g)), "q4_0_f16": _r(d.get("q4_0_f16", {}).get("GB_s"))}
    d = full.get("weight_upload_512MiB")
    if d:
        s["upload_GB_s"] = {k: _r(v["GB_s"], 3) for k, v in d.items()}
    d = full.get("layer_ops")
    if d:
        s["layer_us"] = {k: _r(v["us_per_launch"], 3) for k, v in d.items()}
    d = full.get("gemv_launch_floor")
    if d:
        s["floor"] = {"empty_us": _r(d.get("empty_kernel_us"), 3)}
        s["floor"].update({k.split(" ")[0] + "_" + k.split(" ")[-1]: [_r(v["read_us"], 3), _r(v["gemv_us"], 3)]
                           for k, v in d.items() if isinstance(v, dict)})
    for k in ("cpu_all_cores", "cpu_x86_64_v3_1_thread"):
        if full.get(k):
            s[k] = {"GB_s": _r(full[k]["value"]), "cores": full[k]["cores"]}
    return s


def build_line(*, gbs, med_ms, args, dispatches, launches, kernels, achieved, bytes_per_launch, avg_launch_us,
               ring_us, traffic, cpu, extra_full, full_path, mode, m) -> dict:
    """The one JSON line bench.py prints."""
    extra = summarize_extra(extra_full)
    if full_path:
        p = Path(full_path).resolve()
        # relative to the repository root when it lies inside it (the root
        # is a scratch path on a GPU box)
        extra["full_tables"] = str(p.relative_to(REPO.resolve())) if p.is_relative_to(REPO.resolve()) else str(p)
    line = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": med_ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 weights, f32 activations/accumulate",
        "data": "synthetic (seeded Q4_0 blocks: fp16 scales |N(0,1)|*0.01, codes U{0..15}; x ~ N(0,1))",
        "config": {"workload": f"configs[1] TinyLlama-1.1B Q4_0 decode step, M={m}: 22 layers x "
                               f"{{q,k,v,o,gate,up,down}} + lm_head = {dispatches} fused dequant+GEMV "
                               f"dispatches in {launches} launches ({mode} replay; q/k/v and gate/up read "
                               f"the same activations and are merged); value and ms_per_step are the median "
                               f"of {args.steps} timed steps",
                   "batch": m, "hidden": 2048, "ffn": 5632, "vocab": 32000,
                   "tokens_per_s": _r(m / (med_ms * 1e-3))},
        "roofline": {"bound": "hbm", "kernel": ",".join(kernels), "achieved": round(achieved, 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "bytes_per_launch": round(bytes_per_launch, 1),
                     "avg_launch_us": _r(avg_launch_us, 5), "event_ring_mean_launch_us": _r(ring_us),
                     "traffic_source": str(PMC_SUMMARY.relative_to(REPO)) if traffic is not None else None},
        "cpu_baseline": None if cpu is None else {k: (_r(cpu[k]) if k == "value" else cpu[k])
                                                  for k in ("value", "unit", "cores", "kind", "sample")},
        "extra": extra,
    }
    if len(json.dumps(line)) > LINE_MAX_BYTES:  # keep the headline keys whatever the extras hold
        line["extra"] = {"full_tables": extra.get("full_tables"), "dropped": "extra summary over size limit"}
    return line


def load_pmc_summary():
    if PMC_SUMMARY.exists():
        try:
            d = json.loads(PMC_SUMMARY.read_text())
            return d
        except (OSError, ValueError):
            return None
    return None


# ---------------------------------------------------------------------------

def main(argv=None) -> int:
    args = parse(argv)
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); the path "
              "shards by weight rows across GPUs, which this build does not run", file=sys.stderr)
        return 2
    if args.calibrate_copy:
        return calibrate_copy(args.calibrate_copy)
    from neurofabric_amd import synthetic as syn
    from neurofabric_amd.plugin import Provider
    prov = Provider()
    prov.init()
    if args.only:
        sections = {"c0": lambda: run_c0(prov, args.mode), "c2": lambda: run_c2(prov),
                    "c3": lambda: run_c3(prov, args.mode), "c4": lambda: crossover_sweep(prov),
                    "c7b": lambda: run_step(prov, syn.llama2_7b_step_shapes(), "q4_0", 1, 20, 2, args.mode),
                    "dq": lambda: run_dq(prov), "up": lambda: run_upload(prov),
                    "layer": lambda: run_layer(prov), "floor": lambda: launch_floor(prov)}
        print(json.dumps({args.only: sections[args.only]()}), flush=True)
        return 0

    log(f"[bench] headline: configs[1] decode step M={args.m} mode={args.mode}")
    tiny = WeightSet(prov, syn.tinyllama_step_shapes(), "q4_0")
    st = model_step(prov, tiny, args.m)
    r = time_step(prov, st, args.steps, args.warmup, args.mode)
    gbs = st.bytes / (r["ms_per_step"] * 1e-3) / 1e9
    log(f"[bench] M={args.m}: {r['ms_per_step']*1e3:.1f} us/step, {gbs:.1f} GB/s, "
        f"{r['us_per_launch']:.2f} us/launch, kernels={sorted(st.kernels)}")
    # Dominant kernel = the decode GEMV (every dispatch of the step).  Its mean
    # launch duration is the timed region's HIP-event time on the provider
    # stream / launches: graph replay leaves no host gaps between kernels (the
    # rocprofv3 kernel trace of this command shows them back to back), so
    # this is kernel time.  Per-dispatch event pairs (the timing ring) add
    # ~2 us of event overhead per launch; they are reported as a cross-check.
    launches = r["launches"]
    bytes_per_launch = st.bytes / launches
    avg_launch_us = r["us_per_launch"]
    achieved = bytes_per_launch / (avg_launch_us * 1e-6) / 1e9
    # Cross-check: per-dispatch event pairs (the timing ring; dispatches are
    # not merged while it is on).  --roof-steps 0 skips it (counter runs).
    ring = time_dispatches(prov, st, args.roof_steps) if args.roof_steps > 0 else {"mean_launch_us": None}
    log(f"[bench] dominant kernel: {avg_launch_us:.2f} us/launch, {achieved:.1f} GB/s per launch "
        f"(event-ring cross-check, unmerged dispatches: {ring['mean_launch_us']} us)")
    dispatches = len(st.tasks)
    kernels = sorted(st.kernels)
    st.release()

    extra = {"headline_step": {"median_us_per_step": r["ms_per_step"] * 1e3,
                               "mean_us_per_step": r["mean_ms_per_step"] * 1e3,
                               "min_us_per_step": r["min_ms_per_step"] * 1e3,
                               "wall_us_per_step": r["wall_ms_per_step"] * 1e3, "repetitions": r["repetitions"],
                               "dispatches": dispatches, "launches": launches,
                               "bytes_per_step": bytes_per_launch * launches,
                               "tokens_per_s": args.m / (r["ms_per_step"] * 1e-3)}}
    if not args.no_extra:
        for M in (4, 16):
            if M == args.m:
                continue
            s2 = model_step(prov, tiny, M)
            r2 = time_step(prov, s2, max(20, args.steps // 2), args.warmup, args.mode)
            extra[f"c1_decode_m{M}"] = {"GB_s": s2.bytes / (r2["ms_per_step"] * 1e-3) / 1e9,
                                        "us_per_step": r2["ms_per_step"] * 1e3,
                                        "tokens_per_s": M / (r2["ms_per_step"] * 1e-3),
                                        "kernels": sorted(s2.kernels)}
            log(f"[bench] decode M={M}: {extra[f'c1_decode_m{M}']}")
            s2.release()
    tiny.release()
    if not args.no_extra:
        extra["c0_gemv_5632x2048"] = run_c0(prov, args.mode)
        extra["llama2_7b_q4_0_decode_m1"] = run_step(prov, syn.llama2_7b_step_shapes(), "q4_0", 1, 20, 2, args.mode)
        log(f"[bench] Llama-2-7B Q4_0 decode step M=1: {extra['llama2_7b_q4_0_decode_m1']}")
        extra["c3_llama3_8b_q8_0_decode"] = run_c3(prov, args.mode)
        extra["c2_prefill_f16"] = run_c2(prov)
        extra["c4_crossover"] = crossover_sweep(prov)
        extra["dequant_7b_ffn_weight"] = run_dq(prov)
        extra["weight_upload_512MiB"] = run_upload(prov)
        extra["layer_ops"] = run_layer(prov)
        extra["gemv_launch_floor"] = launch_floor(prov)

    cpu = None
    if not args.no_cpu:
        log("[bench] cpu baseline (1 thread) ...")
        cpu = cpu_baseline(1, args.cpu_seconds)
        log(f"[bench] cpu 1 thread: {cpu['value']:.3f} GB/s over {cpu['seconds']:.1f} s ({cpu['kind']})")
        ncores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
        allc = cpu_baseline(min(ncores, 64), min(args.cpu_seconds, 5.0))
        extra["cpu_all_cores"] = allc
        log(f"[bench] cpu {allc['cores']} threads: {allc['value']:.3f} GB/s")
        if _ref_cpu("v3") is not None:
            v3 = cpu_baseline(1, min(args.cpu_seconds, 5.0), variant="v3")
            extra["cpu_x86_64_v3_1_thread"] = v3
            log(f"[bench] cpu 1 thread, -march=x86-64-v3: {v3['value']:.3f} GB/s")

    pmc = load_pmc_summary()
    traffic = None
    if pmc and pmc.get("kernel_family") == kernels[0]:
        traffic = pmc.get("hbm_bytes_per_launch")
    full_path = None
    if args.full_out:
        full_path = Path(args.full_out)
        try:
            full_path.parent.mkdir(parents=True, exist_ok=True)
            full_path.write_text(json.dumps({"extra": extra, "cpu_baseline": cpu}, indent=1))
            log(f"[bench] full tables written to {full_path}")
        except OSError as e:
            log(f"[bench] could not write {full_path}: {e}")
            full_path = None
    line = build_line(gbs=gbs, med_ms=r["ms_per_step"], args=args, dispatches=dispatches, launches=launches,
                      kernels=kernels, achieved=achieved, bytes_per_launch=bytes_per_launch,
                      avg_launch_us=avg_launch_us, ring_us=ring["mean_launch_us"], traffic=traffic, cpu=cpu,
                      extra_full=extra, full_path=full_path, mode=args.mode, m=args.m)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
