#!/usr/bin/env python3
"""bench.py — throughput of the Q4_0/Q8_0 fused dequant+matmul path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--mode graph|eager] [--m M]

Headline workload: one TinyLlama-1.1B decode step
= the 155 Q4_0 projections of 22 layers + lm_head, f32 activations, batch M
(default 1), dispatched through the provider's C ABI.  A "step" is one pass
over those 155 linears; K steps are timed with HIP events on the provider's
stream (the stream every dispatch is launched on), after W warm-up steps.
`value` is GB/s of algorithmic bytes (Q4_0 weight blocks + activations +
outputs, each counted once per linear) per second, whole job, inputs resident
in HBM.  The 582 MB of weights per step exceed 2x the 256 MB Infinity Cache,
so nothing is served from cache across steps.

Also reported (same JSON line): the decode step at M=4 and 16, the C0 single
GEMV, and Llama-2-7B-shaped Q4_0 prefill GEMMs in TFLOP/s; the
reference CPU path (the oracle's restated dequant + sequential-k loop) timed
on this host's cores on a bounded sample.

Dispatch modes: `graph` captures the step's dispatches (one
nf_hip_run_tasks call) into a HIP graph and replays it; `eager` calls
nf_hip_run_tasks every step (host validation + launch per linear).
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


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--mode", choices=["graph", "eager"], default="graph")
    ap.add_argument("--m", type=int, default=1, help="decode batch of the headline step")
    ap.add_argument("--no-extra", action="store_true", help="only the headline decode step")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    return ap.parse_args(argv)


# ---------------------------------------------------------------------------
# workloads

class Step:
    """A list of prepared dispatches plus the buffers they reference."""

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


def decode_step(prov, M: int, fmt: str = "q4_0") -> Step:
    """22 x {q, k, v, o, gate, up, down} + lm_head, f32 activations."""
    from neurofabric_amd import abi, synthetic as syn
    st = Step(prov)
    qdt = abi.NF_DTYPE_Q4_0 if fmt == "q4_0" else abi.NF_DTYPE_Q8_0
    cache = {}
    shapes = syn.tinyllama_step_shapes()
    acts, outs = {}, {}
    for i, (name, N, K) in enumerate(shapes):
        if (N, K) not in cache:
            cache[(N, K)] = syn.weights(fmt, N, K, seed=N * 7 + K)
        w = prov.alloc_array(cache[(N, K)], qdt)  # a distinct buffer per layer
        st.buffers.append(w)
        if K not in acts:
            acts[K] = prov.alloc_array(syn.activations(M, K, seed=K), abi.NF_DTYPE_F32)
            st.buffers.append(acts[K])
        if N not in outs:
            outs[N] = prov.alloc(abi.NF_DTYPE_F32, M * N * 4)
            st.buffers.append(outs[N])
        st.add(f"dequant_{fmt}_linear", [acts[K], w], [outs[N]], M, N, K)
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
    e0, e1 = hiprt.Event(), hiprt.Event()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        run()
    e1.record(stream)
    e1.synchronize()
    prov.synchronize()
    hiprt.device_synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_ms(e1) / steps
    return {"ms_per_step": ms, "wall_ms_per_step": wall * 1e3 / steps, "launches": len(st.tasks),
            "us_per_launch": ms * 1e3 / len(st.tasks)}


# ---------------------------------------------------------------------------
# CPU baseline (the oracle: restated reference CPU dequant + sequential-k loop)

def cpu_baseline(threads: int) -> dict:
    from neurofabric_amd import synthetic as syn
    from oracle import oracle as orc
    shapes = syn.tinyllama_step_shapes()
    cache = {}
    for _, N, K in shapes:
        if (N, K) not in cache:
            cache[(N, K)] = (syn.q4_0_weights(N, K, seed=N * 7 + K), syn.activations(1, K, seed=K))
    total_bytes = 0
    t0 = time.perf_counter()
    for _, N, K in shapes:
        W, A = cache[(N, K)]
        orc.fused(A, W, "q4_0", 1, N, K, threads=threads)
        total_bytes += W.nbytes + A.nbytes + N * 4
    dt = time.perf_counter() - t0
    return {"value": total_bytes / dt / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "seconds": dt,
            "sample": "one full configs[1] decode step (155 Q4_0 linears, M=1, f32) through the oracle's "
                      "restated reference CPU path (dequant + sequential-k fp32 loop), "
                      f"{threads} thread(s)"}


# ---------------------------------------------------------------------------

def main(argv=None) -> int:
    args = parse(argv)
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the path shards by output rows with no collective, see DESIGN.md", file=sys.stderr)
        return 2
    from neurofabric_amd.plugin import Provider
    prov = Provider()
    prov.init()

    log(f"[bench] headline: configs[1] decode step M={args.m} mode={args.mode}")
    st = decode_step(prov, args.m)
    r = time_step(prov, st, args.steps, args.warmup, args.mode)
    gbs = st.bytes / (r["ms_per_step"] * 1e-3) / 1e9
    log(f"[bench] M={args.m}: {r['ms_per_step']*1e3:.1f} us/step, {gbs:.1f} GB/s, "
        f"{r['us_per_launch']:.2f} us/launch, kernels={sorted(st.kernels)}")
    head = {"step": r, "bytes_per_step": st.bytes, "weight_bytes_per_step": st.weight_bytes,
            "kernels": sorted(st.kernels), "tokens_per_s": args.m / (r["ms_per_step"] * 1e-3)}
    launches = len(st.tasks)
    st.release()

    extra = {}
    if not args.no_extra:
        for M in (4, 16):
            if M == args.m:
                continue
            s2 = decode_step(prov, M)
            r2 = time_step(prov, s2, max(10, args.steps // 2), args.warmup, args.mode)
            extra[f"decode_m{M}"] = {"GB_s": s2.bytes / (r2["ms_per_step"] * 1e-3) / 1e9,
                                     "us_per_step": r2["ms_per_step"] * 1e3,
                                     "tokens_per_s": M / (r2["ms_per_step"] * 1e-3),
                                     "kernels": sorted(s2.kernels)}
            log(f"[bench] decode M={M}: {extra[f'decode_m{M}']}")
            s2.release()
        # one GEMV shape, 80 rotated copies (519 MB > 2x MALL)
        s0 = rotated_linear(prov, "q4_0", 1, 5632, 2048, False, 80)
        r0 = time_step(prov, s0, 20, 3, args.mode)
        extra["c0_gemv_5632x2048"] = {"GB_s": s0.bytes / (r0["ms_per_step"] * 1e-3) / 1e9,
                                      "us_per_launch": r0["us_per_launch"], "kernels": sorted(s0.kernels)}
        log(f"[bench] C0: {extra['c0_gemv_5632x2048']}")
        s0.release()
        pre = {}
        for (name, N, K) in [("qkvo_4096x4096", 4096, 4096), ("gate_up_11008x4096", 11008, 4096),
                             ("down_4096x11008", 4096, 11008)]:
            for M in (512, 2048):
                sp = rotated_linear(prov, "q4_0", M, N, K, True, 4)
                rp = time_step(prov, sp, 5, 2, "eager")
                tf = sp.flops / (rp["ms_per_step"] * 1e-3) / 1e12
                pre[f"{name}_m{M}"] = {"TFLOP_s": tf, "frac_of_mfma_peak": tf / MFMA_F16_PEAK_TFLOPS,
                                       "us_per_launch": rp["us_per_launch"], "kernels": sorted(sp.kernels)}
                log(f"[bench] prefill {name} M={M}: {tf:.1f} TFLOP/s")
                sp.release()
        extra["c2_prefill_f16"] = pre

    cpu = None
    if not args.no_cpu:
        log("[bench] cpu baseline (1 thread) ...")
        cpu = cpu_baseline(1)
        log(f"[bench] cpu 1 thread: {cpu['value']:.3f} GB/s in {cpu['seconds']:.1f} s")
        ncores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
        allc = cpu_baseline(min(ncores, 64))
        extra["cpu_all_cores"] = allc
        log(f"[bench] cpu {allc['cores']} threads: {allc['value']:.3f} GB/s")

    gbs_launch = (head["bytes_per_step"] / launches) / (r["us_per_launch"] * 1e-6) / 1e9
    line = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": r["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded Q4_0 blocks: fp16 scales |N(0,1)|*0.01, codes U{0..15}; x ~ N(0,1))",
        "config": {"workload": f"configs[1] TinyLlama-1.1B Q4_0 decode step, M={args.m}, 22 layers + "
                               f"lm_head = {launches} fused dequant+GEMV dispatches ({args.mode})",
                   "batch": args.m, "hidden": 2048, "ffn": 5632, "vocab": 32000,
                   "tokens_per_s": head["tokens_per_s"]},
        "roofline": {"bound": "hbm", "kernel": ",".join(head["kernels"]), "achieved": round(gbs_launch, 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs_launch / HBM_PEAK_GBS, 4),
                     "traffic": None,
                     "bytes_per_launch": head["bytes_per_step"] / launches,
                     "avg_launch_us": r["us_per_launch"]},
        "cpu_baseline": None if cpu is None else {k: cpu[k] for k in ("value", "unit", "cores", "kind", "sample")},
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
