"""Build libnf_plugin_hip.so for gfx950 in-tree.

    python -m neurofabric_amd.build          # compile every source, link
    python -m neurofabric_amd.build --check  # print the library path if built

The HIP translation units under csrc/ are compiled with hipcc for
--offload-arch=gfx950 only; the pure host planner (plan.cpp) with g++.
All objects land in neurofabric_amd/_build/, the library in
neurofabric_amd/_lib/.  Nothing is installed outside the repository.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIBDIR = PKG / "_lib"
LIB = LIBDIR / "libnf_plugin_hip.so"

ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

HIP_SOURCES = [
    CSRC / "provider.hip",
    CSRC / "kernels" / "dequant.hip",
    CSRC / "kernels" / "gemv.hip",
    CSRC / "kernels" / "gemm.hip",
    CSRC / "kernels" / "skinny.hip",
    CSRC / "kernels" / "generic.hip",
    CSRC / "kernels" / "dense.hip",
    CSRC / "kernels" / "layer.hip",
    CSRC / "kernels" / "attention.hip",
]
CXX_SOURCES = [CSRC / "plan.cpp", CSRC / "plan_layer.cpp", CSRC / "model_ops.cpp"]

COMMON_FLAGS = ["-O3", "-fPIC", "-std=c++17", "-fvisibility=hidden",
                f"-I{REPO / 'include'}", f"-I{CSRC}"]
# Packed-FP32 instructions are disabled for all device code (the host pass
# of hipcc warns that it does not know the feature; that is harmless).
# Kernel arguments are preloaded into SGPRs at wave launch (gfx950 kernarg
# preloading, as many leading arguments as fit in the user SGPRs): a wave
# then starts computing addresses without a scalar load from the argument
# block (measured on MI355X: 2048x2048 Q4_0 GEMV 2.87 against 3.45 us per
# launch).  The compiler adds a fallback prologue that loads the same
# arguments where the firmware does not preload.
HIP_FLAGS = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
             "-packed-fp32-ops", "-Wno-unused-command-line-argument",
             "-mllvm", "-amdgpu-kernarg-preload-count=16"]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines()
                    if "packed-fp32-ops" not in l)  # the harmless host-pass warning
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


def _obj(src: Path) -> Path:
    return BUILD / (src.stem + ("_hip" if src.suffix == ".hip" else "_cxx") + ".o")


def build(jobs: int | None = None, verbose: bool = False, only: list[str] | None = None) -> Path:
    """Compile every source (or, with `only`, the sources whose file names
    are listed, reusing the other objects) and link the provider library;
    returns its path."""
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    BUILD.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    cmds = []
    pick = (lambda src: True) if not only else (lambda src: src.name in only or not _obj(src).exists())
    for src in HIP_SOURCES:
        if pick(src):
            cmds.append([HIPCC, *HIP_FLAGS, *COMMON_FLAGS, "-c", str(src), "-o", str(_obj(src))])
    for src in CXX_SOURCES:
        if pick(src):
            cmds.append(["g++", *COMMON_FLAGS, "-Wall", "-c", str(src), "-o", str(_obj(src))])
    jobs = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for fut in [ex.submit(_run, c) for c in cmds]:
            fut.result()
    objs = [str(_obj(s)) for s in HIP_SOURCES + CXX_SOURCES]
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", str(tmp),
          f"-Wl,-rpath,{ROCM}/lib", "-Wl,--no-undefined"])
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


def library_path() -> Path:
    return LIB


def clean() -> None:
    shutil.rmtree(BUILD, ignore_errors=True)
    shutil.rmtree(LIBDIR, ignore_errors=True)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--check", action="store_true")
    ap.add_argument("--clean", action="store_true")
    ap.add_argument("-j", type=int, default=None)
    ap.add_argument("--only", nargs="+", default=None, metavar="FILE",
                    help="recompile only these source files (e.g. provider.hip), then link")
    a = ap.parse_args(argv)
    if a.clean:
        clean()
        return 0
    if a.check:
        print(LIB if LIB.exists() else "not built")
        return 0 if LIB.exists() else 1
    build(a.j, verbose=True, only=a.only)
    return 0


if __name__ == "__main__":
    sys.exit(main())
