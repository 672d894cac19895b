"""Builds the gfx950 HIP library aiimage_amd/libaexq.so with hipcc (in-tree).

Usage: python -m aiimage_amd.build   (or aiimage_amd.build.build() from Python)
       python -m aiimage_amd.build --stamps   the phase-stamped profiling variant
           aiimage_amd/libaexq_stamps.so (bench.py --decode-phases)
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libaexq.so")
LIB_STAMPS = os.path.join(HERE, "libaexq_stamps.so")
SOURCES = ["aexq_qmv_q8.hip", "aexq_qmv_q4.hip", "aexq_qmm.hip", "aexq_qmmw.hip", "aexq_qgemm.hip",
           "aexq_kernels.hip",
           "aexq_decode.hip", "aexq_step.hip", "aexq_api.hip"]
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the aexq library is built with ROCm's hipcc for gfx950")


def flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        # packed fp32 VALU forms are kept out of the generated code
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
        "-Wno-unused-function",
        "-I", os.path.join(ROOT, "include"),
    ]


def build(verbose: bool = True, jobs: int = 4, stamps: bool = False) -> str:
    """Compile every HIP source to an object in parallel, then link libaexq.so
    (stamps: the profiling variant libaexq_stamps.so, whose fused decode kernel
    records per-phase timestamps; same kernels otherwise)."""
    t0 = time.time()
    lib = LIB_STAMPS if stamps else LIB
    extra = ["-DAEXQ_STEP_STAMPS"] if stamps else []
    objdir = os.path.join(HERE, "_build_stamps" if stamps else "_build")
    os.makedirs(objdir, exist_ok=True)
    cc = hipcc()
    procs = []
    objs = []
    for src in SOURCES:
        path = os.path.join(CSRC, src)
        if not os.path.exists(path):
            continue
        obj = os.path.join(objdir, src.replace(".hip", ".o"))
        objs.append(obj)
        cmd = [cc, *flags(), *extra, "-c", path, "-o", obj]
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
        while len([p for _, p in procs if p.poll() is None]) >= jobs:
            time.sleep(0.2)
    failed = []
    for src, p in procs:
        out, _ = p.communicate()
        text = out.decode(errors="replace")
        if p.returncode != 0:
            failed.append((src, text))
        elif verbose and "error" in text.lower():
            print(text, file=sys.stderr)
    if failed:
        for src, text in failed:
            print(f"--- {src}\n{text}", file=sys.stderr)
        raise RuntimeError("hipcc failed for: " + ", ".join(s for s, _ in failed))
    tmp = lib + ".tmp"
    subprocess.run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], check=True)
    os.replace(tmp, lib)
    if verbose:
        print(f"[aiimage_amd] built {lib} in {time.time() - t0:.1f}s", file=sys.stderr)
    return lib


if __name__ == "__main__":
    build(stamps="--stamps" in sys.argv[1:])
