"""Build the gfx950 HIP libraries of the package, in-tree.

    python mlsys-contest-syfi-fully-agent_amd/build.py

produces
    lib/libmoe_fp8_ds.so   the MoE layer (C ABI: include/moe_fp8_ds.h)
    lib/libmoe_synth.so    the synthetic input generator (include/moe_synth.h)
    lib/libmoe_bench.so    microbenchmarks for bench.py's measured peaks (not the layer)

Every call recompiles.  Objects go to _build/ (not committed); the .so files
are not committed either but travel with the source tree to the GPU host.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
OBJ = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "lib")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    # every fp32 op rounds separately unless the source asks for fmaf
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # no packed-fp32 (v_pk_*_f32) instructions anywhere
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

LIBS = {
    "libmoe_fp8_ds.so": ["route.hip", "gemm1.hip", "gemm2.hip", "combine.hip", "quantize.hip", "moe_api.cpp"],
    "libmoe_synth.so": ["synth.hip"],
    "libmoe_bench.so": ["peaks.hip"],
}


def _compile(src: str) -> str:
    out = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return out


def build(jobs: int | None = None, verbose: bool = False) -> dict:
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIB, exist_ok=True)
    srcs = sorted({s for v in LIBS.values() for s in v})
    jobs = jobs or min(len(srcs), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = dict(zip(srcs, ex.map(_compile, srcs)))
    built = {}
    for lib, parts in LIBS.items():
        dst = os.path.join(LIB, lib)
        tmp = dst + ".tmp"
        cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *[objs[p] for p in parts]]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed for {lib}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
        shutil.move(tmp, dst)
        built[lib] = dst
        if verbose:
            print("built", dst)
    return built


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
