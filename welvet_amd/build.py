"""Builds libwelvet_hip.so in-tree for gfx950.

    python -m welvet_amd.build

HIP sources go through hipcc (device code for gfx950, packed-FP32 codegen
disabled); the host packer goes through g++ with -ffp-contract=off so that its
float expressions round per operation like welvet's Go float32 code.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libwelvet_hip.so")
PROBE_LIB = os.path.join(HERE, "libwv_probe.so")  # bench.py's streaming-read probe, not part of the C ABI
ARCH = os.environ.get("WV_OFFLOAD_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-result",
]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-pthread", "-ffp-contract=off", "-Wall"]

HIP_SOURCES = ["runtime.hip", "gemv.hip", "gemv_rpl.hip", "gemm_rpl.hip", "decode.hip", "native.hip"]
CXX_SOURCES = ["pack.cpp"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + r.stdout + r.stderr)
        raise RuntimeError(f"build failed: {os.path.basename(cmd[-1])}")
    return r


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    jobs = [[HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", os.path.join(OBJ, src + ".o")]
            for src in HIP_SOURCES]
    jobs += [["g++", *CXX_FLAGS, "-c", os.path.join(CSRC, src), "-o", os.path.join(OBJ, src + ".o")]
             for src in CXX_SOURCES]
    workers = max(1, min(len(jobs), int(os.environ.get("MAX_JOBS", "0")) or (os.cpu_count() or 1)))
    with ThreadPoolExecutor(workers) as pool:
        list(pool.map(_run, jobs))
    objs = [j[-1] for j in jobs]
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, "-pthread"])
    os.replace(tmp, LIB)
    tmp = PROBE_LIB + ".tmp"
    _run([HIPCC, *HIP_FLAGS, "-shared", "-o", tmp, os.path.join(CSRC, "probe.hip")])
    os.replace(tmp, PROBE_LIB)
    if verbose:
        print("built", LIB, "and", PROBE_LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
