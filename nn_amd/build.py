"""Build ``nn_amd/libnnq.so`` (HIP kernels for gfx950 + the C ABI) in-tree with hipcc.

Usage: ``python -m nn_amd.build`` (or ``build()`` from Python).  Every call
recompiles; objects go to ``nn_amd/_build/`` (git-ignored).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libnnq.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

# gfx950 device code: no packed-fp32 instructions (v_pk_*_f32) anywhere.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON = ["-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function", "-Wno-unused-variable"]

HIP_SOURCES = ["nnq_gemv.hip", "nnq_gemm.hip", "nnq_gemm_ring.hip", "nnq_gemm_wide.hip", "nnq_gemm_wide8.hip",
               "nnq_gemm_thin.hip", "nnq_gemm_blk.hip", "nnq_moe.hip", "nnq_sample.hip"]
# per-file device flags: the block-scaled GEMM's MFMAs write their partials to VGPRs (the
# FMAs that scale them read VGPRs only; with the default accumulator registers every
# partial costs four extra register reads)
# The decode GEMVs and the probes take their first arguments preloaded into SGPRs at wave
# start (gfx950 kernel-argument preload), so a wave's first loads do not wait for the
# kernel-argument fetch: at 4096x12288 the GEMV is launch- and latency-bound at ~7 us.
PRELOAD = ["-mllvm", "-amdgpu-kernarg-preload-count=16"]
VGPR_MFMA = ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]
EXTRA_FLAGS = {"nnq_gemm_blk.hip": VGPR_MFMA, "nnq_gemm_wide8.hip": VGPR_MFMA, "nnq_gemm_thin.hip": VGPR_MFMA,
               "nnq_gemv.hip": PRELOAD,
               "nnq_probe.hip": PRELOAD}
HOST_SOURCES = ["nnq_abi.cpp", "nnq_plan.cpp", "nnq_repack.cpp", "nnq_host.cpp", "nnq_gguf.cpp"]
# measurement probes for bench.py (streaming-read floor, empty launch), a library of their own
PROBE_SOURCES = ["nnq_probe.hip"]
PROBE_LIB = os.path.join(HERE, "libnnq_probe.so")


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}")
    return r.stdout


def _compile(src: str) -> str:
    path = os.path.join(CSRC, src)
    obj = os.path.join(BUILD, src + ".o")
    if src.endswith(".hip"):
        cmd = [HIPCC, f"--offload-arch={ARCH}", *COMMON, *DEVICE_FLAGS, *EXTRA_FLAGS.get(src, []), "-c", path, "-o",
               obj]
    else:
        # host-only C++ (HIP runtime API): no FMA contraction in the encoders
        cmd = [HIPCC, "-x", "c++", *COMMON, "-ffp-contract=off", f"-I{ROCM}/include", "-D__HIP_PLATFORM_AMD__",
               "-c", path, "-o", obj]
    _run(cmd)
    return obj


def build(verbose: bool = False) -> str:
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(BUILD, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        objs = list(ex.map(_compile, HIP_SOURCES + HOST_SOURCES + PROBE_SOURCES))
    nlib = len(HIP_SOURCES) + len(HOST_SOURCES)
    for out, parts in ((LIB, objs[:nlib]), (PROBE_LIB, objs[nlib:])):
        tmp = out + ".tmp"
        # -z defs: a kernel whose launch stub the host pass dropped fails here, not at load time
        _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-z,defs", "-o", tmp, *parts, "-lpthread"])
        os.replace(tmp, out)
        if verbose:
            print(f"built {out}")
    return LIB


def clean():
    shutil.rmtree(BUILD, ignore_errors=True)


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
