"""Build libomnistack_amd.so (gfx950 HIP kernels + C ABI) in-tree.

    python omnistack-rs_amd/build.py            # -> omnistack_rs/_native/libomnistack_amd.so

Every HIP source is compiled with hipcc for gfx950 with packed-fp32 ops
disabled and fp contraction off (the codec's bit-exactness depends on each
fp32 operation rounding where the reference's torch ops round; kernels that
want fused multiply-adds spell them out).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OBJ_DIR = os.path.join(HERE, "_build")
OUT_DIR = os.path.join(HERE, "omnistack_rs", "_native")
LIB = os.path.join(OUT_DIR, "libomnistack_amd.so")

ARCH = os.environ.get("OMNI_OFFLOAD_ARCH", "gfx950")
SOURCES = ["host_api.cpp", "codec.hip", "attn.hip", "lora.hip", "calib.hip", "dense.hip", "probe.hip"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libomnistack_amd.so)")


def common_flags() -> list[str]:
    return [
        "-O3", "-fPIC", "-std=c++17", f"--offload-arch={ARCH}",
        "-ffp-contract=off",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # keep private arrays in registers: the backend would otherwise move
        # small per-thread arrays into LDS (the decode kernel sizes its LDS
        # explicitly)
        "-mllvm", "-disable-promote-alloca-to-lds",
        "-Wall", "-Wno-unused-function",
        f"-I{INCLUDE}", f"-I{CSRC}",
    ]


# Per-source flags.  attn.hip: the decode kernel's tile claims are one
# lane-0 LDS atomic each; the backend's atomic optimizer would wrap every
# one in a wave reduction (mbcnt / popcount / broadcast) it does not need.
EXTRA_FLAGS = {"attn.hip": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"]}


def compile_one(src: str) -> str:
    obj = os.path.join(OBJ_DIR, os.path.basename(src) + ".o")
    cmd = [hipcc(), *common_flags(), *EXTRA_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".cpp"):
        cmd = [hipcc(), "-O2", "-fPIC", "-std=c++17", f"-I{INCLUDE}", f"-I{CSRC}", "-c",
               os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    if r.stderr.strip():
        # hipcc's host pass warns about the packed-fp32 feature flag; keep other warnings visible.
        lines = [l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip()]
        if lines:
            sys.stderr.write("\n".join(lines) + "\n")
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(OBJ_DIR, exist_ok=True)
    os.makedirs(OUT_DIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(6, len(SOURCES))) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
