"""Build libpgr.so (HIP kernels + C++ host runtime + C ABI) in-tree for gfx950.

Usage: python rust-llm-pager_amd/build.py [--jobs N] [--debug]
"""
from __future__ import annotations

import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libpgr.so")
OBJ_DIR = os.path.join(HERE, "_build")

ARCH = "gfx950"
# Packed FP32 instructions stay disabled for all device code. MFMA results live in VGPRs
# (gfx950 allows it): the decode kernels rescale their accumulators with VALU ops, and
# AGPR accumulators would cost a copy in and out per tile.
# -amdgpu-kernarg-preload-count: leading kernel arguments arrive preloaded in SGPRs (gfx950),
# so a kernel's first dependent loads do not wait for a load of its argument block.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-mllvm", "-amdgpu-mfma-vgpr-form=1",
                "-mllvm", "-amdgpu-kernarg-preload-count=16"]

# (source, language, extra flags)
SOURCES = [
    ("attn_kernels.hip", "hip", []),
    ("kv_kernels.hip", "hip", []),
    ("paged_kv.cpp", "hip", []),
    ("capi.cpp", "hip", []),
    # Host-only placement policy: no fused multiply-add, so f32 rounds like the reference.
    ("pager_core.cpp", "c++", ["-ffp-contract=off"]),
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; ROCm is required to build libpgr.so")
    return path


def compile_one(src: str, lang: str, extra: list[str], opt: list[str]) -> str:
    obj = os.path.join(OBJ_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), "-c", "-fPIC", "-std=c++17", *opt, "-Wall", "-Wno-unused-function"]
    if lang == "hip":
        cmd += ["-x", "hip", f"--offload-arch={ARCH}", *DEVICE_FLAGS]
    else:
        cmd += ["-x", "c++"]
    cmd += [*extra, "-I", CSRC, os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj


def build(jobs: int = 8, debug: bool = False) -> str:
    os.makedirs(OBJ_DIR, exist_ok=True)
    opt = ["-O1", "-g"] if debug else ["-O3"]
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        futures = [pool.submit(compile_one, s, lang, extra, opt) for s, lang, extra in SOURCES]
        objs = [f.result() for f in futures]
    tmp = OUT + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, OUT)
    return OUT


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("--debug", action="store_true")
    args = ap.parse_args()
    print(build(args.jobs, args.debug))
    return 0


if __name__ == "__main__":
    sys.exit(main())
