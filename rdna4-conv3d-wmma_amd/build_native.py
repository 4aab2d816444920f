"""Build librdna4_conv3d_hip.so for gfx950 with hipcc (in-tree, no torch headers).

Each csrc/*.hip translation unit is compiled in parallel into _build/, then
linked into rdna4_conv3d/librdna4_conv3d_hip.so.  The library links the HIP
runtime by SONAME (libamdhip64.so.7); PyTorch-ROCm ships a runtime with the same
SONAME, and the Python loader imports torch first, so one process holds one
HIP runtime.

Usage: python build_native.py [--jobs N] [--verbose]
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import time
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
REPO_ROOT = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
INCLUDE = REPO_ROOT / "include"
BUILD = PKG_ROOT / "_build"
OUT = PKG_ROOT / "rdna4_conv3d" / "librdna4_conv3d_hip.so"
ARCH = "gfx950"

# Packed-fp32 VALU forms are disabled on purpose: the kernels rely only on
# MFMA and scalar fp32 math, and packed v_pk_*_f32 is kept out of the code.
CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the native library)")


def _compile(hipcc: str, src: Path, verbose: bool) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc, *CFLAGS, "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        msg = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if "packed-fp32-ops" not in l)
        raise RuntimeError(f"hipcc failed for {src.name}:\n{msg}")
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    hipcc = _hipcc()
    BUILD.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no sources under {CSRC}")
    jobs = jobs or min(len(sources), max(1, min(16, os.cpu_count() or 1)))
    t0 = time.time()
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(hipcc, s, verbose), sources))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT} in {time.time() - t0:.1f}s", flush=True)
    return OUT


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args()
    build(args.jobs, args.verbose)
    print(OUT)
    return 0


if __name__ == "__main__":
    sys.exit(main())
