"""Builds libgtmoe.so in-tree for gfx950 with hipcc (no cmake, no JIT cache).

Each source compiles to an object under gotransformers_amd/_build/, then one
shared library gotransformers_amd/libgtmoe.so is linked.  The routing source
is compiled with -ffp-contract=off (its float64 arithmetic must round like the
CPU restatement); every HIP source gets -packed-fp32-ops turned off."""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libgtmoe.so")
ARCH = "gfx950"

SOURCES = [
    ("route.hip", ["-ffp-contract=off"]),
    ("experts_gemv.hip", []),
    ("experts_mfma.hip", []),
    ("misc.hip", []),
    ("lora.hip", []),
    ("api.cpp", []),
    ("encode.cpp", ["-ffp-contract=off"]),
    ("weightfile.cpp", []),
]


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _compile(src, extra):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), "-x", "hip", f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-I", os.path.join(ROOT, "include"), "-I", CSRC, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    errors = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                       if "packed-fp32-ops" not in l and l.strip())
    if r.returncode != 0:
        raise RuntimeError(f"compiling {src} failed:\n{errors}")
    return obj, errors


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as pool:
        results = list(pool.map(lambda s: _compile(*s), SOURCES))
    for obj, warnings in results:
        if verbose and warnings:
            print(warnings, file=sys.stderr)
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + [o for o, _ in results]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("linking libgtmoe.so failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
