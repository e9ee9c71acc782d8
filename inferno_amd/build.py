"""Builds libinferno_hip.so (gfx950) in-tree with hipcc.

    python -m inferno_amd.build            # build the HIP library
    python -m inferno_amd.build --jobs 8

Every translation unit is compiled with:
  -ffp-contract=off        float operations stay in the order written, so the
                           kernels reproduce the reference's arithmetic
  -fhip-fp32-correctly-rounded-divide-sqrt
                           1/l, 127/amax and sqrt match IEEE (the reference's
                           CPU results)
  -Xclang -target-feature -Xclang -packed-fp32-ops
                           no packed fp32 instructions are generated
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
CSRC = PKG / "csrc"
INCLUDE = PKG.parent / "include"
LIB = PKG / "libinferno_hip.so"
OBJ_DIR = PKG.parent / "_build" / "obj"
ARCH = "gfx950"

SOURCES = ["api.hip", "attention.hip", "attention_wide.hip", "append.hip", "copy.hip", "bq.hip",
           "prefill.hip", "prefill_sliding.hip", "prefill_wide.hip", "gemm.hip", "sparse.hip"]
# Host-only C++ (page state, scheduler): built with the host compiler.
HOST_SOURCES = ["host_state.cpp", "host_api.cpp"]
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", f"-I{INCLUDE}"]

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-rdc",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}",
]


def hipcc() -> str:
    cand = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    return cand


def host_cxx() -> str:
    return os.environ.get("CXX") or shutil.which("g++") or "c++"


def _compile(src: Path, obj: Path) -> tuple[Path, str]:
    if src.suffix == ".cpp":
        cmd = [host_cxx(), *HOST_FLAGS, "-c", str(src), "-o", str(obj)]
    else:
        cmd = [hipcc(), *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    noise = "is not a recognized feature for this target"
    warn = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    return obj, warn


def build(jobs: int = 8, verbose: bool = False) -> Path:
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    objs = []
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        futs = [ex.submit(_compile, CSRC / s, OBJ_DIR / (s + ".o"))
                for s in SOURCES + HOST_SOURCES]
        for f in futs:
            obj, warn = f.result()
            if warn.strip() and verbose:
                print(warn, file=sys.stderr)
            objs.append(obj)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=8)
    ap.add_argument("-v", "--verbose", action="store_true")
    a = ap.parse_args()
    print(build(a.jobs, a.verbose))


if __name__ == "__main__":
    main()
