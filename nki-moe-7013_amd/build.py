"""Build libqmoe.so (gfx950) in-tree from csrc/.

    python nki-moe-7013_amd/build.py [-j N]

Each csrc/*.hip / *.cpp is compiled by hipcc into _build/*.o (in parallel),
then linked into qmoe/libqmoe.so next to the Python bindings; probes/*.hip
(measurement kernels that bench.py uses for measured peaks, not part of the
C ABI) go into qmoe/libqmoe_probe.so.  Every HIP translation unit is built
with packed-FP32 instruction selection disabled.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import json
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OUT_DIR = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "qmoe", "libqmoe.so")
PROBES = os.path.join(PKG, "probes")
PROBE_LIB = os.path.join(PKG, "qmoe", "libqmoe_probe.so")
BUILD_INFO = os.path.join(PKG, "qmoe", "build_info.json")
ARCH = "gfx950"

COMMON = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-I" + os.path.join(ROOT, "include"),
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libqmoe)")


def _compile(src: str) -> str:
    obj = os.path.join(OUT_DIR, os.path.basename(src) + ".o")
    cmd = [hipcc(), *COMMON, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    msgs = "\n".join(
        l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l
    ).strip()
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {src}\n{msgs}")
    if msgs:
        print(msgs, file=sys.stderr)
    return obj


def build(jobs: int = 8) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    srcs = sorted(
        os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp"))
    )
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, "-lhipblaslt"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, LIB)
    # measurement probes (bench.py's measured peaks): a library of their own
    psrcs = sorted(os.path.join(PROBES, f) for f in os.listdir(PROBES) if f.endswith(".hip"))
    pobjs = [_compile(p) for p in psrcs]
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", PROBE_LIB + ".tmp", *pobjs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("probe link failed:\n" + r.stdout + r.stderr)
    os.replace(PROBE_LIB + ".tmp", PROBE_LIB)
    _write_build_info()
    return LIB


def _write_build_info() -> None:
    """Record the commit the library was built from next to it (a copy of
    the tree without .git can still name its commit: bench.py reads this file)."""
    def git(*args):
        try:
            return subprocess.run(["git", *args], cwd=ROOT, capture_output=True, text=True,
                                  timeout=10).stdout.strip()
        except (OSError, subprocess.SubprocessError):
            return ""
    info = {"git": git("rev-parse", "--short", "HEAD") or None,
            "dirty": bool(git("status", "--porcelain", "--untracked-files=no"))}
    with open(BUILD_INFO, "w") as f:
        json.dump(info, f)


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", "--jobs", type=int, default=min(8, os.cpu_count() or 1))
    a = ap.parse_args()
    print(build(a.jobs))
