"""Build libgrinqh_hip.so (the gfx950 C-ABI library) in-tree with hipcc.

Usage: python vllm-grinqh-plugin_amd/build.py [--jobs N] [--verbose]

Every .hip file under csrc/ is compiled for gfx950 to an object under
_build/, then linked into grinqh/_lib/libgrinqh_hip.so next to the Python
package that loads it.  It always recompiles (this is the "does it build"
check); the objects are independent, so they compile in parallel.  The
compiler's per-kernel resource report (VGPRs, AGPRs, scratch bytes per lane,
occupancy) is written to grinqh/_lib/kernel_resources.json, so that a test can
hold the kernels to their register budgets (no spills beyond the documented
ones).
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import json
import os
import re
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(REPO, "include")
BUILD = os.path.join(HERE, "_build")
LIB_DIR = os.path.join(HERE, "grinqh", "_lib")
LIB = os.path.join(LIB_DIR, "libgrinqh_hip.so")
RESOURCES = os.path.join(LIB_DIR, "kernel_resources.json")
ARCH = "gfx950"

# Packed-fp32 VALU forms are disabled for all device code (known to misbehave on
# this fleet); the host pass prints a harmless "not a recognized feature" note.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    "-Rpass-analysis=kernel-resource-usage",
]

_REMARK = re.compile(r"remark: (?:[^:]*:\d+:\d+: )?\s*(Function Name|VGPRs|AGPRs|ScratchSize \[bytes/lane\]|"
                     r"Occupancy \[waves/SIMD\]): (\S+)")
_FIELDS = {"VGPRs": "vgpr", "AGPRs": "agpr", "ScratchSize [bytes/lane]": "scratch", "Occupancy [waves/SIMD]": "occupancy"}


def _resources(text: str) -> dict:
    """Per kernel (mangled name): the compiler's resource remarks."""
    out, cur = {}, None
    for line in text.splitlines():
        m = _REMARK.search(line)
        if not m:
            continue
        key, val = m.group(1), m.group(2)
        if key == "Function Name":
            cur = out.setdefault(val, {})
        elif cur is not None:
            cur[_FIELDS[key]] = int(val)
    return out


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build the GRINQH HIP library)")


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src: str, verbose: bool):
    obj = os.path.join(BUILD, os.path.basename(src)[:-4] + ".o")
    cmd = [hipcc(), *DEVICE_FLAGS, "-I", INCLUDE, "-I", CSRC, "-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    text = r.stdout + r.stderr
    msg = "\n".join(l for l in text.splitlines() if "packed-fp32-ops" not in l and "remark:" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{msg}")
    if msg.strip() and verbose:
        print(msg)
    return obj, _resources(text)


def build(jobs: int | None = None, verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        results = list(ex.map(lambda s: _compile(s, verbose), srcs))
    objs = [o for o, _ in results]
    resources = {}
    for _, r in results:
        resources.update(r)
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-lhipblaslt", "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    with open(RESOURCES, "w") as f:
        json.dump(resources, f, indent=0, sort_keys=True)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    a = ap.parse_args()
    print(build(a.jobs, a.verbose))
    sys.exit(0)
