"""Build the gfx950 C-ABI library ``libbsx.so`` in-tree.

Each HIP source is compiled for gfx950 only; the host-only sources (planner, error
glue) are compiled with g++.  The objects are linked by hipcc into
``batchspec_amd/libbsx.so``, which is what the Python package loads.

Usage:  python -m batchspec_amd.build   (or batchspec_amd.build.build())
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
INCLUDE = PKG.parent / "include"
OUT = PKG / "libbsx.so"
BUILD_DIR = PKG / "_build"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Packed-fp32 VALU forms are kept off for all device code.  The acceptance and
# softmax translation unit also forbids implicit multiply-add contraction: its
# floating-point operation sequence is part of its bit-exact contract (as is the
# sampling filter's).
HIP_COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result", "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}",
]
HIP_SOURCES = {
    "attn.hip": [],
    "append.hip": [],
    "collate.hip": [],
    "masks.hip": [],
    "page_table.hip": [],
    "plan_device.hip": [],
    "probe.hip": [],
    "custom_mask.hip": [],
    "accept.hip": ["-ffp-contract=off"],
    "filter.hip": ["-ffp-contract=off"],
}
CXX_SOURCES = ["abi.cpp", "plan.cpp"]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        sys.stderr.write(out + "\n")


def build(verbose: bool = False) -> Path:
    """Compile every source and link libbsx.so; always recompiles."""
    BUILD_DIR.mkdir(exist_ok=True)
    jobs = []
    for src, extra in HIP_SOURCES.items():
        obj = BUILD_DIR / (src + ".o")
        jobs.append([HIPCC, *HIP_COMMON, *extra, "-c", str(CSRC / src), "-o", str(obj)])
    for src in CXX_SOURCES:
        obj = BUILD_DIR / (src + ".o")
        jobs.append(["g++", "-O2", "-std=c++17", "-fPIC", f"-I{INCLUDE}",
                     "-c", str(CSRC / src), "-o", str(obj)])
    with ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        for fut in [ex.submit(_run, j) for j in jobs]:
            fut.result()
    objs = [str(BUILD_DIR / (s + ".o")) for s in [*HIP_SOURCES, *CXX_SOURCES]]
    tmp = OUT.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *objs])
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


def clean() -> None:
    shutil.rmtree(BUILD_DIR, ignore_errors=True)
    if OUT.exists():
        OUT.unlink()


if __name__ == "__main__":
    build(verbose=True)
