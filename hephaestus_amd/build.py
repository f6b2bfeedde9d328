"""Offline build of the gfx950 library: every .hip/.cpp under csrc/ is
compiled by hipcc (code objects for gfx950 only, embedded in the shared
library) and linked into hephaestus_amd/lib/libhephaestus_amd.so.  No
run-time compilation happens anywhere on the hot path.

Usage: python -m hephaestus_amd.build   (or hephaestus_amd.build.build()).
"""
from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
LIBDIR = PKG / "lib"
LIB = LIBDIR / "libhephaestus_amd.so"
SOURCES = [
    "csrc/runtime.cpp",
    "csrc/planning.cpp",
    "csrc/ops.cpp",
    "csrc/reduce_full.hip",
    "csrc/reduce_rows.hip",
    "csrc/scan.hip",
    "csrc/segmented.hip",
    "csrc/random.hip",
    "csrc/copy.hip",
    "csrc/map_reduce.hip",
    "csrc/vector.hip",
    "csrc/dense_vector.cpp",
    "csrc/noalloc.hip",
    "csrc/device_api.cpp",
]
HEADERS = ["csrc/hx_device.hpp", "csrc/hx_internal.hpp"]
ARCH = "gfx950"
# Packed FP32 instructions are disabled for every device compile.
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]
_NOISE = "is not a recognized feature for this target"


def hipcc() -> str:
    return os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, cwd=PKG, capture_output=True, text=True)
    out = "\n".join(
        line for line in (proc.stdout + proc.stderr).splitlines() if _NOISE not in line
    ).strip()
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out:
        print(out, file=sys.stderr)


def build(jobs: int = 8) -> Path:
    """Compile every source and link the library; always rebuilds."""
    objdir = LIBDIR / "obj"
    objdir.mkdir(parents=True, exist_ok=True)
    objs = []
    cmds = []
    for src in SOURCES:
        obj = objdir / (Path(src).name + ".o")
        objs.append(str(obj))
        cmds.append([hipcc(), *FLAGS, "-I", str(REPO / "include"), "-c", src, "-o", str(obj)])
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        for fut in [pool.submit(_run, c) for c in cmds]:
            fut.result()
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-lhiprtc", "-o", str(tmp)])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
