"""Build libackvq.so (gfx950) into alelyon_compute_kit/_lib/.

HIP sources are compiled by hipcc for gfx950 only; the host-only calibration
code by g++. Every object is compiled with -ffp-contract=off (the vq4 encode
and AdamW numerics forbid fused multiply-adds; kernels that want an FMA call
fmaf explicitly) and with packed FP32 instructions disabled.

Usage: python alelyon-compute-kit_amd/build.py [--jobs N]
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
INCLUDE = HERE.parent / "include"
BUILD = HERE / "_build"
LIBDIR = HERE / "alelyon_compute_kit" / "_lib"
LIBRARY = LIBDIR / "libackvq.so"

ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")
ARCH = "gfx950"

COMMON = ["-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-Wall", "-Wno-unused-function",
          f"-I{INCLUDE}", f"-I{CSRC}"]
HIP_FLAGS = [f"--offload-arch={ARCH}", "-x", "hip", "-fhip-fp32-correctly-rounded-divide-sqrt",
             "-fno-gpu-flush-denormals-to-zero",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]

HIP_SOURCES = ["vq4_codec.hip", "vq4_matmul.hip", "vq4_gram.hip", "vq4_fit.hip",
               "vq4_direct.hip", "vq4_onehot.hip", "abi.cpp"]
CXX_SOURCES = ["host_fit.cpp"]
# The benchmark's HBM read probe: a library of its own, never linked into
# libackvq.so (bench.py --copy-calibration loads it).
PROBE_SOURCE = "hbm_probe.hip"
PROBE_LIBRARY = LIBDIR / "libackprobe.so"


def _run(cmd: list[str]) -> None:
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        sys.stderr.write(result.stdout + result.stderr)
        raise SystemExit(f"build failed: {' '.join(cmd)}")


def shaders_id() -> int:
    """FNV-1a over the kernel sources (HIP files and headers, in name order):
    the `shaders` identity ack_abi_info reports for this build."""
    h = 0xCBF29CE484222325
    for path in sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.hpp")), key=lambda p: p.name):
        for b in path.read_bytes():
            h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def _compile(source: str) -> Path:
    obj = BUILD / (Path(source).stem + ".o")
    src = CSRC / source
    if source in HIP_SOURCES or source == PROBE_SOURCE:
        defines = [f"-DACK_SHADERS_ID=0x{shaders_id():016x}ull"] if source == "abi.cpp" else []
        cmd = [HIPCC, *HIP_FLAGS, *COMMON, *defines, "-c", str(src), "-o", str(obj)]
    else:
        cmd = ["g++", *COMMON, "-c", str(src), "-o", str(obj)]
    _run(cmd)
    return obj


def build(jobs: int = 4) -> Path:
    """Compile every source and link the library; returns its path."""
    BUILD.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        objects = list(pool.map(_compile, HIP_SOURCES + CXX_SOURCES + [PROBE_SOURCE]))
    probe = objects.pop()
    for lib, objs in ((LIBRARY, objects), (PROBE_LIBRARY, [probe])):
        tmp = lib.with_name(lib.name + ".tmp")
        _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
              *map(str, objs)])
        os.replace(tmp, lib)
    return LIBRARY


def clean() -> None:
    shutil.rmtree(BUILD, ignore_errors=True)


def main(argv=None) -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--jobs", type=int, default=4)
    parser.add_argument("--clean", action="store_true")
    args = parser.parse_args(argv)
    if args.clean:
        clean()
    print(build(args.jobs))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
