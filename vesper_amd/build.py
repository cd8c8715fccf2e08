"""Ahead-of-time build of the gfx950 library and its host-side check library.

  vesper_amd/libmxmoe.so            every HIP translation unit in vesper_amd/csrc, for gfx950
  vesper_amd/libmxmoe_hostcheck.so  csrc/hostcheck.cpp + csrc/mx_numerics.h built by g++: the
                                    device numerics compiled for the CPU so tests can compare
                                    them exhaustively with the oracle without a GPU

Run: python -m vesper_amd.build [--jobs N]. Always recompiles (it is the "does it build" check).
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
BUILD = PKG / "_build"
LIB = PKG / "libmxmoe.so"
HOSTCHECK = PKG / "libmxmoe_hostcheck.so"
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # IEEE-separate multiply/add: results must not depend on contraction choices
    "-ffp-contract=off",
    # keep hipcc from forming packed FP32 instructions on its own
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def hipcc() -> str:
    for candidate in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found: the HIP toolchain is required to build vesper_amd")


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(map(str, cmd))}\n{proc.stdout}")
    return proc.stdout


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError("no HIP sources found")
    compiler = hipcc()
    objects = [BUILD / (src.stem + ".o") for src in sources]
    jobs = jobs or min(len(sources), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        futures = [pool.submit(_run, [compiler, *HIP_FLAGS, "-c", str(src), "-o", str(obj)])
                   for src, obj in zip(sources, objects)]
        for f in futures:
            out = f.result()
            if verbose and out.strip():
                print(out)
    tmp = LIB.with_suffix(".so.tmp")
    # libcrypto: the host digest tables (mx_host_sha256_chunks)
    _run([compiler, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects), "-lcrypto"])
    os.replace(tmp, LIB)
    build_hostcheck()
    return LIB


def build_hostcheck() -> Path:
    tmp = HOSTCHECK.with_suffix(".so.tmp")
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off", "-Wall",
          "-o", str(tmp), str(CSRC / "hostcheck.cpp")])
    os.replace(tmp, HOSTCHECK)
    return HOSTCHECK


def main(argv=None):
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--jobs", type=int, default=None)
    parser.add_argument("-v", "--verbose", action="store_true")
    args = parser.parse_args(argv)
    path = build(args.jobs, args.verbose)
    print(f"built {path} and {HOSTCHECK}")


if __name__ == "__main__":
    sys.exit(main())
