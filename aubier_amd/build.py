"""Build the gfx950 kernel library (aubier_amd/libmla_m4.so) and the CPU oracle
(oracle/libmla_oracle.so), in-tree.

    python -m aubier_amd.build            # both
    python -m aubier_amd.build --lib      # kernels only

Every HIP translation unit is compiled with hipcc for gfx950 only, with packed-FP32 VALU
instructions disabled (-packed-fp32-ops), then linked into one shared library exporting the C ABI
of include/mla_m4.h.
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
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libmla_m4.so"
ORACLE_SRC = ROOT / "oracle" / "mla_oracle.c"
ORACLE_LIB = ROOT / "oracle" / "libmla_oracle.so"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-x", "hip",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l and "is not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))


def build_lib(verbose: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    objs = [BUILD / (s.name + ".o") for s in srcs]

    def one(pair):
        s, o = pair
        _run([HIPCC, *HIP_FLAGS, "-I", str(ROOT / "include"), "-c", str(s), "-o", str(o)])
        return o

    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        list(ex.map(one, zip(srcs, objs)))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB.relative_to(ROOT)} from {len(srcs)} sources")
    return LIB


def build_oracle(verbose: bool = True) -> Path:
    cc = shutil.which("gcc") or "cc"
    tmp = ORACLE_LIB.with_suffix(".so.tmp")
    _run([cc, "-O3", "-march=x86-64-v3", "-fopenmp", "-fPIC", "-shared", "-std=gnu11",
          str(ORACLE_SRC), "-o", str(tmp), "-lm"])
    os.replace(tmp, ORACLE_LIB)
    if verbose:
        print(f"built {ORACLE_LIB.relative_to(ROOT)}")
    return ORACLE_LIB


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--lib", action="store_true", help="kernel library only")
    ap.add_argument("--oracle", action="store_true", help="oracle only")
    args = ap.parse_args(argv)
    every = not (args.lib or args.oracle)
    if args.lib or every:
        build_lib()
    if args.oracle or every:
        build_oracle()
    return 0


if __name__ == "__main__":
    sys.exit(main())
