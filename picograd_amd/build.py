"""Builds libpicograd_amd.so (C11 host + gfx950 HIP kernels) in-tree.

    python -m picograd_amd.build          # library only
    python -m picograd_amd.build --all    # library + oracle checker (+ reference build when present)

Kernels (csrc/kernels/*.hip) go through hipcc for gfx950 only; the host
library (csrc/host/*.c) is plain C11 compiled by gcc against the HIP runtime
and hiprtc headers; hipcc links the shared object.
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
BUILD = HERE / "_build"
LIBDIR = HERE / "lib"
LIB = LIBDIR / "libpicograd_amd.so"

HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    # packed-FP32 instructions are kept out of every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
C_FLAGS = ["-std=c11", "-O2", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter",
           "-D__HIP_PLATFORM_AMD__", f"-I{ROCM / 'include'}", f"-I{ROOT / 'include'}",
           f"-I{HERE / 'csrc'}", f"-I{HERE / 'csrc' / 'host'}"]


def _run(cmd: list[str], quiet: bool = True) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (res.stdout + res.stderr).splitlines()
                    if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip() and not quiet:
        print(out)


def build_library(verbose: bool = False) -> Path:
    hipcc = shutil.which("hipcc") or str(ROCM / "bin" / "hipcc")
    cc = os.environ.get("CC", "gcc")
    BUILD.mkdir(parents=True, exist_ok=True)
    LIBDIR.mkdir(parents=True, exist_ok=True)
    objs = []
    for src in sorted((HERE / "csrc" / "kernels").glob("*.hip")):
        obj = BUILD / (src.stem + ".hip.o")
        _run([hipcc, *HIP_FLAGS, f"-I{HERE / 'csrc' / 'kernels'}", "-c", str(src), "-o", str(obj)])
        objs.append(str(obj))
    for src in sorted((HERE / "csrc" / "host").glob("*.c")):
        obj = BUILD / (src.stem + ".c.o")
        _run([cc, *C_FLAGS, "-c", str(src), "-o", str(obj)], quiet=not verbose)
        objs.append(str(obj))
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *objs,
          f"-L{ROCM / 'lib'}", "-lamdhip64", "-lhiprtc", f"-Wl,-rpath,{ROCM / 'lib'}"])
    os.replace(tmp, LIB)
    return LIB


def build_oracle() -> None:
    """The CPU checker (oracle/liboracle.so) and, where the reference
    checkout exists, its own CPU path (oracle/_ref)."""
    _run(["make", "-s", "-C", str(ROOT / "oracle"), "all"])
    if Path("/root/reference/src").is_dir():
        _run(["make", "-s", "-C", str(ROOT / "oracle"), "ref"])


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--all", action="store_true", help="also build the oracle checker")
    ap.add_argument("-v", "--verbose", action="store_true")
    a = ap.parse_args(argv)
    lib = build_library(a.verbose)
    print(f"built {lib}")
    if a.all:
        build_oracle()
        print("built oracle")
    return 0


if __name__ == "__main__":
    sys.exit(main())
