#!/usr/bin/env python3
r"""Builds libfa2_4d_mask.so (gfx950) in-tree with hipcc.

Usage: python fa2-with-4d-mask_amd/build_ext.py [--jobs N] [--verbose] [--host-sanitize]

Objects go to fa2-with-4d-mask_amd/_build/, the shared library to
fa2-with-4d-mask_amd/tilelang_fa2_4d_mask/_lib/libfa2_4d_mask.so, which is
where the package's loader looks for it.

--host-sanitize builds the same library with its host code (the C ABI's
validation, planning and launch code) under AddressSanitizer and
UndefinedBehaviorSanitizer -- the device code is built as usual -- into
fa2-with-4d-mask_amd/_build_hostsan/libfa2_4d_mask_hostsan.so.  The CPU tests
run against it with the sanitizer runtime loaded first:

  LD_PRELOAD=$(/opt/rocm/llvm/bin/clang++ -print-file-name=libclang_rt.asan-x86_64.so) \
  ASAN_OPTIONS=detect_leaks=0 UBSAN_OPTIONS=halt_on_error=1 \
  FA2_4D_MASK_LIB=fa2-with-4d-mask_amd/_build_hostsan/libfa2_4d_mask_hostsan.so \
  python -m pytest tests -m "not gpu"
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
BUILD = HERE / "_build"
LIBDIR = HERE / "tilelang_fa2_4d_mask" / "_lib"
LIB = LIBDIR / "libfa2_4d_mask.so"
BUILD_SAN = HERE / "_build_hostsan"
LIB_SAN = BUILD_SAN / "libfa2_4d_mask_hostsan.so"
# Host-only sanitizers: each flag applies to the host compilation alone.
HOST_SANITIZE = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                 "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer",
                 "-Xarch_host", "-g"]
SOURCES = ["fa_fwd.hip", "fa_bwd.hip", "fa_bwd_kv.hip", "fa_bwd_dq.hip", "fa_wide.hip", "fa_mask.hip", "fa_noalloc.hip",
           "fa_api.cpp"]
# Per-file extra flags.  fa_bwd_kv.hip keeps its dK/dV accumulators in AGPRs
# through inline asm and wants every other MFMA result in VGPRs (read by
# VALU); fa_wide.hip keeps its MFMA operands in AGPRs and every MFMA result in
# VGPRs.
EXTRA_FLAGS = {"fa_bwd_kv.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"], "fa_wide.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libfa2_4d_mask.so)")


def compile_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-fno-gpu-rdc",
        # Packed fp32 VALU forms are disabled on purpose (kept out of every kernel).
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        f"-I{HERE.parent / 'include'}",
    ]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


def build(jobs: int = 4, verbose: bool = False, host_sanitize: bool = False) -> Path:
    out_dir, lib = (BUILD_SAN, LIB_SAN) if host_sanitize else (BUILD, LIB)
    out_dir.mkdir(exist_ok=True)
    lib.parent.mkdir(exist_ok=True)
    cc = hipcc()
    flags = compile_flags() + (HOST_SANITIZE if host_sanitize else [])

    def obj(src: str) -> Path:
        o = out_dir / (Path(src).stem + ".o")
        _run([cc, *flags, *EXTRA_FLAGS.get(src, []), "-c", str(CSRC / src), "-o", str(o)], verbose)
        return o

    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(obj, SOURCES))
    tmp = lib.with_suffix(".so.tmp")
    if host_sanitize:
        # host link against the shared sanitizer runtime (the device code is
        # already embedded in each object)
        rocm = Path(cc).resolve().parent.parent
        link = [str(rocm / "llvm" / "bin" / "clang++"), "-shared", "-fPIC", "-shared-libsan",
                "-fsanitize=address,undefined", *map(str, objs), f"-L{rocm / 'lib'}", "-lamdhip64",
                f"-Wl,-rpath,{rocm / 'lib'}", "-o", str(tmp)]
        _run(link, verbose)
    else:
        _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)], verbose)
    os.replace(tmp, lib)
    return lib


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=4)
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--host-sanitize", action="store_true",
                    help="host code under ASan + UBSan, into _build_hostsan/ (see the module docstring)")
    args = ap.parse_args()
    lib = build(args.jobs, args.verbose, args.host_sanitize)
    print(f"built {lib}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
