"""Build the fmkv HIP library (libfmkv.so) for gfx950, in-tree.

Usage: python gemma4-moe-flash-mlx-turbo_amd/build.py [--jobs N]

Every .hip file under csrc/ is compiled by hipcc for gfx950 and linked into
one shared library next to this file. Compile flags:
  -ffp-contract=off          the append and readback kernels reproduce the
                             oracle's rounding op by op: no implicit FMA
                             contraction there;
  -ffp-contract=fast-honor-pragmas
                             the attention sources (CONTRACT_SOURCES) let the
                             compiler fuse multiply-adds in their loops; the
                             quantization helpers and new-token columns they
                             share with the append turn contraction off in
                             their bodies (#pragma clang fp contract(off));
  -packed-fp32-ops disabled  no packed FP32 instructions are generated;
  -amdgpu-mfma-vgpr-form=1   MFMA accumulators in VGPRs (see HIP_FLAGS);
  -amdgpu-kernarg-preload-count=14
                             PRELOAD_SOURCES: the leading scalar kernel
                             arguments arrive in SGPRs with the dispatch.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
INCLUDE = PKG_DIR.parent / "include"
BUILD_DIR = PKG_DIR / "_build"
LIB_NAME = "libfmkv.so"
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-mcode-object-version=5",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in ordinary VGPRs: the decode kernel rescales them
    # with VALU ops, and accumulators kept in AGPRs were copied back and
    # forth on every loop iteration
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-Wall",
    "-Wno-unused-result",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


# attention sources: contraction on, except where a pragma turns it off
CONTRACT_SOURCES = {"fmkv_attention.hip", "fmkv_cb_attention.hip", "fmkv_plain_attention.hip",
                    "fmkv_prefill.hip"}
# sources whose kernels take their first 14 argument dwords as scalars that
# the dispatch preloads into SGPRs
PRELOAD_SOURCES = {"fmkv_attention.hip"}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libfmkv.so)")


def _compile(src: Path, obj: Path) -> tuple[Path, str]:
    flags = HIP_FLAGS
    if src.name in CONTRACT_SOURCES:
        flags = ["-ffp-contract=fast-honor-pragmas" if f == "-ffp-contract=off" else f
                 for f in HIP_FLAGS]
    if src.name in PRELOAD_SOURCES:
        flags = [*flags, "-mllvm", "-amdgpu-kernarg-preload-count=14"]
    cmd = [hipcc(), *flags, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = (res.stdout + res.stderr)
    # the host pass does not know the packed-fp32 feature; that note is noise
    lines = [ln for ln in out.splitlines() if "packed-fp32-ops" not in ln]
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n" + "\n".join(lines))
    return obj, "\n".join(lines)


def build(jobs: int = 8, verbose: bool = True) -> Path:
    """Compile all kernels and link libfmkv.so; returns its path."""
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no .hip sources in {CSRC}")
    objs = []
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        futs = {ex.submit(_compile, s, BUILD_DIR / (s.stem + ".o")): s for s in sources}
        for f in cf.as_completed(futs):
            obj, log = f.result()
            objs.append(obj)
            if verbose and log.strip():
                print(log)
    lib = PKG_DIR / LIB_NAME
    tmp = PKG_DIR / (LIB_NAME + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, sorted(objs))]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("link failed:\n" + res.stdout + res.stderr)
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib}")
    return lib


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=8)
    args = ap.parse_args(argv)
    build(jobs=args.jobs)
    return 0


if __name__ == "__main__":
    sys.exit(main())
