"""Builds libfrq_hip.so in-tree with hipcc for gfx950.

    python -m flatrun_amd.build            # compile and link
    python -m flatrun_amd.build --asm      # also write the gfx950 assembly
                                           # (for inspection) under _build/

Flags that matter:
  -ffp-contract=off                    no implicit FMA: the dequant kernels
                                       are bit-exact with the reference's
                                       separately rounded products and sums;
                                       kernels that want FMA call fmaf.
  -fno-gpu-flush-denormals-to-zero     keep fp32 denormals (the reference
                                       never flushes).
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                       no packed-fp32 VALU instructions.
  -mllvm -disable-promote-alloca-to-lds
                                       per-thread arrays stay in registers
                                       (LLVM otherwise moves some into spare
                                       LDS, adding LDS traffic).
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
ROOT = PKG.parent
BUILD = ROOT / "_build"
LIB = PKG / "libfrq_hip.so"

SOURCES = ["frq_dequant.hip", "frq_gemv.hip", "frq_gemv_mx.hip", "frq_gemv_sk.hip", "frq_gemv_mr.hip", "frq_gemv_mb.hip", "frq_gemm.hip", "frq_gemm_f32.hip",
           "frq_noalloc.hip", "frq_act.hip",
           "frq_api.cpp"]
ARCH = os.environ.get("FRQ_OFFLOAD_ARCH", "gfx950")


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libfrq_hip.so)")


def _flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-ffp-contract=off",
        "-fno-gpu-flush-denormals-to-zero",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-mllvm", "-disable-promote-alloca-to-lds",
        "-Wno-unused-command-line-argument",
        f"-I{ROOT / 'include'}",
        f"-I{CSRC}",
    ]


def _compile(src: Path, obj: Path, asm: bool) -> None:
    cmd = [_hipcc(), *_flags(), "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stdout}\n{r.stderr}")
    if asm and src.suffix == ".hip":
        out = BUILD / (src.stem + f"-{ARCH}.s")
        r = subprocess.run([_hipcc(), *_flags(), "--cuda-device-only", "-S", str(src), "-o", str(out)],
                           capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc -S failed on {src.name}:\n{r.stderr}")


def build(asm: bool = False, verbose: bool = False) -> Path:
    """Compile every source (always) and link flatrun_amd/libfrq_hip.so."""
    BUILD.mkdir(exist_ok=True)
    srcs = [CSRC / s for s in SOURCES if (CSRC / s).is_file()]
    objs = [BUILD / (s.stem + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=min(len(srcs), os.cpu_count() or 4)) as ex:
        list(ex.map(lambda so: _compile(so[0], so[1], asm), zip(srcs, objs)))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--asm", action="store_true")
    a = ap.parse_args()
    build(asm=a.asm, verbose=True)
    sys.exit(0)
