"""Builds libfmx.so (the gfx950 HIP library) in-tree with hipcc.

    python -m freemoe_amd.build          # build libfmx.so next to this file

Every HIP source is compiled for gfx950 only, with FMA contraction off (the
kernels spell out each fused multiply-add the reference performs) and packed
FP32 instructions disabled.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "libfmx.so"

SOURCES = ["capi.cpp", "quant.hip", "matvec.hip", "gemm.hip", "moe.hip", "down_pair_q4k.hip", "bucket.hip",
           "prefill.hip", "attention.hip"]

HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-result",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; libfmx needs ROCm's hipcc to build")
    return path


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, cwd=CSRC, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")


def build(jobs: int | None = None) -> Path:
    """Compiles every source to an object in parallel, then links libfmx.so."""
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    cc = hipcc()
    include = ["-I", str(ROOT / "include"), "-I", str(CSRC)]
    srcs = [s for s in SOURCES if (CSRC / s).exists()]
    procs = []
    objs = []
    for src in srcs:
        obj = objdir / (Path(src).stem + ".o")
        objs.append(obj)
        lang = ["-x", "hip"]
        cmd = [cc, *HIP_FLAGS, *include, *lang, "-c", str(CSRC / src), "-o", str(obj)]
        procs.append((cmd, subprocess.Popen(cmd, cwd=CSRC, stdout=subprocess.PIPE,
                                            stderr=subprocess.STDOUT, text=True)))
    errors = []
    for cmd, p in procs:
        out, _ = p.communicate()
        if p.returncode != 0:
            out = "\n".join(l for l in out.splitlines() if "packed-fp32-ops" not in l)
            errors.append(f"{' '.join(cmd)}\n{out}")
    if errors:
        raise RuntimeError("libfmx build failed:\n" + "\n\n".join(errors))
    tmp = LIB.with_suffix(".so.tmp")
    _run([cc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
    sys.exit(0)
