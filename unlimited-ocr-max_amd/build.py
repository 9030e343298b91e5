"""Builds the HIP library ``uocr_moe/libuocr_moe.so`` for gfx950 with hipcc.

Every translation unit is compiled with -ffp-contract=off (the only fused
multiply-adds are explicit) and correctly rounded fp32 division, the two
properties the decode path's bit-exact contract needs; packed fp32 VALU ops are
disabled.  Objects go to ``_build/`` next to this file.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB = HERE / "uocr_moe" / "libuocr_moe.so"
SOURCES = ["gemv.hip", "route.hip", "gemm.hip", "decode.hip", "ngram.hip", "attention.hip", "decoder.hip", "uocr_moe.cpp"]
ARCH = os.environ.get("UOCR_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP library needs ROCm's hipcc")


def _compile(src: str, build_dir: Path = BUILD, defines: tuple[str, ...] = ()) -> Path:
    obj = build_dir / (src + ".o")
    cmd = [hipcc(), *FLAGS, *[f"-D{d}" for d in defines], "-c", str(CSRC / src), "-o", str(obj)]
    if src.endswith(".cpp"):
        cmd.insert(1, "-x")
        cmd.insert(2, "hip")
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{res.stderr}")
    return obj


def build(verbose: bool = False, lib: Path = LIB, build_dir: Path = BUILD, defines: tuple[str, ...] = ()) -> Path:
    """Compile every source (always) and link the shared library; returns its path.

    ``defines`` (``NAME=VALUE``) and a separate ``lib``/``build_dir`` build variants for experiments.
    """
    build_dir.mkdir(parents=True, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 1)) as pool:
        objs = list(pool.map(lambda s: _compile(s, build_dir, defines), SOURCES))
    LIB_ = lib
    tmp = LIB_.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_)
    if verbose:
        print(f"built {LIB_}")
    return LIB_


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
