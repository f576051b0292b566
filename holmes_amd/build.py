"""Compile the HIP sources of holmes_amd into holmes_amd/_lib/libholmes_ckks.so (gfx950).

Run ``python -m holmes_amd.build`` (or ``__graft_entry__.build()``).  Each ``.hip`` file is
compiled to an object in parallel, then linked into one shared library exporting the C ABI of
``include/holmes_ckks.h``.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT_DIR = PKG / "_lib"
LIB = OUT_DIR / "libholmes_ckks.so"
ARCH = os.environ.get("HOLMES_AMD_ARCH", "gfx950")

SOURCES = ["context.hip", "ntt.hip", "poly.hip", "keyswitch.hip", "ksfused.hip", "bsgs.hip", "encode.hip",
           "mul.hip", "noalloc.hip", "wide.hip", "wide_fused.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    # packed FP32 instructions are kept out of every kernel (some of their forms have given
    # wrong results on these boxes); FP64 code does not need them.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-result",
    f"-I{ROOT / 'include'}",
]


def _compile(src: str, build_dir: Path) -> Path:
    obj = build_dir / (Path(src).stem + ".o")
    cmd = [HIPCC, *FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    build_dir = OUT_DIR / "obj"
    build_dir.mkdir(parents=True, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), 8)) as pool:
        objs = list(pool.map(lambda s: _compile(s, build_dir), SOURCES))
    tmp = LIB.with_suffix(f".so.tmp{os.getpid()}")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
