"""Builds libbongard_fp8.so (the gfx950 HIP kernels behind include/bongard_fp8.h) in-tree.

Usage: ``python -m bongard_amd.build`` (also called by ``__graft_entry__.build()``).
Every HIP source is compiled for gfx950 only, with packed-fp32 instruction selection
disabled, into ``bongard_amd/_build/*.o`` and linked into ``bongard_amd/libbongard_fp8.so``.
First ``csrc/gen_gelu_tables.py`` writes ``_build/gelu_tables.inc``, the gated-GELU tables
taken from torch's CPU gelu kernels (the arithmetic the reference's bf16 chain runs).
"""

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "libbongard_fp8.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
    # Packed fp32 ops (v_pk_*_f32) are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-gpu-rdc",
]


def hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the HIP extension cannot be built")
    return path


def _compile(src, extra):
    obj = OBJ / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{OBJ}", *extra, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj, res.stderr


def build(verbose=False, extra=()):
    """Compile every csrc/*.hip for gfx950 and link the shared library. Returns its path."""
    OBJ.mkdir(exist_ok=True)
    res = subprocess.run([sys.executable, str(CSRC / "gen_gelu_tables.py"),
                          str(OBJ / "gelu_tables.inc")], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"gelu table generation failed:\n{res.stdout}\n{res.stderr}")
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    with ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        results = list(ex.map(lambda s: _compile(s, list(extra)), sources))
    for _, log in results:
        if verbose and log.strip():
            print(log, file=sys.stderr)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *[str(o) for o, _ in results]]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
