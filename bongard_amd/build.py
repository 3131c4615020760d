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
    # per-kernel register, scratch and LDS use, summarised into _build/resource_usage.txt
    "-Rpass-analysis=kernel-resource-usage",
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
    usage = []
    for src, (_, log) in zip(sources, results):
        usage += _resource_usage(src.name, log)
        rest = "\n".join(l for l in log.splitlines() if "kernel-resource-usage" not in l)
        if verbose and rest.strip():
            print(rest, file=sys.stderr)
    _write_usage(usage, verbose)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *[str(o) for o, _ in results]]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


_USAGE_KEYS = (("VGPRs", "vgpr"), ("AGPRs", "agpr"), ("ScratchSize [bytes/lane]", "scratch"),
               ("Occupancy [waves/SIMD]", "occupancy"), ("LDS Size [bytes/block]", "lds"))


def _resource_usage(tu, log):
    """Per-kernel figures from the compiler's kernel-resource-usage remarks of one unit."""
    out, cur = [], None
    for line in log.splitlines():
        if "kernel-resource-usage" not in line:
            continue
        body = line.split("remark:", 1)[-1]
        if "Function Name:" in body:
            cur = {"tu": tu, "name": body.split("Function Name:", 1)[1].split()[0]}
            out.append(cur)
            continue
        for key, field in _USAGE_KEYS:
            if cur is not None and f" {key}:" in body:
                cur[field] = int(body.split(f"{key}:", 1)[1].split()[0])
    return out


def _write_usage(usage, verbose):
    """Writes _build/resource_usage.txt (one line per kernel, demangled where c++filt
    exists) and reports the kernels that use scratch (register spills)."""
    names = [u["name"] for u in usage]
    try:
        res = subprocess.run(["c++filt"], input="\n".join(names), capture_output=True,
                             text=True, check=True)
        demangled = res.stdout.splitlines()
        if len(demangled) == len(names):
            names = demangled
    except (OSError, subprocess.CalledProcessError):
        pass
    lines = [f"{'unit':26s} {'vgpr':>4s} {'agpr':>4s} {'scratch':>7s} {'occ':>3s} {'lds':>6s}  kernel"]
    spills = []
    for u, n in zip(usage, names):
        lines.append(f"{u['tu']:26s} {u.get('vgpr', -1):4d} {u.get('agpr', -1):4d} "
                     f"{u.get('scratch', -1):7d} {u.get('occupancy', -1):3d} {u.get('lds', -1):6d}  {n}")
        if u.get("scratch", 0) > 0:
            spills.append(f"  {u['scratch']:4d} B/lane  {n}")
    (OBJ / "resource_usage.txt").write_text("\n".join(lines) + "\n")
    if verbose:
        print(f"{len(usage)} kernels, {len(spills)} with scratch (per-kernel figures in "
              f"{OBJ / 'resource_usage.txt'})", file=sys.stderr)
        for line in spills:
            print(line, file=sys.stderr)


if __name__ == "__main__":
    print(build(verbose=True))
