"""Build libneedle2_native.so (gfx950) in-tree with hipcc.

Usage: ``python -m openneedle_amd.build`` (also called by ``__graft_entry__.build``).
Sources are compiled in parallel into ``openneedle_amd/_build/`` and linked
into ``openneedle_amd/libneedle2_native.so``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT = PKG / "libneedle2_native.so"
BUILD = PKG / "_build"

ARCH = os.environ.get("NEEDLE2_GPU_ARCH", "gfx950")

# -ffp-contract=off: the FP32 and int8 epilogues reproduce the reference's
# separately rounded multiplies and adds. Packed-FP32 VALU forms are disabled
# for the device pass (the host pass warns that it does not know the feature).
COMMON = [
    "-O3", "-std=c++17", "-fPIC", "-DNDEBUG", "-ffp-contract=off",
    "-fno-gpu-flush-denormals-to-zero", "-Wall", "-Wno-unused-function",
]
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
# Per-source extras: the int8 MFMA kernel keeps its accumulators in VGPRs
# (no accumulator-register reads in the per-group epilogue).
EXTRA = {"sdot_kernels": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


def sources():
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))


def _compile(src: Path, build_dir: Path = BUILD, defines=()) -> Path:
    obj = build_dir / (src.stem + ".o")
    cmd = [hipcc(), *COMMON, *DEVICE, *EXTRA.get(src.stem, []), *[f"-D{d}" for d in defines], "-I", str(CSRC), "-c",
           str(src), "-o", str(obj)]
    if src.suffix == ".hip":
        cmd[1:1] = ["-x", "hip"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode:
        raise RuntimeError(f"compile failed: {src.name}\n{' '.join(cmd)}\n{res.stderr}")
    return obj


def build(verbose: bool = False, out: Path = OUT, build_dir: Path = BUILD, defines=()) -> Path:
    """Compile every source and link ``out``; ``defines`` are extra -D tuning macros."""
    build_dir.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda src: _compile(src, build_dir, defines), srcs))
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{res.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
