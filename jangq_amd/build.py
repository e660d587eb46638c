"""Build the gfx950 shared library ``jangq_amd/libjangq_amd.so`` with hipcc.

Each ``csrc/*.hip`` translation unit is compiled to an object in parallel, then linked into
one C-ABI shared library (entry points declared in ``include/jangq_amd.h``). Objects are
rebuilt only when a source or header is newer, so an unchanged tree links in seconds.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "libjangq_amd.so"
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed fp32 VALU forms are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
]
# Per-file extra flags: the codec must round q*s and +b separately (no FMA contraction).
EXTRA = {
    "jq_codec.hip": ["-ffp-contract=off"],
    # decode kernels: keep MFMA results in VGPRs (no accumulator-register round trips)
    "jq_dec.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "jq_decp.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "jq_qmv4.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "jq_dmx.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the jangq_amd kernels need the ROCm toolchain")


def _compile(src: Path, force: bool) -> Path:
    obj = OBJ / (src.stem + ".o")
    deps = [src, *CSRC.glob("*.h"), ROOT / "include" / "jangq_amd.h"]
    if not force and obj.exists() and all(obj.stat().st_mtime >= d.stat().st_mtime for d in deps):
        return obj
    cmd = [hipcc(), *COMMON_FLAGS, *EXTRA.get(src.name, []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr[-6000:]}")
    return obj


def build(force: bool = False, jobs: int | None = None) -> Path:
    """Compile every kernel source for gfx950 and link ``libjangq_amd.so``; returns its path."""
    OBJ.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, force), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr[-6000:]}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(force="--force" in sys.argv))
