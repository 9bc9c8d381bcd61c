"""Builds ``libbioemu2_mi355x.so`` (all HIP kernels + the C ABI) in-tree for gfx950.

Usage: ``python -m bioemu2_amd.build`` (also called by ``__graft_entry__.build()``).
Always recompiles; the ``.so`` lands next to this file so it travels with the
source tree and is what the Python layer loads.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
INCLUDE = PKG_DIR.parent / "include"
LIB_NAME = "libbioemu2_mi355x.so"
ARCH = os.environ.get("BIOEMU_OFFLOAD_ARCH", "gfx950")

# Packed-fp32 VALU ops are disabled for device code; the host pass warns that
# it does not know the feature, which is harmless.
# -fno-honor-nans: no kernel relies on NaN propagation (infinities are still
# honoured: the softmax masks use -inf), and it lets fmaxf lower to a single
# v_max_f32 instead of canonicalise + max.
# -amdgpu-mfma-vgpr-form: MFMA accumulators live in VGPRs, which removes the
# AGPR<->VGPR copies around every softmax / epilogue touch of an accumulator.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-fno-honor-nans",
    "-mllvm",
    "-amdgpu-mfma-vgpr-form",
    f"-I{INCLUDE}",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _compile(src: Path, obj: Path) -> None:
    cmd = [_hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(
        ln for ln in (res.stdout + res.stderr).splitlines() if "packed-fp32-ops" not in ln
    )
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def build(verbose: bool = True) -> Path:
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    target = PKG_DIR / LIB_NAME
    with tempfile.TemporaryDirectory(prefix="bioemu_build_") as tmp:
        objs = [Path(tmp) / (s.stem + ".o") for s in sources]
        with cf.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
            list(ex.map(_compile, sources, objs))
        tmp_lib = Path(tmp) / LIB_NAME
        cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp_lib)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
        # Atomic replace so a running process never maps a half-written file.
        staged = target.with_suffix(".so.tmp")
        shutil.copy2(tmp_lib, staged)
        os.replace(staged, target)
    if verbose:
        print(f"built {target} from {len(sources)} sources for {ARCH}")
    return target


if __name__ == "__main__":
    build()
