"""Compile the HIP sources under ``csrc/`` into ``libctmr_hip.so`` for gfx950.

The library is built in-tree (next to this file) so it travels with the
repository to the GPU host.  ``hipcc`` cross-compiles without a GPU.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_DIR = PACKAGE_DIR.parent
CSRC = PACKAGE_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
LIB_NAME = "libctmr_hip.so"
LIB_PATH = PACKAGE_DIR / LIB_NAME
SOURCES = ("conv.hip", "norm.hip", "attention.hip", "noalloc.hip")
ARCH = "gfx950"

# Packed FP32 VALU ops are disabled for every device pass; hipcc's host pass
# warns that it does not know the feature, which is harmless.
HIP_FLAGS = (
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
)


def hipcc() -> str:
    """Locate hipcc (ROCm's default install first)."""
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found; the ctmr HIP library cannot be built")


# Per-source device flags.  The attention kernel's MFMA accumulators are
# read and rescaled by VALU code; the VGPR form of the MFMAs keeps them out of
# the AGPRs (no v_accvgpr copies in its loop).
EXTRA_FLAGS = {"attention.hip": ("-mllvm", "-amdgpu-mfma-vgpr-form")}


def build(verbose: bool = False) -> Path:
    """Compile every source and link ``libctmr_hip.so``; always rebuilds."""
    compiler = hipcc()
    build_dir = PACKAGE_DIR / "_build"
    build_dir.mkdir(exist_ok=True)
    objects = []
    for name in SOURCES:
        obj = build_dir / (Path(name).stem + ".o")
        cmd = [compiler, *HIP_FLAGS, *EXTRA_FLAGS.get(name, ()), f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(CSRC / name),
               "-o", str(obj)]
        _run(cmd, verbose)
        objects.append(str(obj))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([compiler, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objects, "-o", str(tmp)], verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def _run(cmd: list[str], verbose: bool) -> None:
    """Run one compiler command, keeping only real diagnostics on failure."""
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        lines = [ln for ln in (proc.stdout + proc.stderr).splitlines() if "packed-fp32-ops" not in ln]
        raise RuntimeError("HIP build failed:\n" + " ".join(cmd) + "\n" + "\n".join(lines[-60:]))


if __name__ == "__main__":
    print(build(verbose=True))
