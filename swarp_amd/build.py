"""Build libswarp_hip.so in-tree with hipcc for gfx950.

``python -m swarp_amd.build`` (or ``__graft_entry__.build()``) compiles
``swarp_amd/csrc/swarp_hip.hip`` into ``swarp_amd/libswarp_hip.so``.

Floating-point flags are part of the contract with the parity tests:
``-ffp-contract=off`` keeps every ``a*b + c`` as two rounded operations (the op order
of the reference source), and ``-fhip-fp32-correctly-rounded-divide-sqrt`` keeps fp32
``/`` and ``sqrtf`` IEEE correctly rounded.  Packed-fp32 instructions are disabled.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
SRC = PKG / "csrc" / "swarp_hip.hip"
OUT = PKG / "libswarp_hip.so"
ARCH = os.environ.get("SWARP_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: set HIPCC or install ROCm")


def flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-ffp-contract=off",
        "-fhip-fp32-correctly-rounded-divide-sqrt",
        "-fno-gpu-rdc",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-command-line-argument",
        f"-I{ROOT / 'include'}",
        f"-I{PKG / 'csrc'}",
    ]


def build(verbose: bool = False) -> Path:
    """Compile the HIP library; returns the path of the built .so."""
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), *flags(), str(SRC), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed ({res.returncode}) building {SRC.name}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
