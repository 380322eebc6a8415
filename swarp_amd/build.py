"""Build libswarp_hip.so in-tree with hipcc for gfx950.

``python -m swarp_amd.build`` (or ``__graft_entry__.build()``) compiles the units under
``swarp_amd/csrc`` -- the host side ``swarp_hip.hip`` and one object per kernel family
and scalar type (``k_*.hip`` with ``SWARP_T`` = float / double) -- in parallel, then links
them into ``swarp_amd/libswarp_hip.so``.  ``--incremental`` recompiles only the objects
whose sources, headers (from the compiler's dependency files) or flags changed.

Floating-point flags are part of the contract with the parity tests:
``-ffp-contract=off`` keeps every ``a*b + c`` as two rounded operations (the op order
of the reference source), and ``-fhip-fp32-correctly-rounded-divide-sqrt`` keeps fp32
``/`` and ``sqrtf`` IEEE correctly rounded.  ``-target-feature -packed-fp32-ops`` keeps
the device code free of packed fp32 instructions (v_pk_fma_f32 and friends); the host
pass of hipcc, which does not know the feature, warns that it ignores it.
"""

from __future__ import annotations

import argparse
import hashlib
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
OUT = PKG / "libswarp_hip.so"
ARCH = os.environ.get("SWARP_OFFLOAD_ARCH", "gfx950")

# (object stem, source, extra defines)
FAMILIES = ("k_generic", "k_drone", "k_boxes", "k_holo", "k_bodies", "k_nav", "k_wide",
            "k_wide2", "k_wide4", "k_wbodies")
DTYPES = (("f32", "float", "1"), ("f64", "double", "0"))


def units() -> list[tuple[str, Path, list[str]]]:
    out = [("swarp_hip", CSRC / "swarp_hip.hip", []),
           ("coo_noalloc", CSRC / "coo_noalloc.hip", [])]
    for fam in FAMILIES:
        for tag, ctype, is32 in DTYPES:
            out.append((f"{fam}.{tag}", CSRC / f"{fam}.hip",
                        [f"-DSWARP_T={ctype}", f"-DSWARP_T_IS_F32={is32}"]))
    return out


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
        "-ffp-contract=off",
        "-fhip-fp32-correctly-rounded-divide-sqrt",
        "-fno-gpu-rdc",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-command-line-argument",
        f"-I{ROOT / 'include'}",
        f"-I{CSRC}",
    ]


def _stale(obj: Path, dep: Path, stamp: Path, key: str) -> bool:
    if not obj.exists() or not dep.exists() or not stamp.exists():
        return True
    if stamp.read_text() != key:
        return True
    t = obj.stat().st_mtime
    text = dep.read_text().replace("\\\n", " ")
    paths = text.split(":", 1)[1].split() if ":" in text else []
    for p in paths:
        q = Path(p)
        if not q.exists() or q.stat().st_mtime > t:
            return True
    return False


def _compile(cc: str, stem: str, src: Path, extra: list[str], force: bool,
             verbose: bool) -> tuple[str, bool, str]:
    obj, dep, stamp = OBJ / f"{stem}.o", OBJ / f"{stem}.d", OBJ / f"{stem}.key"
    cmd = [cc, *flags(), *extra, "-c", str(src), "-MD", "-MF", str(dep), "-o", str(obj)]
    key = hashlib.sha256(" ".join(cmd).encode()).hexdigest()
    if not force and not _stale(obj, dep, stamp, key):
        return stem, False, ""
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        return stem, True, res.stdout + res.stderr or f"hipcc failed ({res.returncode})"
    stamp.write_text(key)
    return stem, True, ""


def build(verbose: bool = False, incremental: bool = False, jobs: int | None = None) -> Path:
    """Compile the HIP library; returns the path of the built .so.  Without
    ``incremental`` every unit is recompiled."""
    cc = hipcc()
    OBJ.mkdir(exist_ok=True)
    us = units()
    jobs = jobs or min(len(us), max(1, os.cpu_count() or 1))
    with ThreadPoolExecutor(jobs) as ex:
        res = list(ex.map(lambda u: _compile(cc, *u, not incremental, verbose), us))
    errs = [(s, e) for s, _, e in res if e]
    if errs:
        for s, e in errs:
            sys.stderr.write(f"---- {s}\n{e}\n")
        raise RuntimeError(f"hipcc failed building {', '.join(s for s, _ in errs)}")
    if not incremental or any(r for _, r, _ in res) or not OUT.exists():
        tmp = OUT.with_suffix(".so.tmp")
        cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-fno-gpu-rdc",
               *[str(OBJ / f"{s}.o") for s, _, _ in us], "-o", str(tmp)]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            sys.stderr.write(r.stdout + r.stderr)
            raise RuntimeError(f"linking {OUT.name} failed ({r.returncode})")
        os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--incremental", action="store_true")
    ap.add_argument("-q", "--quiet", action="store_true")
    ap.add_argument("-j", "--jobs", type=int, default=None)
    a = ap.parse_args()
    print(build(verbose=not a.quiet, incremental=a.incremental, jobs=a.jobs))
