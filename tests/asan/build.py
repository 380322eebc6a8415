"""Builds tests/asan/_build/driver: the library's host code and kernels compiled for the
CPU with g++ under AddressSanitizer + UndefinedBehaviorSanitizer, the kernels running on
the host emulation of the HIP device model in emu/hip/hip_runtime.h (test infrastructure
only; see driver.cpp for the cases).

The sources are copied from swarp_amd/csrc and include/ with two mechanical rewrites the
emulation needs: the dynamic-LDS declaration becomes a pointer to the launch's heap
block, and empty `asm volatile` scheduling barriers are dropped.  Objects are rebuilt when
a source or flag changes.
"""

from __future__ import annotations

import hashlib
import re
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
OUT = HERE / "_build"
SRC = OUT / "src"
EXE = OUT / "driver"

FLAGS = ["-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
         "-fno-sanitize-recover=undefined", "-ffp-contract=off", "-pthread",
         "-Wno-unused-result", "-Wno-ignored-attributes", "-Wno-attributes"]
UNITS = [("swarp_hip", "swarp_hip.hip", [])]
for fam in ("k_generic", "k_drone", "k_boxes", "k_holo", "k_bodies", "k_nav", "k_wide",
            "k_wide2", "k_wide4", "k_wbodies"):
    for tag, ctype, is32 in (("f32", "float", "1"), ("f64", "double", "0")):
        UNITS.append((f"{fam}.{tag}", f"{fam}.hip", [f"-DSWARP_T={ctype}", f"-DSWARP_T_IS_F32={is32}"]))

DYN = re.compile(r"extern\s+__shared__\s+__align__\(16\)\s+unsigned\s+char\s+(\w+)\[\];")
ASM = re.compile(r"asm\s+volatile\s*\([^;]*\);")


def stage() -> None:
    SRC.mkdir(parents=True, exist_ok=True)
    files = list((ROOT / "swarp_amd" / "csrc").glob("*.hpp")) + \
        list((ROOT / "swarp_amd" / "csrc").glob("*.hip")) + list((ROOT / "include").glob("*.h"))
    for f in files:
        t = f.read_text()
        t = DYN.sub(r"unsigned char *\1 = ::emu::dyn_lds();", t)
        t = ASM.sub(";", t)
        dst = SRC / f.name
        if not dst.exists() or dst.read_text() != t:
            dst.write_text(t)


def _compile(stem: str, src: str, extra: list[str]) -> str:
    obj = OUT / f"{stem}.o"
    cmd = ["g++", *FLAGS, *extra, f"-I{HERE / 'emu'}", f"-I{SRC}", "-x", "c++", "-c",
           str(SRC / src), "-o", str(obj)]
    key = hashlib.sha256((" ".join(cmd) + "".join(
        p.read_text() for p in sorted(SRC.iterdir())) + (HERE / "emu/hip/hip_runtime.h").read_text()
    ).encode()).hexdigest()
    stamp = OUT / f"{stem}.key"
    if obj.exists() and stamp.exists() and stamp.read_text() == key:
        return ""
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        return f"---- {stem}\n{r.stdout}{r.stderr}"
    stamp.write_text(key)
    return ""


def build(jobs: int = 8) -> Path:
    OUT.mkdir(exist_ok=True)
    stage()
    with ThreadPoolExecutor(jobs) as ex:
        errs = [e for e in ex.map(lambda u: _compile(*u), UNITS) if e]
    if errs:
        raise RuntimeError("sanitizer build failed:\n" + "\n".join(errs)[-6000:])
    cmd = ["g++", *FLAGS, f"-I{SRC}", f"-I{HERE / 'emu'}", str(HERE / "driver.cpp"),
           *[str(OUT / f"{s}.o") for s, _, _ in UNITS], "-o", str(EXE)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError("sanitizer link failed:\n" + (r.stdout + r.stderr)[-6000:])
    return EXE


if __name__ == "__main__":
    print(build())
    sys.exit(0)
