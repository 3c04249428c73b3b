"""Build libbpdecode_hip.so in-tree with hipcc for gfx950.

Each translation unit under ``csrc/`` is compiled to an object in
``csrc/_build/`` (in parallel), then linked into ``libbpdecode_hip.so`` next
to this file.  The build always recompiles; callers that only need the
library load the existing one.
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
OBJ = CSRC / "_build"
LIB = PKG / "libbpdecode_hip.so"
SOURCES = ["dense.hip", "fsa.hip", "pda.hip", "soft.hip", "stage.hip", "frames.hip", "host.cpp"]
ARCH = os.environ.get("BPDECODE_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
    # packed-FP32 VALU forms (v_pk_*_f32) stay off: some of their forms have
    # given silently wrong results on this hardware
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.sep not in cand or Path(cand).exists()):
            return cand
    raise RuntimeError("hipcc not found")


def _compile(src: str) -> Path:
    obj = OBJ / (Path(src).stem + ".o")
    cmd = [_hipcc(), *FLAGS, "-x", "hip", "-c", str(CSRC / src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stdout}\n{res.stderr}")
    return obj


def build_library(verbose: bool = False) -> Path:
    OBJ.mkdir(exist_ok=True)
    present = [s for s in SOURCES if (CSRC / s).exists()]
    with ThreadPoolExecutor(max_workers=min(4, len(present))) as ex:
        objs = list(ex.map(_compile, present))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build_library(verbose=True)
