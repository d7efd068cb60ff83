"""Builds libraftinfer_amd.so (gfx950) in-tree with hipcc.

Every HIP / C++ source under csrc/ is compiled for --offload-arch=gfx950 with
packed-FP32 instruction selection disabled, then linked into one shared
library next to this file.  Run ``python -m raftinfer_amd.build``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import pathlib
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libraftinfer_amd.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC", "-Wall",
    "-Wno-unused-function", "-Wno-unused-variable",
    # packed FP32 arithmetic stays off (compiler-generated v_pk_*_f32 are not used).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}", f"-I{CSRC}",
]


def _compile(src: pathlib.Path) -> pathlib.Path:
    obj = BUILD / (src.name + ".o")
    lang = ["-x", "hip"] if src.suffix == ".hip" else []
    cmd = [HIPCC, *FLAGS, *lang, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(jobs: int | None = None) -> pathlib.Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))
    jobs = jobs or min(8, len(sources))
    with cf.ThreadPoolExecutor(jobs) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
                    *map(str, objs)], check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
