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


# Sources whose kernels issue MFMAs from inline asm; their gfx950 assembly is
# checked for reads of an MFMA result inside its latency (asm_check.py).
ASM_CHECKED = ("attention_prefill_mfma.hip",)


def _check_asm(name: str) -> None:
    try:
        from .asm_check import asm_mfma_hazards
    except ImportError:  # run as a script
        sys.path.insert(0, str(PKG))
        from asm_check import asm_mfma_hazards

    src = CSRC / name
    out = BUILD / (name + ".s")
    cmd = [HIPCC, *FLAGS, "-x", "hip", "--cuda-device-only", "-S", str(src), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc -S failed for {name}:\n{res.stderr}")
    hazards = asm_mfma_hazards(out.read_text())
    if hazards:
        raise RuntimeError(f"{name}: inline-asm MFMA results read too early "
                           f"({len(hazards)}):\n" + "\n".join(hazards[:10]))


def build(jobs: int | None = None) -> pathlib.Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))
    jobs = jobs or min(8, len(sources) + len(ASM_CHECKED))
    with cf.ThreadPoolExecutor(jobs) as pool:
        checks = [pool.submit(_check_asm, name) for name in ASM_CHECKED]
        objs = list(pool.map(_compile, sources))
        for c in checks:
            c.result()
    tmp = LIB.with_suffix(".so.tmp")
    subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
                    *map(str, objs)], check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
