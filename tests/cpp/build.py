"""Builds tests/cpp/executor_caller (a C++ caller of the drop-in headers)
against raftinfer_amd/libraftinfer_amd.so with hipcc."""
from __future__ import annotations

import os
import pathlib
import subprocess

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parent.parent
BIN = HERE / "executor_caller"


def build() -> pathlib.Path:
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    cmd = [hipcc, "--offload-arch=gfx950", "-std=c++20", "-O2", "-Wall",
           f"-I{ROOT / 'include'}", str(HERE / "executor_caller.cpp"),
           f"-L{ROOT / 'raftinfer_amd'}", "-lraftinfer_amd",
           "-Wl,-rpath,$ORIGIN/../../raftinfer_amd", "-o", str(BIN)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"building the C++ caller failed:\n{res.stderr}")
    return BIN


if __name__ == "__main__":
    print(build())
