"""A compiled C++ caller of the drop-in headers (tests/cpp/executor_caller.cpp),
written like the reference executor's call sites
(cpp/execution/qwen35_executor.cu:2017-2057, :2105-2126).  The host checks run
without a GPU (sizing, plans, operator==, error types); the GPU run's outputs
are checked against the CPU oracle."""
import pathlib
import subprocess

import numpy as np
import pytest

from helpers import HKV, HQ, D, assert_bf16_close, close_enough, rel_l2
from oracle import pyoracle as orc

HERE = pathlib.Path(__file__).resolve().parent
BIN = HERE / "cpp" / "executor_caller"


def _stale():
    """The binary is missing or older than its source, a drop-in header or the library."""
    if not BIN.exists():
        return True
    deps = [HERE / "cpp" / "executor_caller.cpp", HERE.parent / "raftinfer_amd" / "libraftinfer_amd.so"]
    deps += sorted((HERE.parent / "include").rglob("*.h*"))
    built = BIN.stat().st_mtime
    return any(d.exists() and d.stat().st_mtime > built for d in deps)


def _binary():
    if _stale():
        import sys
        sys.path.insert(0, str(HERE / "cpp"))
        import build as cpp_build
        cpp_build.build()
    return BIN


def test_cpp_caller_host_checks():
    res = subprocess.run([str(_binary()), "host"], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "host checks ok" in res.stdout


@pytest.mark.gpu
def test_cpp_caller_gpu_matches_oracle(gpu, tmp_path):
    res = subprocess.run([str(_binary()), "gpu", str(tmp_path)], capture_output=True, text=True,
                         timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    ld = lambda n, *shape: np.fromfile(tmp_path / f"{n}.f32", np.float32).reshape(*shape)
    # decode at position 700 of a 1024-token head-major cache (split-K 256)
    max_ctx, pos = 1024, 700
    q, g = ld("decode_q", HQ, D), ld("decode_g", HQ, D)
    k, v = ld("decode_k", HKV, D), ld("decode_v", HKV, D)
    cache = ld("decode_cache", 2, HKV, max_ctx, D)
    assert np.array_equal(cache[0, :, pos], k) and np.array_equal(cache[1, :, pos], v)
    keys = cache[0, :, :pos + 1].transpose(1, 0, 2)
    vals = cache[1, :, :pos + 1].transpose(1, 0, 2)
    want = orc.attention_core(q[None], keys, vals, g[None], pos)[0]
    assert_bf16_close(ld("decode_out", HQ, D), want, what="C++ caller decode")
    # prefill, 40 tokens
    T = 40
    qp, gp = ld("prefill_q", T, HQ, D), ld("prefill_g", T, HQ, D)
    kp, vp = ld("prefill_k", T, HKV, D), ld("prefill_v", T, HKV, D)
    want = orc.attention_core(qp, kp, vp, gp, 0)
    assert_bf16_close(ld("prefill_out", T, HQ, D), want, what="C++ caller prefill")
    # gated delta, 5 tokens at the model shape from zero states
    tokens = 5
    wo, _, wrec = orc.gated_delta_prefill(
        ld("delta_input", tokens * 12352), ld("delta_conv_w", 8192 * 4), ld("delta_a", 32),
        ld("delta_dt", 32), ld("delta_norm_w", 128), np.zeros(8192 * 3, np.float32),
        np.zeros(32 * 128 * 128, np.float32), tokens=tokens, hidden=4096, hk=16, hv=32, dk=128,
        dv=128, width=4, eps=1e-6)
    assert close_enough(ld("delta_out", tokens * 4096), wo)
    assert rel_l2(ld("delta_rec", 32 * 128 * 128), wrec) < 1e-4
