"""Seeded random sweeps of the three entry families against the C oracle.

Each case draws its shape and options from a fixed seed, so a failure names a
reproducible configuration: decode over context, cache capacity, layout, plan
mode, activation / cache dtype and host / device position; prefill over
prompt length, past length, layout and dtypes; the gated-delta entry at the
model shape over length, activation / weight dtype and schedule.  The
per-feature tests pin the edges; these cover the combinations between them.
"""
import numpy as np
import pytest

from helpers import HKV, HQ, D, close_enough, normal, rel_l2, rng
from test_attention_gpu import run_decode, run_prefill
from test_delta_gpu import fixture_for, model_shape, run_gpu, run_ref
from raftinfer_amd import ops

pytestmark = pytest.mark.gpu


def _decode_case(i):
    r = np.random.default_rng(7000 + i)
    ctx = int(r.integers(1, 3000))
    return dict(ctx=ctx, max_ctx=ctx + int(r.integers(0, 600)), layout=int(r.integers(0, 2)),
                mode=int(r.integers(0, 4)), dt=[(3, 1), (1, 1), (3, 0), (1, 0)][int(r.integers(0, 4))],
                dev=bool(r.integers(0, 2)))


@pytest.mark.parametrize("i", range(40))
def test_random_decode(gpu, i):
    c = _decode_case(i)
    out, expect, cache, keys, vals, _, _ = run_decode(c["dt"][0], c["dt"][1], c["layout"], c["ctx"], c["max_ctx"],
                                                      mode=c["mode"], device_position=c["dev"], seed=i,
                                                      heavy_rows=0.01)
    assert close_enough(out, expect), c


@pytest.mark.parametrize("i", range(16))
def test_random_prefill(gpu, i):
    r = np.random.default_rng(8000 + i)
    T = int(r.integers(1, 600))
    past = int(r.integers(0, 400)) if r.random() < 0.6 else 0
    layout = int(r.integers(0, 2))
    act, cdt = [(3, 1), (3, 1), (1, 1), (3, 0)][int(r.integers(0, 4))]
    out, expect, *_ = run_prefill(act, cdt, layout, T, HQ, HKV, D, past, seed=1000 + i)
    assert np.isfinite(out).all() and close_enough(out, expect), (T, past, layout, act, cdt)


@pytest.mark.parametrize("i", range(16))
def test_random_gated_delta(gpu, i):
    r = np.random.default_rng(9000 + i)
    T = int(r.choice([1, 2, 5, 33, 63, 64, 65, 100, 129, 200]))
    dt, wdt = [(3, 3), (3, 3), (1, 1), (2, 2), (1, 3)][int(r.integers(0, 5))]
    sched = int(r.integers(0, 2)) if T > 1 else int(r.integers(0, 3))
    sh = model_shape(T)
    fx = fixture_for(sh, seed=500 + i)
    g = rng(900 + i)
    rec0, conv0 = normal(g, 32 * 128 * 128, scale=0.05), normal(g, 8192 * 3)
    got = run_gpu(sh, fx, dt, wdt, conv0, rec0, policy=ops.GatedDeltaLaunchPolicy(sched))
    want = run_ref(sh, fx, dt, wdt, conv0, rec0)
    assert all(close_enough(a, b) for a, b in zip(got, want)), (T, dt, wdt, sched)
    assert rel_l2(got[2], want[2]) < 1e-4
