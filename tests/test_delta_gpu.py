"""GPU parity of the gfx950 gated-delta path against the CPU oracle.

Mirrors cpp/tests/qwen35_cuda_delta_test.cu (prefill lengths, continued
prefill, decode after prefill, f32 auxiliary weights, f32 activations, the
model-shape register path, both schedules) and benchmark config 5 (chunked
prefill T=512 in chunks of 64, then 32 recurrent decode steps).  Operands are
quantised to the activation dtype before the fp32 oracle runs
(cpp/tests/qwen35_cuda_delta_test.cu:258-276).  Gates: the reference's
abs-or-rel 2e-2 for the full entry point; fp32 state within relative-L2 1e-4
and bf16 outputs within max-abs 1e-2 / relative-L2 5e-3 for config 5.
"""
import numpy as np
import pytest
import torch

from helpers import assert_bf16_close, bf16, close_enough, from_dev, normal, rel_l2, rng, sequence, to_dev
from oracle import pyoracle as orc
from raftinfer_amd import ops

pytestmark = pytest.mark.gpu
TDT = {1: torch.float32, 2: torch.float16, 3: torch.bfloat16}


def quantize(a, dt):
    return from_dev(to_dev(a, TDT[dt]))


def small_shape(T):
    # cpp/tests/qwen35_cuda_delta_test.cu:194-205
    return dict(tokens=T, hidden=28, hk=2, hv=4, dk=5, dv=7, width=3, eps=1e-6)


def fixture_for(sh, seed=None):
    cd = 2 * sh["hk"] * sh["dk"] + sh["hv"] * sh["dv"]
    stride = cd + 2 * sh["hv"] + sh["hidden"]
    if seed is None:  # the reference test's deterministic sequences (:236-248)
        return dict(inp=sequence(sh["tokens"] * stride, 0.017, -0.03, 29, 17),
                    cw=sequence(cd * sh["width"], 0.011, 0.04, 29, 17),
                    a=sequence(sh["hv"], 0.03, -1.2, 29, 17),
                    dt=sequence(sh["hv"], 0.025, -0.4, 29, 17),
                    nw=sequence(sh["dv"], 0.02, 0.7, 29, 17))
    r = rng(seed)
    return dict(inp=normal(r, sh["tokens"] * stride), cw=normal(r, cd * sh["width"], scale=0.3),
                a=-np.exp(normal(r, sh["hv"], scale=0.5)), dt=normal(r, sh["hv"]),
                nw=normal(r, sh["dv"]))


def run_gpu(sh, fx, dt, wdt, conv0=None, rec0=None, policy=None):
    cd = 2 * sh["hk"] * sh["dk"] + sh["hv"] * sh["dv"]
    shape = ops.GatedDeltaShape(sh["tokens"], sh["hidden"], sh["hk"], sh["hv"], sh["dk"], sh["dv"],
                                sh["width"], sh["eps"])
    conv = torch.zeros(cd * (sh["width"] - 1), device="cuda") if conv0 is None else to_dev(conv0, torch.float32)
    rec = torch.zeros(sh["hv"] * sh["dk"] * sh["dv"], device="cuda") if rec0 is None else to_dev(rec0, torch.float32)
    ws = torch.empty(ops.qwen35_gated_delta_workspace_bytes(shape) // 4, device="cuda")
    out = torch.empty(sh["tokens"] * sh["hidden"], device="cuda", dtype=TDT[dt])
    ops.qwen35_gated_delta(to_dev(fx["inp"], TDT[dt]), to_dev(fx["cw"], TDT[wdt]),
                           to_dev(fx["a"], TDT[wdt]), to_dev(fx["dt"], TDT[wdt]),
                           to_dev(fx["nw"], TDT[wdt]), out, conv if conv.numel() else None, rec, ws,
                           shape, dt, wdt, policy=policy)
    torch.cuda.synchronize()
    return from_dev(out), from_dev(conv), from_dev(rec)


def run_ref(sh, fx, dt, wdt, conv0=None, rec0=None):
    cd = 2 * sh["hk"] * sh["dk"] + sh["hv"] * sh["dv"]
    q = {k: quantize(v, dt if k == "inp" else wdt) for k, v in fx.items()}
    conv0 = np.zeros(cd * (sh["width"] - 1), np.float32) if conv0 is None else conv0
    rec0 = np.zeros(sh["hv"] * sh["dk"] * sh["dv"], np.float32) if rec0 is None else rec0
    kw = {k: sh[k] for k in ("tokens", "hidden", "hk", "hv", "dk", "dv", "width", "eps")}
    return orc.gated_delta_prefill(q["inp"], q["cw"], q["a"], q["dt"], q["nw"], conv0, rec0, **kw)


def check(got, want):
    for g, w in zip(got, want):
        assert close_enough(g, w), np.abs(np.asarray(g) - np.asarray(w)).max()


@pytest.mark.parametrize("dt", [2, 3])
@pytest.mark.parametrize("T", [1, 2, 4, 17])
def test_prefill_lengths(gpu, dt, T):
    sh = small_shape(T)
    fx = fixture_for(sh)
    check(run_gpu(sh, fx, dt, dt), run_ref(sh, fx, dt, dt))


def test_continued_prefill_and_decode(gpu):
    # cpp/tests/qwen35_cuda_delta_test.cu:352-440
    sh4, sh2, sh1 = small_shape(4), small_shape(2), small_shape(1)
    f4 = fixture_for(sh4)
    g4, w4 = run_gpu(sh4, f4, 3, 3), run_ref(sh4, f4, 3, 3)
    check(g4, w4)
    f2 = fixture_for(sh2)
    f2["inp"] = f2["inp"] + 0.037
    check(run_gpu(sh2, f2, 3, 3, g4[1], g4[2]), run_ref(sh2, f2, 3, 3, w4[1], w4[2]))
    f1 = fixture_for(sh1, seed=5)
    check(run_gpu(sh1, f1, 3, 3, g4[1], g4[2]), run_ref(sh1, f1, 3, 3, w4[1], w4[2]))


def test_f32_auxiliary_weights_and_f32_activations(gpu):
    sh = small_shape(4)
    fx = fixture_for(sh)
    check(run_gpu(sh, fx, 3, 1), run_ref(sh, fx, 3, 1))
    check(run_gpu(sh, fx, 1, 1), run_ref(sh, fx, 1, 1))
    check(run_gpu(sh, fx, 1, 3), run_ref(sh, fx, 1, 3))


def test_saturation_edges(gpu):
    # cpp/tests/qwen35_cuda_delta_test.cu:569-605: large |b|, |a| exercise the
    # sigmoid / softplus branches.
    sh = small_shape(4)
    fx = fixture_for(sh)
    cd = 2 * 2 * 5 + 4 * 7
    stride = cd + 8 + 28
    inp = fx["inp"].reshape(4, stride)
    inp[:, cd:cd + 4] = [[30.0, -30.0, 0.0, 5.0]] * 4
    inp[:, cd + 4:cd + 8] = [[40.0, -40.0, 20.5, -20.5]] * 4
    fx["inp"] = inp.ravel()
    check(run_gpu(sh, fx, 1, 1), run_ref(sh, fx, 1, 1))


def model_shape(T):
    return dict(tokens=T, hidden=4096, hk=16, hv=32, dk=128, dv=128, width=4, eps=1e-6)


@pytest.mark.parametrize("T,schedule", [(3, 0), (2, 0), (1, 2), (1, 0), (17, 1), (64, 0), (128, 0), (150, 0),
                                        (257, 0)])
def test_model_shape_schedules(gpu, T, schedule):
    # cpp/tests/qwen35_cuda_delta_test.cu:631-650 plus both gfx950 schedules.
    sh = model_shape(T)
    fx = fixture_for(sh, seed=T)
    r = rng(T + 1)
    rec0 = normal(r, 32 * 128 * 128, scale=0.05)
    conv0 = normal(r, 8192 * 3)
    got = run_gpu(sh, fx, 3, 3, conv0, rec0, policy=ops.GatedDeltaLaunchPolicy(schedule))
    want = run_ref(sh, fx, 3, 3, conv0, rec0)
    check(got, want)
    assert rel_l2(got[2], want[2]) < 1e-4


@pytest.mark.parametrize("dt,wdt", [(1, 1), (2, 2), (1, 3)])
def test_model_shape_chunked_f32_f16_activations(gpu, dt, wdt):
    # The chunked path (T >= 64, two chunks with a ragged tail) with f32 / f16 activations and
    # f32 or bf16 auxiliary weights: the convolution writes q / k / v as (hi, lo) bf16 planes
    # and the T-record prep and split scan take every product over them in three parts.
    T = 100
    sh = model_shape(T)
    fx = fixture_for(sh, seed=T + dt)
    r = rng(T + 7)
    rec0 = normal(r, 32 * 128 * 128, scale=0.05)
    conv0 = normal(r, 8192 * 3)
    got = run_gpu(sh, fx, dt, wdt, conv0, rec0)
    want = run_ref(sh, fx, dt, wdt, conv0, rec0)
    check(got, want)
    assert rel_l2(got[2], want[2]) < 1e-4


def cfg5_inputs(T, seed):
    """benchmark config 5: q, k ~ N(0,1) L2-normalised per head, v ~ N(0,1),
    beta = sigmoid(N), g = -softplus(N); bf16 q/k/v."""
    r = rng(seed)
    q, k = normal(r, T, 16, 128), normal(r, T, 16, 128)
    q = bf16(q / np.linalg.norm(q, axis=-1, keepdims=True))
    k = bf16(k / np.linalg.norm(k, axis=-1, keepdims=True))
    v = bf16(normal(r, T, 32, 128))
    beta = (1 / (1 + np.exp(-normal(r, T, 32)))).astype(np.float32)
    g = (-np.log1p(np.exp(normal(r, T, 32)))).astype(np.float32)
    return q, k, v, beta, g


def run_core(q, k, v, beta, g, state, chunked):
    T = q.shape[0]
    st = to_dev(state, torch.float32)
    out = torch.empty(T, 32, 128, device="cuda", dtype=torch.bfloat16)
    ws = torch.empty(ops.qwen35_gated_delta_core_workspace_bytes(T, 16, 32, 128, 128),
                     device="cuda", dtype=torch.uint8)
    bt = lambda a: to_dev(a, torch.bfloat16)
    ops.qwen35_gated_delta_core(bt(q), bt(k), bt(v), to_dev(beta, torch.float32),
                                to_dev(g, torch.float32), 1 / np.sqrt(128), st, out, ws, chunked)
    torch.cuda.synchronize()
    return from_dev(out), from_dev(st)


def test_cfg5_chunked_prefill_then_32_decode_steps(gpu):
    T = 512
    q, k, v, beta, g = cfg5_inputs(T + 32, 2026)
    s0 = np.zeros((32, 128, 128), np.float32)
    want_o, want_s = orc.delta_core(q[:T], k[:T], v[:T], beta[:T], g[:T], 1 / np.sqrt(128), s0)
    got_o, got_s = run_core(q[:T], k[:T], v[:T], beta[:T], g[:T], s0, chunked=True)
    assert rel_l2(got_s, want_s) < 1e-4
    assert_bf16_close(got_o, want_o, what="cfg5 chunked prefill")
    s = got_s
    ws_ = want_s
    for t in range(T, T + 32):
        sl = slice(t, t + 1)
        wo, ws_ = orc.delta_core(q[sl], k[sl], v[sl], beta[sl], g[sl], 1 / np.sqrt(128), ws_)
        go, s = run_core(q[sl], k[sl], v[sl], beta[sl], g[sl], s, chunked=False)
        assert_bf16_close(go, wo, what=f"cfg5 decode step {t - T}")
    assert rel_l2(s, ws_) < 1e-4


@pytest.mark.parametrize("T", [1, 63, 64, 65, 130, 257])
def test_core_chunked_ragged_lengths_with_state(gpu, T):
    """Chunked core on a last chunk of every fill (1, 63, 64, 65 tokens ...)
    from a non-zero state, against the oracle's token recurrence."""
    q, k, v, beta, g = cfg5_inputs(T, 100 + T)
    s0 = normal(rng(200 + T), 32, 128, 128, scale=0.05)
    want_o, want_s = orc.delta_core(q, k, v, beta, g, 1 / np.sqrt(128), s0)
    got_o, got_s = run_core(q, k, v, beta, g, s0, chunked=True)
    assert rel_l2(got_s, want_s) < 1e-4
    assert_bf16_close(got_o, want_o, what=f"chunked core T={T}")


def test_core_chunked_long_prompt(gpu):
    """T=2048 (32 chunks): the state carried through a long scan stays within
    rel-L2 1e-4 of the token recurrence, and every output row within the bf16 gate."""
    T = 2048
    q, k, v, beta, g = cfg5_inputs(T, 4242)
    s0 = normal(rng(4243), 32, 128, 128, scale=0.05)
    want_o, want_s = orc.delta_core(q, k, v, beta, g, 1 / np.sqrt(128), s0)
    got_o, got_s = run_core(q, k, v, beta, g, s0, chunked=True)
    assert rel_l2(got_s, want_s) < 1e-4
    assert_bf16_close(got_o, want_o, what="chunked core T=2048")


def test_full_entry_long_prompt(gpu):
    # The drop-in entry at T=1024 (16 chunks through the split-plane path) from non-zero states.
    sh = model_shape(1024)
    fx = fixture_for(sh, seed=1024)
    r = rng(1025)
    rec0 = normal(r, 32 * 128 * 128, scale=0.05)
    conv0 = normal(r, 8192 * 3)
    got = run_gpu(sh, fx, 3, 3, conv0, rec0)
    want = run_ref(sh, fx, 3, 3, conv0, rec0)
    check(got, want)
    assert rel_l2(got[2], want[2]) < 1e-4


@pytest.mark.parametrize("hk,hv", [(8, 32), (32, 32), (4, 8)])
def test_core_chunked_head_groupings(gpu, hk, hv):
    """Value head h reads key head h % Hk; the chunk kernels index K and Q
    rows by it, so other groupings than 16 / 32 must hold too."""
    T = 100
    r = rng(300 + hk)
    q, k = normal(r, T, hk, 128), normal(r, T, hk, 128)
    q = bf16(q / np.linalg.norm(q, axis=-1, keepdims=True))
    k = bf16(k / np.linalg.norm(k, axis=-1, keepdims=True))
    v = bf16(normal(r, T, hv, 128))
    beta = (1 / (1 + np.exp(-normal(r, T, hv)))).astype(np.float32)
    g = (-np.log1p(np.exp(normal(r, T, hv)))).astype(np.float32)
    s0 = normal(r, hv, 128, 128, scale=0.05)
    want_o, want_s = orc.delta_core(q, k, v, beta, g, 1 / np.sqrt(128), s0)
    st = to_dev(s0, torch.float32)
    out = torch.empty(T, hv, 128, device="cuda", dtype=torch.bfloat16)
    ws = torch.empty(ops.qwen35_gated_delta_core_workspace_bytes(T, hk, hv, 128, 128), device="cuda",
                     dtype=torch.uint8)
    bt = lambda a: to_dev(a, torch.bfloat16)
    ops.qwen35_gated_delta_core(bt(q), bt(k), bt(v), to_dev(beta, torch.float32), to_dev(g, torch.float32),
                                1 / np.sqrt(128), st, out, ws, True)
    torch.cuda.synchronize()
    assert rel_l2(from_dev(st), want_s) < 1e-4
    assert_bf16_close(from_dev(out), want_o, what=f"chunked core hk={hk} hv={hv}")


@pytest.mark.parametrize("hk,hv", [(8, 16), (16, 16), (8, 32)])
@pytest.mark.parametrize("T", [1, 130])
def test_full_entry_head_groupings(gpu, hk, hv, T):
    """The full entry on head counts other than 16 / 32 whose widths still take
    the channel-spread convolution: (8, 16) the fused one-token step with 8
    workgroups, (16, 16) and (8, 32) key groups of 1 and 4 (the recurrent and
    chunked kernels behind the wide convolution), from non-zero states."""
    sh = dict(tokens=T, hidden=hv * 128, hk=hk, hv=hv, dk=128, dv=128, width=4, eps=1e-6)
    cd = 2 * hk * 128 + hv * 128
    fx = fixture_for(sh, seed=700 + hk + hv + T)
    r = rng(701 + hk + hv + T)
    rec0 = normal(r, hv * 128 * 128, scale=0.05)
    conv0 = normal(r, cd * 3)
    got = run_gpu(sh, fx, 3, 3, conv0, rec0)
    want = run_ref(sh, fx, 3, 3, conv0, rec0)
    check(got, want)
    assert rel_l2(got[2], want[2]) < 1e-4
    assert np.array_equal(got[1], want[1]) or rel_l2(got[1], want[1]) < 1e-6


def test_core_chunked_equals_recurrent(gpu):
    T = 200
    q, k, v, beta, g = cfg5_inputs(T, 7)
    s0 = normal(rng(8), 32, 128, 128, scale=0.05)
    a_o, a_s = run_core(q, k, v, beta, g, s0, chunked=True)
    b_o, b_s = run_core(q, k, v, beta, g, s0, chunked=False)
    assert rel_l2(a_s, b_s) < 1e-4
    assert_bf16_close(a_o, b_o, what="chunked vs recurrent", both_bf16=True)


def test_cfg5_full_entry_prefill_512_then_32_decode_steps(gpu):
    # The drop-in qwen35_gated_delta (conv + SiLU + l2norm + chunked recurrence + out-norm,
    # cpp/kernels/qwen35_delta.cu:811-897) at the benchmark's config-5 shape: a T=512 prefill
    # from zero states, then 32 single-token calls continuing from the returned states,
    # each against the oracle's token-sequential prefill (cpp/reference/qwen35.cpp:384-549).
    sh = model_shape(512)
    fx = fixture_for(sh, seed=5120)
    got = run_gpu(sh, fx, 3, 3)
    want = run_ref(sh, fx, 3, 3)
    check(got, want)
    assert rel_l2(got[2], want[2]) < 1e-4
    assert_bf16_close(got[0], want[0], what="cfg5 entry prefill T=512")
    g_conv, g_rec, w_conv, w_rec = got[1], got[2], want[1], want[2]
    sh1 = model_shape(1)
    for step in range(32):
        f1 = fixture_for(sh1, seed=6000 + step)
        f1["cw"], f1["a"], f1["dt"], f1["nw"] = fx["cw"], fx["a"], fx["dt"], fx["nw"]
        go, g_conv, g_rec = run_gpu(sh1, f1, 3, 3, g_conv, g_rec)
        wo, w_conv, w_rec = run_ref(sh1, f1, 3, 3, w_conv, w_rec)
        assert close_enough(go, wo), f"decode step {step}"
        assert_bf16_close(go, wo, what=f"cfg5 entry decode step {step}")
    assert rel_l2(g_rec, w_rec) < 1e-4
    assert np.array_equal(g_conv, w_conv) or rel_l2(g_conv, w_conv) < 1e-6


@pytest.mark.parametrize("sh", [small_shape(4), model_shape(1), model_shape(3), model_shape(100),
                                model_shape(512)], ids=["small4", "m1", "m3", "m100", "m512"])
@pytest.mark.parametrize("dt", [1, 3])
def test_unpacked_entry_equals_pack_then_delta(gpu, sh, dt):
    # qwen35_gated_delta_unpacked reads the four projection outputs in place; it must give
    # exactly what qwen35_pack_linear_delta_input + qwen35_gated_delta give
    # (cpp/kernels/qwen35_primitives.cu:388-420, cpp/kernels/qwen35_delta.cu:811-897): the
    # same kernels run, only the row addressing differs, so outputs and states are compared
    # bit for bit, and the packed path against the oracle.
    T = sh["tokens"]
    cd = 2 * sh["hk"] * sh["dk"] + sh["hv"] * sh["dv"]
    r = rng(T * 31 + dt)
    qkv, beta = normal(r, T, cd), normal(r, T, sh["hv"])
    alpha, gate = normal(r, T, sh["hv"]), normal(r, T, sh["hidden"])
    fx = fixture_for(sh, seed=T + 11)
    fx["inp"] = orc.pack_linear_delta_input(qkv, beta, alpha, gate).ravel()
    conv0 = normal(r, cd * (sh["width"] - 1))
    rec0 = normal(r, sh["hv"] * sh["dk"] * sh["dv"], scale=0.05)
    want = run_gpu(sh, fx, dt, dt, conv0, rec0)
    check(want, run_ref(sh, fx, dt, dt, conv0, rec0))
    shape = ops.GatedDeltaShape(T, sh["hidden"], sh["hk"], sh["hv"], sh["dk"], sh["dv"], sh["width"],
                                sh["eps"])
    conv = to_dev(conv0, torch.float32)
    rec = to_dev(rec0, torch.float32)
    ws = torch.empty(ops.qwen35_gated_delta_workspace_bytes(shape) // 4, device="cuda")
    out = torch.empty(T * sh["hidden"], device="cuda", dtype=TDT[dt])
    t = lambda a: to_dev(a, TDT[dt])
    ops.qwen35_gated_delta_unpacked(t(qkv), t(beta), t(alpha), t(gate), t(fx["cw"]), t(fx["a"]),
                                    t(fx["dt"]), t(fx["nw"]), out, conv, rec, ws, shape, dt, dt)
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(out), want[0])
    assert np.array_equal(from_dev(conv), want[1])
    assert np.array_equal(from_dev(rec), want[2])


def test_unpacked_entry_validation(gpu):
    shape = ops.GatedDeltaShape(2, 4096, 16, 32, 128, 128, 4, 1e-6)
    z = torch.zeros(2 * 12352, device="cuda", dtype=torch.bfloat16)
    st = torch.zeros(32 * 128 * 128, device="cuda")
    ws = torch.empty(ops.qwen35_gated_delta_workspace_bytes(shape), device="cuda", dtype=torch.uint8)
    with pytest.raises(ops.Qwen35DeltaError, match="beta pointer is null"):
        ops.qwen35_gated_delta_unpacked(z, None, z, z, z, z, z, z, z, st, st, ws, shape, 3, 3)
    with pytest.raises(ops.Qwen35DeltaError, match="alpha is not dtype-aligned"):
        # f32 activations need 4-byte alignment; one bf16 element in is 2-byte aligned
        ops.qwen35_gated_delta_unpacked(z, z, z[1:], z, z, z, z, z, z, st, st, ws, shape, 1, 1)


def test_channel_spread_shape_off_the_wide_path_stays_in_its_workspace(gpu):
    # A model-shape prefill long enough to be chunked (T = 128) whose packed input is not
    # 16-byte aligned, so the channel-spread convolution cannot run.  The workspace of this
    # shape holds T-records only (33,024 B each), so the call must take the recurrent kernels
    # rather than the W/U-record path: checked against the oracle, with a guard region after
    # the workspace that must come back untouched.
    sh = model_shape(128)
    fx = fixture_for(sh, seed=1280)
    r = rng(1281)
    cd = 2 * sh["hk"] * 128 + sh["hv"] * 128
    conv0 = normal(r, cd * 3)
    rec0 = normal(r, sh["hv"] * 128 * 128, scale=0.05)
    shape = ops.GatedDeltaShape(128, sh["hidden"], sh["hk"], sh["hv"], 128, 128, 4, sh["eps"])
    need = ops.qwen35_gated_delta_workspace_bytes(shape)
    guard = 1 << 16
    buf = torch.full((need + guard,), 0x5A, device="cuda", dtype=torch.uint8)
    ws = buf[:need]
    inp = to_dev(fx["inp"], torch.bfloat16)
    shifted = torch.empty(inp.numel() + 1, device="cuda", dtype=torch.bfloat16)
    shifted[1:].copy_(inp)
    conv = to_dev(conv0, torch.float32)
    rec = to_dev(rec0, torch.float32)
    out = torch.empty(128 * sh["hidden"], device="cuda", dtype=torch.bfloat16)
    w = {k: to_dev(fx[k], torch.bfloat16) for k in ("cw", "a", "dt", "nw")}
    ops.qwen35_gated_delta(shifted[1:], w["cw"], w["a"], w["dt"], w["nw"], out, conv, rec, ws, shape, 3, 3)
    torch.cuda.synchronize()
    assert bool((buf[need:] == 0x5A).all()), "the call wrote past its workspace"
    want = run_ref(sh, fx, 3, 3, conv0, rec0)
    got = (from_dev(out), from_dev(conv), from_dev(rec))
    check(got, want)
    assert rel_l2(got[2], want[2]) < 1e-4
    assert_bf16_close(got[0], want[0], what="off-wide T=128")
