"""GPU parity of the attention producers (the q/gate split and the per-head
RMSNorm + partial RoPE) against the CPU oracle, which is bit-exact with the
reference's own cpp/reference/qwen35.cpp helpers.

Mirrors cpp/tests/qwen35_cuda_primitives_test.cu:325-420 (3 heads x 13 dims,
rotary 8, position 5, base 1e4, eps 1e-5, every activation dtype, f32 weights
for 16-bit activations and 16-bit weights for f32 activations) plus the
Qwen3.5 model shape (16 q / 4 k heads x 256, rotary 64, base 1e7, T = 512).
Inputs are quantised to the activation dtype before the fp32 oracle runs.
Gates: the reference's abs-or-rel 2e-2 elementwise; for bf16 model-shape
outputs also max-abs max(1e-2, 1 ulp) and relative-L2 5e-3; f32 within 1e-5.
The split is a copy and must be bit-exact.
"""
import numpy as np
import pytest
import torch

from helpers import assert_bf16_close, close_enough, from_dev, normal, rng, sequence, to_dev
from oracle import pyoracle as orc
from raftinfer_amd import ops

pytestmark = pytest.mark.gpu
TDT = {1: torch.float32, 2: torch.float16, 3: torch.bfloat16}
Q = ops.QkNormRopeShape


def quantize(a, dt):
    return from_dev(to_dev(a, TDT[dt]))


def run_norm_rope(x, w, shape, eps, dt, wdt, device_position=None):
    out = torch.empty(x.size, device="cuda", dtype=TDT[dt])
    ops.qwen35_qk_norm_rope(to_dev(x, TDT[dt]), to_dev(w, TDT[wdt]), out, shape, eps, dt, wdt,
                            device_position=device_position)
    torch.cuda.synchronize()
    return from_dev(out).reshape(x.shape)


@pytest.mark.parametrize("dt,wdt", [(1, 1), (2, 2), (3, 3), (2, 1), (3, 1), (1, 2), (1, 3)])
def test_reference_shapes_every_dtype(gpu, dt, wdt):
    rows, heads, d, rot = 2, 3, 13, 8
    shape = Q(rows, heads, d, rot, 5, 1e4)
    x = quantize(sequence(rows * heads * d, 0.019, -0.4).reshape(rows, heads, d), dt)
    w = quantize(sequence(d, 0.005, 0.0), wdt)
    got = run_norm_rope(x, w, shape, 1e-5, dt, wdt)
    want = orc.qk_norm_rope(x, w, rot, 5, 1e4, 1e-5)
    assert close_enough(got, want)
    if dt == 1:
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("heads", [16, 4])
@pytest.mark.parametrize("pos", [0, 1000])
def test_model_shape_bf16(gpu, heads, pos):
    T, d, rot = 512, 256, 64
    r = rng(heads + pos)
    x = quantize(normal(r, T * heads * d).reshape(T, heads, d), 3)
    w = quantize(normal(r, d, scale=0.3) + 1.0, 3)
    got = run_norm_rope(x, w, Q(T, heads, d, rot, pos, 1e7), 1e-6, 3, 3)
    want = orc.qk_norm_rope(x, w, rot, pos, 1e7, 1e-6)
    assert_bf16_close(got, want, what=f"qk_norm_rope heads {heads} pos {pos}")


def test_device_position_equals_host_offset(gpu):
    T, heads, d, rot = 7, 4, 256, 64
    r = rng(5)
    x = quantize(normal(r, T * heads * d).reshape(T, heads, d), 3)
    w = quantize(normal(r, d, scale=0.3) + 1.0, 3)
    pos = torch.tensor([4321], device="cuda", dtype=torch.int32)
    a = run_norm_rope(x, w, Q(T, heads, d, rot, 0, 1e7), 1e-6, 3, 3, device_position=pos)
    b = run_norm_rope(x, w, Q(T, heads, d, rot, 4321, 1e7), 1e-6, 3, 3)
    np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("dt", [1, 2, 3])
@pytest.mark.parametrize("heads,d", [(3, 5), (16, 256), (2, 12)])
def test_split_is_exact(gpu, dt, heads, d):
    rows = 3
    qg = to_dev(sequence(rows * heads * 2 * d, 0.013, 0.2), TDT[dt])
    q = torch.empty(rows * heads * d, device="cuda", dtype=TDT[dt])
    g = torch.empty_like(q)
    ops.qwen35_split_full_query_gate(qg, q, g, rows, heads, d, dt)
    torch.cuda.synchronize()
    blocks = from_dev(qg).reshape(rows, heads, 2, d)
    np.testing.assert_array_equal(from_dev(q).reshape(rows, heads, d), blocks[:, :, 0])
    np.testing.assert_array_equal(from_dev(g).reshape(rows, heads, d), blocks[:, :, 1])


def test_fused_split_norm_rope_equals_two_steps(gpu):
    T, heads, d, rot = 128, 16, 256, 64
    r = rng(9)
    qg = quantize(normal(r, T * heads * 2 * d), 3)
    w = quantize(normal(r, d, scale=0.3) + 1.0, 3)
    shape = Q(T, heads, d, rot, 77, 1e7)
    dq = to_dev(qg, torch.bfloat16)
    q1, g1 = (torch.empty(T * heads * d, device="cuda", dtype=torch.bfloat16) for _ in range(2))
    ops.qwen35_split_full_query_gate(dq, q1, g1, T, heads, d, 3)
    q2 = torch.empty_like(q1)
    ops.qwen35_qk_norm_rope(q1, to_dev(w, torch.bfloat16), q2, shape, 1e-6, 3, 3)
    q3, g3 = torch.empty_like(q1), torch.empty_like(g1)
    ops.qwen35_split_query_gate_norm_rope(dq, to_dev(w, torch.bfloat16), q3, g3, shape, 1e-6, 3, 3)
    torch.cuda.synchronize()
    assert torch.equal(q2, q3) and torch.equal(g1, g3)
    want = orc.qk_norm_rope(qg.reshape(T, heads, 2, d)[:, :, 0], w, rot, 77, 1e7, 1e-6)
    assert_bf16_close(from_dev(q3).reshape(T, heads, d), want, what="fused producer")


@pytest.mark.parametrize("dt", [1, 2, 3])
@pytest.mark.parametrize("widths", [(8192, 32, 32, 4096), (7, 3, 3, 5), (16, 8, 8, 24)])
def test_pack_linear_delta_input_is_exact(gpu, dt, widths):
    # cpp/tests/qwen35_cuda_primitives_test.cu (pack cases) and the model widths
    # (qkv 2*16*128 + 32*128, beta 32, alpha 32, gate 32*128).
    tokens = 5
    srcs = [sequence(tokens * w, 0.011 * (k + 1), 0.1 * k).reshape(tokens, w) for k, w in enumerate(widths)]
    dev = [to_dev(x, TDT[dt]) for x in srcs]
    packed = torch.empty(tokens * sum(widths), device="cuda", dtype=TDT[dt])
    ops.qwen35_pack_linear_delta_input(*dev, packed, tokens, *widths, dt)
    torch.cuda.synchronize()
    want = orc.pack_linear_delta_input(*[from_dev(d).reshape(tokens, -1) for d in dev])
    np.testing.assert_array_equal(from_dev(packed).reshape(tokens, -1), want)
