"""The producers fused into the attention kernels.

The reference runs the q / gate split and the per-head RMSNorm + partial RoPE of
q and k as separate kernels before the attention (cpp/execution/qwen35_executor.cu:
1989-2013, cpp/kernels/qwen35_primitives.cu:158-210).  The fused entry points do
that work inside the attention kernels from the raw projections.  They must give
bit for bit what the separate producers followed by the unfused attention give
(outputs and appended cache rows), and that sequence is checked against the CPU
oracle (RMSNorm + RoPE: cpp/reference/qwen35.cpp:169-186; attention:
:316-370).
"""
import numpy as np
import pytest
import torch

from helpers import HKV, HQ, D, assert_bf16_close, bf16, from_dev, make_cache, normal, read_cache, rng, to_dev
from oracle import pyoracle as orc
from raftinfer_amd import ops

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def _norm_weights(r, wdt):
    wq = normal(r, D, scale=0.2) + 1.0
    wk = normal(r, D, scale=0.2) + 1.0
    if wdt == torch.bfloat16:
        wq, wk = bf16(wq), bf16(wk)
    return wq, wk


def _decode_case(ctx, max_ctx, mode, rot, wdt, layout, device_position, seed):
    r = rng(seed)
    past_k, past_v = bf16(normal(r, ctx - 1, HKV, D)), bf16(normal(r, ctx - 1, HKV, D))
    qg = bf16(normal(r, HQ, 2, D))
    kraw, v = bf16(normal(r, HKV, D)), bf16(normal(r, HKV, D))
    wq, wk = _norm_weights(r, wdt)
    base, eps = 1e7, 1e-6
    cache0 = to_dev(make_cache(past_k, past_v, layout, max_ctx), BF)
    shape = ops.Qwen35AttentionShape(1, HQ, HKV, D, max_ctx, ctx - 1)
    plan = ops.qwen35_online_decode_plan(shape, mode, max_ctx)
    nbytes = ops.qwen35_online_decode_workspace_layout(shape, plan[0])[4]
    mk_ws = lambda: torch.zeros(nbytes, device="cuda", dtype=torch.uint8) if nbytes else None
    pos = torch.tensor([ctx - 1], device="cuda", dtype=torch.int32) if device_position else None
    dqg, dk, dv = to_dev(qg, BF), to_dev(kraw, BF), to_dev(v, BF)
    dwq, dwk = to_dev(wq, wdt), to_dev(wk, wdt)
    wcode = ops.DTYPE_F32 if wdt == torch.float32 else ops.DTYPE_BF16
    # separate producers, then the unfused decode
    q1 = torch.empty(HQ * D, device="cuda", dtype=BF)
    g1 = torch.empty(HQ * D, device="cuda", dtype=BF)
    k1 = torch.empty(HKV * D, device="cuda", dtype=BF)
    ops.qwen35_split_query_gate_norm_rope(dqg, dwq, q1, g1, ops.QkNormRopeShape(1, HQ, D, rot, ctx - 1, base),
                                          eps, ops.DTYPE_BF16, wcode)
    ops.qwen35_qk_norm_rope(dk, dwk, k1, ops.QkNormRopeShape(1, HKV, D, rot, ctx - 1, base), eps,
                            ops.DTYPE_BF16, wcode)
    out1 = torch.empty(HQ * D, device="cuda", dtype=BF)
    cache1 = cache0.clone()
    ops.qwen35_online_attention_decode(q1, k1, dv, g1, out1, cache1, mk_ws(), shape, ops.DTYPE_BF16,
                                       ops.CACHE_BF16, layout, plan=plan, device_position=pos)
    # fused
    out2 = torch.empty(HQ * D, device="cuda", dtype=BF)
    cache2 = cache0.clone()
    norm = ops.Qwen35FusedNormRope(dwq, dwk, rot, base, eps)
    ops.qwen35_online_attention_decode_fused(dqg, dk, dv, out2, cache2, mk_ws(), shape, norm,
                                             ops.CACHE_BF16, layout, plan, device_position=pos)
    torch.cuda.synchronize()
    return dict(out1=out1, out2=out2, cache1=cache1, cache2=cache2, q1=q1, g1=g1, k1=k1,
                past_k=past_k, past_v=past_v, qg=qg, kraw=kraw, v=v, wq=wq, wk=wk)


@pytest.mark.parametrize("ctx,max_ctx,mode", [(100, 1024, ops.SPLIT_K_256), (300, 1024, ops.SPLIT_K_256),
                                              (4096, 4096, ops.AUTO), (512, 512, ops.SINGLE_BLOCK),
                                              (1000, 1024, ops.SINGLE_BLOCK), (1500, 2048, ops.SPLIT_K_512)])
@pytest.mark.parametrize("device_position", [False, True])
def test_fused_decode_equals_producers_then_decode(gpu, ctx, max_ctx, mode, device_position):
    c = _decode_case(ctx, max_ctx, mode, 64, torch.bfloat16, ops.HEAD_MAJOR, device_position,
                     seed=ctx + 7 * device_position)
    assert torch.equal(c["out1"], c["out2"])
    assert torch.equal(c["cache1"], c["cache2"])


@pytest.mark.parametrize("rot,wdt,layout", [(256, torch.float32, ops.HEAD_MAJOR),
                                            (8, torch.bfloat16, ops.TOKEN_MAJOR),
                                            (128, torch.float32, ops.TOKEN_MAJOR)])
def test_fused_decode_rotary_weights_layouts(gpu, rot, wdt, layout):
    c = _decode_case(777, 1024, ops.SPLIT_K_256, rot, wdt, layout, True, seed=rot)
    assert torch.equal(c["out1"], c["out2"])
    assert torch.equal(c["cache1"], c["cache2"])


def test_fused_decode_against_oracle(gpu):
    ctx, rot, base, eps = 2049, 64, 1e7, 1e-6
    c = _decode_case(ctx, 4096, ops.AUTO, rot, torch.bfloat16, ops.HEAD_MAJOR, False, seed=5)
    q = orc.qk_norm_rope(c["qg"][None, :, 0], c["wq"], rot, ctx - 1, base, eps)
    k = orc.qk_norm_rope(c["kraw"][None], c["wk"], rot, ctx - 1, base, eps)
    kb = bf16(k[0])
    keys = np.concatenate([c["past_k"], kb[None]])
    vals = np.concatenate([c["past_v"], c["v"][None]])
    want = orc.attention_core(bf16(q), keys, vals, c["qg"][None, :, 1], ctx - 1)[0]
    assert_bf16_close(from_dev(c["out2"]).reshape(HQ, D), want, what="fused decode")
    ck, _ = read_cache(from_dev(c["cache2"]), 1, ctx, 4096)
    assert_bf16_close(ck[ctx - 1], kb, what="appended k", both_bf16=True)


def _prefill_case(T, past, rot, wdt, layout, seed):
    r = rng(seed)
    max_ctx = past + T
    pk, pv = bf16(normal(r, past, HKV, D)), bf16(normal(r, past, HKV, D))
    qg = bf16(normal(r, T, HQ, 2, D))
    kraw, v = bf16(normal(r, T, HKV, D)), bf16(normal(r, T, HKV, D))
    wq, wk = _norm_weights(r, wdt)
    base, eps = 1e7, 1e-6
    cache0 = to_dev(make_cache(pk, pv, layout, max_ctx), BF)
    shape = ops.Qwen35AttentionShape(T, HQ, HKV, D, max_ctx, past)
    dqg, dk, dv = to_dev(qg, BF), to_dev(kraw, BF), to_dev(v, BF)
    dwq, dwk = to_dev(wq, wdt), to_dev(wk, wdt)
    wcode = ops.DTYPE_F32 if wdt == torch.float32 else ops.DTYPE_BF16
    q1 = torch.empty(T * HQ * D, device="cuda", dtype=BF)
    g1 = torch.empty(T * HQ * D, device="cuda", dtype=BF)
    k1 = torch.empty(T * HKV * D, device="cuda", dtype=BF)
    ops.qwen35_split_query_gate_norm_rope(dqg, dwq, q1, g1, ops.QkNormRopeShape(T, HQ, D, rot, past, base),
                                          eps, ops.DTYPE_BF16, wcode)
    ops.qwen35_qk_norm_rope(dk, dwk, k1, ops.QkNormRopeShape(T, HKV, D, rot, past, base), eps,
                            ops.DTYPE_BF16, wcode)
    out1 = torch.empty(T * HQ * D, device="cuda", dtype=BF)
    cache1 = cache0.clone()
    ops.qwen35_causal_attention(q1, k1, dv, g1, out1, cache1, None, shape, ops.DTYPE_BF16,
                                ops.Qwen35AttentionLaunchPolicy(1, ops.CACHE_BF16, layout))
    out2 = torch.empty(T * HQ * D, device="cuda", dtype=BF)
    cache2 = cache0.clone()
    ops.qwen35_online_attention_prefill_fused(dqg, dk, dv, out2, cache2, shape,
                                              ops.Qwen35FusedNormRope(dwq, dwk, rot, base, eps),
                                              ops.CACHE_BF16, layout)
    torch.cuda.synchronize()
    return dict(out1=out1, out2=out2, cache1=cache1, cache2=cache2, qg=qg, kraw=kraw, v=v, wq=wq,
                wk=wk, pk=pk, pv=pv)


@pytest.mark.parametrize("T,past", [(2, 0), (7, 0), (40, 0), (128, 0), (512, 0), (17, 111), (300, 33)])
def test_fused_prefill_equals_producers_then_attention(gpu, T, past):
    c = _prefill_case(T, past, 64, torch.bfloat16, ops.HEAD_MAJOR, seed=T + past)
    assert torch.equal(c["cache1"], c["cache2"])
    assert torch.equal(c["out1"], c["out2"])


@pytest.mark.parametrize("rot,wdt,layout", [(256, torch.float32, ops.HEAD_MAJOR),
                                            (8, torch.bfloat16, ops.TOKEN_MAJOR),
                                            (128, torch.float32, ops.TOKEN_MAJOR),
                                            (192, torch.bfloat16, ops.HEAD_MAJOR)])
def test_fused_prefill_rotary_weights_layouts(gpu, rot, wdt, layout):
    c = _prefill_case(70, 5, rot, wdt, layout, seed=rot + 1)
    assert torch.equal(c["cache1"], c["cache2"])
    assert torch.equal(c["out1"], c["out2"])


def test_fused_prefill_against_oracle(gpu):
    T, past, rot, base, eps = 96, 20, 64, 1e7, 1e-6
    c = _prefill_case(T, past, rot, torch.bfloat16, ops.HEAD_MAJOR, seed=9)
    q = bf16(orc.qk_norm_rope(c["qg"][:, :, 0], c["wq"], rot, past, base, eps))
    k = bf16(orc.qk_norm_rope(c["kraw"], c["wk"], rot, past, base, eps))
    keys = np.concatenate([c["pk"], k])
    vals = np.concatenate([c["pv"], c["v"]])
    want = orc.attention_core(q, keys, vals, c["qg"][:, :, 1], past)
    assert_bf16_close(from_dev(c["out2"]).reshape(T, HQ, D), want, what="fused prefill")
    ck, cv = read_cache(from_dev(c["cache2"]), 1, past + T, past + T)
    assert_bf16_close(ck[past:], k, what="appended k", both_bf16=True)
    assert np.array_equal(cv[past:], c["v"])
