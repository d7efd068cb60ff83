"""The allocation-free decode entry point against the workspace-taking one.

raftinfer_amd_online_attention_decode_static_workspace runs the same kernels
as raftinfer_amd_online_attention_decode, with the split-K partials in the
library's static device array instead of a caller workspace, so outputs and
appended cache rows must be bit-identical.  Two calls in a row, the second
smaller (shorter context, smaller maximum context), check that the array's
contents from the first call do not leak into the second.
"""
import numpy as np
import pytest
import torch

from helpers import HKV, HQ, D, bf16, make_cache, normal, rng, to_dev
from raftinfer_amd import ops

pytestmark = pytest.mark.gpu
S = ops.Qwen35AttentionShape


def _case(ctx, max_ctx, seed, layout=1):
    r = rng(seed)
    pk, pv = bf16(normal(r, ctx - 1, HKV, D)), bf16(normal(r, ctx - 1, HKV, D))
    pk[r.random(ctx - 1) < 0.01] *= 8.0
    cache = to_dev(make_cache(pk, pv, layout, max_ctx), torch.bfloat16)
    x = [to_dev(bf16(normal(r, *s)), torch.bfloat16) for s in ((HQ * D,), (HKV * D,), (HKV * D,), (HQ * D,))]
    return x, cache


def _both(ctx, max_ctx, seed, mode=ops.SPLIT_K_256, device_position=False, layout=1):
    x, cache = _case(ctx, max_ctx, seed, layout)
    shape = S(1, HQ, HKV, D, max_ctx, ctx - 1)
    plan = ops.qwen35_online_decode_plan(shape, mode, max_ctx)
    pos = torch.tensor([ctx - 1], device="cuda", dtype=torch.int32) if device_position else None
    ws = torch.full((ops.qwen35_online_decode_workspace_layout(shape, plan[0])[4],), 0x7F,
                    device="cuda", dtype=torch.uint8)
    ref_out = torch.empty(HQ * D, device="cuda", dtype=torch.bfloat16)
    ref_cache = cache.clone()
    ops.qwen35_online_attention_decode(*x, ref_out, ref_cache, ws, shape, 3, 1, layout, plan=plan,
                                       device_position=pos)
    out = torch.empty(HQ * D, device="cuda", dtype=torch.bfloat16)
    ops.qwen35_online_attention_decode_static_workspace(*x, out, cache, shape, 3, 1, layout, plan,
                                                        device_position=pos)
    torch.cuda.synchronize()
    return ref_out, out, ref_cache, cache


def test_static_workspace_matches_workspace_entry_two_calls(gpu):
    assert ops.qwen35_online_attention_static_workspace_bytes() == 16 * 512 * 258 * 4
    # first call: the benchmark's ctx 4096 (16 partitions), heavy rows
    a, b, ca, cb = _both(4096, 4096, 41)
    assert torch.isfinite(b.float()).all()
    assert torch.equal(a, b) and torch.equal(ca, cb)
    # second call, smaller: ctx 700 in a 1024-token cache (3 of 4 partitions), device position
    a, b, ca, cb = _both(700, 1024, 42, device_position=True)
    assert torch.equal(a, b) and torch.equal(ca, cb)


def test_static_workspace_largest_and_too_large(gpu):
    # the largest supported plan at split_k_512, a short context in it, token-major cache
    a, b, ca, cb = _both(1500, 262144, 43, mode=ops.SPLIT_K_512, layout=0)
    assert torch.equal(a, b) and torch.equal(ca, cb)
    # single-block plans take no workspace
    a, b, ca, cb = _both(300, 512, 44, mode=ops.SINGLE_BLOCK)
    assert torch.equal(a, b) and torch.equal(ca, cb)
    # one token beyond the array's capacity is rejected before anything is enqueued
    shape = S(1, HQ, HKV, D, 131073, 0)
    plan = ops.qwen35_online_decode_plan(shape, ops.SPLIT_K_256, 1)
    z = torch.zeros(16, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(ops.Qwen35PrimitiveError, match="static decode workspace is too small"):
        ops.qwen35_online_attention_decode_static_workspace(z, z, z, z, z, z, shape, 3, 1, 1, plan)


def test_static_workspace_under_graph_capture(gpu):
    # After one eager call on the device, the allocation-free entry point is captured into a
    # HIP graph (torch.cuda.graph) and replayed; each replay, with eager work and
    # synchronisations between replays, must give exactly the workspace entry point's output.
    ctx, max_ctx = 3000, 4096
    ref_out, _, _, _ = _both(ctx, max_ctx, 45)  # also the eager first call on this device
    x, cache = _case(ctx, max_ctx, 45)
    shape = S(1, HQ, HKV, D, max_ctx, ctx - 1)
    plan = ops.qwen35_online_decode_plan(shape, ops.SPLIT_K_256, max_ctx)
    pos = torch.tensor([ctx - 1], device="cuda", dtype=torch.int32)
    out = torch.empty(HQ * D, device="cuda", dtype=torch.bfloat16)
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        ops.qwen35_online_attention_decode_static_workspace(*x, out, cache, shape, 3, 1, 1, plan,
                                                            device_position=pos,
                                                            stream=side)
    for replay in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref_out), f"replay {replay}"
