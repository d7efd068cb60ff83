"""Decode under HIP graph capture with a device-resident position, as the
reference's decode graphs run it (cpp/tests/qwen35_cuda_graph_test.cu:115-183,
cpp/kernels/qwen35_online_attention.cu:947-1014): the captured kernels read the
position from device memory, so one graph replays every step while a captured
kernel advances the position.  Every replay is checked against the CPU oracle,
with eager work and synchronizations between replays.
"""
import numpy as np
import pytest
import torch

from helpers import HKV, HQ, D, assert_bf16_close, bf16, from_dev, make_cache, normal, rng, to_dev
from oracle import pyoracle as orc
from raftinfer_amd import ops

pytestmark = pytest.mark.gpu


def test_rope_graph_follows_device_position(gpu):
    # cpp/tests/qwen35_cuda_graph_test.cu:115-183
    x = torch.tensor([1.0, -2.0, 0.5, 3.0], device="cuda")
    w = torch.ones(4, device="cuda")
    out = torch.empty(4, device="cuda")
    pos = torch.tensor([128], device="cuda", dtype=torch.int32)
    shape = ops.QkNormRopeShape(1, 1, 4, 2, 0, 1e4)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=gpu):
        ops.qwen35_qk_norm_rope(x, w, out, shape, 1e-6, 1, 1, stream=gpu, device_position=pos)
        pos.add_(1)
    for expected_position in (128, 129, 130):
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        ref = torch.empty(4, device="cuda")
        ops.qwen35_qk_norm_rope(x, w, ref, ops.QkNormRopeShape(1, 1, 4, 2, expected_position, 1e4),
                                1e-6, 1, 1, stream=gpu)
        torch.cuda.synchronize()
        assert torch.allclose(got, ref, atol=1e-5, rtol=0)
        want = orc.qk_norm_rope(from_dev(x).reshape(1, 1, 4), from_dev(w), 2, expected_position, 1e4, 1e-6)
        np.testing.assert_allclose(from_dev(got), want.ravel(), atol=1e-5)


def test_captured_decode_step_crosses_split_threshold(gpu):
    """Producers (fused q split + norm + RoPE, k norm + RoPE) and the online
    decode (append + single-block or split-K by the device position) captured
    once; replayed for contexts 253 .. 260, across the 256-token threshold."""
    max_ctx, start, steps, rot, base = 320, 252, 8, 64, 1e7
    r = rng(2024)
    past_k = bf16(normal(r, start, HKV, D))
    past_v = bf16(normal(r, start, HKV, D))
    cache = to_dev(make_cache(past_k, past_v, 1, max_ctx), torch.bfloat16)
    wq = to_dev(bf16(normal(r, D, scale=0.2) + 1.0), torch.bfloat16)
    wk = to_dev(bf16(normal(r, D, scale=0.2) + 1.0), torch.bfloat16)
    qg_in = torch.empty(HQ * 2 * D, device="cuda", dtype=torch.bfloat16)
    k_in = torch.empty(HKV * D, device="cuda", dtype=torch.bfloat16)
    v_in = torch.empty(HKV * D, device="cuda", dtype=torch.bfloat16)
    q_out, g_out = (torch.empty(HQ * D, device="cuda", dtype=torch.bfloat16) for _ in range(2))
    k_out = torch.empty(HKV * D, device="cuda", dtype=torch.bfloat16)
    out = torch.empty(HQ * D, device="cuda", dtype=torch.bfloat16)
    pos = torch.tensor([start], device="cuda", dtype=torch.int32)
    shape = ops.Qwen35AttentionShape(1, HQ, HKV, D, max_ctx, start)
    plan = ops.qwen35_online_decode_plan(shape, ops.AUTO, max_ctx)
    ws = torch.zeros(ops.qwen35_online_decode_workspace_layout(shape, plan[0])[4], device="cuda",
                     dtype=torch.uint8)
    qshape = ops.QkNormRopeShape(1, HQ, D, rot, 0, base)
    kshape = ops.QkNormRopeShape(1, HKV, D, rot, 0, base)

    def step():
        ops.qwen35_split_query_gate_norm_rope(qg_in, wq, q_out, g_out, qshape, 1e-6, 3, 3,
                                              stream=gpu, device_position=pos)
        ops.qwen35_qk_norm_rope(k_in, wk, k_out, kshape, 1e-6, 3, 3, stream=gpu,
                                device_position=pos)
        ops.qwen35_online_attention_decode(q_out, k_out, v_in, g_out, out, cache, ws, shape,
                                           ops.DTYPE_BF16, ops.CACHE_BF16, ops.HEAD_MAJOR,
                                           plan=plan, device_position=pos, stream=gpu)
        pos.add_(1)

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=gpu):
        step()
    # Capture does not run the work: the position and cache are unchanged.
    keys, vals = list(past_k), list(past_v)
    for s in range(steps):
        p = start + s
        qg = bf16(normal(r, HQ * 2 * D))
        kn, vn = bf16(normal(r, HKV * D)), bf16(normal(r, HKV * D))
        qg_in.copy_(to_dev(qg, torch.bfloat16))
        k_in.copy_(to_dev(kn, torch.bfloat16))
        v_in.copy_(to_dev(vn, torch.bfloat16))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert int(pos.item()) == p + 1
        qg3 = qg.reshape(1, HQ, 2, D)
        q_want = orc.qk_norm_rope(qg3[:, :, 0], from_dev(wq), rot, p, base, 1e-6)
        k_want = orc.qk_norm_rope(kn.reshape(1, HKV, D), from_dev(wk), rot, p, base, 1e-6)
        q_got = from_dev(q_out).reshape(HQ, D)
        k_got = from_dev(k_out).reshape(HKV, D)
        assert_bf16_close(q_got, q_want[0], what=f"q at position {p}")
        assert_bf16_close(k_got, k_want[0], what=f"k at position {p}")
        np.testing.assert_array_equal(from_dev(g_out).reshape(HQ, D), qg3[0, :, 1])
        keys.append(k_got)
        vals.append(vn.reshape(HKV, D))
        want = orc.attention_core(q_got[None], np.stack(keys), np.stack(vals),
                                  qg3[:, :, 1], p)[0]
        assert_bf16_close(from_dev(out).reshape(HQ, D), want, what=f"decode at context {p + 1}")
        ck = from_dev(cache)[: HKV * max_ctx * D].reshape(HKV, max_ctx, D)
        np.testing.assert_array_equal(ck[:, p], k_got)  # the appended row is the produced k


def test_captured_prefill_and_delta_core_replay(gpu):
    """The bf16 MFMA prefill (with its fused cache append) and the chunked gated-delta core
    captured once each and replayed three times, with eager work and synchronizations between
    the replays; every replay must reproduce the eager result bit for bit (the delta state is
    restored eagerly before each replay)."""
    gen = torch.Generator(device="cuda").manual_seed(77)
    rnd = lambda *s: torch.randn(*s, device="cuda", generator=gen).to(torch.bfloat16)
    T = 512
    q, g, k, v = rnd(T, HQ, D), rnd(T, HQ, D), rnd(T, HKV, D), rnd(T, HKV, D)
    cache = torch.zeros(2 * T * HKV * D, device="cuda", dtype=torch.bfloat16)
    out = torch.empty(T, HQ, D, device="cuda", dtype=torch.bfloat16)
    shape = ops.Qwen35AttentionShape(T, HQ, HKV, D, T, 0)
    pol = ops.Qwen35AttentionLaunchPolicy(1, 1, 1)
    run_prefill = lambda: ops.qwen35_causal_attention(q, k, v, g, out, cache, None, shape, 3, pol, stream=gpu)

    dq = torch.nn.functional.normalize(torch.randn(T, 16, 128, device="cuda", generator=gen), dim=-1).to(torch.bfloat16)
    dk = torch.nn.functional.normalize(torch.randn(T, 16, 128, device="cuda", generator=gen), dim=-1).to(torch.bfloat16)
    dv = torch.randn(T, 32, 128, device="cuda", generator=gen).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(T, 32, device="cuda", generator=gen))
    lg = -torch.nn.functional.softplus(torch.randn(T, 32, device="cuda", generator=gen))
    s0 = torch.randn(32, 128, 128, device="cuda", generator=gen) * 0.05
    st = s0.clone()
    dout = torch.empty(T, 32, 128, device="cuda", dtype=torch.bfloat16)
    ws = torch.empty(ops.qwen35_gated_delta_core_workspace_bytes(T, 16, 32, 128, 128), device="cuda",
                     dtype=torch.uint8)
    run_delta = lambda: ops.qwen35_gated_delta_core(dq, dk, dv, beta, lg, 128 ** -0.5, st, dout, ws, True,
                                                    stream=gpu)

    with torch.cuda.stream(gpu):
        run_prefill()
        run_delta()
    torch.cuda.synchronize()
    want_out, want_cache, want_dout, want_st = out.clone(), cache.clone(), dout.clone(), st.clone()

    graph_p, graph_d = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph_p, stream=gpu):
        run_prefill()
    with torch.cuda.graph(graph_d, stream=gpu):
        run_delta()
    for replay in range(3):
        out.zero_()
        cache.zero_()
        dout.zero_()
        st.copy_(s0)
        torch.cuda.synchronize()
        graph_p.replay()
        graph_d.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want_out), f"prefill replay {replay}"
        assert torch.equal(cache, want_cache), f"prefill append replay {replay}"
        assert torch.equal(dout, want_dout), f"delta output replay {replay}"
        assert torch.equal(st, want_st), f"delta state replay {replay}"


def test_decode_graph_variants_across_bucket_boundaries(gpu):
    """The per-bucket variant table (cpp/execution/qwen35_executor.cu:2191-2226) captured by
    the library's HipGraphDecode (cpp/execution/cuda_graph_decode.cu:20-61): one single-block
    variant below the split threshold, then one per distinct split-K plan.  Replayed across
    the 256 threshold and the 512 / 1024 bucket edges, each replay against the oracle."""
    max_ctx = 1100
    r = rng(3030)
    keys, vals = bf16(normal(r, max_ctx, HKV, D)), bf16(normal(r, max_ctx, HKV, D))
    keys[r.random(max_ctx) < 0.01] *= 8.0
    cache = to_dev(make_cache(keys, vals, 1, max_ctx), torch.bfloat16)
    q_np, g_np = bf16(normal(r, HQ, D)), bf16(normal(r, HQ, D))
    q, g = to_dev(q_np, torch.bfloat16), to_dev(g_np, torch.bfloat16)
    k_in = torch.empty(HKV * D, device="cuda", dtype=torch.bfloat16)
    v_in = torch.empty(HKV * D, device="cuda", dtype=torch.bfloat16)
    out = torch.empty(HQ * D, device="cuda", dtype=torch.bfloat16)
    shape = ops.Qwen35AttentionShape(1, HQ, HKV, D, max_ctx, 0)
    ws = torch.empty(ops.qwen35_online_decode_workspace_layout(shape, ops.SPLIT_K_256)[4],
                     device="cuda", dtype=torch.uint8)
    pos = torch.zeros(1, device="cuda", dtype=torch.int32)
    graphs = ops.Qwen35DecodeAttentionGraphs(shape, ops.SPLIT_K_256, 3, 1, 1, q, k_in, v_in, g, out,
                                             cache, ws, pos, stream=gpu)
    # single-block, then buckets 512 (cap 2), 1024 (cap 4), 1100 (cap 5)
    assert graphs.variant_count() == 4
    assert [graphs.variant_for(p) for p in (0, 254, 255, 510, 511, 1022, 1023, 1099)] == \
        [0, 0, 1, 1, 1, 2, 2, 3]
    for position in (254, 255, 256, 510, 511, 512, 1022, 1023, 1024, 1099, 100):
        k_in.copy_(to_dev(keys[position], torch.bfloat16).flatten())
        v_in.copy_(to_dev(vals[position], torch.bfloat16).flatten())
        pos.fill_(position)
        graphs.replay(position)
        torch.cuda.synchronize()
        want = orc.attention_core(q_np[None], keys[:position + 1], vals[:position + 1], g_np[None],
                                  position)[0]
        assert_bf16_close(from_dev(out).reshape(HQ, D), want, what=f"graph position {position}")
    graphs.close()
    # auto_select and single_block build only the single-block variant, as the reference
    # executor does (qwen35_executor.cu:2199-2205: threshold 0), and replay it at any position.
    for mode in (ops.AUTO, ops.SINGLE_BLOCK):
        g2 = ops.Qwen35DecodeAttentionGraphs(shape, mode, 3, 1, 1, q, k_in, v_in, g, out, cache, ws,
                                             pos, stream=gpu)
        assert g2.variant_count() == 1
        assert [g2.variant_for(p) for p in (0, 255, 511, 1099)] == [0, 0, 0, 0]
        position = 700
        k_in.copy_(to_dev(keys[position], torch.bfloat16).flatten())
        v_in.copy_(to_dev(vals[position], torch.bfloat16).flatten())
        pos.fill_(position)
        g2.replay(position)
        torch.cuda.synchronize()
        want = orc.attention_core(q_np[None], keys[:position + 1], vals[:position + 1], g_np[None],
                                  position)[0]
        assert_bf16_close(from_dev(out).reshape(HQ, D), want, what=f"mode {mode} position {position}")
        g2.close()
