"""GPU parity of the gfx950 attention path against the CPU oracle.

Mirrors the reference's cpp/tests/qwen35_cuda_attention_test.cu cases
(decode in every layout / dtype, split-K boundary contexts with partial-state
checks, the capacity guard, online prefill incl. causality and adversarial
rescaling, the materialized path) plus the benchmark shapes.  Gates:
 * bf16 outputs: max-abs 1e-2 (or one bf16 ulp of the expected value) and
   relative-L2 5e-3 against the fp32-accumulated oracle;
 * reference-style cases: abs <= 2e-2 or rel <= 2e-2 elementwise;
 * cache appends and split-K bookkeeping (which partials are written, where):
   bit-exact.
"""
import numpy as np
import pytest
import torch

from helpers import (HKV, HQ, D, assert_bf16_close, bf16, close_enough, from_dev,
                     make_cache, normal, read_cache, rng, to_dev)
from oracle import pyoracle as orc
from raftinfer_amd import ops

pytestmark = pytest.mark.gpu
S = ops.Qwen35AttentionShape
TDT = {1: torch.float32, 3: torch.bfloat16}
CDT = {0: torch.float32, 1: torch.bfloat16}


def quant(a, dt):
    return bf16(a) if dt in (3, 1) and dt is not None else a


def decode_inputs(seed, ctx, heavy_rows=0.0):
    """Past keys/values for positions 0..ctx-2 plus the new token's q/k/v/gate."""
    r = rng(seed)
    past_k, past_v = normal(r, ctx - 1, HKV, D), normal(r, ctx - 1, HKV, D)
    if heavy_rows:
        past_k[r.random(ctx - 1) < heavy_rows] *= 8.0
    q, g = normal(r, HQ, D), normal(r, HQ, D)
    k, v = normal(r, HKV, D), normal(r, HKV, D)
    return past_k, past_v, q, k, v, g


def run_decode(act, cdt, layout, ctx, max_ctx, mode=None, device_position=True, seed=0,
               heavy_rows=0.0, ws_fill=None):
    past_k, past_v, q, k, v, g = decode_inputs(seed, ctx, heavy_rows)
    qa, ka, va, ga = (bf16(x) if act == 3 else x for x in (q, k, v, g))
    cache_np = make_cache(past_k, past_v, layout, max_ctx)
    if cdt == 1:
        cache_np = bf16(cache_np)
    cache = to_dev(cache_np, CDT[cdt])
    out = torch.empty(HQ * D, device="cuda", dtype=TDT[act])
    shape = S(1, HQ, HKV, D, max_ctx, ctx - 1)
    ws = None
    plan = None
    if mode is not None:
        plan = ops.qwen35_online_decode_plan(shape, mode, max_ctx)
        nbytes = ops.qwen35_online_decode_workspace_layout(shape, plan[0])[4]
        if nbytes:
            ws = torch.full((nbytes,), ws_fill if ws_fill is not None else 0, device="cuda",
                            dtype=torch.uint8)
    pos = torch.tensor([ctx - 1], device="cuda", dtype=torch.int32) if device_position else None
    ops.qwen35_online_attention_decode(to_dev(qa, TDT[act]), to_dev(ka, TDT[act]),
                                       to_dev(va, TDT[act]), to_dev(ga, TDT[act]), out, cache, ws,
                                       shape, act, cdt, layout, plan=plan, device_position=pos)
    torch.cuda.synchronize()
    keys = np.concatenate([past_k, ka[None]])
    vals = np.concatenate([past_v, va[None]])
    if cdt == 1:
        keys, vals = bf16(keys), bf16(vals)
    expect = orc.attention_core(qa[None], keys, vals, ga[None], ctx - 1)[0]
    return from_dev(out).reshape(HQ, D), expect, from_dev(cache), keys, vals, ws, plan


def test_decode_cfg1_single_block_ctx512(gpu):
    # benchmark config 1: ctx 512, bf16 head-major cache, single-block, no split.
    out, expect, cache, keys, vals, _, _ = run_decode(3, 1, 1, 512, 512, mode=None,
                                                      device_position=False, seed=11)
    assert_bf16_close(out, expect, what="cfg1 decode")
    ck, cv = read_cache(cache, 1, 512, 512)
    assert np.array_equal(ck, keys) and np.array_equal(cv, vals)  # append is bit-exact


@pytest.mark.parametrize("T,past", [(8, 30), (3, 62), (5, 91), (9, 123)])
def test_prefill_mfma_key_tile_past_first_query(gpu, T, past):
    # Regression: a key-split wave whose first key tile starts after some
    # query positions of the workgroup sees only masked scores for those
    # columns; their probabilities must be 0, not exp2(-inf + inf) = NaN.
    out, expect, *_ = run_prefill(3, 1, 1, T, HQ, HKV, D, past, seed=T * 1000 + past)
    assert np.isfinite(out).all()
    assert_bf16_close(out, expect, what=f"prefill T={T} past={past}")


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("act,cdt", [(1, 0), (1, 1), (3, 0), (3, 1)])
@pytest.mark.parametrize("ctx", [32, 128, 512])
def test_decode_layouts_and_dtypes(gpu, layout, act, cdt, ctx):
    # cpp/tests/qwen35_cuda_attention_test.cu:1067-1076
    for device_position in (True, False):
        out, expect, cache, keys, vals, _, _ = run_decode(act, cdt, layout, ctx, ctx + 1,
                                                          mode=1, device_position=device_position,
                                                          seed=ctx + layout)
        assert close_enough(out, expect), (layout, act, cdt, ctx)
        ck, cv = read_cache(cache, layout, ctx, ctx + 1)
        assert np.array_equal(ck, keys) and np.array_equal(cv, vals)


@pytest.mark.parametrize("ctx", [1, 255, 256, 257, 511, 512, 513, 777, 1024])
def test_split_k_256_boundaries_and_partials(gpu, ctx):
    # cpp/tests/qwen35_cuda_attention_test.cu:1078-1101, partials :883-957
    max_ctx = 1025
    out, expect, cache, keys, vals, ws, plan = run_decode(3, 1, 1, ctx, max_ctx, mode=2, seed=ctx,
                                                          ws_fill=0xA5)
    assert close_enough(out, expect)
    assert_bf16_close(out, expect, what=f"split-256 ctx {ctx}")
    wsb = ws.cpu().numpy()
    if ctx < plan[2]:
        assert np.all(wsb == 0xA5)  # below the threshold the workspace is untouched
        return
    lay = ops.qwen35_online_decode_workspace_layout(S(1, HQ, HKV, D, max_ctx, 0), 2)
    f = wsb.view(np.float32)
    maxp = -(-max_ctx // 256)
    pm = f[lay[1] // 4:lay[1] // 4 + lay[0]].reshape(HQ, maxp)
    ps = f[lay[2] // 4:lay[2] // 4 + lay[0]].reshape(HQ, maxp)
    pv = f[lay[3] // 4:lay[3] // 4 + lay[0] * D].reshape(HQ, maxp, D)
    em, es, ev = orc.decode_partials(bf16(decode_inputs(ctx, ctx)[2]), keys, vals, ctx, 256, maxp)
    active = -(-ctx // 256)
    sentinel = np.frombuffer(np.full(4, 0xA5, np.uint8).tobytes(), np.float32)[0]
    assert np.all(pm[:, active:].view(np.uint32) == sentinel.view(np.uint32))  # untouched
    assert close_enough(pm[:, :active], em.reshape(HQ, maxp)[:, :active])
    assert close_enough(ps[:, :active], es.reshape(HQ, maxp)[:, :active])
    assert close_enough(pv[:, :active], ev.reshape(HQ, maxp, D)[:, :active])


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("ctx", [2, 33, 300, 1000, 2049, 3000])
def test_split_k_256_layout_sweep(gpu, layout, ctx):
    # Split-K 256 on the bf16 MFMA path in both cache layouts, odd contexts with a plan
    # capacity above the active partitions (max_ctx 4096), device position, ~1% heavy rows.
    out, expect, cache, keys, vals, *_ = run_decode(3, 1, layout, ctx, 4096, mode=2, seed=ctx + 31 * layout,
                                                    heavy_rows=0.01)
    assert_bf16_close(out, expect, what=f"split-256 layout {layout} ctx {ctx}")
    ck, cv = read_cache(cache, layout, ctx, 4096)
    assert np.array_equal(ck, keys) and np.array_equal(cv, vals)


@pytest.mark.parametrize("ctx", [2, 300, 2049, 5000, 16384])
def test_split_k_row_merge_sparse_waves(gpu, ctx):
    # max_ctx 16384 gives a plan capacity of 64 partitions, so the 8-wave row merge runs;
    # at ctx 2 and 300 (1-2 active partitions) most of its waves have no partition.
    out, expect, *_ = run_decode(3, 1, 1, ctx, 16384, mode=2, seed=ctx + 7, heavy_rows=0.01)
    assert_bf16_close(out, expect, what=f"row merge ctx {ctx}")


@pytest.mark.parametrize("ctx", [513, 777])
def test_split_k_512(gpu, ctx):
    out, expect, *_ = run_decode(3, 1, 1, ctx, 1025, mode=3, seed=ctx + 5)
    assert close_enough(out, expect)


@pytest.mark.parametrize("ctx", [4096, 16384])
def test_split_k_cfg2_long_context(gpu, ctx):
    # benchmark config 2: auto (split-K 256), ~1% of K rows x8, host position.
    out, expect, *_ = run_decode(3, 1, 1, ctx, ctx, mode=0, device_position=False, seed=ctx,
                                 heavy_rows=0.01)
    assert_bf16_close(out, expect, what=f"cfg2 ctx {ctx}")


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("ctx", [385, 512, 513, 777, 1024, 1500])
def test_single_block_staged_scan(gpu, layout, ctx):
    # Above 384 tokens the single-block kernel feeds its scan through an LDS
    # stage (the next chunk streams in under the current one); ragged last
    # chunks, both cache layouts, host and device positions.
    for device_position in (False, True):
        out, expect, cache, keys, vals, _, _ = run_decode(3, 1, layout, ctx, ctx + 7, mode=1,
                                                          device_position=device_position,
                                                          seed=ctx * 3 + layout, heavy_rows=0.01)
        assert_bf16_close(out, expect, what=f"single-block ctx {ctx} layout {layout}")
        ck, cv = read_cache(cache, layout, ctx, ctx + 7)
        assert np.array_equal(ck, keys) and np.array_equal(cv, vals)


@pytest.mark.parametrize("ctx", [1, 2, 31, 33, 100, 300])
def test_single_block_staged_scan_short_context(gpu, ctx):
    # A device position with max_ctx above 384 selects the staged scan whatever
    # the position, so short contexts (waves with no chunk, one ragged chunk)
    # run through it too.
    out, expect, cache, keys, vals, _, _ = run_decode(3, 1, 1, ctx, 2048, mode=1, device_position=True,
                                                      seed=ctx + 4000, heavy_rows=0.01)
    assert_bf16_close(out, expect, what=f"staged single-block ctx {ctx}")
    ck, cv = read_cache(cache, 1, ctx, 2048)
    assert np.array_equal(ck, keys) and np.array_equal(cv, vals)


def test_single_block_equals_split(gpu):
    a, *_ = run_decode(3, 1, 1, 1500, 2048, mode=1, seed=99)
    b, *_ = run_decode(3, 1, 1, 1500, 2048, mode=2, seed=99)
    assert_bf16_close(a, b, what="single vs split", both_bf16=True)


def test_capacity_guard_reports_instead_of_trapping(gpu):
    # cpp/tests/qwen35_cuda_attention_test.cu:1103-1164 (there: a device trap).  The
    # reference appends before attention (qwen35_online_attention.cu:936-945), so the
    # new row must reach the cache even when the merge reports the capacity error.
    ops.consume_capacity_errors()
    max_ctx = 1024
    shape = S(1, HQ, HKV, D, max_ctx, 0)
    plan = ops.qwen35_online_decode_plan(shape, 2, 256)
    assert plan[3] == 512 and plan[4] == 2
    nbytes = ops.qwen35_online_decode_workspace_layout(shape, 2)[4]
    r = rng(512)
    k, v = bf16(normal(r, HKV, D)), bf16(normal(r, HKV, D))
    z = lambda n: torch.zeros(n, device="cuda", dtype=torch.bfloat16)
    out = z(HQ * D)
    cache = z(2 * max_ctx * HKV * D)
    ws = torch.zeros(nbytes, device="cuda", dtype=torch.uint8)
    pos = torch.tensor([512], device="cuda", dtype=torch.int32)
    ops.qwen35_online_attention_decode(z(HQ * D), to_dev(k, torch.bfloat16), to_dev(v, torch.bfloat16),
                                       z(HQ * D), out, cache, ws, shape, 3, 1, 1, plan=plan,
                                       device_position=pos)
    assert ops.consume_capacity_errors() == 1
    assert torch.isnan(out.float()).all()
    ck, cv = read_cache(from_dev(cache), 1, max_ctx, max_ctx)
    assert np.array_equal(ck[512], k) and np.array_equal(cv[512], v)
    assert not ck[:512].any() and not ck[513:].any()  # no other row written
    assert ops.consume_capacity_errors() == 0


@pytest.mark.parametrize("ctx", [33000, 40000])
def test_split_k_row_merge_multi_chunk(gpu, ctx):
    # max_ctx 40960: 160 partitions, so each of the row merge's 8 waves merges up to 20
    # partitions in two chunks (the running max is rescaled across chunks and the second
    # chunk is partial).  Heavy rows in early and late partitions move the max both ways.
    past_k, past_v, q, k, v, g = decode_inputs(ctx, ctx)
    past_k[5] *= 8.0
    past_k[ctx - 300] *= 8.0
    past_k[ctx // 2] *= 8.0
    max_ctx = 40960
    cache = to_dev(bf16(make_cache(past_k, past_v, 1, max_ctx)), torch.bfloat16)
    qa, ka, va, ga = (bf16(x) for x in (q, k, v, g))
    shape = S(1, HQ, HKV, D, max_ctx, ctx - 1)
    plan = ops.qwen35_online_decode_plan(shape, 2, ctx)
    assert plan[4] == 160
    ws = torch.zeros(ops.qwen35_online_decode_workspace_layout(shape, 2)[4], device="cuda",
                     dtype=torch.uint8)
    out = torch.empty(HQ * D, device="cuda", dtype=torch.bfloat16)
    ops.qwen35_online_attention_decode(*(to_dev(x, torch.bfloat16) for x in (qa, ka, va, ga)), out,
                                       cache, ws, shape, 3, 1, 1, plan=plan)
    torch.cuda.synchronize()
    keys = bf16(np.concatenate([past_k, ka[None]]))
    vals = bf16(np.concatenate([past_v, va[None]]))
    expect = orc.attention_core(qa[None], keys, vals, ga[None], ctx - 1)[0]
    assert_bf16_close(from_dev(out).reshape(HQ, D), expect, what=f"row merge ctx {ctx}")


def prefill_case(act, cdt, layout, T, hq, hkv, d, past, seed, q_scale=1.0):
    r = rng(seed)
    q, g = normal(r, T, hq, d), normal(r, T, hq, d)
    k, v = normal(r, T, hkv, d), normal(r, T, hkv, d)
    pk, pv = normal(r, past, hkv, d), normal(r, past, hkv, d)
    return q, g, k, v, pk, pv


def run_prefill(act, cdt, layout, T, hq, hkv, d, past, seed=0, inputs=None):
    q, g, k, v, pk, pv = inputs if inputs is not None else prefill_case(act, cdt, layout, T, hq,
                                                                         hkv, d, past, seed)
    if act == 3:
        q, g, k, v = (bf16(x) for x in (q, g, k, v))
    max_ctx = past + T
    cache_np = make_cache(pk, pv, layout, max_ctx, hkv, d)
    if cdt == 1:
        cache_np = bf16(cache_np)
    cache = to_dev(cache_np, CDT[cdt])
    out = torch.empty(T * hq * d, device="cuda", dtype=TDT[act])
    shape = S(T, hq, hkv, d, max_ctx, past)
    policy = ops.Qwen35AttentionLaunchPolicy(1, cdt, layout)
    ops.qwen35_causal_attention(to_dev(q, TDT[act]), to_dev(k, TDT[act]), to_dev(v, TDT[act]),
                                to_dev(g, TDT[act]), out, cache, None, shape, act, policy)
    torch.cuda.synchronize()
    keys = np.concatenate([pk, k]) if past else k
    vals = np.concatenate([pv, v]) if past else v
    if cdt == 1:
        keys, vals = bf16(keys), bf16(vals)
        if past:
            keys[:past], vals[:past] = bf16(pk), bf16(pv)
    expect = orc.attention_core(q, keys, vals, g, past)
    return from_dev(out).reshape(T, hq, d), expect, from_dev(cache), keys, vals


@pytest.mark.parametrize("T", [17, 128, 512])
@pytest.mark.parametrize("past", [0, 111])
def test_prefill_mfma_model_shape(gpu, T, past):
    # benchmark config 3 (PP128 / PP512) and the reference's {17,16,4,256,111} case.
    out, expect, cache, keys, vals = run_prefill(3, 1, 1, T, HQ, HKV, D, past, seed=T + past)
    assert_bf16_close(out, expect, what=f"prefill T={T} past={past}")
    ck, cv = read_cache(cache, 1, past + T, past + T)
    assert np.array_equal(ck, keys) and np.array_equal(cv, vals)


@pytest.mark.parametrize("past", [0, 1, 33])
@pytest.mark.parametrize("T", [1, 2, 7, 9, 15, 31, 33, 63, 65, 100, 255, 257])
def test_prefill_mfma_ragged_sweep(gpu, T, past):
    # Ragged query tiles (T not a multiple of 8), partial last key tiles (past + T not a
    # multiple of 32) and the diagonal mask at several offsets, on the bf16 MFMA path
    # (with past == 0 the kernel also writes the cache rows itself).
    out, expect, cache, keys, vals = run_prefill(3, 1, 1, T, HQ, HKV, D, past, seed=7 * T + past)
    assert np.isfinite(out).all()
    assert_bf16_close(out, expect, what=f"prefill T={T} past={past}")
    ck, cv = read_cache(cache, 1, past + T, past + T)
    assert np.array_equal(ck, keys) and np.array_equal(cv, vals)


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("act,cdt", [(1, 0), (1, 1), (3, 0), (3, 1)])
@pytest.mark.parametrize("case", [(4, 4, 2, 64, 0), (17, 16, 4, 256, 0), (17, 16, 4, 256, 111),
                                  (9, 6, 3, 40, 5)])
def test_prefill_layouts_dtypes_shapes(gpu, layout, act, cdt, case):
    # cpp/tests/qwen35_cuda_attention_test.cu:753-766
    T, hq, hkv, d, past = case
    out, expect, *_ = run_prefill(act, cdt, layout, T, hq, hkv, d, past, seed=sum(case))
    assert close_enough(out, expect), (layout, act, cdt, case)


@pytest.mark.parametrize("act,cdt,layout", [(3, 1, 1), (1, 0, 0)])
def test_prefill_causality(gpu, act, cdt, layout):
    # cpp/tests/qwen35_cuda_attention_test.cu:688-705: the last token's K/V
    # cannot change any earlier row (bit-identical).
    T = 40
    inputs = list(prefill_case(act, cdt, layout, T, HQ, HKV, D, 0, 5))
    a, *_ = run_prefill(act, cdt, layout, T, HQ, HKV, D, 0, inputs=inputs)
    inputs[2] = inputs[2].copy()
    inputs[3] = inputs[3].copy()
    inputs[2][-1] += 7.0
    inputs[3][-1] -= 9.0
    b, *_ = run_prefill(act, cdt, layout, T, HQ, HKV, D, 0, inputs=inputs)
    assert np.array_equal(a[:-1], b[:-1])
    assert not np.array_equal(a[-1], b[-1])


@pytest.mark.parametrize("act,cdt", [(3, 1), (1, 0)])
def test_prefill_adversarial_rescaling(gpu, act, cdt):
    # cpp/tests/qwen35_cuda_attention_test.cu:709-750: scores -80 .. +80.
    T, hq, hkv, d = 17, 4, 2, 64
    q = np.zeros((T, hq, d), np.float32)
    k = np.zeros((T, hkv, d), np.float32)
    v = np.zeros((T, hkv, d), np.float32)
    q[:, :, 0] = np.sqrt(d)
    for t in range(T):
        k[t, :, 0] = -80.0 + 10.0 * t
        for h in range(hkv):
            v[t, h] = 0.01 * (t + np.arange(d) + h)
    g = np.zeros((T, hq, d), np.float32)
    e = np.zeros((0, hkv, d), np.float32)
    out, expect, *_ = run_prefill(act, cdt, 1, T, hq, hkv, d, 0, inputs=(q, g, k, v, e, e))
    assert close_enough(out, expect)


@pytest.mark.parametrize("direction", [1, -1])
@pytest.mark.parametrize("past", [0, 64])
def test_prefill_mfma_adversarial_rescaling_model_shape(gpu, direction, past):
    # The -80 .. +80 score ramp of cpp/tests/qwen35_cuda_attention_test.cu:709-750 at the
    # model shape, so the bf16 MFMA kernel runs.  Ascending, every 32-key tile raises the
    # running max by ~14 log2 units (a rescale each tile, past the lazy threshold); descending,
    # the first keys dominate and later tiles underflow.  past > 0 reads keys from the cache.
    T = 512
    n = past + T
    ramp = (-80.0 + 160.0 * np.arange(n) / (n - 1)) * direction
    q = np.zeros((T, HQ, D), np.float32)
    q[:, :, 0] = 16.0  # score = q.k / 16 = k[0]
    kall = np.zeros((n, HKV, D), np.float32)
    kall[:, :, 0] = ramp[:, None]
    vall = np.zeros((n, HKV, D), np.float32)
    for h in range(HKV):
        vall[:, h] = 0.01 * (np.arange(n)[:, None] % 97 + np.arange(D)[None, :] + h)
    g = normal(rng(5), T, HQ, D)
    out, expect, *_ = run_prefill(3, 1, 1, T, HQ, HKV, D, past,
                                  inputs=(q, g, kall[past:], vall[past:], kall[:past], vall[:past]))
    assert np.isfinite(out).all()
    assert_bf16_close(out, expect, what=f"adversarial ramp dir {direction} past {past}")


def test_prefill_mfma_pp2048_vs_torch_fp32(gpu):
    # PP2048 (the size bench.py also times) against a torch fp32 causal attention on the
    # same bf16 inputs: the C oracle takes minutes at this size.  Same bf16 gates.
    T = 2048
    gen = torch.Generator(device="cuda").manual_seed(2048)
    rnd = lambda *shape: torch.randn(*shape, device="cuda", generator=gen).to(torch.bfloat16)
    q, g, k, v = rnd(T, HQ, D), rnd(T, HQ, D), rnd(T, HKV, D), rnd(T, HKV, D)
    cache = torch.zeros(2 * T * HKV * D, device="cuda", dtype=torch.bfloat16)
    out = torch.empty(T, HQ, D, device="cuda", dtype=torch.bfloat16)
    shape = S(T, HQ, HKV, D, T, 0)
    ops.qwen35_causal_attention(q, k, v, g, out, cache, None, shape, 3,
                                ops.Qwen35AttentionLaunchPolicy(1, 1, 1))
    torch.cuda.synchronize()
    qf = q.float().permute(1, 0, 2)                                # [16][T][256]
    kf = k.float().repeat_interleave(HQ // HKV, dim=1).permute(1, 0, 2)
    vf = v.float().repeat_interleave(HQ // HKV, dim=1).permute(1, 0, 2)
    s = torch.matmul(qf, kf.transpose(1, 2)) / 16.0
    s = s.masked_fill(torch.triu(torch.ones(T, T, device="cuda", dtype=torch.bool), 1), float("-inf"))
    ref = torch.matmul(torch.softmax(s, dim=-1), vf).permute(1, 0, 2) * torch.sigmoid(g.float())
    assert_bf16_close(from_dev(out), from_dev(ref), what="PP2048 vs torch fp32")


@pytest.mark.parametrize("act", [1, 2, 3])
@pytest.mark.parametrize("T,past", [(17, 0), (1, 40), (5, 7)])
def test_materialized_path(gpu, act, T, past):
    # cpp/kernels/qwen35_attention.cu:463-563 (f32 token-major cache + logits workspace)
    r = rng(T * 10 + act)
    hq, hkv, d = 16, 4, 256
    q, g = normal(r, T, hq, d), normal(r, T, hq, d)
    k, v = normal(r, T, hkv, d), normal(r, T, hkv, d)
    pk, pv = normal(r, past, hkv, d), normal(r, past, hkv, d)
    tdt = {1: torch.float32, 2: torch.float16, 3: torch.bfloat16}[act]
    enc = lambda a: from_dev(to_dev(a, tdt))
    q, g, k, v = map(enc, (q, g, k, v))
    max_ctx = past + T + 3
    cache = to_dev(make_cache(pk, pv, 0, max_ctx, hkv, d), torch.float32)
    shape = S(T, hq, hkv, d, max_ctx, past)
    policy = ops.Qwen35AttentionLaunchPolicy(0, 0, 0)
    ws = torch.empty(ops.qwen35_attention_workspace_bytes(shape, policy) // 4, device="cuda")
    out = torch.empty(T * hq * d, device="cuda", dtype=tdt)
    ops.qwen35_causal_attention(to_dev(q, tdt), to_dev(k, tdt), to_dev(v, tdt), to_dev(g, tdt), out,
                                cache, ws, shape, act, policy)
    torch.cuda.synchronize()
    keys = np.concatenate([pk, k])
    vals = np.concatenate([pv, v])
    expect = orc.attention_core(q, keys, vals, g, past)
    assert close_enough(from_dev(out).reshape(T, hq, d), expect)


@pytest.mark.parametrize("lengths,max_ctx", [
    ([1, 100, 511, 512, 513, 777, 2000, 4096], 4096),
    # 66 partitions: the merge takes a second chunk of partials.
    ([16641, 700], 16896),
])
def test_batched_ragged_decode(gpu, lengths, max_ctx):
    # benchmark config 4 at reduced length: per-sequence oracle, mixed policies.
    B = len(lengths)
    r = rng(77)
    per = 2 * max_ctx * HKV * D
    cache_np = np.zeros(B * per, np.float32)
    q, g = bf16(normal(r, B, HQ, D)), bf16(normal(r, B, HQ, D))
    k, v = bf16(normal(r, B, HKV, D)), bf16(normal(r, B, HKV, D))
    expects = []
    for b, L in enumerate(lengths):
        pk, pv = bf16(normal(r, L - 1, HKV, D)), bf16(normal(r, L - 1, HKV, D))
        cache_np[b * per:(b + 1) * per] = make_cache(pk, pv, 1, max_ctx)
        keys = np.concatenate([pk, k[b:b + 1]])
        vals = np.concatenate([pv, v[b:b + 1]])
        expects.append(orc.attention_core(q[b:b + 1], keys, vals, g[b:b + 1], L - 1)[0])
    cache = to_dev(cache_np, torch.bfloat16)
    lens = torch.tensor(lengths, device="cuda", dtype=torch.int32)
    stride = per * 2
    wsb = ops.qwen35_batched_decode_workspace_bytes(B, max_ctx, stride)
    ws = torch.empty(wsb, device="cuda", dtype=torch.uint8)
    out = torch.empty(B, HQ, D, device="cuda", dtype=torch.bfloat16)
    bt = lambda a: to_dev(a, torch.bfloat16)
    ops.qwen35_online_attention_decode_batched(bt(q), bt(k), bt(v), bt(g), out, cache, lens, ws,
                                               max_ctx, stride)
    torch.cuda.synchronize()
    got = from_dev(out)
    for b in range(B):
        assert_bf16_close(got[b], expects[b], what=f"batched seq {b} len {lengths[b]}")


@pytest.mark.parametrize("act", [1, 3])
def test_batched_out_of_range_lengths_report_nan(gpu, act):
    # Lengths 0, above max_ctx, and -1 (read as 0xFFFFFFFF) have no valid context: their
    # output rows become NaN and each is counted once; the valid sequences are unaffected
    # and no cache row of an invalid sequence is written.
    ops.consume_capacity_errors()
    lengths, max_ctx = [300, 0, 700, 1025, -1], 1024
    B = len(lengths)
    r = rng(99)
    per = 2 * max_ctx * HKV * D
    cache_np = np.zeros(B * per, np.float32)
    q, g = bf16(normal(r, B, HQ, D)), bf16(normal(r, B, HQ, D))
    k, v = bf16(normal(r, B, HKV, D)), bf16(normal(r, B, HKV, D))
    expects = {}
    for b, L in enumerate(lengths):
        if not 0 < L <= max_ctx:
            continue
        pk, pv = bf16(normal(r, L - 1, HKV, D)), bf16(normal(r, L - 1, HKV, D))
        cache_np[b * per:(b + 1) * per] = make_cache(pk, pv, 1, max_ctx)
        expects[b] = orc.attention_core(q[b:b + 1], np.concatenate([pk, k[b:b + 1]]),
                                        np.concatenate([pv, v[b:b + 1]]), g[b:b + 1], L - 1)[0]
    cache = to_dev(cache_np, torch.bfloat16)
    lens = torch.tensor(lengths, device="cuda", dtype=torch.int32)
    ws = torch.empty(ops.qwen35_batched_decode_workspace_bytes(B, max_ctx, per * 2), device="cuda",
                     dtype=torch.uint8)
    out = torch.zeros(B, HQ, D, device="cuda", dtype=TDT[act])
    t = lambda a: to_dev(a, TDT[act])
    ops.qwen35_online_attention_decode_batched(t(q), t(k), t(v), t(g), out, cache, lens, ws,
                                               max_ctx, per * 2, activation_dtype=act)
    torch.cuda.synchronize()
    got = from_dev(out)
    assert ops.consume_capacity_errors() == 3
    cache_out = from_dev(cache)
    for b, L in enumerate(lengths):
        if b in expects:
            assert close_enough(got[b], expects[b]), f"seq {b}"
        else:
            assert np.isnan(got[b]).all(), f"seq {b}"
            assert not cache_out[b * per:(b + 1) * per].any(), f"seq {b} cache written"


def test_batched_ragged_decode_cfg4_full_size(gpu):
    # benchmark config 4 at full size: 32 sequences with lengths U{1..32768} from the bench's
    # seed, max_ctx 32768, bf16 head-major caches (4.3 GB).  Every sequence is checked against
    # the single-sequence decode entry point (pinned to the oracle by the tests above) on the
    # same, already appended cache; the shortest, the longest and two others also against the
    # C oracle directly.
    lengths = np.random.default_rng(0x5241465449 + 4).integers(1, 32769, size=32)
    B, max_ctx = len(lengths), 32768
    per = 2 * HKV * max_ctx * D
    gen = torch.Generator(device="cuda").manual_seed(44)
    cache = torch.empty(B * per, device="cuda", dtype=torch.bfloat16)
    for b in range(B):
        cache[b * per:(b + 1) * per].copy_(torch.randn(per, device="cuda", generator=gen))
    q, g = (torch.randn(B, HQ, D, device="cuda", generator=gen).to(torch.bfloat16) for _ in range(2))
    k, v = (torch.randn(B, HKV, D, device="cuda", generator=gen).to(torch.bfloat16) for _ in range(2))
    lens = torch.tensor(lengths, device="cuda", dtype=torch.int32)
    ws = torch.empty(ops.qwen35_batched_decode_workspace_bytes(B, max_ctx, per * 2), device="cuda",
                     dtype=torch.uint8)
    out = torch.empty(B, HQ, D, device="cuda", dtype=torch.bfloat16)
    ops.qwen35_online_attention_decode_batched(q, k, v, g, out, cache, lens, ws, max_ctx, per * 2)
    torch.cuda.synchronize()
    got = from_dev(out)
    for b in range(B):
        L = int(lengths[b])
        shape = S(1, HQ, HKV, D, max_ctx, L - 1)
        plan = ops.qwen35_online_decode_plan(shape, ops.AUTO, max_ctx)
        nbytes = ops.qwen35_online_decode_workspace_layout(shape, plan[0])[4]
        ws1 = torch.empty(nbytes, device="cuda", dtype=torch.uint8) if nbytes else None
        one = torch.empty(HQ * D, device="cuda", dtype=torch.bfloat16)
        ops.qwen35_online_attention_decode(q[b].flatten(), k[b].flatten(), v[b].flatten(), g[b].flatten(),
                                           one, cache[b * per:(b + 1) * per], ws1, shape, 3, 1, 1,
                                           plan=plan)
        torch.cuda.synchronize()
        assert_bf16_close(got[b], from_dev(one).reshape(HQ, D), what=f"cfg4 seq {b} len {L} vs single", both_bf16=True)
    order = np.argsort(lengths)
    for b in {int(order[0]), int(order[-1]), int(order[len(order) // 3]), int(order[2 * len(order) // 3])}:
        L = int(lengths[b])
        c = from_dev(cache[b * per:(b + 1) * per]).reshape(2, HKV, max_ctx, D)[:, :, :L]
        keys, vals = c[0].transpose(1, 0, 2), c[1].transpose(1, 0, 2)
        expect = orc.attention_core(from_dev(q[b])[None], keys, vals, from_dev(g[b])[None], L - 1)[0]
        assert_bf16_close(got[b], expect, what=f"cfg4 seq {b} len {L} vs oracle")
