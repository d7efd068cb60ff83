"""Benchmark of the gfx950 attention / gated-delta hot path.

A "step" is one split-K GQA decode call at context 4096 (benchmark config 2:
16 query / 4 KV heads, head_dim 256, BF16 head-major cache, 256-token
partitions + fp32 LSE merge, ~1% of K rows x8), with inputs resident in HBM.
Every timed call reads a cache of its own, and the L2 / 256 MB MALL are
flushed (a 1 GiB read-modify-write) between the warm replay and the timed one,
so each call streams its K/V from HBM.  ``value`` is that call's algorithmic
HBM throughput (KV bytes + q/gate/out bytes per call / event-timed call time).

The other benchmark configs are reported under ``configs``:
  cfg1 single-block decode ctx 512 (cold), cfg2 ctx 16384 and the
  device-position (graph-replay) form of ctx 4096, cfg3 PP128 / PP512 prefill
  (hot: the same inputs every call; cold: a fresh input set per call after a
  flush), cfg4 batched ragged decode x32, cfg5 gated delta (the recurrence
  core and the full qwen35_gated_delta entry, prefill T=512 and decode
  steps, hot and cold), and the PP512 attention producers.
``roofline`` prices the dominant kernel (the split-K partition kernel, cold)
timed alone with HIP events on its own stream.  ``cpu_baseline`` times the CPU
oracle (the restated cpp/reference path) on the host cores, one thread and
one thread per head, for every config, on bounded samples.

    python bench.py [--gpus 1] [--steps 50] [--warmup 5] [--no-cpu] [--quick]
    python bench.py --counters     # eager launches for rocprofv3 --pmc passes

``--counters`` launches the ctx-4096 partition kernel eagerly (no graph) 20
times on 20 distinct caches, then copies a 64 MiB buffer 20 times with a
plain device-to-device copy kernel of known size, so that FETCH_SIZE and
WRITE_SIZE per dispatch can be scaled by what the counters read for the copy;
then 20 PP512 prefill kernels, 10 delta prefills (T=512) and 20 delta decode
steps, for their traffic and MFMA counters.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import ctypes
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, published
BF16_PEAK_TFLOPS = 2500.0    # MI355X dense bf16 MFMA, published
HQ, HKV, D = 16, 4, 256
METRIC = json.loads((ROOT / "BASELINE.json").read_text())["metric"]
SEED = 0x5241465449
CACHE_POOL_BYTES = 16 << 30  # at most this much distinct cache per decode config


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def decode_bytes(ctx):
    # K and V rows read once per call + q, gate read and out written (bf16).
    return 2 * HKV * ctx * D * 2 + 3 * HQ * D * 2


def prefill_flops(T):
    return 8192 * T * (T + 1)


def delta_prefill_bytes(T):
    # q, k (16 heads) and v, out (32 heads) in bf16, beta and log-decay fp32,
    # the fp32 state read and written once.
    return T * (16 * 128 * 2 * 2 + 32 * 128 * 2 * 2 + 32 * 8) + 2 * 32 * 128 * 128 * 4


def delta_entry_bytes(T):
    # qwen35_gated_delta: the packed input row (12,352 bf16) read, the output
    # row (4,096 bf16) written, the conv state [8192][3] and the recurrent
    # state read and written.
    return T * (12352 + 4096) * 2 + 2 * (8192 * 3 * 4 + 32 * 128 * 128 * 4)


def cpu_description():
    model = "unknown"
    ids = {}
    try:
        for line in open("/proc/cpuinfo"):
            key, _, val = line.partition(":")
            key = key.strip()
            if key == "model name" and model == "unknown":
                model = val.strip()
            elif key in ("cpu family", "model", "stepping") and key not in ids:
                ids[key] = val.strip()
            elif not line.strip() and ids:
                break  # the first processor's block is enough
    except OSError:
        pass
    if ids:  # a virtualised host may report only the product line as its name
        model += " (" + ", ".join(f"{k} {v}" for k, v in ids.items()) + ")"
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count()
    return model, avail


# ------------------------------------------------------------------ CPU leg
def cpu_baselines(threads):
    """The oracle (plain-C restatement of cpp/reference/qwen35.cpp, -O3) on the
    host: one thread running the reference's loop over all heads, and
    `threads` threads each running one head's share (the C calls release the
    GIL).  Each figure is timed on a bounded sample; returns per-config dicts."""
    import numpy as np

    from oracle import pyoracle as orc

    r = np.random.default_rng(SEED)
    bf = orc.bf16_round
    pool = cf.ThreadPoolExecutor(threads)

    def clock(fn, budget, max_reps):
        n, t0 = 0, time.perf_counter()
        while n < max_reps and (n == 0 or time.perf_counter() - t0 < budget):
            fn()
            n += 1
        return (time.perf_counter() - t0) / n, n

    def attn_inputs(T, past):
        q = bf(r.standard_normal((T, HQ, D)).astype(np.float32))
        g = bf(r.standard_normal((T, HQ, D)).astype(np.float32))
        k = bf(r.standard_normal((past + T, HKV, D)).astype(np.float32))
        v = bf(r.standard_normal((past + T, HKV, D)).astype(np.float32))
        return q, k, v, g

    def attn_heads(q, k, v, g, past):
        # one task per query head: (q, gate) of that head and its KV head's rows
        ks = [np.ascontiguousarray(k[:, j:j + 1]) for j in range(HKV)]
        vs = [np.ascontiguousarray(v[:, j:j + 1]) for j in range(HKV)]
        qs = [np.ascontiguousarray(q[:, h:h + 1]) for h in range(HQ)]
        gs = [np.ascontiguousarray(g[:, h:h + 1]) for h in range(HQ)]
        grp = HQ // HKV
        return lambda: list(pool.map(
            lambda h: orc.attention_core(qs[h], ks[h // grp], vs[h // grp], gs[h], past), range(HQ)))

    out = {}

    def attn_case(name, T, past, budget, max_reps, work, unit):
        q, k, v, g = attn_inputs(T, past)
        s1, n1 = clock(lambda: orc.attention_core(q, k, v, g, past), budget, max_reps)
        sm, nm = clock(attn_heads(q, k, v, g, past), budget / 2, max_reps)
        scale = 1e9 if unit == "GB/s" else 1e12
        out[name] = {"unit": unit, "value_1_thread": work / s1 / scale, "ms_per_call_1_thread": s1 * 1e3,
                     "calls_1_thread": n1, "value_threads": work / sm / scale,
                     "ms_per_call_threads": sm * 1e3, "calls_threads": nm, "threads": threads}
        log(f"cpu {name}: {s1 * 1e3:.1f} ms/call (1 thread), {sm * 1e3:.1f} ms/call ({threads} threads)")

    attn_case("cfg1_decode_ctx512", 1, 511, 2.0, 400, decode_bytes(512), "GB/s")
    attn_case("cfg2_decode_ctx4096", 1, 4095, 3.0, 200, decode_bytes(4096), "GB/s")
    attn_case("cfg2_decode_ctx16384", 1, 16383, 3.0, 50, decode_bytes(16384), "GB/s")
    attn_case("cfg3_prefill_pp128", 128, 0, 2.0, 20, prefill_flops(128), "TFLOP/s")
    attn_case("cfg3_prefill_pp512", 512, 0, 3.0, 3, prefill_flops(512), "TFLOP/s")

    # cfg4: the first 4 sequences of the benchmark's length draw, decoded one
    # after another (1 thread) and as (sequence, head) tasks (threads).
    lengths = [int(x) for x in np.random.default_rng(SEED + 4).integers(1, 32769, size=32)][:4]
    seqs = [attn_inputs(1, L - 1) for L in lengths]
    sample_bytes = sum(decode_bytes(L) for L in lengths)
    t0 = time.perf_counter()
    for (q, k, v, g), L in zip(seqs, lengths):
        orc.attention_core(q, k, v, g, L - 1)
    s1 = time.perf_counter() - t0
    fns = [attn_heads(q, k, v, g, L - 1) for (q, k, v, g), L in zip(seqs, lengths)]
    t0 = time.perf_counter()
    for fn in fns:
        fn()
    sm = time.perf_counter() - t0
    out["cfg4_batched_ragged_decode_x32"] = {
        "unit": "GB/s", "value_1_thread": sample_bytes / s1 / 1e9, "value_threads": sample_bytes / sm / 1e9,
        "threads": threads, "sample": f"sequences of length {lengths} (the first 4 of the benchmark draw)",
        "ms_sample_1_thread": s1 * 1e3, "ms_sample_threads": sm * 1e3}
    log(f"cpu cfg4 sample: {s1 * 1e3:.0f} ms (1 thread), {sm * 1e3:.0f} ms ({threads} threads)")

    # cfg5: the token-sequential recurrence (cpp/reference/qwen35.cpp:459-549)
    T = 512
    qd = r.standard_normal((T, 16, 128)); kd = r.standard_normal((T, 16, 128))
    qd = bf(qd / np.linalg.norm(qd, axis=-1, keepdims=True))
    kd = bf(kd / np.linalg.norm(kd, axis=-1, keepdims=True))
    vd = bf(r.standard_normal((T, 32, 128)))
    beta = (1 / (1 + np.exp(-r.standard_normal((T, 32))))).astype(np.float32)
    lg = (-np.log1p(np.exp(r.standard_normal((T, 32))))).astype(np.float32)
    s0 = np.zeros((32, 128, 128), np.float32)
    sc = 128 ** -0.5
    s1, n1 = clock(lambda: orc.delta_core(qd, kd, vd, beta, lg, sc, s0), 3.0, 3)
    per_head = [tuple(np.ascontiguousarray(x) for x in (qd[:, h % 16:h % 16 + 1], kd[:, h % 16:h % 16 + 1],
                                                        vd[:, h:h + 1], beta[:, h:h + 1], lg[:, h:h + 1],
                                                        s0[h:h + 1])) for h in range(32)]
    sm, nm = clock(lambda: list(pool.map(lambda a: orc.delta_core(*a[:5], sc, a[5]), per_head)), 2.0, 3)
    d1, _ = clock(lambda: orc.delta_core(qd[:1], kd[:1], vd[:1], beta[:1], lg[:1], sc, s0), 1.0, 200)
    flop = 6 * 128 * 128 * 32 * T
    out["cfg5_gated_delta"] = {
        "unit": "GFLOP/s", "prefill_T512_ms_1_thread": s1 * 1e3, "prefill_T512_ms_threads": sm * 1e3,
        "value_1_thread": flop / s1 / 1e9, "value_threads": flop / sm / 1e9, "threads": threads,
        "decode_step_ms_1_thread": d1 * 1e3}
    log(f"cpu cfg5: prefill {s1 * 1e3:.0f} ms (1 thread), {sm * 1e3:.0f} ms ({threads} threads), "
        f"step {d1 * 1e3:.2f} ms")
    pool.shutdown()
    return out


# ------------------------------------------------------------------ GPU leg
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--quick", action="store_true", help="headline config only")
    ap.add_argument("--counters", action="store_true",
                    help="eager partition-kernel and copy launches for counter passes")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the path would shard over KV heads and value heads); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from raftinfer_amd import _lib, ops

    lib = _lib.load()
    vp = lambda t: ctypes.c_void_p(t.data_ptr())
    torch.manual_seed(SEED)
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    ev = lambda: torch.cuda.Event(enable_timing=True)
    flush_buf = torch.zeros(1 << 28, device="cuda", dtype=torch.float32)  # 1 GiB

    def flush():
        flush_buf.add_(1.0)  # 1 GiB read + 1 GiB written: evicts L2 and the MALL

    def timed(fn, steps, warmup, cold):
        """Mean GPU time per call (us).  The `steps` calls are captured into
        one HIP graph (how a serving loop replays decode), replayed once warm,
        then (cold) the caches are flushed, and the replay is bracketed by
        events on the launch stream, so host dispatch cost is excluded."""
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(steps):
                fn(i)
        graph.replay()
        if cold:
            flush()
        a, b = ev(), ev()
        a.record(stream)
        graph.replay()
        b.record(stream)
        torch.cuda.synchronize()
        del graph
        return a.elapsed_time(b) / steps * 1e3

    def rand_bf16(*shape):
        return torch.randn(*shape, device="cuda", dtype=torch.float32).to(torch.bfloat16)

    results = {}

    # ---------------------------------------------------------- config 2
    def make_caches(ctx, n, heavy=True):
        caches = torch.empty(n, 2 * HKV * ctx * D, device="cuda", dtype=torch.bfloat16)
        for i in range(n):
            caches[i].copy_(rand_bf16(2 * HKV * ctx * D))
            if heavy:
                rows = torch.rand(ctx, device="cuda") < 0.01  # ~1% of K rows x8
                kview = caches[i][:HKV * ctx * D].view(HKV, ctx, D)
                kview[:, rows] *= 8
        return caches

    def n_caches(ctx, steps):
        return max(1, min(steps, CACHE_POOL_BYTES // (2 * HKV * ctx * D * 2)))

    def split_decode(ctx, counters=False):
        ncache = 20 if counters else n_caches(ctx, args.steps)
        shape = ops.Qwen35AttentionShape(1, HQ, HKV, D, ctx, ctx - 1)
        caches = make_caches(ctx, ncache)
        q, k, v, g = rand_bf16(HQ * D), rand_bf16(HKV * D), rand_bf16(HKV * D), rand_bf16(HQ * D)
        out = torch.empty(HQ * D, device="cuda", dtype=torch.bfloat16)
        plan = ops.qwen35_online_decode_plan(shape, ops.AUTO, ctx)
        ws = torch.empty(ops.qwen35_online_decode_workspace_layout(shape, plan[0])[4],
                         device="cuda", dtype=torch.uint8)
        call = lambda i: ops.qwen35_online_attention_decode(
            q, k, v, g, out, caches[i % ncache], ws, shape, ops.DTYPE_BF16, ops.CACHE_BF16,
            ops.HEAD_MAJOR, plan=plan, stream=stream)
        cplan = _lib.DecodePlan(*plan)
        nbytes = caches[0].numel() * 2

        def part(i):
            _lib.check(lib.raftinfer_amd_online_attention_decode_partition_only(
                vp(q), vp(k), vp(v), vp(g), vp(out), vp(caches[i % ncache]), nbytes, vp(ws),
                ws.numel(), shape.c(), ops.DTYPE_BF16, ops.CACHE_BF16, ops.HEAD_MAJOR, cplan,
                None, ctypes.c_void_p(stream.cuda_stream)))
        if counters:
            for i in range(ncache):
                part(i)
            torch.cuda.synchronize()
            return None
        res = {"us": timed(call, args.steps, args.warmup, cold=True),
               "kernel_us": timed(part, args.steps, args.warmup, cold=True),
               "caches": ncache}
        if ctx == 4096:
            # Device-position form, as a serving loop replays it from a graph
            # (cpp/execution/qwen35_executor.cu:755-765): the plan of the 4096
            # bucket, the position read on the device, every kernel of the plan
            # enqueued (the single-block kernel exits early).
            pos = torch.tensor([ctx - 1], device="cuda", dtype=torch.int32)
            dshape = ops.Qwen35AttentionShape(1, HQ, HKV, D, ctx, 0)
            dplan = ops.qwen35_online_decode_plan(dshape, ops.AUTO, ctx)
            res["device_position_us"] = timed(lambda i: ops.qwen35_online_attention_decode(
                q, k, v, g, out, caches[i % ncache], ws, dshape, ops.DTYPE_BF16, ops.CACHE_BF16,
                ops.HEAD_MAJOR, plan=dplan, device_position=pos, stream=stream),
                args.steps, args.warmup, cold=True)
        del caches
        torch.cuda.empty_cache()
        return res

    if args.counters:
        split_decode(4096, counters=True)
        # The ctx 4096 split-K call in its device-position form, 20 times with a
        # valid position and 20 times with position == max_ctx, where both of
        # its kernels return right after reading the position: the second set
        # is the merge kernel's fixed fetch (code, arguments, position) with the
        # same grid and arguments and no partial read.
        mshape = ops.Qwen35AttentionShape(1, HQ, HKV, D, 4096, 0)
        mplan = ops.qwen35_online_decode_plan(mshape, ops.AUTO, 4096)
        mws = torch.empty(ops.qwen35_online_decode_workspace_layout(mshape, mplan[0])[4],
                          device="cuda", dtype=torch.uint8)
        mcache = make_caches(4096, 1)[0]
        mq, mk, mv, mg = rand_bf16(HQ * D), rand_bf16(HKV * D), rand_bf16(HKV * D), rand_bf16(HQ * D)
        mout = torch.empty(HQ * D, device="cuda", dtype=torch.bfloat16)
        for position in (4095, 4096):
            mpos = torch.tensor([position], device="cuda", dtype=torch.int32)
            for _ in range(20):
                ops.qwen35_online_attention_decode(mq, mk, mv, mg, mout, mcache, mws, mshape,
                                                   ops.DTYPE_BF16, ops.CACHE_BF16, ops.HEAD_MAJOR,
                                                   plan=mplan, device_position=mpos, stream=stream)
        torch.cuda.synchronize()
        del mcache
        src = torch.empty(64 << 20, device="cuda", dtype=torch.uint8)
        dst = torch.empty_like(src)
        src.fill_(1)
        torch.cuda.synchronize()
        for _ in range(20):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        # PP512 prefill (kernel with the fused append) and the cfg5 delta
        # prefill / decode step, launched eagerly for per-dispatch counters.
        T = 512
        shape = ops.Qwen35AttentionShape(T, HQ, HKV, D, T, 0)
        qp, gp = rand_bf16(T * HQ * D), rand_bf16(T * HQ * D)
        kp, vp_ = rand_bf16(T * HKV * D), rand_bf16(T * HKV * D)
        cache = torch.zeros(2 * T * HKV * D, device="cuda", dtype=torch.bfloat16)
        outp = torch.empty(T * HQ * D, device="cuda", dtype=torch.bfloat16)
        for _ in range(20):
            _lib.check(lib.raftinfer_amd_online_attention_prefill_kernel_only(
                *[vp(t) for t in (qp, kp, vp_, gp, outp, cache)],
                cache.numel() * 2, shape.c(), ops.DTYPE_BF16, ops.CACHE_BF16, ops.HEAD_MAJOR,
                ctypes.c_void_p(stream.cuda_stream)))
        q5 = torch.nn.functional.normalize(torch.randn(T, 16, 128, device="cuda"), dim=-1).to(torch.bfloat16)
        k5 = torch.nn.functional.normalize(torch.randn(T, 16, 128, device="cuda"), dim=-1).to(torch.bfloat16)
        v5 = rand_bf16(T, 32, 128)
        beta = torch.sigmoid(torch.randn(T, 32, device="cuda"))
        lg = -torch.nn.functional.softplus(torch.randn(T, 32, device="cuda"))
        st = torch.zeros(32, 128, 128, device="cuda")
        o5 = torch.empty(T, 32, 128, device="cuda", dtype=torch.bfloat16)
        ws5 = torch.empty(ops.qwen35_gated_delta_core_workspace_bytes(T, 16, 32, 128, 128),
                          device="cuda", dtype=torch.uint8)
        for _ in range(10):
            ops.qwen35_gated_delta_core(q5, k5, v5, beta, lg, 128 ** -0.5, st, o5, ws5, True,
                                        stream=stream)
        for i in range(20):
            ops.qwen35_gated_delta_core(q5[i:i + 1], k5[i:i + 1], v5[i:i + 1], beta[i:i + 1],
                                        lg[i:i + 1], 128 ** -0.5, st, o5[:1], None, False,
                                        stream=stream)
        torch.cuda.synchronize()
        log("counters run: 20 partition launches (ctx 4096), 20 + 20 device-position decode calls "
            "(valid, then past the maximum context), 20 copies of 64 MiB, 20 PP512 "
            "prefill kernels, 10 delta prefills (T=512), 20 delta decode steps")
        return

    r4096 = split_decode(4096)
    us4096, kus4096 = r4096["us"], r4096["kernel_us"]
    log(f"cfg2 ctx4096: {us4096:.2f} us/call, partition kernel {kus4096:.2f} us, "
        f"device-position {r4096['device_position_us']:.2f} us ({r4096['caches']} caches)")
    results["cfg2_split_k_decode_ctx4096"] = {
        "us_per_call": us4096, "GB_per_s": decode_bytes(4096) / us4096 / 1e3,
        "partition_kernel_us": kus4096, "bytes_per_call": decode_bytes(4096),
        "device_position_graph_us_per_call": r4096["device_position_us"],
        "device_position_GB_per_s": decode_bytes(4096) / r4096["device_position_us"] / 1e3,
        "distinct_caches": r4096["caches"], "cold": True}

    if not args.quick:
        r16k = split_decode(16384)
        log(f"cfg2 ctx16384: {r16k['us']:.2f} us/call, partition kernel {r16k['kernel_us']:.2f} us")
        results["cfg2_split_k_decode_ctx16384"] = {
            "us_per_call": r16k["us"], "GB_per_s": decode_bytes(16384) / r16k["us"] / 1e3,
            "partition_kernel_us": r16k["kernel_us"], "bytes_per_call": decode_bytes(16384),
            "distinct_caches": r16k["caches"], "cold": True}

        # ------------------------------------------------------ config 1
        ctx = 512
        ncache = n_caches(ctx, args.steps)
        shape = ops.Qwen35AttentionShape(1, HQ, HKV, D, ctx, ctx - 1)
        caches = make_caches(ctx, ncache, heavy=False)
        q, k, v, g = rand_bf16(HQ * D), rand_bf16(HKV * D), rand_bf16(HKV * D), rand_bf16(HQ * D)
        out = torch.empty(HQ * D, device="cuda", dtype=torch.bfloat16)
        call1 = lambda i: ops.qwen35_online_attention_decode(
            q, k, v, g, out, caches[i % ncache], None, shape, ops.DTYPE_BF16, ops.CACHE_BF16,
            ops.HEAD_MAJOR, stream=stream)
        us = timed(call1, args.steps, args.warmup, cold=True)
        us_hot = timed(lambda i: call1(0), args.steps, args.warmup, cold=False)
        results["cfg1_single_block_decode_ctx512"] = {
            "us_per_call": us, "GB_per_s": decode_bytes(512) / us / 1e3, "distinct_caches": ncache,
            "cold": True, "hot_us_per_call": us_hot}
        log(f"cfg1 ctx512: {us:.2f} us/call cold, {us_hot:.2f} us hot")
        del caches

        # ------------------------------------------------------ config 3
        for T in (128, 512):
            shape = ops.Qwen35AttentionShape(T, HQ, HKV, D, T, 0)
            nset = max(1, min(args.steps, 64))
            sets = [dict(q=rand_bf16(T * HQ * D), g=rand_bf16(T * HQ * D), k=rand_bf16(T * HKV * D),
                         v=rand_bf16(T * HKV * D),
                         cache=torch.zeros(2 * T * HKV * D, device="cuda", dtype=torch.bfloat16),
                         out=torch.empty(T * HQ * D, device="cuda", dtype=torch.bfloat16))
                    for _ in range(nset)]
            pol = ops.Qwen35AttentionLaunchPolicy()

            def full(i, s=sets):
                x = s[i % nset]
                ops.qwen35_causal_attention(x["q"], x["k"], x["v"], x["g"], x["out"], x["cache"], None,
                                            shape, ops.DTYPE_BF16, pol, stream=stream)

            def kern(i, s=sets):
                x = s[i % nset]
                _lib.check(lib.raftinfer_amd_online_attention_prefill_kernel_only(
                    *[vp(x[n]) for n in ("q", "k", "v", "g", "out", "cache")],
                    x["cache"].numel() * 2, shape.c(), ops.DTYPE_BF16, ops.CACHE_BF16,
                    ops.HEAD_MAJOR, ctypes.c_void_p(stream.cuda_stream)))
            us = timed(lambda i: full(0), args.steps, args.warmup, cold=False)
            kus = timed(lambda i: kern(0), args.steps, args.warmup, cold=False)
            us_c = timed(full, args.steps, args.warmup, cold=True)
            kus_c = timed(kern, args.steps, args.warmup, cold=True)
            flops = prefill_flops(T)
            results[f"cfg3_prefill_pp{T}"] = {
                "us_per_call": us, "TFLOP_per_s": flops / us / 1e6, "kernel_us": kus,
                "kernel_TFLOP_per_s": flops / kus / 1e6, "flop": flops,
                "mfma_frac": flops / kus / 1e6 / BF16_PEAK_TFLOPS,
                "cold_us_per_call": us_c, "cold_TFLOP_per_s": flops / us_c / 1e6,
                "cold_kernel_us": kus_c, "cold_input_sets": nset}
            log(f"cfg3 PP{T}: {us:.2f} us/call, kernel {kus:.2f} us ({flops / kus / 1e6:.1f} TFLOP/s); "
                f"cold {us_c:.2f} / kernel {kus_c:.2f} us")
            del sets

        # ------------------------------------------------------ config 4
        rng = np.random.default_rng(SEED + 4)
        lengths = rng.integers(1, 32769, size=32)
        max_ctx = 32768
        per = 2 * HKV * max_ctx * D
        cache = torch.empty(32 * per, device="cuda", dtype=torch.bfloat16)
        for b in range(32):
            cache[b * per:(b + 1) * per].copy_(rand_bf16(per))
        lens = torch.tensor(lengths, device="cuda", dtype=torch.int32)
        qb, gb = rand_bf16(32, HQ, D), rand_bf16(32, HQ, D)
        kb, vb = rand_bf16(32, HKV, D), rand_bf16(32, HKV, D)
        outb = torch.empty(32, HQ, D, device="cuda", dtype=torch.bfloat16)
        wsb = torch.empty(ops.qwen35_batched_decode_workspace_bytes(32, max_ctx, per * 2),
                          device="cuda", dtype=torch.uint8)
        us = timed(lambda i: ops.qwen35_online_attention_decode_batched(
            qb, kb, vb, gb, outb, cache, lens, wsb, max_ctx, per * 2, stream=stream),
            max(5, args.steps // 5), 2, cold=True)
        kv_bytes = int(sum(4096 * int(L) for L in lengths)) + 32 * 24576
        results["cfg4_batched_ragged_decode_x32"] = {
            "us_per_call": us, "GB_per_s": kv_bytes / us / 1e3, "bytes_per_call": kv_bytes,
            "lengths_seed": SEED + 4}
        log(f"cfg4 batched: {us:.2f} us/call, {kv_bytes / us / 1e3:.0f} GB/s")
        del cache
        torch.cuda.empty_cache()

        # ------------------------------------------------------ config 5
        T = 512
        nset = max(1, min(args.steps, 64))

        def core_set(T):
            return dict(
                q=torch.nn.functional.normalize(torch.randn(T, 16, 128, device="cuda"), dim=-1).to(torch.bfloat16),
                k=torch.nn.functional.normalize(torch.randn(T, 16, 128, device="cuda"), dim=-1).to(torch.bfloat16),
                v=rand_bf16(T, 32, 128), beta=torch.sigmoid(torch.randn(T, 32, device="cuda")),
                lg=-torch.nn.functional.softplus(torch.randn(T, 32, device="cuda")),
                st=torch.zeros(32, 128, 128, device="cuda"),
                o=torch.empty(T, 32, 128, device="cuda", dtype=torch.bfloat16))
        csets = [core_set(T) for _ in range(nset)]
        ws5 = torch.empty(ops.qwen35_gated_delta_core_workspace_bytes(T, 16, 32, 128, 128),
                          device="cuda", dtype=torch.uint8)

        def core_prefill(i):
            x = csets[i % nset]
            ops.qwen35_gated_delta_core(x["q"], x["k"], x["v"], x["beta"], x["lg"], 128 ** -0.5, x["st"],
                                        x["o"], ws5, True, stream=stream)

        def core_step(i, sets=csets):
            x = sets[i % len(sets)]
            t = i % T
            ops.qwen35_gated_delta_core(x["q"][t:t + 1], x["k"][t:t + 1], x["v"][t:t + 1],
                                        x["beta"][t:t + 1], x["lg"][t:t + 1], 128 ** -0.5, x["st"],
                                        x["o"][:1], None, False, stream=stream)
        us_p = timed(lambda i: core_prefill(0), args.steps, args.warmup, cold=False)
        us_pc = timed(core_prefill, args.steps, args.warmup, cold=True)
        us_d = timed(lambda i: core_step(i, csets[:1]), max(args.steps, 32), args.warmup, cold=False)
        us_dc = timed(core_step, max(args.steps, 32), args.warmup, cold=True)
        del csets

        # the full drop-in entry (conv + SiLU + l2norm + recurrence + out-norm)
        dshape = ops.GatedDeltaShape(T, 4096, 16, 32, 128, 128, 4, 1e-6)
        dshape1 = ops.GatedDeltaShape(1, 4096, 16, 32, 128, 128, 4, 1e-6)
        wsf = torch.empty(ops.qwen35_gated_delta_workspace_bytes(dshape), device="cuda", dtype=torch.uint8)
        cw = rand_bf16(8192 * 4) * 0.3
        a_ = -torch.exp(torch.randn(32, device="cuda") * 0.5).to(torch.bfloat16)
        dtb, nw = rand_bf16(32), rand_bf16(128)
        fsets = [dict(inp=rand_bf16(T * 12352), out=torch.empty(T * 4096, device="cuda", dtype=torch.bfloat16),
                      conv=torch.zeros(8192 * 3, device="cuda"), rec=torch.zeros(32 * 128 * 128, device="cuda"))
                 for _ in range(nset)]

        def entry(i, tokens, sets=fsets):
            x = sets[i % len(sets)]
            sh = dshape if tokens == T else dshape1
            t = (i % T) if tokens == 1 else 0
            ops.qwen35_gated_delta(x["inp"][t * 12352:(t + tokens) * 12352], cw, a_, dtb, nw,
                                   x["out"][:tokens * 4096], x["conv"], x["rec"], wsf, sh, ops.DTYPE_BF16,
                                   ops.DTYPE_BF16, stream=stream)
        ue_p = timed(lambda i: entry(0, T), args.steps, args.warmup, cold=False)
        ue_pc = timed(lambda i: entry(i, T), args.steps, args.warmup, cold=True)
        ue_d = timed(lambda i: entry(i, 1, fsets[:1]), max(args.steps, 32), args.warmup, cold=False)
        ue_dc = timed(lambda i: entry(i, 1), max(args.steps, 32), args.warmup, cold=True)
        del fsets
        pbytes = delta_prefill_bytes(T)
        dbytes = 2 * 32 * 128 * 128 * 4 + (16 * 128 * 2 * 2 + 32 * 128 * 2 * 2 + 32 * 8)
        results["cfg5_gated_delta"] = {
            "prefill_T512_us": us_p, "prefill_GB_per_s": pbytes / us_p / 1e3,
            "prefill_GFLOP_per_s": 6 * 128 * 128 * 32 * T / us_p / 1e3,
            "prefill_T512_cold_us": us_pc,
            "decode_step_us": us_d, "decode_GB_per_s": dbytes / us_d / 1e3,
            "decode_step_cold_us": us_dc, "decode_cold_GB_per_s": dbytes / us_dc / 1e3,
            "entry_prefill_T512_us": ue_p, "entry_prefill_T512_cold_us": ue_pc,
            "entry_prefill_GB_per_s": delta_entry_bytes(T) / ue_p / 1e3,
            "entry_decode_step_us": ue_d, "entry_decode_step_cold_us": ue_dc,
            "entry_decode_GB_per_s": delta_entry_bytes(1) / ue_d / 1e3,
            "cold_sets": nset}
        log(f"cfg5 delta core: prefill {us_p:.1f} us (cold {us_pc:.1f}), step {us_d:.2f} us "
            f"(cold {us_dc:.2f}); entry: prefill {ue_p:.1f} us (cold {ue_pc:.1f}), step {ue_d:.2f} us "
            f"(cold {ue_dc:.2f})")

        # ------------------------------------- attention producers (PP512)
        # q projection [T][16][2][256] -> split + RMSNorm + RoPE of q (fused),
        # and RMSNorm + RoPE of k [T][4][256]; rotary 64, base 1e7.
        T = 512
        qg = rand_bf16(T * HQ * 2 * D)
        kin = rand_bf16(T * HKV * D)
        wq, wk = rand_bf16(D), rand_bf16(D)
        qo, go = (torch.empty(T * HQ * D, device="cuda", dtype=torch.bfloat16) for _ in range(2))
        ko = torch.empty(T * HKV * D, device="cuda", dtype=torch.bfloat16)
        qshape = ops.QkNormRopeShape(T, HQ, D, 64, 0, 1e7)
        kshape = ops.QkNormRopeShape(T, HKV, D, 64, 0, 1e7)
        us_f = timed(lambda i: ops.qwen35_split_query_gate_norm_rope(
            qg, wq, qo, go, qshape, 1e-6, 3, 3, stream=stream), args.steps, args.warmup, cold=False)
        us_k = timed(lambda i: ops.qwen35_qk_norm_rope(kin, wk, ko, kshape, 1e-6, 3, 3,
                                                       stream=stream), args.steps, args.warmup, cold=False)
        us_s = timed(lambda i: ops.qwen35_split_full_query_gate(qg, qo, go, T, HQ, D, 3,
                                                                stream=stream),
                     args.steps, args.warmup, cold=False)
        fbytes = T * HQ * D * 2 * 4  # read q and gate halves, write query and gate
        kbytes_p = T * HKV * D * 2 * 2
        results["producers_pp512"] = {
            "split_norm_rope_q_us": us_f, "split_norm_rope_q_GB_per_s": fbytes / us_f / 1e3,
            "norm_rope_k_us": us_k, "norm_rope_k_GB_per_s": kbytes_p / us_k / 1e3,
            "split_only_us": us_s, "split_only_GB_per_s": fbytes / us_s / 1e3}
        log(f"producers PP512: fused q {us_f:.1f} us, k {us_k:.1f} us, split {us_s:.1f} us")

        # ------------- whole attention steps: producers separate vs fused in
        # PP512 prefill: q split+norm+RoPE, k norm+RoPE, prefill (3 launches)
        # against the fused entry (2 launches); hot inputs.
        wq32 = torch.randn(D, device="cuda") * 0.2 + 1.0
        wk32 = torch.randn(D, device="cuda") * 0.2 + 1.0
        wqb, wkb = wq32.to(torch.bfloat16), wk32.to(torch.bfloat16)
        norm = ops.Qwen35FusedNormRope(wqb, wkb, 64, 1e7, 1e-6)
        pshape = ops.Qwen35AttentionShape(T, HQ, HKV, D, T, 0)
        vin = rand_bf16(T * HKV * D)
        pcache = torch.zeros(2 * T * HKV * D, device="cuda", dtype=torch.bfloat16)
        pout = torch.empty(T * HQ * D, device="cuda", dtype=torch.bfloat16)
        pol = ops.Qwen35AttentionLaunchPolicy()

        def prefill_step(i):
            ops.qwen35_split_query_gate_norm_rope(qg, wqb, qo, go, qshape, 1e-6, 3, 3, stream=stream)
            ops.qwen35_qk_norm_rope(kin, wkb, ko, kshape, 1e-6, 3, 3, stream=stream)
            ops.qwen35_causal_attention(qo, ko, vin, go, pout, pcache, None, pshape, ops.DTYPE_BF16, pol,
                                        stream=stream)
        us_sep = timed(prefill_step, args.steps, args.warmup, cold=False)
        us_fus = timed(lambda i: ops.qwen35_online_attention_prefill_fused(
            qg, kin, vin, pout, pcache, pshape, norm, stream=stream), args.steps, args.warmup, cold=False)
        # ctx 4096 decode step: producers + split-K decode (4 launches) against
        # the fused decode (2 launches); a distinct cache per call, cold.
        ctx = 4096
        ncache = n_caches(ctx, args.steps)
        caches = make_caches(ctx, ncache)
        dshape = ops.Qwen35AttentionShape(1, HQ, HKV, D, ctx, ctx - 1)
        dplan = ops.qwen35_online_decode_plan(dshape, ops.AUTO, ctx)
        dws = torch.empty(ops.qwen35_online_decode_workspace_layout(dshape, dplan[0])[4], device="cuda",
                          dtype=torch.uint8)
        qg1, k1raw, v1 = rand_bf16(HQ * 2 * D), rand_bf16(HKV * D), rand_bf16(HKV * D)
        q1, g1 = (torch.empty(HQ * D, device="cuda", dtype=torch.bfloat16) for _ in range(2))
        k1 = torch.empty(HKV * D, device="cuda", dtype=torch.bfloat16)
        o1 = torch.empty(HQ * D, device="cuda", dtype=torch.bfloat16)
        q1s = ops.QkNormRopeShape(1, HQ, D, 64, ctx - 1, 1e7)
        k1s = ops.QkNormRopeShape(1, HKV, D, 64, ctx - 1, 1e7)

        def decode_step(i):
            ops.qwen35_split_query_gate_norm_rope(qg1, wqb, q1, g1, q1s, 1e-6, 3, 3, stream=stream)
            ops.qwen35_qk_norm_rope(k1raw, wkb, k1, k1s, 1e-6, 3, 3, stream=stream)
            ops.qwen35_online_attention_decode(q1, k1, v1, g1, o1, caches[i % ncache], dws, dshape,
                                               ops.DTYPE_BF16, ops.CACHE_BF16, ops.HEAD_MAJOR, plan=dplan,
                                               stream=stream)
        ud_sep = timed(decode_step, args.steps, args.warmup, cold=True)
        ud_fus = timed(lambda i: ops.qwen35_online_attention_decode_fused(
            qg1, k1raw, v1, o1, caches[i % ncache], dws, dshape, norm, ops.CACHE_BF16, ops.HEAD_MAJOR,
            dplan, stream=stream), args.steps, args.warmup, cold=True)
        del caches
        torch.cuda.empty_cache()
        results["fused_producers"] = {
            "prefill_pp512_separate_us": us_sep, "prefill_pp512_fused_us": us_fus,
            "decode_ctx4096_separate_us": ud_sep, "decode_ctx4096_fused_us": ud_fus,
            "note": "separate = q split+norm+RoPE, k norm+RoPE, then attention; fused = the producers "
                    "inside the attention kernels (bit-identical results)"}
        log(f"attention step with producers: PP512 {us_sep:.1f} -> {us_fus:.1f} us fused; "
            f"decode ctx4096 {ud_sep:.1f} -> {ud_fus:.1f} us fused")

    # ------------------------------------------------------ CPU baseline
    cpu = None
    if not args.no_cpu:
        model, avail = cpu_description()
        threads = max(1, min(16, avail))
        per = cpu_baselines(threads)
        head = per["cfg2_decode_ctx4096"]
        cpu = {"value": head["value_1_thread"], "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": f"{head['calls_1_thread']} single-token decode calls at ctx 4096 (16q/4kv, D=256) "
                         f"through the C oracle (restated cpp/reference/qwen35.cpp:316-370, -O3, 1 thread), "
                         f"{head['ms_per_call_1_thread']:.1f} ms/call; with {threads} threads (one query head "
                         f"per task) {head['value_threads']:.2f} GB/s",
               "cpu_model": model, "host_cpus_available": avail,
               "threaded": {"value": head["value_threads"], "cores": threads},
               "configs": per}

    traffic = None
    prof = ROOT / "profiles" / "decode_partition_ctx4096_traffic.json"
    if prof.exists():
        traffic = json.loads(prof.read_text()).get("hbm_bytes_per_launch")
    kbytes = 2 * HKV * 4096 * D * 2 + HQ * D * 2  # K/V rows + q read by the partition kernel
    achieved = kbytes / kus4096 / 1e3
    line = {
        "metric": METRIC, "value": results["cfg2_split_k_decode_ctx4096"]["GB_per_s"],
        "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": us4096 / 1e3, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded N(0,1), bf16)",
        "config": {"workload": "split-K GQA decode attention, ctx 4096, 16 q / 4 kv heads, "
                               "head_dim 256, bf16 head-major KV cache, P=256 + LSE merge, "
                               f"1% K rows x8, a distinct cache per timed call ({r4096['caches']}), "
                               "L2/MALL flushed before the timed replay",
                   "global_batch": 1, "seq_len": 4096, "parallelism": "none (1 GPU)",
                   "decode_us_per_call": us4096,
                   "prefill_pp512_TFLOP_per_s": results.get("cfg3_prefill_pp512", {}).get("TFLOP_per_s")},
        "roofline": {"bound": "hbm", "kernel": "decode_split_mfma_kernel<4, 8> (ctx 4096, cold)",
                     "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                     "kernel_us": kus4096, "algorithmic_bytes": kbytes},
        "cpu_baseline": cpu,
        "configs": results,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
