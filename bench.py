"""Benchmark of the gfx950 attention / gated-delta hot path.

A "step" is one split-K GQA decode call at context 4096 (benchmark config 2:
16 query / 4 KV heads, head_dim 256, BF16 head-major cache, 256-token
partitions + fp32 LSE merge), with inputs resident in HBM and 40 distinct
caches (671 MB) rotated so the 256 MB MALL cannot serve them.  ``value`` is
that call's algorithmic HBM throughput (KV bytes + q/gate/out bytes per call /
event-timed call time).  The other benchmark configs are reported under
``configs``; ``roofline`` prices the dominant kernel (the split-K partition
kernel) timed alone with HIP events on its own stream; ``cpu_baseline`` times
the CPU oracle's decode on one host core over a bounded sample.

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
import json
import math
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


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def decode_bytes(ctx):
    # K and V rows read once per call + q, gate read and out written (bf16).
    return 2 * HKV * ctx * D * 2 + 3 * HQ * D * 2


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

    from raftinfer_amd import ops

    torch.manual_seed(0x5241465449)
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    ev = lambda: torch.cuda.Event(enable_timing=True)

    def timed(fn, steps, warmup):
        """Mean GPU time per call: the `steps` calls are captured into one HIP
        graph (how a serving loop replays decode) and the replay is bracketed by
        events on the launch stream, so host dispatch cost is excluded."""
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(steps):
                fn(i)
        graph.replay()
        torch.cuda.synchronize()
        a, b = ev(), ev()
        a.record(stream)
        graph.replay()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / steps * 1e3  # us per call

    timed_each = timed

    def rand_bf16(*shape):
        return torch.randn(*shape, device="cuda", dtype=torch.float32).to(torch.bfloat16)

    results = {}

    # ---------------------------------------------------------- config 2
    def split_decode(ctx, ncache, counters=False):
        shape = ops.Qwen35AttentionShape(1, HQ, HKV, D, ctx, ctx - 1)
        caches = torch.empty(ncache, 2 * HKV * ctx * D, device="cuda", dtype=torch.bfloat16)
        for i in range(ncache):
            caches[i].copy_(rand_bf16(2 * HKV * ctx * D))
            rows = torch.rand(ctx, device="cuda") < 0.01  # ~1% of K rows x8
            kview = caches[i][:HKV * ctx * D].view(HKV, ctx, D)
            kview[:, rows] *= 8
        q, k, v, g = rand_bf16(HQ * D), rand_bf16(HKV * D), rand_bf16(HKV * D), rand_bf16(HQ * D)
        out = torch.empty(HQ * D, device="cuda", dtype=torch.bfloat16)
        plan = ops.qwen35_online_decode_plan(shape, ops.AUTO, ctx)
        ws = torch.empty(ops.qwen35_online_decode_workspace_layout(shape, plan[0])[4],
                         device="cuda", dtype=torch.uint8)
        call = lambda i: ops.qwen35_online_attention_decode(
            q, k, v, g, out, caches[i % ncache], ws, shape, ops.DTYPE_BF16, ops.CACHE_BF16,
            ops.HEAD_MAJOR, plan=plan, stream=stream)
        from raftinfer_amd import _lib
        lib = _lib.load()
        import ctypes
        cplan = _lib.DecodePlan(*plan)
        nbytes = caches[0].numel() * 2

        def part(i):
            _lib.check(lib.raftinfer_amd_online_attention_decode_partition_only(
                ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(k.data_ptr()),
                ctypes.c_void_p(v.data_ptr()), ctypes.c_void_p(g.data_ptr()),
                ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(caches[i % ncache].data_ptr()),
                nbytes, ctypes.c_void_p(ws.data_ptr()), ws.numel(), shape.c(), ops.DTYPE_BF16,
                ops.CACHE_BF16, ops.HEAD_MAJOR, cplan, None, ctypes.c_void_p(stream.cuda_stream)))
        if counters:
            for i in range(ncache):
                part(i)
            torch.cuda.synchronize()
            return None
        us = timed(call, args.steps, args.warmup)
        kus = timed_each(part, args.steps, args.warmup)
        del caches
        torch.cuda.empty_cache()
        return us, kus

    if args.counters:
        split_decode(4096, 20, counters=True)
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
        from raftinfer_amd import _lib
        import ctypes
        lib = _lib.load()
        T = 512
        shape = ops.Qwen35AttentionShape(T, HQ, HKV, D, T, 0)
        qp, gp = rand_bf16(T * HQ * D), rand_bf16(T * HQ * D)
        kp, vp = rand_bf16(T * HKV * D), rand_bf16(T * HKV * D)
        cache = torch.zeros(2 * T * HKV * D, device="cuda", dtype=torch.bfloat16)
        outp = torch.empty(T * HQ * D, device="cuda", dtype=torch.bfloat16)
        for _ in range(20):
            _lib.check(lib.raftinfer_amd_online_attention_prefill_kernel_only(
                *[ctypes.c_void_p(t.data_ptr()) for t in (qp, kp, vp, gp, outp, cache)],
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
        log("counters run: 20 partition launches (ctx 4096), 20 copies of 64 MiB, 20 PP512 "
            "prefill kernels, 10 delta prefills (T=512), 20 delta decode steps")
        return

    us4096, kus4096 = split_decode(4096, 40)
    log(f"cfg2 ctx4096: {us4096:.2f} us/call, partition kernel {kus4096:.2f} us")
    results["cfg2_split_k_decode_ctx4096"] = {
        "us_per_call": us4096, "GB_per_s": decode_bytes(4096) / us4096 / 1e3,
        "partition_kernel_us": kus4096, "bytes_per_call": decode_bytes(4096)}

    if not args.quick:
        us16k, kus16k = split_decode(16384, 10)
        log(f"cfg2 ctx16384: {us16k:.2f} us/call, partition kernel {kus16k:.2f} us")
        results["cfg2_split_k_decode_ctx16384"] = {
            "us_per_call": us16k, "GB_per_s": decode_bytes(16384) / us16k / 1e3,
            "partition_kernel_us": kus16k, "bytes_per_call": decode_bytes(16384)}

        # ------------------------------------------------------ config 1
        ctx, ncache = 512, 256
        shape = ops.Qwen35AttentionShape(1, HQ, HKV, D, ctx, ctx - 1)
        caches = rand_bf16(ncache, 2 * HKV * ctx * D)
        q, k, v, g = rand_bf16(HQ * D), rand_bf16(HKV * D), rand_bf16(HKV * D), rand_bf16(HQ * D)
        out = torch.empty(HQ * D, device="cuda", dtype=torch.bfloat16)
        us = timed(lambda i: ops.qwen35_online_attention_decode(
            q, k, v, g, out, caches[i % ncache], None, shape, ops.DTYPE_BF16, ops.CACHE_BF16,
            ops.HEAD_MAJOR, stream=stream), args.steps, args.warmup)
        results["cfg1_single_block_decode_ctx512"] = {
            "us_per_call": us, "GB_per_s": decode_bytes(512) / us / 1e3}
        log(f"cfg1 ctx512: {us:.2f} us/call")
        del caches

        # ------------------------------------------------------ config 3
        for T in (128, 512):
            shape = ops.Qwen35AttentionShape(T, HQ, HKV, D, T, 0)
            qp, gp = rand_bf16(T * HQ * D), rand_bf16(T * HQ * D)
            kp, vp = rand_bf16(T * HKV * D), rand_bf16(T * HKV * D)
            cache = torch.zeros(2 * T * HKV * D, device="cuda", dtype=torch.bfloat16)
            outp = torch.empty(T * HQ * D, device="cuda", dtype=torch.bfloat16)
            pol = ops.Qwen35AttentionLaunchPolicy()
            us = timed(lambda i: ops.qwen35_causal_attention(
                qp, kp, vp, gp, outp, cache, None, shape, ops.DTYPE_BF16, pol, stream=stream),
                args.steps, args.warmup)
            from raftinfer_amd import _lib
            import ctypes
            lib = _lib.load()
            kern = lambda i: _lib.check(lib.raftinfer_amd_online_attention_prefill_kernel_only(
                *[ctypes.c_void_p(t.data_ptr()) for t in (qp, kp, vp, gp, outp, cache)],
                cache.numel() * 2, shape.c(), ops.DTYPE_BF16, ops.CACHE_BF16, ops.HEAD_MAJOR,
                ctypes.c_void_p(stream.cuda_stream)))
            kus = timed_each(kern, args.steps, args.warmup)
            flops = 8192 * T * (T + 1)
            results[f"cfg3_prefill_pp{T}"] = {
                "us_per_call": us, "TFLOP_per_s": flops / us / 1e6, "kernel_us": kus,
                "kernel_TFLOP_per_s": flops / kus / 1e6, "flop": flops,
                "mfma_frac": flops / kus / 1e6 / BF16_PEAK_TFLOPS}
            log(f"cfg3 PP{T}: {us:.2f} us/call, kernel {kus:.2f} us, {flops / kus / 1e6:.1f} TFLOP/s")

        # ------------------------------------------------------ config 4
        rng = np.random.default_rng(0x5241465449 + 4)
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
            max(5, args.steps // 5), 2)
        kv_bytes = int(sum(4096 * int(L) for L in lengths)) + 32 * 24576
        results["cfg4_batched_ragged_decode_x32"] = {
            "us_per_call": us, "GB_per_s": kv_bytes / us / 1e3, "bytes_per_call": kv_bytes,
            "lengths_seed": 0x5241465449 + 4}
        log(f"cfg4 batched: {us:.2f} us/call, {kv_bytes / us / 1e3:.0f} GB/s")
        del cache
        torch.cuda.empty_cache()

        # ------------------------------------------------------ config 5
        T = 512
        q5 = torch.nn.functional.normalize(torch.randn(T, 16, 128, device="cuda"), dim=-1).to(torch.bfloat16)
        k5 = torch.nn.functional.normalize(torch.randn(T, 16, 128, device="cuda"), dim=-1).to(torch.bfloat16)
        v5 = rand_bf16(T, 32, 128)
        beta = torch.sigmoid(torch.randn(T, 32, device="cuda"))
        lg = -torch.nn.functional.softplus(torch.randn(T, 32, device="cuda"))
        st = torch.zeros(32, 128, 128, device="cuda")
        o5 = torch.empty(T, 32, 128, device="cuda", dtype=torch.bfloat16)
        ws5 = torch.empty(ops.qwen35_gated_delta_core_workspace_bytes(T, 16, 32, 128, 128),
                          device="cuda", dtype=torch.uint8)
        us_p = timed(lambda i: ops.qwen35_gated_delta_core(
            q5, k5, v5, beta, lg, 128 ** -0.5, st, o5, ws5, True, stream=stream),
            args.steps, args.warmup)
        us_d = timed(lambda i: ops.qwen35_gated_delta_core(
            q5[i % T:i % T + 1], k5[i % T:i % T + 1], v5[i % T:i % T + 1], beta[i % T:i % T + 1],
            lg[i % T:i % T + 1], 128 ** -0.5, st, o5[:1], None, False, stream=stream),
            max(args.steps, 32), args.warmup)
        pbytes = T * (16 * 128 * 2 * 2 + 32 * 128 * 2 * 2 + 32 * 8) + 2 * 32 * 128 * 128 * 4
        dbytes = 2 * 32 * 128 * 128 * 4 + (16 * 128 * 2 * 2 + 32 * 128 * 2 * 2 + 32 * 8)
        results["cfg5_gated_delta"] = {
            "prefill_T512_us": us_p, "prefill_GB_per_s": pbytes / us_p / 1e3,
            "prefill_GFLOP_per_s": 6 * 128 * 128 * 32 * T / us_p / 1e3,
            "decode_step_us": us_d, "decode_GB_per_s": dbytes / us_d / 1e3}
        log(f"cfg5 delta: prefill {us_p:.1f} us, decode step {us_d:.2f} us")

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
            qg, wq, qo, go, qshape, 1e-6, 3, 3, stream=stream), args.steps, args.warmup)
        us_k = timed(lambda i: ops.qwen35_qk_norm_rope(kin, wk, ko, kshape, 1e-6, 3, 3,
                                                       stream=stream), args.steps, args.warmup)
        us_s = timed(lambda i: ops.qwen35_split_full_query_gate(qg, qo, go, T, HQ, D, 3,
                                                                stream=stream),
                     args.steps, args.warmup)
        fbytes = T * HQ * D * 2 * 4  # read q and gate halves, write query and gate
        kbytes_p = T * HKV * D * 2 * 2
        results["producers_pp512"] = {
            "split_norm_rope_q_us": us_f, "split_norm_rope_q_GB_per_s": fbytes / us_f / 1e3,
            "norm_rope_k_us": us_k, "norm_rope_k_GB_per_s": kbytes_p / us_k / 1e3,
            "split_only_us": us_s, "split_only_GB_per_s": fbytes / us_s / 1e3}
        log(f"producers PP512: fused q {us_f:.1f} us, k {us_k:.1f} us, split {us_s:.1f} us")

    # ------------------------------------------------------ CPU baseline
    cpu = None
    if not args.no_cpu:
        from oracle import pyoracle as orc
        r = np.random.default_rng(1)
        ctx = 4096
        keys = orc.bf16_round(r.standard_normal((ctx, HKV, D)).astype(np.float32))
        vals = orc.bf16_round(r.standard_normal((ctx, HKV, D)).astype(np.float32))
        qn = orc.bf16_round(r.standard_normal((1, HQ, D)).astype(np.float32))
        gn = orc.bf16_round(r.standard_normal((1, HQ, D)).astype(np.float32))
        n, t0 = 0, time.perf_counter()
        while n < 200 and time.perf_counter() - t0 < 10.0:
            orc.attention_core(qn, keys, vals, gn, ctx - 1)
            n += 1
        per_call = (time.perf_counter() - t0) / n
        cpu = {"value": decode_bytes(ctx) / per_call / 1e9, "unit": "GB/s", "cores": 1,
               "kind": "port",
               "sample": f"{n} single-token decode calls at ctx 4096 (16q/4kv, D=256) through the "
                         f"C oracle (restated cpp/reference/qwen35.cpp:316-370, -O3, 1 thread), "
                         f"{per_call * 1e3:.1f} ms/call; host {os.cpu_count()} logical CPUs"}
        log(f"cpu baseline: {per_call * 1e3:.1f} ms/call")

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
                               "1% K rows x8, 40 rotating caches (671 MB)",
                   "global_batch": 1, "seq_len": 4096, "parallelism": "none (1 GPU)",
                   "decode_us_per_call": us4096,
                   "prefill_pp512_TFLOP_per_s": results.get("cfg3_prefill_pp512", {}).get("TFLOP_per_s")},
        "roofline": {"bound": "hbm", "kernel": "decode_split_mfma_kernel<4, 8> (ctx 4096)",
                     "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                     "kernel_us": kus4096, "algorithmic_bytes": kbytes},
        "cpu_baseline": cpu,
        "configs": results,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
