"""Shared helpers for the parity tests: seeded inputs, cache construction in
either layout / dtype, and tolerance checks.  Expected values always come from
the CPU oracle (oracle/pyoracle.py)."""
from __future__ import annotations

import numpy as np

from oracle import pyoracle as orc

HQ, HKV, D = 16, 4, 256


def rng(seed):
    return np.random.default_rng(seed)


def normal(r, *shape, scale=1.0):
    return (r.standard_normal(shape) * scale).astype(np.float32)


def bf16(a):
    return orc.bf16_round(a)


def sequence(n, scale, bias, mod=19, mul=13):
    """cpp/tests/qwen35_cuda_attention_test.cu:180-187 (mod 19, x13) and
    cpp/tests/qwen35_cuda_delta_test.cu:183-191 (mod 29, x17)."""
    i = np.arange(n, dtype=np.int64)
    return (bias + scale * (((i * mul) % mod) - (mod // 2)).astype(np.float32)).astype(np.float32)


def to_dev(a, dtype):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))
    return t.to(device="cuda", dtype=dtype)


def from_dev(t):
    import torch
    return t.detach().to(dtype=torch.float32).cpu().numpy()


def cache_index(layout, token, kvh, max_ctx, hkv=HKV, d=D):
    """Element index of (token, kv_head, 0) in one plane
    (cpp/kernels/qwen35_online_attention.cu:240-252)."""
    if layout == 1:  # head-major
        return (kvh * max_ctx + token) * d
    return (token * hkv + kvh) * d


def make_cache(keys, values, layout, max_ctx, hkv=HKV, d=D):
    """keys/values [n][hkv][d] float -> flat float cache [2][plane]."""
    n = keys.shape[0]
    plane = max_ctx * hkv * d
    cache = np.zeros(2 * plane, np.float32)
    if layout == 1:
        c = cache.reshape(2, hkv, max_ctx, d)
        c[0, :, :n] = keys.transpose(1, 0, 2)
        c[1, :, :n] = values.transpose(1, 0, 2)
    else:
        c = cache.reshape(2, max_ctx, hkv, d)
        c[0, :n] = keys
        c[1, :n] = values
    return cache


def read_cache(cache, layout, n, max_ctx, hkv=HKV, d=D):
    if layout == 1:
        c = cache.reshape(2, hkv, max_ctx, d)
        return c[0, :, :n].transpose(1, 0, 2), c[1, :, :n].transpose(1, 0, 2)
    c = cache.reshape(2, max_ctx, hkv, d)
    return c[0, :n], c[1, :n]


def assert_bf16_close(actual, expected, max_abs=1e-2, rel_l2=5e-3, what="", both_bf16=False):
    """The bf16-output gate of the fp32-accumulated reference: every element
    within max_abs and the whole tensor within rel_l2 (relative L2).

    `expected` is the oracle's fp32 output, not rounded.  Only where the bf16
    grid itself is coarser than the gate (|e| >= 4, where half an ulp of bf16 is
    1.56e-2 and no bf16 value need lie within 1e-2 of e) does an element get
    half an ulp of e plus 2e-3 instead; below |e| = 4 the bound is max_abs
    exactly.  both_bf16: `expected` is itself a bf16 result (one GPU path
    against another), so the two may sit one bf16 ulp of e apart."""
    a = np.asarray(actual, np.float64).ravel()
    e = np.asarray(expected, np.float64).ravel()
    assert np.all(np.isfinite(a)), f"{what}: non-finite output"
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(e), 1e-30))) - 7)
    grid = ulp if both_bf16 else 0.5 * ulp + 2e-3
    err = np.abs(a - e)
    bad = err > np.maximum(max_abs, grid)
    assert not bad.any(), (f"{what}: {bad.sum()} elements off, worst {err.max():.3e} "
                           f"at expected {e[np.argmax(err)]:.4f}")
    r = np.linalg.norm(a - e) / max(np.linalg.norm(e), 1e-30)
    assert r <= rel_l2, f"{what}: rel-L2 {r:.3e} > {rel_l2}"


def close_enough(actual, expected, tol=2e-2):
    """The reference tests' elementwise gate: abs <= 2e-2 or rel <= 2e-2
    (cpp/tests/qwen35_cuda_attention_test.cu:189-193)."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    ab = np.abs(a - e)
    rel = ab / np.maximum(np.abs(e), 1e-6)
    return bool(np.all((ab <= tol) | (rel <= tol)) and np.all(np.isfinite(a)))


def rel_l2(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))
