"""ctypes binding of the CPU oracle (liboracle.so) and of the compiled
reference shim (oracle/_ref/libqwen35_ref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by ``__graft_entry__.smoke()``
as the checker, and by ``bench.py``'s cpu_baseline leg.  The product package
``raftinfer_amd`` never imports it.
"""
from __future__ import annotations

import ctypes
import os
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
_LIB = None
_REF = None

MODE_AUTO, MODE_SINGLE_BLOCK, MODE_SPLIT_K_256, MODE_SPLIT_K_512 = 0, 1, 2, 3

_f = ctypes.POINTER(ctypes.c_float)
_sz = ctypes.c_size_t


class DecodePlan(ctypes.Structure):
    _fields_ = [("resolved_mode", ctypes.c_int), ("partition_tokens", _sz),
                ("split_k_threshold_tokens", _sz), ("context_bucket_tokens", _sz),
                ("active_partition_capacity", _sz)]


class DecodeLayout(ctypes.Structure):
    _fields_ = [("partial_count", _sz), ("max_offset_bytes", _sz),
                ("sum_offset_bytes", _sz), ("value_offset_bytes", _sz), ("bytes", _sz)]


def build() -> None:
    """Compile liboracle.so (and oracle/_ref when the reference is present)."""
    subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)


def lib():
    global _LIB
    if _LIB is None:
        path = HERE / "liboracle.so"
        if not path.exists():
            build()
        _LIB = ctypes.CDLL(str(path))
    return _LIB


def ref_lib():
    """The compiled reference shim, or None when it was not built."""
    global _REF
    if _REF is None:
        path = HERE / "_ref" / "libqwen35_ref.so"
        if not path.exists():
            return None
        _REF = ctypes.CDLL(str(path))
    return _REF


def _p(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_f)


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def bf16_round(a: np.ndarray) -> np.ndarray:
    a = f32(a)
    out = np.empty_like(a)
    lib().orc_bf16_round_array(_p(a), _p(out), _sz(a.size))
    return out


def decode_plan(shape, requested: int, context_tokens: int):
    """shape = (tokens, Hq, Hkv, D, max_ctx); returns DecodePlan or None."""
    out = DecodePlan()
    rc = lib().orc_decode_plan(*[_sz(x) for x in shape], ctypes.c_int(requested),
                               _sz(context_tokens), ctypes.byref(out))
    return None if rc != 0 else out


def decode_layout(shape, resolved: int):
    out = DecodeLayout()
    rc = lib().orc_decode_workspace_layout(*[_sz(x) for x in shape], ctypes.c_int(resolved),
                                           ctypes.byref(out))
    return None if rc != 0 else out


def attention_core(q, keys, values, gate, past_tokens: int):
    """q, gate: [T,Hq,D]; keys, values: [past+T,Hkv,D] -> out [T,Hq,D]."""
    q, keys, values, gate = map(f32, (q, keys, values, gate))
    T, hq, d = q.shape
    hkv = keys.shape[1]
    assert keys.shape[0] == past_tokens + T
    out = np.empty_like(q)
    lib().orc_attention_core(_p(q), _p(keys), _p(values), _p(gate), _p(out), _sz(T), _sz(hq),
                             _sz(hkv), _sz(d), _sz(past_tokens))
    return out


def gated_full_attention(inp, qnw, knw, ow, *, tokens, hidden, hq, hkv, d, rotary_dim,
                         position, rope_base, eps, use_reference=False):
    inp, qnw, knw, ow = map(f32, (inp, qnw, knw, ow))
    out = np.zeros(tokens * hidden, np.float32)
    fn = ref_lib().ref_gated_full_attention if use_reference else lib().orc_gated_full_attention
    fn.argtypes = [_f] * 5 + [_sz] * 7 + [ctypes.c_float, ctypes.c_float]
    rc = fn(_p(inp), _p(qnw), _p(knw), _p(ow), _p(out), tokens, hidden, hq, hkv, d,
            rotary_dim, position, rope_base, eps)
    assert rc in (None, 0)
    return out


def decode_partials(q, keys, values, context_tokens, partition_tokens, max_partitions):
    q, keys, values = map(f32, (q, keys, values))
    hq, d = q.shape
    hkv = keys.shape[1]
    pm = np.full(hq * max_partitions, np.nan, np.float32)
    ps = np.full(hq * max_partitions, np.nan, np.float32)
    pv = np.full(hq * max_partitions * d, np.nan, np.float32)
    lib().orc_decode_partials(_p(q), _p(keys), _p(values), _sz(context_tokens), _sz(hq),
                              _sz(hkv), _sz(d), _sz(partition_tokens), _sz(max_partitions),
                              _p(pm), _p(ps), _p(pv))
    return pm, ps, pv


def decode_merge(gate, pm, ps, pv, context_tokens, partition_tokens, max_partitions):
    gate = f32(gate)
    hq, d = gate.shape
    out = np.empty_like(gate)
    lib().orc_decode_merge(_p(gate), _p(f32(pm)), _p(f32(ps)), _p(f32(pv)),
                           _sz(context_tokens), _sz(hq), _sz(d), _sz(partition_tokens),
                           _sz(max_partitions), _p(out))
    return out


def gated_delta_prefill(inp, conv_w, a, dt_bias, norm_w, conv_state, rec_state, *, tokens,
                        hidden, hk, hv, dk, dv, width, eps, use_reference=False):
    """Returns (output, conv_state, rec_state); states are copied, not mutated."""
    inp, conv_w, a, dt_bias, norm_w = map(f32, (inp, conv_w, a, dt_bias, norm_w))
    cs = f32(conv_state).copy()
    rs = f32(rec_state).copy()
    out = np.zeros(tokens * hidden, np.float32)
    fn = ref_lib().ref_gated_delta_prefill if use_reference else lib().orc_gated_delta_prefill
    fn.argtypes = [_f] * 8 + [_sz] * 7 + [ctypes.c_float]
    rc = fn(_p(inp), _p(conv_w), _p(a), _p(dt_bias), _p(norm_w), _p(out), _p(cs), _p(rs),
            tokens, hidden, hk, hv, dk, dv, width, eps)
    assert rc in (None, 0)
    return out, cs, rs


def delta_core(q, k, v, beta, log_decay, q_scale, state):
    """q,k [T,Hk,dk]; v [T,Hv,dv]; beta, log_decay [T,Hv]; state [Hv,dk,dv] (copied)."""
    q, k, v, beta, log_decay = map(f32, (q, k, v, beta, log_decay))
    T, hk, dk = q.shape
    hv, dv = v.shape[1], v.shape[2]
    st = f32(state).copy()
    raw = np.zeros((T, hv, dv), np.float32)
    lib().orc_delta_core(_p(q), _p(k), _p(v), _p(beta), _p(log_decay), ctypes.c_float(q_scale),
                         _p(st), _p(raw), _sz(T), _sz(hk), _sz(hv), _sz(dk), _sz(dv))
    return raw, st


def qk_norm_rope(x, weight, rotary_dim, position_offset, rope_base, eps, use_reference=False):
    """x [tokens][heads][head_dim] -> RMSNorm * weight, then partial RoPE."""
    x = f32(x)
    tokens, heads, head_dim = x.shape
    out = np.zeros_like(x)
    fn = ref_lib().ref_qk_norm_rope if use_reference else lib().orc_qk_norm_rope
    fn.argtypes = [_f] * 3 + [_sz] * 5 + [ctypes.c_float, ctypes.c_float]
    fn.restype = ctypes.c_int if use_reference else None
    rc = fn(_p(x), _p(f32(weight)), _p(out), tokens, heads, head_dim, rotary_dim,
            position_offset, rope_base, eps)
    assert rc in (None, 0)
    return out


def split_full_query_gate(query_gate, heads, head_dim):
    """[tokens][heads][2][head_dim] -> (query, gate), each [tokens][heads][head_dim]."""
    qg = f32(query_gate)
    tokens = qg.size // (2 * heads * head_dim)
    q = np.zeros((tokens, heads, head_dim), np.float32)
    g = np.zeros_like(q)
    lib().orc_split_full_query_gate(_p(qg), _p(q), _p(g), _sz(tokens), _sz(heads), _sz(head_dim))
    return q, g


def pack_linear_delta_input(qkv, beta, alpha, gate):
    """Each [tokens][width] -> [tokens][sum of widths]."""
    parts = [f32(x) for x in (qkv, beta, alpha, gate)]
    tokens = parts[0].shape[0]
    widths = [x.shape[1] for x in parts]
    out = np.zeros((tokens, sum(widths)), np.float32)
    fn = lib().orc_pack_linear_delta_input
    fn.restype = None
    fn(*[_p(x) for x in parts], _p(out), _sz(tokens), *[_sz(w) for w in widths])
    return out


def compare(candidate, reference, relative_floor=1e-12):
    c, r = f32(candidate).ravel(), f32(reference).ravel()
    assert c.size == r.size
    out = (ctypes.c_double * 5)()
    lib().orc_compare(_p(c), _p(r), _sz(c.size), ctypes.c_double(relative_floor), out)
    return {"max_abs": out[0], "max_rel": out[1], "cosine": out[2], "nonfinite": int(out[3]),
            "rel_l2": out[4]}
