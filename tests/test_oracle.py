"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker:
the reference's own known-answer vectors and HF fixture, the compiled
reference (oracle/_ref, when built), and closed-form / brute-force checks."""
import json
import pathlib

import numpy as np
import pytest

import fixture
from helpers import bf16, normal, rng
from oracle import pyoracle as orc

KAT = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_kat.json").read_text())


def test_bf16_rne_matches_reference_rules():
    # cpp/reference/bf16.hpp:16-32: ties to even, NaN stays NaN, inf stays inf.
    x = np.array([1.0, 1.00390625, 1.005859375, 1.01171875, -2.5, np.inf, -np.inf, 3.4e38],
                 np.float32)
    got = bf16(x)
    assert got[0] == 1.0 and got[1] == 1.0  # tie 0x3F808000 -> even 0x3F80
    assert got[2] == np.float32(1.0078125)  # 0x3F80C000: above the half -> 0x3F81
    assert got[3] == np.float32(1.015625)
    assert got[4] == -2.5 and np.isposinf(got[5]) and np.isneginf(got[6])
    assert np.isnan(bf16(np.array([np.nan], np.float32)))[0]
    r = rng(1)
    v = normal(r, 10000)
    b = bf16(v)
    bits = b.view(np.uint32)
    assert np.all(bits & 0xFFFF == 0)
    assert np.all(np.abs(b - v) <= np.abs(v) * 2.0 ** -8 + 1e-38)


def test_full_attention_known_answer():
    k = KAT["full_attention"]
    out = orc.gated_full_attention(k["input"], k["query_norm_weight"], k["key_norm_weight"],
                                   k["output_weight"], tokens=2, hidden=4, hq=2, hkv=1, d=2,
                                   rotary_dim=2, position=0, rope_base=1e4, eps=1e-6)
    np.testing.assert_allclose(out, k["expected"], atol=k["tolerance"], rtol=0)


def test_gated_delta_known_answer_and_step_equals_prefill():
    k = KAT["gated_delta"]
    cd = 2 * 1 * 2 + 2 * 2
    out, cs, rs = orc.gated_delta_prefill(k["input"], k["conv_weight"], k["recurrent_a"],
                                          k["dt_bias"], k["output_norm_weight"],
                                          np.zeros(cd * 3), np.zeros(8), tokens=3, hidden=4,
                                          hk=1, hv=2, dk=2, dv=2, width=4, eps=1e-6)
    np.testing.assert_allclose(out, k["expected"], atol=k["tolerance"], rtol=0)
    # step-by-step == prefill (cpp/tests/qwen35_reference_test.cpp:136-155)
    inp = np.asarray(k["input"], np.float32).reshape(3, 16)
    c2, r2, outs = np.zeros(cd * 3, np.float32), np.zeros(8, np.float32), []
    for t in range(3):
        o, c2, r2 = orc.gated_delta_prefill(inp[t], k["conv_weight"], k["recurrent_a"], k["dt_bias"],
                                            k["output_norm_weight"], c2, r2, tokens=1, hidden=4,
                                            hk=1, hv=2, dk=2, dv=2, width=4, eps=1e-6)
        outs.append(o)
    np.testing.assert_allclose(np.concatenate(outs), out, atol=1e-6)
    np.testing.assert_allclose(c2, cs, atol=1e-6)
    np.testing.assert_allclose(r2, rs, atol=1e-6)


def _within(actual, expected, tol=1e-5):
    a, e = np.asarray(actual), np.asarray(expected)
    diff = np.abs(a - e)
    return np.all((diff <= tol) | (diff <= tol * np.maximum(np.abs(a), np.abs(e))))


def test_hf_fixture_full_attention_and_delta():
    f = fixture.load()
    F, D = f["full"], f["delta"]
    out = orc.gated_full_attention(f["full_input"], f["full_query_norm_weight"],
                                   f["full_key_norm_weight"], f["full_output_weight"],
                                   tokens=F["tokens"], hidden=F["hidden_size"], hq=F["query_heads"],
                                   hkv=F["kv_heads"], d=F["head_dim"], rotary_dim=F["rotary_dim"],
                                   position=F["position_offset"], rope_base=F["rope_base"],
                                   eps=F["epsilon"])
    assert _within(out, f["full_expected_output"])
    o, cs, rs = orc.gated_delta_prefill(
        f["delta_input"], f["delta_conv_weight"], f["delta_recurrent_a"], f["delta_dt_bias"],
        f["delta_output_norm_weight"], f["delta_initial_convolution"], f["delta_initial_recurrent"],
        tokens=D["tokens"], hidden=D["hidden_size"], hk=D["key_heads"], hv=D["value_heads"],
        dk=D["key_dim"], dv=D["value_dim"], width=D["conv_width"], eps=D["epsilon"])
    assert _within(o, f["delta_expected_output"])
    assert _within(cs, f["delta_expected_convolution"])
    assert _within(rs, f["delta_expected_recurrent"])


def test_fixture_parser_rejects_corruption():
    # cpp/tests/qwen35_fixture_test.cpp:205-225
    data = bytearray(fixture.PATH.read_bytes())
    for mutate in (lambda b: b.__setitem__(0, b[0] ^ 0xFF),
                   lambda b: b.__setitem__(slice(8, 12), (2).to_bytes(4, "little")),
                   lambda b: b.__setitem__(slice(16, 24), (len(b) + 1).to_bytes(8, "little")),
                   lambda b: b.pop()):
        bad = bytearray(data)
        mutate(bad)
        with pytest.raises(ValueError):
            fixture.parse(bytes(bad))


ref_needed = pytest.mark.skipif(orc.ref_lib() is None, reason="oracle/_ref not built")


@ref_needed
@pytest.mark.parametrize("tokens,hq,hkv,d,rot,pos", [(17, 16, 4, 256, 64, 3), (5, 4, 2, 64, 0, 0),
                                                     (9, 2, 1, 8, 4, 11)])
def test_attention_restatement_matches_compiled_reference(tokens, hq, hkv, d, rot, pos):
    r = rng(tokens * 7 + d)
    hid = hq * d
    inp = normal(r, tokens * (hid + 2 * hkv * d + hid))
    qn, kn = normal(r, d), normal(r, d)
    ow = normal(r, hid * hid, scale=0.05)
    kw = dict(tokens=tokens, hidden=hid, hq=hq, hkv=hkv, d=d, rotary_dim=rot, position=pos,
              rope_base=1e7, eps=1e-6)
    a = orc.gated_full_attention(inp, qn, kn, ow, **kw)
    b = orc.gated_full_attention(inp, qn, kn, ow, use_reference=True, **kw)
    np.testing.assert_array_equal(a, b)


@ref_needed
@pytest.mark.parametrize("tokens,hk,hv,dk,dv,w", [(5, 2, 4, 5, 7, 3), (3, 16, 32, 128, 128, 4),
                                                  (17, 1, 2, 4, 4, 4), (2, 2, 2, 8, 8, 1)])
def test_delta_restatement_matches_compiled_reference(tokens, hk, hv, dk, dv, w):
    r = rng(tokens + 100 * dk)
    hid = hv * dv
    cd = 2 * hk * dk + hv * dv
    inp = normal(r, tokens * (cd + 2 * hv + hid))
    cw = normal(r, cd * w, scale=0.3)
    a_w = -np.exp(normal(r, hv))
    dt = normal(r, hv)
    nw = normal(r, dv)
    cs = normal(r, cd * max(w - 1, 0))
    rs = normal(r, hv * dk * dv, scale=0.1)
    kw = dict(tokens=tokens, hidden=hid, hk=hk, hv=hv, dk=dk, dv=dv, width=w, eps=1e-6)
    a = orc.gated_delta_prefill(inp, cw, a_w, dt, nw, cs, rs, **kw)
    b = orc.gated_delta_prefill(inp, cw, a_w, dt, nw, cs, rs, use_reference=True, **kw)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)


def _brute_attention(q, keys, values, gate, past):
    """Textbook softmax attention in float64 (no shared code with the oracle)."""
    T, hq, d = q.shape
    hkv = keys.shape[1]
    out = np.zeros_like(q, dtype=np.float64)
    for t in range(T):
        for h in range(hq):
            kk = keys[:past + t + 1, h // (hq // hkv)].astype(np.float64)
            vv = values[:past + t + 1, h // (hq // hkv)].astype(np.float64)
            s = kk @ q[t, h].astype(np.float64) / np.sqrt(d)
            p = np.exp(s - s.max())
            p /= p.sum()
            out[t, h] = (p @ vv) / (1 + np.exp(-gate[t, h].astype(np.float64)))
    return out


def test_attention_core_matches_brute_force_and_gqa_mapping():
    r = rng(3)
    T, past, hq, hkv, d = 6, 5, 8, 2, 16
    q, gate = normal(r, T, hq, d), normal(r, T, hq, d)
    keys, values = normal(r, past + T, hkv, d), normal(r, past + T, hkv, d)
    got = orc.attention_core(q, keys, values, gate, past)
    np.testing.assert_allclose(got, _brute_attention(q, keys, values, gate, past), atol=2e-6)
    # GQA mapping is qh / (Hq/Hkv): perturbing kv head 1 changes only heads 4..7.
    keys2 = keys.copy()
    keys2[:, 1] += 1.0
    got2 = orc.attention_core(q, keys2, values, gate, past)
    assert np.array_equal(got[:, :4], got2[:, :4]) and not np.array_equal(got[:, 4:], got2[:, 4:])


def test_attention_core_causality():
    r = rng(4)
    T, hq, hkv, d = 7, 4, 2, 32
    q, gate = normal(r, T, hq, d), normal(r, T, hq, d)
    keys, values = normal(r, T, hkv, d), normal(r, T, hkv, d)
    a = orc.attention_core(q, keys, values, gate, 0)
    keys[-1] += 7.0
    values[-1] -= 9.0
    b = orc.attention_core(q, keys, values, gate, 0)
    assert np.array_equal(a[:-1], b[:-1]) and not np.array_equal(a[-1], b[-1])


@pytest.mark.parametrize("ctx,P", [(1, 256), (255, 256), (256, 256), (257, 256), (777, 256),
                                   (1024, 256), (513, 512), (777, 512)])
def test_split_partials_merge_to_single_pass(ctx, P):
    r = rng(ctx)
    hq, hkv, d = 16, 4, 256
    q, gate = normal(r, hq, d), normal(r, hq, d)
    keys, values = normal(r, ctx, hkv, d), normal(r, ctx, hkv, d)
    keys[r.random(ctx) < 0.01] *= 8
    maxp = -(-1025 // P)
    pm, ps, pv = orc.decode_partials(q, keys, values, ctx, P, maxp)
    out = orc.decode_merge(gate, pm, ps, pv, ctx, P, maxp)
    ref = orc.attention_core(q[None], keys, values, gate[None], ctx - 1)[0]
    np.testing.assert_allclose(out, ref, atol=2e-5, rtol=1e-4)
    # inactive partitions untouched
    active = -(-ctx // P)
    pm2 = pm.reshape(hq, maxp)
    assert np.all(np.isnan(pm2[:, active:])) and np.all(np.isfinite(pm2[:, :active]))


@pytest.mark.parametrize("ctx,P", [(300, 256), (777, 256), (1024, 512)])
def test_split_partials_representation_brute_force(ctx, P):
    # Pins the partial representation itself (cpp/kernels/qwen35_online_attention.cu:602-691):
    # per (head, partition) m is the partition's true max score in natural-log units
    # (q.k / sqrt(D)), l = sum exp(score - m) and o = sum exp(score - m) v, unnormalised;
    # a log2 max, a normalised o or a shifted sum would pass the merge invariant above but
    # fails here.  float64 brute force, GQA head h reads KV head h // 4.
    r = rng(ctx + P)
    hq, hkv, d = 16, 4, 256
    q = normal(r, hq, d)
    keys, values = normal(r, ctx, hkv, d), normal(r, ctx, hkv, d)
    keys[r.random(ctx) < 0.02] *= 8
    maxp = -(-1025 // P)
    pm, ps, pv = orc.decode_partials(q, keys, values, ctx, P, maxp)
    pm, ps, pv = pm.reshape(hq, maxp), ps.reshape(hq, maxp), pv.reshape(hq, maxp, d)
    for h in range(hq):
        kv = h // (hq // hkv)
        for p in range(-(-ctx // P)):
            k = keys[p * P:min(ctx, (p + 1) * P), kv].astype(np.float64)
            v = values[p * P:min(ctx, (p + 1) * P), kv].astype(np.float64)
            sc = k @ q[h].astype(np.float64) / np.sqrt(d)
            m = sc.max()
            w = np.exp(sc - m)
            assert abs(pm[h, p] - m) <= 1e-5 * max(1.0, abs(m))
            np.testing.assert_allclose(ps[h, p], w.sum(), rtol=1e-5)
            np.testing.assert_allclose(pv[h, p], w @ v, rtol=1e-4, atol=1e-4)


def test_decode_plan_table_matches_reference_test():
    t = KAT["decode_plan_table"]
    shape = tuple(t["shape"])
    modes = {"auto": 0, "single_block": 1, "split_k_256": 2, "split_k_512": 3}
    for c in t["cases"]:
        p = orc.decode_plan(shape, modes[c["requested"]], c["context"])
        assert p.resolved_mode == modes[c["resolved"]]
        assert p.context_bucket_tokens == c["bucket"]
        assert p.active_partition_capacity == c["capacity"]
        if "partition" in c:
            assert p.partition_tokens == c["partition"] and p.split_k_threshold_tokens == c["threshold"]
    lay = orc.decode_layout(shape, 2)
    assert (lay.partial_count, lay.max_offset_bytes, lay.sum_offset_bytes, lay.value_offset_bytes,
            lay.bytes) == tuple(t["layout_split_k_256"].values())
    assert orc.decode_layout(shape, 1).bytes == 0
    for e in t["errors"]:
        s = list(shape)
        if "head_dim" in e:
            s[3] = e["head_dim"]
        assert orc.decode_plan(tuple(s), modes[e["requested"]], e["context"]) is None


def test_decode_plan_closed_forms():
    # bucket = min(max_ctx, smallest 512*2^k >= ctx); capacity = ceil(bucket / P).
    for max_ctx in (1, 300, 512, 1025, 4096, 16384, 32768):
        for ctx in sorted({1, 2, 255, 256, 257, 511, 512, 513, max_ctx // 2 + 1, max_ctx}):
            if ctx < 1 or ctx > max_ctx:
                continue
            b = 512
            while b < ctx and b < max_ctx:
                b *= 2
            b = min(b, max_ctx)
            p = orc.decode_plan((1, 16, 4, 256, max_ctx), 2, ctx)
            assert p.context_bucket_tokens == b and p.active_partition_capacity == -(-b // 256)


@pytest.mark.parametrize("tokens,hk,hv,dk,dv", [(6, 2, 4, 5, 7), (9, 1, 2, 8, 8), (4, 16, 32, 128, 128)])
def test_delta_core_matches_reference_layer(tokens, hk, hv, dk, dv):
    """orc_delta_core (the recurrence the GPU core kernels are checked against)
    against the full reference layer (cpp/reference/qwen35.cpp:384-549): with a
    width-1 conv of weight 1 the layer is silu -> l2norm -> core -> RMSNorm x w x
    silu(z), so the core's inputs and the layer's output follow elementwise
    from the same raw token rows.  Uses the compiled reference when built,
    else the restatement pinned to it above."""
    r = rng(tokens * 31 + dk)
    hid = hv * dv
    cd = 2 * hk * dk + hv * dv
    stride = cd + 2 * hv + hid
    inp = normal(r, tokens * stride).reshape(tokens, stride)
    a_w = -np.exp(normal(r, hv))
    dt = normal(r, hv)
    nw = normal(r, dv)
    rs = normal(r, hv * dk * dv, scale=0.1)
    kw = dict(tokens=tokens, hidden=hid, hk=hk, hv=hv, dk=dk, dv=dv, width=1, eps=1e-6)
    want, _, want_state = orc.gated_delta_prefill(
        inp.ravel(), np.ones(cd, np.float32), a_w, dt, nw, np.zeros(0, np.float32), rs,
        use_reference=orc.ref_lib() is not None, **kw)

    x = inp.astype(np.float64)
    silu = lambda t: t / (1 + np.exp(-t))
    conv = silu(x[:, :cd])
    def l2(t):
        t = t.reshape(tokens, hk, dk)
        return t / np.sqrt((t * t).sum(-1, keepdims=True) + 1e-6)
    q = l2(conv[:, :hk * dk])
    k = l2(conv[:, hk * dk:2 * hk * dk])
    v = conv[:, 2 * hk * dk:].reshape(tokens, hv, dv)
    beta = 1 / (1 + np.exp(-x[:, cd:cd + hv]))
    log_decay = a_w * np.logaddexp(0, x[:, cd + hv:cd + 2 * hv] + dt)
    raw, state = orc.delta_core(q, k, v, beta, log_decay, 1 / np.sqrt(dk), rs.reshape(hv, dk, dv))
    raw = raw.astype(np.float64)
    norm = raw / np.sqrt((raw * raw).mean(-1, keepdims=True) + 1e-6) * nw
    got = norm.reshape(tokens, hid) * silu(x[:, cd + 2 * hv:])
    np.testing.assert_allclose(got.ravel(), want, rtol=2e-4, atol=2e-5)
    np.testing.assert_allclose(state.ravel(), want_state, rtol=2e-4, atol=2e-6)


# ---------------------------------------------------- attention producers
@ref_needed
@pytest.mark.parametrize("tokens,heads,d,rot,pos,base", [(3, 3, 13, 8, 5, 1e4), (2, 1, 256, 64, 0, 1e7),
                                                         (4, 16, 256, 64, 1000, 1e7), (1, 2, 8, 8, 7, 10.0)])
def test_qk_norm_rope_matches_compiled_reference(tokens, heads, d, rot, pos, base):
    r = rng(tokens * d + rot)
    x = normal(r, tokens * heads * d).reshape(tokens, heads, d)
    w = normal(r, d, scale=0.5)
    a = orc.qk_norm_rope(x, w, rot, pos, base, 1e-5)
    b = orc.qk_norm_rope(x, w, rot, pos, base, 1e-5, use_reference=True)
    np.testing.assert_array_equal(a, b)


def test_qk_norm_rope_invariants():
    """What the mathematics fixes, independent of the restatement's code:
    position 0 is no rotation; rotation keeps each (p, p + rot/2) pair's norm;
    RoPE is the complex product (x_p + i x_{p+rot/2}) e^{i pos base^(-2p/rot)};
    and after RoPE q(m).k(n) depends on m - n only."""
    r = rng(77)
    d, rot, base = 32, 16, 100.0
    x = normal(r, d).reshape(1, 1, d)
    w = normal(r, d, scale=0.5) + 1.0
    ms = np.sqrt((x.astype(np.float64) ** 2).mean() + 1e-6)
    normed = (x / ms * w).astype(np.float64)
    at0 = orc.qk_norm_rope(x, w, rot, 0, base, 1e-6)
    np.testing.assert_allclose(at0, normed, rtol=1e-6, atol=1e-6)
    pos = 37
    y = orc.qk_norm_rope(x, w, rot, pos, base, 1e-6)[0, 0].astype(np.float64)
    n = normed[0, 0]
    half = rot // 2
    z = (n[:half] + 1j * n[half:rot]) * np.exp(1j * pos * base ** (-2.0 * np.arange(half) / rot))
    np.testing.assert_allclose(y[:half], z.real, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(y[half:rot], z.imag, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(y[rot:], n[rot:], rtol=1e-6, atol=1e-6)  # untouched dims
    np.testing.assert_allclose(y[:half] ** 2 + y[half:rot] ** 2, n[:half] ** 2 + n[half:rot] ** 2,
                               rtol=1e-5)
    q, k = normal(r, d).reshape(1, 1, d), normal(r, d).reshape(1, 1, d)
    ones = np.ones(d, np.float32)
    def dot(m, nn):
        a = orc.qk_norm_rope(q, ones, rot, m, base, 1e-6)[0, 0].astype(np.float64)
        b = orc.qk_norm_rope(k, ones, rot, nn, base, 1e-6)[0, 0].astype(np.float64)
        return a @ b
    assert abs(dot(10, 3) - dot(107, 100)) < 1e-4 and abs(dot(10, 3) - dot(3, 10)) > 1e-3


def test_split_full_query_gate_layout():
    heads, d = 3, 5
    qg = np.arange(2 * 2 * heads * d, dtype=np.float32)  # 2 tokens
    q, g = orc.split_full_query_gate(qg, heads, d)
    blocks = qg.reshape(2, heads, 2, d)
    np.testing.assert_array_equal(q, blocks[:, :, 0])
    np.testing.assert_array_equal(g, blocks[:, :, 1])


def test_pack_linear_delta_input_layout():
    a = np.arange(6, dtype=np.float32).reshape(2, 3)
    b = np.array([[100.], [101.]], np.float32)
    got = orc.pack_linear_delta_input(a, b, b + 10, a + 50)
    np.testing.assert_array_equal(got, np.concatenate([a, b, b + 10, a + 50], axis=1))
