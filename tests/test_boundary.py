"""CPU tests of the drop-in boundary: the C-ABI library loads and exports every
symbol include/raftinfer_amd.h declares; host-side planning and sizing are
bit-exact with the oracle; validation failures are raised before any launch
(so no GPU is needed)."""
import ctypes
import pathlib
import re

import numpy as np
import pytest

from oracle import pyoracle as orc
from raftinfer_amd import _lib, ops

ROOT = pathlib.Path(__file__).resolve().parent.parent
S = ops.Qwen35AttentionShape


def declared_symbols():
    text = (ROOT / "include" / "raftinfer_amd.h").read_text()
    return sorted(set(re.findall(r"\b(raftinfer_amd_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_symbols()
    assert len(names) >= 20
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)


def test_product_does_not_reference_oracle():
    for p in (ROOT / "raftinfer_amd").rglob("*"):
        if p.suffix in (".py", ".hip", ".cpp", ".hpp", ".h"):
            assert "oracle" not in p.read_text().replace("Oracle", ""), p


@pytest.mark.parametrize("max_ctx", [1, 17, 255, 256, 257, 512, 1025, 4096, 16384, 32768])
@pytest.mark.parametrize("mode", [0, 1, 2, 3])
def test_decode_plan_bit_exact_with_oracle(max_ctx, mode):
    ctxs = sorted({1, 2, 128, 255, 256, 257, 511, 512, 513, 777, 1024, 1025, 4095, 4096,
                   max_ctx - 1, max_ctx, max_ctx + 1})
    for ctx in ctxs:
        shape = S(1, 16, 4, 256, max_ctx, 0)
        want = orc.decode_plan((1, 16, 4, 256, max_ctx), mode, ctx)
        if want is None:
            with pytest.raises(ops.Qwen35PrimitiveError):
                ops.qwen35_online_decode_plan(shape, mode, ctx)
            continue
        got = ops.qwen35_online_decode_plan(shape, mode, ctx)
        assert got == (want.resolved_mode, want.partition_tokens, want.split_k_threshold_tokens,
                       want.context_bucket_tokens, want.active_partition_capacity)


def test_decode_plan_bucket_at_the_size_limit():
    # The bucket's overflow guard (cpp/kernels/qwen35_online_attention.cu:188-191): contexts
    # next to and past the largest power of two a size_t holds, single-block plans.
    top = 2 ** 64 - 1
    for ctx in (2 ** 62 + 1, 2 ** 63 - 1, 2 ** 63, 2 ** 63 + 1, top - 1, top):
        for max_ctx in (ctx, top):
            want = orc.decode_plan((1, 16, 4, 256, max_ctx), 1, ctx)
            got = ops.qwen35_online_decode_plan(S(1, 16, 4, 256, max_ctx, 0), 1, ctx)
            assert got == (want.resolved_mode, want.partition_tokens, want.split_k_threshold_tokens,
                           want.context_bucket_tokens, want.active_partition_capacity), (ctx, max_ctx)


@pytest.mark.parametrize("shape", [(1, 16, 4, 256, 4096), (1, 16, 4, 256, 1025), (1, 16, 4, 256, 1),
                                   (1, 16, 4, 255, 4096), (2, 16, 4, 256, 64), (1, 8, 4, 256, 64)])
def test_workspace_layout_bit_exact_with_oracle(shape):
    for mode in (1, 2, 3, 0, 7):
        want = orc.decode_layout(shape, mode)
        if want is None:
            with pytest.raises(ops.Qwen35PrimitiveError):
                ops.qwen35_online_decode_workspace_layout(S(*shape, 0), mode)
            continue
        got = ops.qwen35_online_decode_workspace_layout(S(*shape, 0), mode)
        assert got == (want.partial_count, want.max_offset_bytes, want.sum_offset_bytes,
                       want.value_offset_bytes, want.bytes)


def test_headline_workspace_is_264192_bytes():
    # docs/benchmarks.md:17-20 of the reference: max_ctx 4096, P = 256.
    assert ops.qwen35_online_decode_workspace_layout(S(1, 16, 4, 256, 4096, 0), 2)[4] == 264192


def test_sizing_formulas():
    # cpp/tests/qwen35_cuda_attention_test.cu:277-287
    shape = S(1, 2, 1, 7, 4, 0)
    mat = ops.Qwen35AttentionLaunchPolicy(0, 0, 0)
    onl = ops.Qwen35AttentionLaunchPolicy(1, 1, 0)
    assert ops.qwen35_attention_cache_bytes(shape, mat) == 2 * 4 * 1 * 7 * 4
    assert ops.qwen35_attention_workspace_bytes(shape, mat) == 1 * 2 * 1 * 4
    assert ops.qwen35_attention_cache_bytes(shape, onl) == 2 * 4 * 1 * 7 * 2
    assert ops.qwen35_attention_workspace_bytes(shape, onl) == 0
    assert ops.qwen35_attention_workspace_floats(S(3, 4, 2, 8, 10, 5)) == 3 * 4 * 8


def test_prefill_supported_contract():
    # cpp/tests/qwen35_cuda_attention_test.cu:221-259
    sp = S(4, 4, 2, 64, 4, 0)
    f32_online = ops.Qwen35AttentionLaunchPolicy(1, 0, 0)
    bf16_online = ops.Qwen35AttentionLaunchPolicy(1, 1, 0)
    ref = ops.Qwen35AttentionLaunchPolicy(0, 0, 0)
    assert ops.qwen35_online_attention_prefill_supported(sp, 1, f32_online)
    assert ops.qwen35_online_attention_prefill_supported(sp, 3, bf16_online)
    assert not ops.qwen35_online_attention_prefill_supported(sp, 2, f32_online)
    assert not ops.qwen35_online_attention_prefill_supported(sp, 1, ref)
    assert ops.qwen35_online_attention_prefill_supported(sp, 1, ops.Qwen35AttentionLaunchPolicy(1, 0, 1))
    assert not ops.qwen35_online_attention_prefill_supported(sp, 1, ops.Qwen35AttentionLaunchPolicy(1, 0, 99))
    assert not ops.qwen35_online_attention_prefill_supported(S(1, 4, 2, 64, 4, 0), 1, f32_online)
    assert not ops.qwen35_online_attention_prefill_supported(S(4, 4, 2, 257, 4, 0), 1, f32_online)


class FakeTensor:
    """A host stand-in with a non-null address; validation rejects the call
    before any device access."""

    def __init__(self, nbytes=1 << 20, addr=0x100000):
        self._n, self._a = nbytes, addr

    def data_ptr(self):
        return self._a

    def numel(self):
        return self._n

    def element_size(self):
        return 1


def test_attention_validation_errors_before_launch():
    f = FakeTensor()
    shape = S(1, 2, 1, 7, 4, 0)
    bf16_online = ops.Qwen35AttentionLaunchPolicy(1, 1, 0)
    bf16_mat = ops.Qwen35AttentionLaunchPolicy(0, 1, 0)
    stream = 0x1234
    need = ops.qwen35_attention_cache_bytes(shape, bf16_online)
    with pytest.raises(ops.Qwen35PrimitiveError, match="too small"):
        ops.qwen35_causal_attention(f, f, f, f, f, f, f, shape, 3, bf16_online, stream,
                                    kv_cache_bytes=need - 1, workspace_bytes=0)
    with pytest.raises(ops.Qwen35PrimitiveError, match="F32 KV cache"):
        ops.qwen35_causal_attention(f, f, f, f, f, f, f, shape, 3, bf16_mat, stream,
                                    workspace_bytes=8)
    with pytest.raises(ops.Qwen35PrimitiveError, match="forbids logits workspace"):
        ops.qwen35_causal_attention(f, f, f, f, f, f, f, S(4, 4, 2, 64, 4, 0), 1,
                                    ops.Qwen35AttentionLaunchPolicy(1, 0, 0), stream,
                                    workspace_bytes=0)
    with pytest.raises(ops.Qwen35PrimitiveError, match="stream is null"):
        ops.qwen35_causal_attention(f, f, f, f, f, f, None, S(4, 4, 2, 64, 4, 0), 1,
                                    ops.Qwen35AttentionLaunchPolicy(1, 0, 0), 0)
    with pytest.raises(ops.Qwen35PrimitiveError, match="unsupported"):
        ops.qwen35_causal_attention(f, f, f, f, f, f, None, S(4, 4, 2, 257, 4, 0), 1,
                                    ops.Qwen35AttentionLaunchPolicy(1, 0, 0), stream)


def test_decode_validation_errors_before_launch():
    f = FakeTensor()
    model = S(1, 16, 4, 256, 32, 0)
    plan = ops.qwen35_online_decode_plan(model, 1, 1)
    stream = 0x1234
    for shape, act, layout, cache_bytes in [(S(1, 16, 4, 255, 32, 0), 1, 0, 1 << 40),
                                            (model, 2, 0, 1 << 40), (model, 1, 0, 4),
                                            (model, 1, 99, 1 << 40)]:
        with pytest.raises(ops.Qwen35PrimitiveError):
            ops.qwen35_online_attention_decode(f, f, f, f, f, f, None, shape, act, 0, layout,
                                               plan=plan, stream=stream, kv_cache_bytes=cache_bytes)
    split = ops.qwen35_online_decode_plan(S(1, 16, 4, 256, 1025, 0), 2, 257)
    lay = ops.qwen35_online_decode_workspace_layout(S(1, 16, 4, 256, 1025, 0), 2)
    with pytest.raises(ops.Qwen35PrimitiveError, match="workspace is too small"):
        ops.qwen35_online_attention_decode(f, f, f, f, f, f, f, S(1, 16, 4, 256, 1025, 256), 3, 1,
                                           1, plan=split, stream=stream, workspace_bytes=lay[4] - 1)
    bad = list(split)
    bad[4] += 1
    with pytest.raises(ops.Qwen35PrimitiveError, match="capacity is inconsistent"):
        ops.qwen35_online_attention_decode(f, f, f, f, f, f, f, S(1, 16, 4, 256, 1025, 256), 3, 1,
                                           1, plan=tuple(bad), stream=stream)
    with pytest.raises(ops.Qwen35PrimitiveError, match="exceeds the planned bucket"):
        ops.qwen35_online_attention_decode(f, f, f, f, f, f, f, S(1, 16, 4, 256, 1025, 600), 3, 1,
                                           1, plan=split, stream=stream)


def test_delta_workspace_linear_and_validation():
    G = ops.GatedDeltaShape
    one, four = G(1, 28, 2, 4, 5, 7, 3, 1e-6), G(4, 28, 2, 4, 5, 7, 3, 1e-6)
    # cpp/tests/qwen35_cuda_delta_test.cu:785-787
    assert ops.qwen35_gated_delta_workspace_bytes(four) == 4 * ops.qwen35_gated_delta_workspace_bytes(one)
    # The model shape at T=512: the per-token buffers (conv outputs, raw output, beta and
    # decay: T (conv_dim + hidden + 2 hv) fp32) plus one 33,024-byte T-record per (value
    # head, 64-token chunk); the reference's own workspace is T (conv_dim + hidden) fp32
    # (cpp/kernels/qwen35_delta.cu:757-759), 25,165,824 bytes here.
    model = G(512, 4096, 16, 32, 128, 128, 4, 1e-6)
    per_token = 512 * (8192 + 4096 + 64) * 4
    want = ((per_token + 255) // 256) * 256 + 32 * 8 * 33024
    assert ops.qwen35_gated_delta_workspace_bytes(model) == want
    assert want <= 1.4 * 512 * (8192 + 4096) * 4
    # other dk = dv = 128 shapes keep the W/U records (147,712 bytes each)
    small = G(512, 512, 2, 4, 128, 128, 4, 1e-6)
    per_token = 512 * (1024 + 512 + 8) * 4
    assert ops.qwen35_gated_delta_workspace_bytes(small) == ((per_token + 255) // 256) * 256 + 4 * 8 * 147712
    f = FakeTensor()
    bad_shapes = [G(0, 28, 2, 4, 5, 7, 3, 1e-6), G(1, 29, 2, 4, 5, 7, 3, 1e-6),
                  G(1, 21, 2, 3, 5, 7, 3, 1e-6), G(1, 28, 2, 4, 5, 7, 0, 1e-6),
                  G(1, 28, 2, 4, 5, 7, 3, float("nan")), G(2 ** 63, 28, 2, 4, 5, 7, 3, 1e-6)]
    for s in bad_shapes:
        with pytest.raises(ops.Qwen35DeltaError):
            ops.qwen35_gated_delta(f, f, f, f, f, f, f, f, f, s, 2, 2, stream=0x1234)
    ws = ops.qwen35_gated_delta_workspace_bytes(one)
    with pytest.raises(ops.Qwen35DeltaError, match="workspace is too small"):
        ops.qwen35_gated_delta(f, f, f, f, f, f, f, f, f, one, 2, 2, stream=0x1234,
                               workspace_bytes=ws - 1)
    with pytest.raises(ops.Qwen35DeltaError, match="dtype"):
        ops.qwen35_gated_delta(f, f, f, f, f, f, f, f, f, one, 100, 100, stream=0x1234,
                               workspace_bytes=ws)
    with pytest.raises(ops.Qwen35DeltaError, match="unknown gated-delta schedule"):
        ops.qwen35_gated_delta(f, f, f, f, f, f, f, f, f, one, 2, 2, stream=0x1234,
                               workspace_bytes=ws, policy=ops.GatedDeltaLaunchPolicy(99))
    mis = FakeTensor(addr=0x100001)
    with pytest.raises(ops.Qwen35DeltaError, match="not dtype-aligned"):
        ops.qwen35_gated_delta(mis, f, f, f, f, f, f, f, f, one, 2, 2, stream=0x1234,
                               workspace_bytes=ws)


def test_producer_validation_errors_before_launch():
    # cpp/tests/qwen35_cuda_primitives_test.cu:608-660 (the qk_norm_rope cases)
    f = FakeTensor()
    Q = ops.QkNormRopeShape
    inf, nan = float("inf"), float("nan")
    cases = [(Q(1, 1, 7, 9, 0, 1e4), 1e-5, "rotary_dim exceeds head_dim"),
             (Q(1, 1, 8, 5, 0, 1e4), 1e-5, "rotary_dim must be even"),
             (Q(1, 1, 8, 0, 0, 1e4), 1e-5, "rotary_dim must be positive"),
             (Q(1, 1, 8, 4, 0, inf), 1e-5, "rope_base must be finite"),
             (Q(1, 1, 8, 4, 0, nan), 1e-5, "rope_base must be finite"),
             (Q(1, 1, 8, 4, 0, 1e4), inf, "epsilon must be finite"),
             (Q(1, 1, 8, 4, 0, 1e4), nan, "epsilon must be finite"),
             (Q(2, 1, 8, 4, 2 ** 64 - 1, 1e4), 1e-5, "position range overflow"),
             (Q(0, 1, 8, 4, 0, 1e4), 1e-5, "tokens must be positive")]
    for shape, eps, msg in cases:
        with pytest.raises(ops.Qwen35PrimitiveError, match=msg):
            ops.qwen35_qk_norm_rope(f, f, f, shape, eps, 2, 2, stream=0x1234)
    with pytest.raises(ops.Qwen35PrimitiveError, match="weight dtype is incompatible"):
        ops.qwen35_qk_norm_rope(f, f, f, Q(1, 1, 8, 4, 0, 1e4), 1e-5, 3, 2, stream=0x1234)
    with pytest.raises(ops.Qwen35PrimitiveError, match="unsupported Qwen3.5 primitive dtype"):
        ops.qwen35_split_full_query_gate(f, f, f, 1, 1, 8, 7, stream=0x1234)
    with pytest.raises(ops.Qwen35PrimitiveError, match="stream is null"):
        ops.qwen35_split_full_query_gate(f, f, f, 1, 1, 8, 1, stream=0)
    with pytest.raises(ops.Qwen35PrimitiveError, match="input pointer is null"):
        ops.qwen35_split_full_query_gate(None, f, f, 1, 1, 8, 1, stream=0x1234)


def test_pack_validation_errors_before_launch():
    # cpp/kernels/qwen35_primitives.cu:768-793: every null pointer, zero width
    f = FakeTensor()
    for i, msg in enumerate(["qkv pointer", "beta pointer", "alpha pointer", "gate pointer",
                             "output pointer"]):
        args = [f] * 5
        args[i] = None
        with pytest.raises(ops.Qwen35PrimitiveError, match=msg):
            ops.qwen35_pack_linear_delta_input(*args, 1, 4, 1, 1, 4, 3, stream=0x1234)
    for i, msg in enumerate(["qkv_width", "beta_width", "alpha_width", "gate_width"]):
        w = [4, 1, 1, 4]
        w[i] = 0
        with pytest.raises(ops.Qwen35PrimitiveError, match=msg):
            ops.qwen35_pack_linear_delta_input(f, f, f, f, f, 1, *w, 3, stream=0x1234)
    with pytest.raises(ops.Qwen35PrimitiveError, match="width overflow"):
        ops.qwen35_pack_linear_delta_input(f, f, f, f, f, 1, 2 ** 64 - 2, 1, 1, 4, 3, stream=0x1234)


def test_c_abi_null_result_pointer_is_an_invalid_argument():
    # A sizing / planning call with a null result pointer returns an error status with a
    # message instead of writing through it.
    import ctypes
    from raftinfer_amd import _lib
    lib = _lib.load()
    shape = _lib.AttentionShape(1, 16, 4, 256, 4096, 4095)
    rc = lib.raftinfer_amd_attention_workspace_floats(shape, None)
    assert rc == 1  # RAFTINFER_AMD_INVALID_ARGUMENT
    assert b"result pointer is null" in lib.raftinfer_amd_last_error_message()
    rc = lib.raftinfer_amd_gated_delta_core_workspace_bytes(_lib.DeltaCoreShape(512, 16, 32, 128, 128), None)
    assert rc == 1


def test_batched_decode_requires_aligned_workspace():
    # The batched merge reads whole partial rows with 16-byte loads.
    big = FakeTensor(nbytes=1 << 40)
    lens = FakeTensor(addr=0x200000)
    q = FakeTensor(nbytes=1 << 40, addr=0x300000)
    q.shape = (2, 16, 256)
    stride = 2 * 4 * 1024 * 256 * 2
    with pytest.raises(ops.Qwen35PrimitiveError, match="workspace must be 16-byte aligned"):
        ops.qwen35_online_attention_decode_batched(
            q, big, big, big, big, big, lens, FakeTensor(nbytes=1 << 40, addr=0x400004), 1024,
            stride, stream=0x1234)
