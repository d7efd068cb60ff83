"""Host-side mirror of the reference kernel interface for the attention /
gated-delta hot path, over torch device tensors.

Names, argument meaning and error behaviour follow the reference's
cpp/kernels/qwen35_attention.cuh, qwen35_online_attention.cuh and
qwen35_delta.cuh: validation failures raise Qwen35PrimitiveError (attention)
or Qwen35DeltaError (delta) before anything is enqueued.  Every call goes
through libraftinfer_amd.so; nothing here computes on the CPU.  Tensors are
caller-owned device buffers; byte sizes passed to the library are the tensors'
own sizes.  ``stream`` is a torch.cuda.Stream (or raw hipStream_t int); the
default is the current stream, which must not be the null stream.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

from . import _lib
from ._lib import (AttentionPolicy, AttentionShape, BatchedDecodeShape, DecodeLayout, DecodePlan,
                   DeltaCoreShape, DeltaPolicy, DeltaShape, RaftInferError)

# cpp/execution/qwen35_execution_policy.hpp:7-27 and cpp/include/raftinfer/tensor.h:10-15
MATERIALIZED, ONLINE_TILED = 0, 1
AUTO, SINGLE_BLOCK, SPLIT_K_256, SPLIT_K_512 = 0, 1, 2, 3
CACHE_F32, CACHE_BF16 = 0, 1
TOKEN_MAJOR, HEAD_MAJOR = 0, 1
DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 1, 2, 3
SCHEDULE_CURRENT, SCHEDULE_PREFILL_CANDIDATE, SCHEDULE_DECODE_CANDIDATE = 0, 1, 2


class Qwen35PrimitiveError(RaftInferError):
    """Attention validation / launch failure (cpp/kernels/qwen35_primitives.cuh:15-19)."""


class Qwen35DeltaError(RaftInferError):
    """Gated-delta validation / launch failure (cpp/kernels/qwen35_delta.cuh:14-18)."""


def _call(err_type, status: int) -> None:
    try:
        _lib.check(status)
    except RaftInferError as e:
        raise err_type(e.status, str(e)) from None


@dataclass(frozen=True)
class Qwen35AttentionShape:
    tokens: int
    query_heads: int
    kv_heads: int
    head_dim: int
    max_context_tokens: int
    past_tokens: int

    def c(self) -> AttentionShape:
        return AttentionShape(self.tokens, self.query_heads, self.kv_heads, self.head_dim,
                              self.max_context_tokens, self.past_tokens)


@dataclass(frozen=True)
class Qwen35AttentionLaunchPolicy:
    implementation: int = ONLINE_TILED
    kv_cache_dtype: int = CACHE_BF16
    kv_cache_layout: int = HEAD_MAJOR

    def c(self) -> AttentionPolicy:
        return AttentionPolicy(self.implementation, self.kv_cache_dtype, self.kv_cache_layout)


@dataclass(frozen=True)
class GatedDeltaShape:
    tokens: int
    hidden_size: int
    key_heads: int
    value_heads: int
    key_dim: int
    value_dim: int
    conv_width: int
    epsilon: float

    def c(self) -> DeltaShape:
        return DeltaShape(self.tokens, self.hidden_size, self.key_heads, self.value_heads,
                          self.key_dim, self.value_dim, self.conv_width, self.epsilon)


@dataclass(frozen=True)
class GatedDeltaLaunchPolicy:
    schedule: int = SCHEDULE_CURRENT
    warps_per_block: int = 4
    transposed_boundary_state: bool = False

    def c(self) -> DeltaPolicy:
        return DeltaPolicy(self.schedule, self.warps_per_block, int(self.transposed_boundary_state))


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _fptr(t):
    return None if t is None else ctypes.cast(t.data_ptr(), ctypes.POINTER(ctypes.c_float))


def _nbytes(t) -> int:
    return 0 if t is None else t.numel() * t.element_size()


def _stream(stream) -> ctypes.c_void_p:
    if stream is None:
        import torch
        stream = torch.cuda.current_stream()
    handle = stream if isinstance(stream, int) else stream.cuda_stream
    return ctypes.c_void_p(handle)


def _dtype_code(t) -> int:
    import torch
    return {torch.float32: DTYPE_F32, torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16}.get(
        t.dtype, 0)


# ------------------------------------------------------------- sizing API

def qwen35_attention_workspace_floats(shape: Qwen35AttentionShape) -> int:
    out = ctypes.c_size_t()
    _call(Qwen35PrimitiveError,
          _lib.load().raftinfer_amd_attention_workspace_floats(shape.c(), ctypes.byref(out)))
    return out.value


def qwen35_attention_cache_bytes(shape, policy: Qwen35AttentionLaunchPolicy) -> int:
    out = ctypes.c_size_t()
    _call(Qwen35PrimitiveError,
          _lib.load().raftinfer_amd_attention_cache_bytes(shape.c(), policy.c(), ctypes.byref(out)))
    return out.value


def qwen35_attention_workspace_bytes(shape, policy: Qwen35AttentionLaunchPolicy) -> int:
    out = ctypes.c_size_t()
    _call(Qwen35PrimitiveError, _lib.load().raftinfer_amd_attention_workspace_bytes(
        shape.c(), policy.c(), ctypes.byref(out)))
    return out.value


def qwen35_online_decode_plan(shape, requested: int, context_tokens: int) -> tuple:
    """(resolved_mode, partition_tokens, split_k_threshold_tokens, context_bucket_tokens,
    active_partition_capacity) -- cpp/kernels/qwen35_online_attention.cu:1071-1109."""
    out = DecodePlan()
    _call(Qwen35PrimitiveError, _lib.load().raftinfer_amd_online_decode_plan(
        shape.c(), requested, context_tokens, ctypes.byref(out)))
    return out.as_tuple()


def qwen35_online_decode_workspace_layout(shape, resolved_mode: int) -> tuple:
    """(partial_count, max_offset, sum_offset, value_offset, bytes) -- :1111-1143."""
    out = DecodeLayout()
    _call(Qwen35PrimitiveError, _lib.load().raftinfer_amd_online_decode_workspace_layout(
        shape.c(), resolved_mode, ctypes.byref(out)))
    return out.as_tuple()


def qwen35_online_attention_prefill_supported(shape, activation_dtype: int,
                                              policy: Qwen35AttentionLaunchPolicy) -> bool:
    return bool(_lib.load().raftinfer_amd_online_attention_prefill_supported(
        shape.c(), activation_dtype, policy.c()))


def qwen35_gated_delta_workspace_bytes(shape: GatedDeltaShape) -> int:
    out = ctypes.c_size_t()
    _call(Qwen35DeltaError,
          _lib.load().raftinfer_amd_gated_delta_workspace_bytes(shape.c(), ctypes.byref(out)))
    return out.value


def qwen35_gated_delta_core_workspace_bytes(tokens, key_heads, value_heads, key_dim,
                                            value_dim) -> int:
    out = ctypes.c_size_t()
    _call(Qwen35DeltaError, _lib.load().raftinfer_amd_gated_delta_core_workspace_bytes(
        DeltaCoreShape(tokens, key_heads, value_heads, key_dim, value_dim), ctypes.byref(out)))
    return out.value


def qwen35_batched_decode_workspace_bytes(sequences, max_context_tokens, cache_stride_bytes,
                                          single_block_max_tokens=512) -> int:
    out = ctypes.c_size_t()
    _call(Qwen35PrimitiveError, _lib.load().raftinfer_amd_batched_decode_workspace_bytes(
        BatchedDecodeShape(sequences, max_context_tokens, cache_stride_bytes,
                           single_block_max_tokens), ctypes.byref(out)))
    return out.value


# ------------------------------------------------------------ enqueue API

def qwen35_causal_attention(query, key, value, gate, output, kv_cache, workspace, shape,
                            activation_dtype: int, policy: Qwen35AttentionLaunchPolicy,
                            stream=None, kv_cache_bytes=None, workspace_bytes=None) -> None:
    _call(Qwen35PrimitiveError, _lib.load().raftinfer_amd_causal_attention(
        _ptr(query), _ptr(key), _ptr(value), _ptr(gate), _ptr(output), _ptr(kv_cache),
        _nbytes(kv_cache) if kv_cache_bytes is None else kv_cache_bytes, _ptr(workspace),
        _nbytes(workspace) if workspace_bytes is None else workspace_bytes, shape.c(),
        activation_dtype, policy.c(), _stream(stream)))


def qwen35_online_attention_prefill(query, key, value, gate, output, kv_cache, shape,
                                    activation_dtype, cache_dtype, cache_layout, stream=None,
                                    kv_cache_bytes=None) -> None:
    _call(Qwen35PrimitiveError, _lib.load().raftinfer_amd_online_attention_prefill(
        _ptr(query), _ptr(key), _ptr(value), _ptr(gate), _ptr(output), _ptr(kv_cache),
        _nbytes(kv_cache) if kv_cache_bytes is None else kv_cache_bytes, shape.c(),
        activation_dtype, cache_dtype, cache_layout, _stream(stream)))


def qwen35_online_attention_decode(query, key, value, gate, output, kv_cache, workspace, shape,
                                   activation_dtype, cache_dtype, cache_layout, plan=None,
                                   device_position=None, stream=None, kv_cache_bytes=None,
                                   workspace_bytes=None) -> None:
    """plan=None selects the plan-less single-block overload
    (cpp/kernels/qwen35_online_attention.cu:1316-1328)."""
    lib = _lib.load()
    pos = None if device_position is None else ctypes.cast(device_position.data_ptr(),
                                                           ctypes.POINTER(ctypes.c_uint32))
    cache_bytes = _nbytes(kv_cache) if kv_cache_bytes is None else kv_cache_bytes
    if plan is None:
        _call(Qwen35PrimitiveError, lib.raftinfer_amd_online_attention_decode_single(
            _ptr(query), _ptr(key), _ptr(value), _ptr(gate), _ptr(output), _ptr(kv_cache),
            cache_bytes, shape.c(), activation_dtype, cache_dtype, cache_layout, pos,
            _stream(stream)))
        return
    _call(Qwen35PrimitiveError, lib.raftinfer_amd_online_attention_decode(
        _ptr(query), _ptr(key), _ptr(value), _ptr(gate), _ptr(output), _ptr(kv_cache), cache_bytes,
        _ptr(workspace), _nbytes(workspace) if workspace_bytes is None else workspace_bytes,
        shape.c(), activation_dtype, cache_dtype, cache_layout, DecodePlan(*plan), pos,
        _stream(stream)))


@dataclass
class Qwen35FusedNormRope:
    """The producer parameters of the fused attention entry points."""
    query_norm_weight: object  # device tensor [head_dim]
    key_norm_weight: object
    rotary_dim: int
    rope_base: float
    epsilon: float

    def c(self):
        wd = _dtype_code(self.query_norm_weight)
        return _lib.FusedNormRope(_ptr(self.query_norm_weight), _ptr(self.key_norm_weight), wd,
                                  self.rotary_dim, self.rope_base, self.epsilon)


def qwen35_online_attention_decode_fused(query_gate, key, value, output, kv_cache, workspace, shape,
                                         norm: Qwen35FusedNormRope, cache_dtype, cache_layout, plan,
                                         device_position=None, stream=None) -> None:
    """The q split + RMSNorm + RoPE of q and k fused into the decode attention."""
    pos = None if device_position is None else ctypes.cast(device_position.data_ptr(),
                                                           ctypes.POINTER(ctypes.c_uint32))
    _call(Qwen35PrimitiveError, _lib.load().raftinfer_amd_online_attention_decode_fused(
        _ptr(query_gate), _ptr(key), _ptr(value), _ptr(output), _ptr(kv_cache), _nbytes(kv_cache),
        _ptr(workspace), _nbytes(workspace), shape.c(), norm.c(), cache_dtype, cache_layout,
        DecodePlan(*plan), pos, _stream(stream)))


def qwen35_online_attention_prefill_fused(query_gate, key, value, output, kv_cache, shape,
                                          norm: Qwen35FusedNormRope, cache_dtype=CACHE_BF16,
                                          cache_layout=HEAD_MAJOR, stream=None) -> None:
    """The q split + RMSNorm + RoPE of q and k fused into the causal gated prefill."""
    _call(Qwen35PrimitiveError, _lib.load().raftinfer_amd_online_attention_prefill_fused(
        _ptr(query_gate), _ptr(key), _ptr(value), _ptr(output), _ptr(kv_cache), _nbytes(kv_cache),
        shape.c(), norm.c(), cache_dtype, cache_layout, _stream(stream)))


def qwen35_online_attention_static_workspace_bytes() -> int:
    return int(_lib.load().raftinfer_amd_online_attention_static_workspace_bytes())


def qwen35_online_attention_decode_static_workspace(query, key, value, gate, output, kv_cache, shape,
                                                    activation_dtype, cache_dtype, cache_layout,
                                                    plan, device_position=None, stream=None) -> None:
    """The allocation-free decode: as qwen35_online_attention_decode with a
    plan, with the split-K workspace in the library's static device array."""
    pos = None if device_position is None else ctypes.cast(device_position.data_ptr(),
                                                           ctypes.POINTER(ctypes.c_uint32))
    _call(Qwen35PrimitiveError, _lib.load().raftinfer_amd_online_attention_decode_static_workspace(
        _ptr(query), _ptr(key), _ptr(value), _ptr(gate), _ptr(output), _ptr(kv_cache),
        _nbytes(kv_cache), shape.c(), activation_dtype, cache_dtype, cache_layout, DecodePlan(*plan),
        pos, _stream(stream)))


def qwen35_online_attention_decode_batched(query, key, value, gate, output, kv_cache,
                                           context_lengths, workspace, max_context_tokens,
                                           cache_stride_bytes, single_block_max_tokens=512,
                                           activation_dtype=DTYPE_BF16, stream=None) -> None:
    shape = BatchedDecodeShape(query.shape[0], max_context_tokens, cache_stride_bytes,
                               single_block_max_tokens)
    _call(Qwen35PrimitiveError, _lib.load().raftinfer_amd_online_attention_decode_batched(
        _ptr(query), _ptr(key), _ptr(value), _ptr(gate), _ptr(output), _ptr(kv_cache),
        _nbytes(kv_cache), ctypes.cast(context_lengths.data_ptr(), ctypes.POINTER(ctypes.c_uint32)),
        _ptr(workspace), _nbytes(workspace), shape, activation_dtype, _stream(stream)))


class Qwen35DecodeAttentionGraphs:
    """Per-context-bucket captured decode steps (include/raftinfer_amd/hip_graph_decode.hpp),
    the variant table of cpp/execution/qwen35_executor.cu:2191-2226 on hipGraph.  The
    tensors must outlive the object; ``device_position`` (int32/uint32, 1 element) is read
    by the kernels at replay time."""

    def __init__(self, shape, mode, activation_dtype, cache_dtype, cache_layout, query, key, value,
                 gate, output, kv_cache, workspace, device_position, stream=None, device_id=0):
        self._lib = _lib.load()
        self._keep = (query, key, value, gate, output, kv_cache, workspace, device_position)
        pos = ctypes.cast(device_position.data_ptr(), ctypes.POINTER(ctypes.c_uint32))
        buf = _lib.DecodeBuffers(_ptr(query), _ptr(key), _ptr(value), _ptr(gate), _ptr(output),
                                 _ptr(kv_cache), _nbytes(kv_cache), _ptr(workspace),
                                 _nbytes(workspace), pos)
        handle = ctypes.c_void_p()
        _call(Qwen35PrimitiveError, self._lib.raftinfer_amd_decode_graphs_create(
            device_id, _stream(stream), shape.c(), mode, activation_dtype, cache_dtype, cache_layout,
            buf, ctypes.byref(handle)))
        self._handle = handle

    def variant_count(self) -> int:
        out = ctypes.c_size_t()
        _call(Qwen35PrimitiveError, self._lib.raftinfer_amd_decode_graphs_variant_count(
            self._handle, ctypes.byref(out)))
        return out.value

    def variant_for(self, position: int) -> int:
        out = ctypes.c_size_t()
        _call(Qwen35PrimitiveError, self._lib.raftinfer_amd_decode_graphs_variant_for(
            self._handle, position, ctypes.byref(out)))
        return out.value

    def replay(self, position: int) -> None:
        _call(Qwen35PrimitiveError, self._lib.raftinfer_amd_decode_graphs_replay(self._handle, position))

    def close(self) -> None:
        if self._handle:
            self._lib.raftinfer_amd_decode_graphs_destroy(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def consume_capacity_errors() -> int:
    out = ctypes.c_uint32()
    _call(Qwen35PrimitiveError, _lib.load().raftinfer_amd_consume_capacity_errors(ctypes.byref(out)))
    return out.value


def qwen35_gated_delta(input, conv_weight, recurrent_a, dt_bias, output_norm_weight, output,
                       convolution_state, recurrent_state, workspace, shape: GatedDeltaShape,
                       dtype: int, weight_dtype: int, policy: GatedDeltaLaunchPolicy | None = None,
                       stream=None, workspace_bytes=None) -> None:
    lib = _lib.load()
    ws_bytes = _nbytes(workspace) if workspace_bytes is None else workspace_bytes
    common = (_ptr(input), _ptr(conv_weight), _ptr(recurrent_a), _ptr(dt_bias),
              _ptr(output_norm_weight), _ptr(output), _fptr(convolution_state),
              _fptr(recurrent_state), _ptr(workspace), ws_bytes, shape.c())
    if policy is None:
        _call(Qwen35DeltaError, lib.raftinfer_amd_gated_delta_auto(
            *common, dtype, weight_dtype, _stream(stream)))
    else:
        _call(Qwen35DeltaError, lib.raftinfer_amd_gated_delta(
            *common, policy.c(), dtype, weight_dtype, _stream(stream)))


def qwen35_gated_delta_unpacked(qkv, beta, alpha, gate, conv_weight, recurrent_a, dt_bias,
                                output_norm_weight, output, convolution_state, recurrent_state,
                                workspace, shape: GatedDeltaShape, dtype: int, weight_dtype: int,
                                policy: GatedDeltaLaunchPolicy | None = None, stream=None) -> None:
    """qwen35_pack_linear_delta_input + qwen35_gated_delta in one call, reading the four
    projection outputs in place (no packed copy)."""
    policy = policy or GatedDeltaLaunchPolicy()
    _call(Qwen35DeltaError, _lib.load().raftinfer_amd_gated_delta_unpacked(
        _ptr(qkv), _ptr(beta), _ptr(alpha), _ptr(gate), _ptr(conv_weight), _ptr(recurrent_a),
        _ptr(dt_bias), _ptr(output_norm_weight), _ptr(output), _fptr(convolution_state),
        _fptr(recurrent_state), _ptr(workspace), _nbytes(workspace), shape.c(), policy.c(), dtype,
        weight_dtype, _stream(stream)))


def qwen35_gated_delta_core(q, k, v, beta, log_decay, q_scale, state, output, workspace=None,
                            chunked=True, stream=None) -> None:
    T, hk, dk = q.shape
    hv, dv = v.shape[1], v.shape[2]
    _call(Qwen35DeltaError, _lib.load().raftinfer_amd_gated_delta_core(
        _ptr(q), _ptr(k), _ptr(v), _fptr(beta), _fptr(log_decay), ctypes.c_float(q_scale),
        _fptr(state), _ptr(output), _ptr(workspace), _nbytes(workspace),
        DeltaCoreShape(T, hk, hv, dk, dv), int(chunked), _stream(stream)))


# ------------------------------------------------------ attention producers
# cpp/kernels/qwen35_primitives.cuh:34-41, :63-67, :93-96.
@dataclass
class QkNormRopeShape:
    tokens: int
    heads: int
    head_dim: int
    rotary_dim: int
    position_offset: int
    rope_base: float

    def c(self):
        return _lib.QkNormRopeShape(self.tokens, self.heads, self.head_dim, self.rotary_dim,
                                    self.position_offset, self.rope_base)


def qwen35_qk_norm_rope(input, weight, output, shape: QkNormRopeShape, epsilon, dtype,
                        weight_dtype, stream=None, device_position=None) -> None:
    _call(Qwen35PrimitiveError, _lib.load().raftinfer_amd_qk_norm_rope(
        _ptr(input), _ptr(weight), _ptr(output), shape.c(), ctypes.c_float(epsilon), dtype,
        weight_dtype, _stream(stream), _ptr(device_position)))


def qwen35_split_full_query_gate(query_gate, query, gate, tokens, heads, head_dim, dtype,
                                 stream=None) -> None:
    _call(Qwen35PrimitiveError, _lib.load().raftinfer_amd_split_full_query_gate(
        _ptr(query_gate), _ptr(query), _ptr(gate), tokens, heads, head_dim, dtype,
        _stream(stream)))


def qwen35_split_query_gate_norm_rope(query_gate, weight, query, gate, shape: QkNormRopeShape,
                                      epsilon, dtype, weight_dtype, stream=None,
                                      device_position=None) -> None:
    """Additive: qwen35_split_full_query_gate then qwen35_qk_norm_rope on the query, fused."""
    _call(Qwen35PrimitiveError, _lib.load().raftinfer_amd_split_query_gate_norm_rope(
        _ptr(query_gate), _ptr(weight), _ptr(query), _ptr(gate), shape.c(),
        ctypes.c_float(epsilon), dtype, weight_dtype, _stream(stream), _ptr(device_position)))


def qwen35_pack_linear_delta_input(qkv, beta, alpha, gate, packed, tokens, qkv_width, beta_width,
                                   alpha_width, gate_width, dtype, stream=None) -> None:
    """cpp/kernels/qwen35_primitives.cuh:98-102."""
    _call(Qwen35PrimitiveError, _lib.load().raftinfer_amd_pack_linear_delta_input(
        _ptr(qkv), _ptr(beta), _ptr(alpha), _ptr(gate), _ptr(packed), tokens, qkv_width,
        beta_width, alpha_width, gate_width, dtype, _stream(stream)))
