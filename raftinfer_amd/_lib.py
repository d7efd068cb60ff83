"""ctypes binding of libraftinfer_amd.so (the C ABI in include/raftinfer_amd.h).

Loading fails loudly when the library is missing: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import pathlib

_SO = pathlib.Path(__file__).resolve().parent / "libraftinfer_amd.so"

_sz = ctypes.c_size_t
_u8 = ctypes.c_uint8
_vp = ctypes.c_void_p


class AttentionShape(ctypes.Structure):
    _fields_ = [("tokens", _sz), ("query_heads", _sz), ("kv_heads", _sz), ("head_dim", _sz),
                ("max_context_tokens", _sz), ("past_tokens", _sz)]


class AttentionPolicy(ctypes.Structure):
    _fields_ = [("implementation", _u8), ("kv_cache_dtype", _u8), ("kv_cache_layout", _u8)]


class DecodePlan(ctypes.Structure):
    _fields_ = [("resolved_mode", _u8), ("partition_tokens", _sz),
                ("split_k_threshold_tokens", _sz), ("context_bucket_tokens", _sz),
                ("active_partition_capacity", _sz)]

    def as_tuple(self):
        return (self.resolved_mode, self.partition_tokens, self.split_k_threshold_tokens,
                self.context_bucket_tokens, self.active_partition_capacity)


class DecodeLayout(ctypes.Structure):
    _fields_ = [("partial_count", _sz), ("max_offset_bytes", _sz), ("sum_offset_bytes", _sz),
                ("value_offset_bytes", _sz), ("bytes", _sz)]

    def as_tuple(self):
        return (self.partial_count, self.max_offset_bytes, self.sum_offset_bytes,
                self.value_offset_bytes, self.bytes)


class DeltaShape(ctypes.Structure):
    _fields_ = [("tokens", _sz), ("hidden_size", _sz), ("key_heads", _sz), ("value_heads", _sz),
                ("key_dim", _sz), ("value_dim", _sz), ("conv_width", _sz),
                ("epsilon", ctypes.c_float)]


class DeltaPolicy(ctypes.Structure):
    _fields_ = [("schedule", _u8), ("warps_per_block", ctypes.c_uint32),
                ("transposed_boundary_state", _u8)]


class BatchedDecodeShape(ctypes.Structure):
    _fields_ = [("sequences", _sz), ("max_context_tokens", _sz), ("cache_stride_bytes", _sz),
                ("single_block_max_tokens", _sz)]


class DeltaCoreShape(ctypes.Structure):
    _fields_ = [("tokens", _sz), ("key_heads", _sz), ("value_heads", _sz), ("key_dim", _sz),
                ("value_dim", _sz)]


class QkNormRopeShape(ctypes.Structure):
    _fields_ = [("tokens", _sz), ("heads", _sz), ("head_dim", _sz), ("rotary_dim", _sz),
                ("position_offset", _sz), ("rope_base", ctypes.c_float)]


class FusedNormRope(ctypes.Structure):
    _fields_ = [("query_norm_weight", _vp), ("key_norm_weight", _vp), ("weight_dtype", ctypes.c_int),
                ("rotary_dim", _sz), ("rope_base", ctypes.c_float), ("epsilon", ctypes.c_float)]


class DecodeBuffers(ctypes.Structure):
    _fields_ = [("query", _vp), ("key", _vp), ("value", _vp), ("gate", _vp), ("output", _vp),
                ("kv_cache", _vp), ("kv_cache_bytes", _sz), ("workspace", _vp),
                ("workspace_bytes", _sz), ("device_position", ctypes.POINTER(ctypes.c_uint32))]


# Every symbol include/raftinfer_amd.h declares, with its argument types.
_I, _F = ctypes.c_int, ctypes.c_float
_PF = ctypes.POINTER(ctypes.c_float)
_PSZ = ctypes.POINTER(_sz)
_PU32 = ctypes.POINTER(ctypes.c_uint32)
SIGNATURES = {
    "raftinfer_amd_last_error_message": ([], ctypes.c_char_p),
    "raftinfer_amd_attention_workspace_floats": ([AttentionShape, _PSZ], _I),
    "raftinfer_amd_attention_cache_bytes": ([AttentionShape, AttentionPolicy, _PSZ], _I),
    "raftinfer_amd_attention_workspace_bytes": ([AttentionShape, AttentionPolicy, _PSZ], _I),
    "raftinfer_amd_online_decode_plan": ([AttentionShape, _u8, _sz, ctypes.POINTER(DecodePlan)], _I),
    "raftinfer_amd_online_decode_workspace_layout":
        ([AttentionShape, _u8, ctypes.POINTER(DecodeLayout)], _I),
    "raftinfer_amd_online_attention_prefill_supported": ([AttentionShape, _I, AttentionPolicy], _I),
    "raftinfer_amd_gated_delta_workspace_bytes": ([DeltaShape, _PSZ], _I),
    "raftinfer_amd_gated_delta_select_policy": ([DeltaShape, _sz, ctypes.POINTER(DeltaPolicy)], _I),
    "raftinfer_amd_batched_decode_workspace_bytes": ([BatchedDecodeShape, _PSZ], _I),
    "raftinfer_amd_causal_attention":
        ([_vp] * 6 + [_sz, _vp, _sz, AttentionShape, _I, AttentionPolicy, _vp], _I),
    "raftinfer_amd_causal_attention_materialized":
        ([_vp] * 5 + [_PF, _PF, _sz, AttentionShape, _I, _vp], _I),
    "raftinfer_amd_online_attention_prefill":
        ([_vp] * 6 + [_sz, AttentionShape, _I, _u8, _u8, _vp], _I),
    "raftinfer_amd_online_attention_decode":
        ([_vp] * 6 + [_sz, _vp, _sz, AttentionShape, _I, _u8, _u8, DecodePlan, _PU32, _vp], _I),
    "raftinfer_amd_online_attention_decode_single":
        ([_vp] * 6 + [_sz, AttentionShape, _I, _u8, _u8, _PU32, _vp], _I),
    "raftinfer_amd_online_attention_decode_batched":
        ([_vp] * 6 + [_sz, _PU32, _vp, _sz, BatchedDecodeShape, _I, _vp], _I),
    "raftinfer_amd_online_attention_decode_partition_only":
        ([_vp] * 6 + [_sz, _vp, _sz, AttentionShape, _I, _u8, _u8, DecodePlan, _PU32, _vp], _I),
    "raftinfer_amd_online_attention_decode_fused":
        ([_vp] * 5 + [_sz, _vp, _sz, AttentionShape, FusedNormRope, _u8, _u8, DecodePlan, _PU32, _vp], _I),
    "raftinfer_amd_online_attention_prefill_fused":
        ([_vp] * 5 + [_sz, AttentionShape, FusedNormRope, _u8, _u8, _vp], _I),
    "raftinfer_amd_online_attention_static_workspace_bytes": ([], _sz),
    "raftinfer_amd_online_attention_decode_static_workspace":
        ([_vp] * 6 + [_sz, AttentionShape, _I, _u8, _u8, DecodePlan, _PU32, _vp], _I),
    "raftinfer_amd_online_attention_prefill_kernel_only":
        ([_vp] * 6 + [_sz, AttentionShape, _I, _u8, _u8, _vp], _I),
    "raftinfer_amd_consume_capacity_errors": ([_PU32], _I),
    "raftinfer_amd_decode_graphs_create":
        ([_I, _vp, AttentionShape, _u8, _I, _u8, _u8, DecodeBuffers, ctypes.POINTER(_vp)], _I),
    "raftinfer_amd_decode_graphs_variant_count": ([_vp, _PSZ], _I),
    "raftinfer_amd_decode_graphs_variant_for": ([_vp, _sz, _PSZ], _I),
    "raftinfer_amd_decode_graphs_replay": ([_vp, _sz], _I),
    "raftinfer_amd_decode_graphs_destroy": ([_vp], None),
    "raftinfer_amd_gated_delta":
        ([_vp] * 6 + [_PF, _PF, _vp, _sz, DeltaShape, DeltaPolicy, _I, _I, _vp], _I),
    "raftinfer_amd_gated_delta_auto":
        ([_vp] * 6 + [_PF, _PF, _vp, _sz, DeltaShape, _I, _I, _vp], _I),
    "raftinfer_amd_gated_delta_unpacked":
        ([_vp] * 9 + [_PF, _PF, _vp, _sz, DeltaShape, DeltaPolicy, _I, _I, _vp], _I),
    "raftinfer_amd_gated_delta_core_workspace_bytes": ([DeltaCoreShape, _PSZ], _I),
    "raftinfer_amd_gated_delta_core":
        ([_vp, _vp, _vp, _PF, _PF, _F, _PF, _vp, _vp, _sz, DeltaCoreShape, _I, _vp], _I),
    "raftinfer_amd_qk_norm_rope":
        ([_vp, _vp, _vp, QkNormRopeShape, _F, _I, _I, _vp, _vp], _I),
    "raftinfer_amd_split_full_query_gate": ([_vp, _vp, _vp, _sz, _sz, _sz, _I, _vp], _I),
    "raftinfer_amd_pack_linear_delta_input":
        ([_vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _I, _vp], _I),
    "raftinfer_amd_split_query_gate_norm_rope":
        ([_vp, _vp, _vp, _vp, QkNormRopeShape, _F, _I, _I, _vp, _vp], _I),
}

_lib = None


def path() -> pathlib.Path:
    return _SO


def load():
    """Loads the HIP library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not _SO.exists():
            raise RuntimeError(f"{_SO} is missing: build it with `python -m raftinfer_amd.build` "
                               "(there is no CPU fallback)")
        lib = ctypes.CDLL(str(_SO))
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib


class RaftInferError(RuntimeError):
    """A non-OK status from the C ABI; `status` is the raftinfer_amd_status code."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


def check(status: int) -> None:
    if status != 0:
        msg = load().raftinfer_amd_last_error_message().decode()
        raise RaftInferError(status, msg)
