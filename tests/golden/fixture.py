"""Reader for tiny-layer-v1.bin, the HF-generated fixture the reference's own
tests hold (tests/fixtures/qwen35/tiny-layer-v1.bin, format in the reference's
tests/fixtures/qwen35/README.md; parser behaviour follows
cpp/tests/qwen35_fixture_test.cpp:104-160).  Data only: copied byte-for-byte,
SHA-256 800878611016996887aa9828ee97eb165e6bf1066543a8797b4c99e6eaf167e0."""
from __future__ import annotations

import pathlib
import struct

import numpy as np

PATH = pathlib.Path(__file__).resolve().parent / "tiny-layer-v1.bin"
MAGIC = b"RIFQ35F1"
VECTORS = [
    "full_input", "full_query_norm_weight", "full_key_norm_weight", "full_output_weight",
    "full_expected_output", "delta_input", "delta_conv_weight", "delta_recurrent_a",
    "delta_dt_bias", "delta_output_norm_weight", "delta_initial_convolution",
    "delta_initial_recurrent", "delta_expected_output", "delta_expected_convolution",
    "delta_expected_recurrent",
]


def parse(data: bytes) -> dict:
    off = 0

    def take(n):
        nonlocal off
        if n > len(data) - off:
            raise ValueError("truncated Qwen3.5 fixture")
        chunk = data[off:off + n]
        off += n
        return chunk

    if take(8) != MAGIC:
        raise ValueError("invalid Qwen3.5 fixture magic")
    if struct.unpack("<I", take(4))[0] != 1:
        raise ValueError("unsupported Qwen3.5 fixture version")
    if struct.unpack("<I", take(4))[0] != 0x01020304:
        raise ValueError("invalid Qwen3.5 fixture endian marker")
    if struct.unpack("<Q", take(8))[0] != len(data):
        raise ValueError("Qwen3.5 fixture length mismatch")
    full = dict(zip(["tokens", "hidden_size", "query_heads", "kv_heads", "head_dim", "rotary_dim",
                     "position_offset"], struct.unpack("<7I", take(28))))
    full["rope_base"], full["epsilon"] = struct.unpack("<2f", take(8))
    delta = dict(zip(["tokens", "hidden_size", "key_heads", "value_heads", "key_dim", "value_dim",
                      "conv_width"], struct.unpack("<7I", take(28))))
    delta["epsilon"] = struct.unpack("<f", take(4))[0]
    out = {"full": full, "delta": delta}
    for name in VECTORS:
        count = struct.unpack("<Q", take(8))[0]
        out[name] = np.frombuffer(take(4 * count), dtype="<f4").astype(np.float32)
    if off != len(data):
        raise ValueError("Qwen3.5 fixture has trailing bytes")
    return out


def load() -> dict:
    return parse(PATH.read_bytes())
