"""raftinfer_amd: MI355X (gfx950) attention / gated-delta hot path of Qwen3.5.

The compute lives in libraftinfer_amd.so (hand-written HIP); ``ops`` mirrors
the reference's kernel interface over torch device tensors.
"""
from . import _lib, ops  # noqa: F401

__all__ = ["ops"]
