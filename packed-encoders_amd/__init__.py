"""packed-encoders for MI355X: the packed varlen attention path, rebuilt for gfx950.

The hot path of packed-encoders — packed (padding-free) attention over a flat
``[total_tokens, H, D]`` bf16 Q/K/V with int32 ``cu_seqlens`` — as hand-written HIP kernels
behind a C ABI (``include/pe_attn.h``, ``libpe_attn.so``) registered as ``pe_hip::*`` torch
ops, with the reference's Python operator surface on top:

    import packed_encoders_amd as pe
    pe.hip_attention.varlen_attention(q, k, v, cu_seqlens, max_seqlen, window=(64, 64))
    pe.hip_attention.packed_short_attention(q, k, v, cu, max_seqlen, half_window=None,
                                            softmax_scale=0.125)

The directory is named ``packed-encoders_amd``; ``packed_encoders_amd`` (a module at the
repository root) is its importable alias.
"""

from __future__ import annotations

from . import errors, workloads
from . import _lib, attention_dispatch, hip_attention
from .errors import PackedEncodersError, UnsupportedTargetError, ValidationError
from .hip_attention import (
    packed_short_attention,
    packed_short_attention_supported,
    select_packed_short_attention_config,
    varlen_attention,
)

__all__ = [
    "PackedEncodersError",
    "UnsupportedTargetError",
    "ValidationError",
    "errors",
    "hip_attention",
    "packed_short_attention",
    "packed_short_attention_supported",
    "select_packed_short_attention_config",
    "varlen_attention",
    "workloads",
]
