"""packed-encoders for MI355X: the packed varlen attention path, rebuilt for gfx950.

The hot path of packed-encoders — packed (padding-free) attention over a flat
``[total_tokens, H, D]`` bf16 Q/K/V with int32 ``cu_seqlens`` — as hand-written HIP kernels
behind a C ABI (``include/pe_attn.h``, ``libpe_attn.so``) registered as ``pe_hip::*`` torch
ops, with the reference's operator and model surface on top:

    import packed_encoders_amd as pe
    pe.pack(model)                                   # HF ModernBertModel (or a wrapper), in place
    pe.varlen_attention(q, k, v, cu_seqlens, max_seqlen, window=(64, 64))
    pe.packed_short_attention(q, k, v, cu, max_seqlen, half_window=None, softmax_scale=0.125)

The directory is named ``packed-encoders_amd``; ``packed_encoders_amd`` (a module at the
repository root) is its importable alias.
"""

from __future__ import annotations

from . import errors, workloads
from . import _lib, attention_dispatch, hip_attention
from . import batch, config, locate, state, staging, ops, pieces, forward, graph, runtime_attention, pack as _pack_module
from .batch import PackedBatch
from .errors import PackedEncodersError, UnsupportedTargetError, ValidationError
from .forward import packed_forward
from .graph import GraphConfig
from .hip_attention import (
    packed_short_attention,
    packed_short_attention_supported,
    select_packed_short_attention_config,
    shared_plans,
    varlen_attention,
)
from .pack import get_engine, no_cuda_graph, pack, set_cuda_graph, unpack, validate
from .runtime_attention import select_attention

__all__ = [
    "GraphConfig",
    "PackedBatch",
    "PackedEncodersError",
    "UnsupportedTargetError",
    "ValidationError",
    "errors",
    "get_engine",
    "hip_attention",
    "no_cuda_graph",
    "pack",
    "packed_forward",
    "packed_short_attention",
    "packed_short_attention_supported",
    "select_attention",
    "select_packed_short_attention_config",
    "set_cuda_graph",
    "shared_plans",
    "unpack",
    "validate",
    "varlen_attention",
    "workloads",
]
