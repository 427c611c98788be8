"""The packed ModernBERT forward around the HIP attention path (packed_encoders/forward.py).

``packed_forward`` (forward.py:426-531) runs the encoder on an already-packed batch: ids
``[T]``, int32 ``cu_seqlens [N+1]``, host ``max_seqlen``, positions ``[T]``, and returns
``[T, hidden]``. Every layer's attention is the varlen HIP call on ``[T, H, D]`` with the layer's
window (global or ``±local_attention/2``); the layer loop runs inside
``hip_attention.shared_plans()``, so the tiled kernel's work list is built once per window kind
for the whole forward. ``fused_forward`` (forward.py:660-710) is the padded ``[B, S]`` entry:
with the HIP backend it unpads, runs ``packed_forward`` and re-pads (``_varlen_forward``,
forward.py:634-657); with ``"sdpa"`` it runs the dense rectangular path with additive masks.

Backend resolution is host-only and never reads ``cu_seqlens`` values, so it is the same
before eager execution and before graph capture (forward.py:301-371, 534-590).
"""

from __future__ import annotations

import os
import warnings
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from . import attention_dispatch, ops
from .config import ModernBertParams
from .state import ATTR

GRAPH_ENV = "PACKED_ENCODERS_GRAPH"


@dataclass(frozen=True)
class Prologue:
    x: Tensor
    cos_global: Tensor
    sin_global: Tensor
    cos_local: Tensor
    sin_local: Tensor
    full_mask: Tensor | None
    sliding_mask: Tensor | None


def _execution_for(model, execution=None):
    if execution is not None:
        return execution
    state = getattr(model, ATTR, None)
    if state is not None and state.execution is not None:
        return state.execution
    from .pieces import default_execution

    return default_execution()


# ----------------------------------------------------------------------------- backend resolution


def hip_supported(params: ModernBertParams, *, device: torch.device, dtype: torch.dtype) -> bool:
    """Whether this call can run on the HIP kernels: no autograd, a HIP device, bf16, a head
    dim the kernels serve, and the library loaded (the reference's invariants,
    forward.py:351-371, for its Triton kernel)."""
    return (not torch.is_grad_enabled() and device.type == "cuda" and dtype == torch.bfloat16
            and params.head_dim in (64, 128, 256) and ops.hip_available())


def resolve_backend(backend: str, params: ModernBertParams, *, device: torch.device, dtype: torch.dtype) -> str:
    """``"hip"`` or ``"sdpa"`` for one call. ``"hip"`` outside its invariants (autograd, fp32
    weights, CPU) runs the dense SDPA path, as the reference's ``"triton"`` does outside its
    envelope; ``"auto"`` is ``"hip"`` wherever the kernels serve the call."""
    if backend == "sdpa":
        return "sdpa"
    if backend in ("hip", "auto"):
        return "hip" if hip_supported(params, device=device, dtype=dtype) else "sdpa"
    raise ValueError(f"unknown attention backend {backend!r}")


def attention_workload(params: ModernBertParams, input_ids: Tensor,
                       attention_mask: Tensor | None) -> attention_dispatch.AttentionWorkload:
    """Shape statistics of a padded batch (forward.py:374-392); a mask costs one device-to-host
    read of ``B`` lengths."""
    b, s = input_ids.shape
    if attention_mask is None:
        lengths = (s,) * b
    else:
        lengths = tuple(int(n) for n in attention_mask.sum(dim=1, dtype=torch.int64).tolist())
    return attention_dispatch.AttentionWorkload.from_lengths(lengths)


def packed_workload(*, total_tokens: int, n_sequences: int, max_seqlen: int) -> attention_dispatch.AttentionWorkload:
    return attention_dispatch.AttentionWorkload.from_summary(n_sequences=n_sequences, live_tokens=total_tokens,
                                                             max_seqlen=max_seqlen)


# ----------------------------------------------------------------------------- layers


@dataclass(frozen=True)
class LayerKind:
    """What a layer's attention sees: RoPE tables, the dense path's additive mask, and the
    (left, right) window the varlen kernels take — (-1, -1) for global layers."""

    cos: Tensor
    sin: Tensor
    mask: Tensor | None
    window: tuple[int, int]


def layer_schedule(model: nn.Module, params: ModernBertParams) -> list[bool]:
    """Per encoder layer, whether it attends globally: the layer's own ``attention_type`` when
    Hugging Face set one, else the config's period of global layers (config.py)."""
    kinds = {"full_attention": True, "sliding_attention": False}
    return [kinds.get(getattr(layer, "attention_type", None), params.is_global_layer(i))
            for i, layer in enumerate(model.layers)]


def _qkv_projection(x: Tensor, residual: Tensor | None, layer: nn.Module, execution) -> tuple[Tensor, Tensor]:
    """Fold the previous layer's unapplied MLP residual into ``x`` (inside the add+LayerNorm when
    the layer has an attention norm) and project the normed stream to ``qkv``. Returns
    ``(x, qkv)``; a layer with ``nn.Identity`` as its attention norm projects ``x`` as is."""
    norm = layer.attn_norm
    if isinstance(norm, nn.Identity):
        x = x if residual is None else x + residual
        return x, execution.dense_linear(x, layer.attn.Wqkv.weight)
    if residual is None:
        normed = execution.layer_norm(x, norm.weight, norm.eps)
    else:
        x, normed = execution.add_layer_norm(x, residual, norm.weight, norm.eps)
    return x, execution.linear(normed, layer.attn.Wqkv.weight)


def _attention_context(qkv: Tensor, kind: LayerKind, params: ModernBertParams, backend: str, execution,
                       cu_seqlens: Tensor | None, max_seqlen: int | None) -> Tensor:
    """RoPE and attention over ``qkv [B, S, 3*H*D]``; returns the context ``[B, S, H*D]``.
    The HIP path rotates q and k straight out of ``qkv`` into contiguous ``[B, S, H, D]`` and
    leaves v a strided view (token stride 3HD) that the kernels read in place, or, with the
    default pieces on short segments, lets the attention kernel rotate them itself
    (``ops.flash_attention_qkv_bshd``); the dense path splits and transposes to
    ``[B, H, S, D]``."""
    b, s = qkv.shape[:2]
    h, d = params.num_attention_heads, params.head_dim
    if ops.use_bshd_rope(backend, h, d, cu_seqlens):
        if execution.rope_qkv is ops.rope_qkv and execution.attention_bshd is ops.attention_bshd:
            # the default pieces: one call, with RoPE fused into the attention kernel when it fits
            return ops.flash_attention_qkv_bshd(qkv, h, d, cos=kind.cos, sin=kind.sin, window=kind.window,
                                                scaling=params.scaling, cu_seqlens=cu_seqlens, max_seqlen=max_seqlen,
                                                backend=backend)
        q, k = execution.rope_qkv(qkv, h, d, kind.cos, kind.sin)
        v = qkv.view(b, s, 3, h, d).select(2, 2)
        return execution.attention_bshd(q, k, v, window=kind.window, scaling=params.scaling,
                                        cu_seqlens=cu_seqlens, max_seqlen=max_seqlen, backend=backend)
    q, k, v = (t.transpose(1, 2) for t in qkv.view(b, s, 3, h, d).unbind(dim=2))
    q, k = execution.rope(q, k, kind.cos, kind.sin)
    return execution.attention(q, k, v, mask=kind.mask, window=kind.window, scaling=params.scaling,
                               backend=backend, cu_seqlens=cu_seqlens, max_seqlen=max_seqlen)


def encoder_layer(x: Tensor, residual: Tensor | None, layer: nn.Module, params: ModernBertParams, kind: LayerKind,
                  backend: str, execution, cu_seqlens: Tensor | None = None,
                  max_seqlen: int | None = None) -> tuple[Tensor, Tensor]:
    """One ModernBERT layer in Hugging Face's order (attention half, then GeGLU MLP half). The
    MLP's output is returned unapplied as the next residual: the next layer's attention norm,
    or the final norm, adds it inside its add+LayerNorm (forward.py:164-234)."""
    x, qkv = _qkv_projection(x, residual, layer, execution)
    ctx = _attention_context(qkv, kind, params, backend, execution, cu_seqlens, max_seqlen)
    x, normed = execution.add_layer_norm(x, execution.linear(ctx, layer.attn.Wo.weight), layer.mlp_norm.weight,
                                         layer.mlp_norm.eps)
    hidden = execution.geglu(execution.linear(normed, layer.mlp.Wi.weight))
    return x, execution.linear(hidden, layer.mlp.Wo.weight)


def core(model: nn.Module, params: ModernBertParams, x: Tensor, cos_global: Tensor, sin_global: Tensor,
         cos_local: Tensor, sin_local: Tensor, full_mask: Tensor | None, sliding_mask: Tensor | None, *,
         execution=None, backend: str = "sdpa", cu_seqlens: Tensor | None = None,
         max_seqlen: int | None = None, min_seqlen: int = 0) -> Tensor:
    """The encoder layers and the final norm: device work only, so it can be captured
    (forward.py:237-288). ``min_seqlen`` is the host's lower bound on the packed segment lengths
    (0 unknown), shared by every layer's HIP attention call."""
    execution = _execution_for(model, execution)
    half = params.sliding_half_window
    kinds = {True: LayerKind(cos_global, sin_global, full_mask, (-1, -1)),
             False: LayerKind(cos_local, sin_local, sliding_mask, (half, half))}
    residual = None
    with _plan_scope(backend, cu_seqlens, min_seqlen):
        for layer, is_global in zip(model.layers, layer_schedule(model, params)):
            x, residual = encoder_layer(x, residual, layer, params, kinds[is_global], backend, execution,
                                        cu_seqlens=cu_seqlens, max_seqlen=max_seqlen)
    final = model.final_norm
    if residual is None:
        return execution.layer_norm(x, final.weight, final.eps)
    return execution.add_layer_norm(x, residual, final.weight, final.eps)[1]


class _NullScope:
    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


def _plan_scope(backend: str, cu_seqlens: Tensor | None, min_seqlen: int = 0):
    """The layers of one packed forward share ``cu_seqlens``: under the HIP backend they share
    the device-built tile plans and the host's length bound (``hip_attention.shared_plans``)."""
    if backend == "hip" and cu_seqlens is not None:
        from .hip_attention import shared_plans

        return shared_plans(min_seqlen)
    return _NullScope()


# ----------------------------------------------------------------------------- dense (SDPA) path


def _build_masks(attention_mask: Tensor | None, seq_len: int, half_window: int, device) -> tuple[Tensor | None, Tensor]:
    """(full, sliding) additive fp32 masks broadcastable to ``[B, 1, S, S]``; ``full`` is None
    without padding."""
    pad = None
    if attention_mask is not None:
        pad = torch.zeros(attention_mask.shape, dtype=torch.float32, device=device)
        pad = pad.masked_fill(attention_mask == 0, float("-inf"))[:, None, None, :]
    pos = torch.arange(seq_len, device=device)
    outside = (pos[:, None] - pos[None, :]).abs() > half_window
    band = torch.zeros((seq_len, seq_len), dtype=torch.float32, device=device).masked_fill(outside, float("-inf"))
    band = band[None, None]
    return pad, band if pad is None else band + pad


def _finite(mask: Tensor | None, dtype) -> Tensor | None:
    """SDPA wants a finite additive mask in the activation dtype."""
    if mask is None:
        return None
    m = mask.to(dtype)
    return m.masked_fill(torch.isinf(m), torch.finfo(dtype).min)


def prologue(model: nn.Module, params: ModernBertParams, input_ids: Tensor, attention_mask: Tensor | None, *,
             execution=None) -> Prologue:
    """Embeddings, RoPE tables and SDPA masks of the rectangular path (forward.py:107-150)."""
    execution = _execution_for(model, execution)
    _, s = input_ids.shape
    device = input_ids.device
    norm = model.embeddings.norm
    x = execution.layer_norm(model.embeddings.tok_embeddings(input_ids), norm.weight, norm.eps)
    cos_g, sin_g = execution.rope_tables(s, params.head_dim, params.global_rope_theta, device, x.dtype)
    if params.local_rope_theta == params.global_rope_theta:
        cos_l, sin_l = cos_g, sin_g
    else:
        cos_l, sin_l = execution.rope_tables(s, params.head_dim, params.local_rope_theta, device, x.dtype)
    full, sliding = _build_masks(attention_mask, s, params.sliding_half_window, device)
    return Prologue(x, cos_g, sin_g, cos_l, sin_l, _finite(full, x.dtype), _finite(sliding, x.dtype))


# ----------------------------------------------------------------------------- packed path


def unpad(x: Tensor, attention_mask: Tensor | None) -> tuple[Tensor, Tensor, Tensor, int, Tensor]:
    """Strip padding from ``x [B, S, ...]`` with ``attention_mask [B, S]`` (1 = real token):
    packed rows, their flat ``indices`` (for re-padding), int32 ``cu_seqlens``, ``max_seqlen``
    and ``position_ids = indices % S`` — the token's column, which is the RoPE position
    Hugging Face ModernBERT gives it (forward.py:395-415).

    Synchronisation: a device mask costs two device-to-host reads, as in the reference (the
    packed length and ``max_seqlen``). A host mask with device ``x`` costs none: the layout is
    built on the host and staged in one pinned non-blocking copy (``staging``). No mask (every
    token real) costs none either: the layout is a set of device ``arange``s."""
    if attention_mask is None:
        return _unpad_dense(x)
    if attention_mask.device.type == "cpu" and x.device.type == "cuda":
        return _unpad_host_mask(x, attention_mask)
    b, s = attention_mask.shape
    seqlens = attention_mask.sum(dim=1, dtype=torch.int32)
    indices = torch.nonzero(attention_mask.flatten(), as_tuple=False).flatten()
    cu_seqlens = F.pad(seqlens.cumsum(0, dtype=torch.int32), (1, 0))
    max_seqlen = int(seqlens.max())
    packed = x.reshape(b * s, *x.shape[2:]).index_select(0, indices)
    return packed, indices, cu_seqlens, max_seqlen, indices % s


def _unpad_dense(x: Tensor) -> tuple[Tensor, Tensor, Tensor, int, Tensor]:
    b, s = x.shape[:2]
    dev = x.device
    indices = torch.arange(b * s, device=dev)
    cu_seqlens = torch.arange(0, (b + 1) * s, s, dtype=torch.int32, device=dev)
    return x.reshape(b * s, *x.shape[2:]), indices, cu_seqlens, s, indices % s


def _unpad_host_mask(x: Tensor, attention_mask: Tensor) -> tuple[Tensor, Tensor, Tensor, int, Tensor]:
    from .staging import padded_layout_host, stager_for

    b, s = attention_mask.shape
    indices, cu, positions, max_seqlen = padded_layout_host(attention_mask)
    d_indices, d_cu, d_positions = stager_for(x.device).put([indices, cu, positions])
    packed = x.reshape(b * s, *x.shape[2:]).index_select(0, d_indices)
    return packed, d_indices, d_cu.to(torch.int32), max_seqlen, d_positions


def repad(x_packed: Tensor, indices: Tensor, b: int, s: int) -> Tensor:
    """Scatter packed rows back into a zero-filled ``[B, S, ...]`` (the inverse of ``unpad``)."""
    out = x_packed.new_zeros(b * s, *x_packed.shape[1:])
    out.index_copy_(0, indices, x_packed)
    return out.reshape(b, s, *x_packed.shape[1:])


def packed_forward(model: nn.Module, params: ModernBertParams, packed_ids: Tensor, cu_seqlens: Tensor,
                   max_seqlen: int, position_ids: Tensor, *, execution=None, backend: str | None = None,
                   _allow_graph: bool = True, min_seqlen: int = 0) -> Tensor:
    """Encode an already-packed batch; returns ``[total, hidden]`` in input order.

    ``packed_ids [T]`` int64, ``cu_seqlens [N+1]`` int32 on the device, ``max_seqlen`` a host
    int bounding every length, ``position_ids [T]`` int64 positions within each sequence
    (``arange`` per sequence, as ``unpad`` makes them). ``min_seqlen`` is an optional host lower
    bound on the lengths (0 unknown): with every segment longer than the short kernel's
    boundary, no layer launches the short pass. With an active packed graph runner (no
    autograd, no autocast) the call replays a captured graph instead (captured for any lengths).
    """
    state = getattr(model, ATTR, None)
    requested = backend if backend is not None else (state.attention_backend if state is not None else "hip")
    if (_allow_graph and state is not None and state.graph_enabled and state.packed_graph_runner is not None
            and (execution is None or execution is state.execution) and requested == state.attention_backend
            and os.environ.get(GRAPH_ENV, "1") != "0" and not torch.is_grad_enabled()
            and not torch.is_autocast_enabled("cuda")):
        return state.packed_graph_runner(packed_ids, cu_seqlens, max_seqlen, position_ids)

    execution = _execution_for(model, execution)
    norm = model.embeddings.norm
    x = execution.layer_norm(model.embeddings.tok_embeddings(packed_ids), norm.weight, norm.eps)
    resolved = resolve_backend(requested, params, device=x.device, dtype=x.dtype)
    if resolved == "sdpa":
        return packed_sdpa_fallback(model, params, packed_ids, cu_seqlens, max_seqlen, position_ids,
                                    execution=execution)
    return packed_core(model, params, x, cu_seqlens, max_seqlen, position_ids, execution=execution,
                       min_seqlen=min_seqlen)


def packed_core(model: nn.Module, params: ModernBertParams, x: Tensor, cu_seqlens: Tensor, max_seqlen: int,
                position_ids: Tensor, *, execution, min_seqlen: int = 0) -> Tensor:
    """RoPE tables up to ``max_seqlen`` gathered per token, then ``core`` on ``[1, T, hidden]``
    with the HIP backend. Shared by the eager packed forward and the graph runner's capture."""
    device, dtype, d = x.device, x.dtype, params.head_dim
    cos_g, sin_g = execution.rope_tables(max_seqlen, d, params.global_rope_theta, device, dtype)
    if params.local_rope_theta == params.global_rope_theta:
        cos_l, sin_l = cos_g, sin_g
    else:
        cos_l, sin_l = execution.rope_tables(max_seqlen, d, params.local_rope_theta, device, dtype)

    def gather(t: Tensor) -> Tensor:
        return t[0].index_select(0, position_ids)[None]

    out = core(model, params, x[None], gather(cos_g), gather(sin_g), gather(cos_l), gather(sin_l), None, None,
               execution=execution, backend="hip", cu_seqlens=cu_seqlens, max_seqlen=int(max_seqlen),
               min_seqlen=min(int(min_seqlen), int(max_seqlen)))
    return out[0]


def packed_sdpa_fallback(model: nn.Module, params: ModernBertParams, packed_ids: Tensor, cu_seqlens: Tensor,
                         max_seqlen: int, position_ids: Tensor, *, execution=None) -> Tensor:
    """Re-pad a packed batch to ``[N, max_seqlen]`` for the dense SDPA path and pack the result
    again (forward.py:593-620)."""
    n = cu_seqlens.numel() - 1
    total = packed_ids.numel()
    seq_of = torch.bucketize(torch.arange(total, device=packed_ids.device), cu_seqlens[1:], right=True)
    flat = seq_of * int(max_seqlen) + position_ids
    ids = packed_ids.new_zeros(n * int(max_seqlen)).index_copy_(0, flat, packed_ids)
    mask = packed_ids.new_zeros(n * int(max_seqlen)).index_fill_(0, flat, 1)
    out = fused_forward(model, params, ids.view(n, int(max_seqlen)), mask.view(n, int(max_seqlen)), backend="sdpa",
                        execution=execution)
    return out.reshape(-1, out.shape[-1]).index_select(0, flat)


def varlen_forward(model: nn.Module, params: ModernBertParams, input_ids: Tensor, attention_mask: Tensor | None, *,
                   backend: str = "hip", execution=None) -> Tensor:
    """Padded batch through the packed path: ``unpad`` → ``packed_forward`` → ``repad``
    (``attention_mask`` None: every token is real)."""
    b, s = input_ids.shape
    ids, indices, cu, max_seqlen, positions = unpad(input_ids, attention_mask)
    # the shortest row when the host holds the mask (or there is none): no device read
    if attention_mask is None:
        shortest = s
    elif attention_mask.device.type == "cpu":
        shortest = int(attention_mask.sum(dim=1).min()) if b else 0
    else:
        shortest = 0
    out = packed_forward(model, params, ids, cu, max_seqlen, positions, backend=backend, execution=execution,
                         _allow_graph=True, min_seqlen=shortest)
    return repad(out, indices, b, s)


def fused_forward(model: nn.Module, params: ModernBertParams, input_ids: Tensor, attention_mask: Tensor | None, *,
                  execution=None, backend: str = "sdpa") -> Tensor:
    """Padded ``[B, S]`` forward; returns the final-normed hidden states ``[B, S, hidden]``.
    The HIP backend goes through the packed path (padding is never computed); SDPA runs the
    rectangular path with dense masks."""
    dtype = model.embeddings.tok_embeddings.weight.dtype
    resolved = resolve_backend(backend, params, device=input_ids.device, dtype=dtype)
    if resolved == "hip":
        return varlen_forward(model, params, input_ids, attention_mask, backend=resolved, execution=execution)
    p = prologue(model, params, input_ids, attention_mask, execution=execution)
    return core(model, params, p.x, p.cos_global, p.sin_global, p.cos_local, p.sin_local, p.full_mask,
                p.sliding_mask, execution=execution, backend="sdpa")


def warn_once(state, message: str) -> None:
    if not state.graph_skip_warned:
        state.graph_skip_warned = True
        warnings.warn(message, stacklevel=3)
