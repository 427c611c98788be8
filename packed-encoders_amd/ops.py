"""Operations of the packed ModernBERT forward (packed_encoders/ops.py:322-555 for attention).

Attention — the hot path — goes to the HIP kernels (``hip_attention``): ``attention_bshd`` with
``backend="hip"`` replaces the reference's Triton-else-FlashAttention switch
(``ops.attention_bshd``, ops.py:502-538) by one varlen call that routes every segment to the
short or the tiled kernel on the device. ``"sdpa"`` is the reference's dependency-free dense
fallback (ops.py:327-339), reached only when it is asked for.

The rest of the layer (LayerNorm, the projections, GeGLU, RoPE) is outside this build's scope
and runs as plain torch ops with Hugging Face ModernBERT's numerics: LayerNorm without bias,
bias-free linears, ``gelu(input) * gate``, split-half RoPE applied in fp32 with tables rounded to
the model dtype.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor

BACKENDS = ("hip", "sdpa", "auto")


# ----------------------------------------------------------------------------- dense tail


def layer_norm(x: Tensor, weight: Tensor, eps: float) -> Tensor:
    return F.layer_norm(x, (x.shape[-1],), weight, None, eps)


def add_layer_norm(x: Tensor, residual: Tensor, weight: Tensor, eps: float) -> tuple[Tensor, Tensor]:
    """``(x + residual, LayerNorm(x + residual))``: the residual stream and the next input."""
    summed = x + residual
    return summed, layer_norm(summed, weight, eps)


def linear(x: Tensor, weight: Tensor) -> Tensor:
    return F.linear(x, weight)


def dense_linear(x: Tensor, weight: Tensor) -> Tensor:
    return F.linear(x, weight)


def geglu(proj: Tensor) -> Tensor:
    """ModernBERT's MLP gate: the projection's halves ``(input, gate)`` → ``gelu(input) * gate``."""
    inp, gate = proj.chunk(2, dim=-1)
    return F.gelu(inp) * gate


def rope_tables(seq_len: int, head_dim: int, theta: float, device, dtype) -> tuple[Tensor, Tensor]:
    """Split-half RoPE ``cos``/``sin`` ``[1, seq_len, head_dim]`` for positions ``0..seq_len-1``:
    frequencies ``theta ** (-2i / head_dim)``, angles in fp32, rounded to ``dtype``."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, device=device, dtype=torch.float32) / head_dim))
    pos = torch.arange(seq_len, device=device, dtype=torch.float32)
    angles = torch.outer(pos, inv_freq)
    emb = torch.cat((angles, angles), dim=-1)
    return emb.cos()[None].to(dtype), emb.sin()[None].to(dtype)


def _rotate(x: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
    xf = x.float()
    half = xf.shape[-1] // 2
    rotated = torch.cat((-xf[..., half:], xf[..., :half]), dim=-1)
    return (xf * cos.float() + rotated * sin.float()).to(x.dtype)


def rope(q: Tensor, k: Tensor, cos: Tensor, sin: Tensor) -> tuple[Tensor, Tensor]:
    """RoPE on ``[B, H, S, D]`` q and k; ``cos``/``sin`` ``[B or 1, S, D]``."""
    return _rotate(q, cos[:, None], sin[:, None]), _rotate(k, cos[:, None], sin[:, None])


def rope_qkv(qkv: Tensor, h: int, d: int, cos: Tensor, sin: Tensor) -> tuple[Tensor, Tensor]:
    """RoPE read straight from the packed projection ``qkv [B, S, 3*h*d]``: returns contiguous
    ``[B, S, h, d]`` q and k, the layout the varlen kernels read. ``cos``/``sin`` are
    ``[B or 1, S, d]`` (for packed input: the tables gathered by each token's position).
    On the GPU in bf16 this is the HIP kernel (``hip_attention.rope_qkv``, the reference's
    apply_rope_bshd, _kernels/rope.py:302-349); fp32 inputs (the pieces' oracles) and CPU
    tensors take the same formula in torch."""
    if qkv.is_cuda and qkv.dtype == torch.bfloat16:
        from .hip_attention import rope_qkv as hip_rope_qkv

        return hip_rope_qkv(qkv, h, d, cos, sin)
    view = qkv.view(*qkv.shape[:-1], 3, h, d)
    c, s = cos[..., None, :], sin[..., None, :]
    return _rotate(view[..., 0, :, :], c, s).contiguous(), _rotate(view[..., 1, :, :], c, s).contiguous()


# ----------------------------------------------------------------------------- attention


def _load_packed_short_attention():
    """The short-segment operator pair, loaded lazily (the reference's loader, ops.py:345-352).
    ``ImportError`` when the HIP library is not built or loadable."""
    from . import _lib
    from .hip_attention import packed_short_attention, packed_short_attention_supported

    _lib.library()
    return packed_short_attention, packed_short_attention_supported


def _load_hip_attention():
    """The general varlen operator; ``ImportError`` when the HIP library is unavailable."""
    from . import _lib
    from .hip_attention import varlen_attention

    _lib.library()
    return varlen_attention


def hip_available() -> bool:
    try:
        _load_hip_attention()
    except ImportError:
        return False
    return torch.cuda.is_available()


def sdpa_attention(q: Tensor, k: Tensor, v: Tensor, additive_mask: Tensor | None, scaling: float) -> Tensor:
    """Dense SDPA over ``[B, H, S, D]`` (views allowed); returns ``[B, S, H*D]``."""
    out = F.scaled_dot_product_attention(q, k, v, attn_mask=additive_mask, dropout_p=0.0, is_causal=False,
                                         scale=scaling)
    b, _, s, _ = out.shape
    return out.transpose(1, 2).reshape(b, s, -1)


def use_bshd_rope(backend: str, h: int, d: int, cu_seqlens: Tensor | None) -> bool:
    """Whether the layer takes the packed BSHD path (RoPE straight from qkv, then varlen
    attention on ``[T, H, D]``): the HIP backend, a head dim its kernels serve, and no autograd
    (the kernels are forward-only)."""
    return backend == "hip" and d in (64, 128, 256) and not torch.is_grad_enabled()


def attention_bshd(q: Tensor, k: Tensor, v: Tensor, *, window: tuple[int, int], scaling: float,
                   cu_seqlens: Tensor | None = None, max_seqlen: int | None = None,
                   backend: str = "hip") -> Tensor:
    """BSHD attention: q, k ``[B, S, H, D]`` (contiguous), v possibly a strided view. With
    ``cu_seqlens`` (B = 1) every segment attends within itself; without, each batch row is one
    segment. Returns ``[B, S, H*D]``."""
    if backend != "hip":
        raise ValueError(f"BSHD attention runs on the HIP kernels only (backend={backend!r})")
    varlen_attention = _load_hip_attention()
    b, s, h, d = q.shape
    floor = None  # packed: the enclosing shared_plans scope's host bound
    if cu_seqlens is None:
        cu_seqlens = torch.arange(0, (b + 1) * s, s, dtype=torch.int32, device=q.device)
        max_seqlen = floor = s  # every row one segment of exactly s tokens
    elif b != 1:
        raise ValueError("packed attention takes a batch of one flat sequence")
    out = varlen_attention(q.reshape(b * s, h, d), k.reshape(b * s, k.shape[2], d), v.reshape(b * s, v.shape[2], d),
                           cu_seqlens, int(max_seqlen), softmax_scale=scaling, window=tuple(window),
                           min_seqlen=floor)
    return out.reshape(b, s, h * d)


def fused_rope_applies(qkv: Tensor, d: int, seq: int) -> bool:
    """Whether ``flash_attention_qkv_bshd`` fuses RoPE into the attention call: bf16 on the
    GPU, head_dim 64 or 128, and segments of at most 128 tokens, which the short kernel (the one
    that carries the fused prologue) serves whole."""
    return qkv.is_cuda and qkv.dtype == torch.bfloat16 and d in (64, 128) and 0 < seq <= 128


def flash_attention_qkv_bshd(qkv: Tensor, h: int, d: int, *, cos: Tensor, sin: Tensor, window: tuple[int, int],
                             scaling: float, cu_seqlens: Tensor | None = None, max_seqlen: int | None = None,
                             backend: str = "hip") -> Tensor:
    """RoPE + attention reading ``qkv [B, S, 3*h*d]`` directly (the reference's
    ``flash_attention_qkv_bshd``, ops.py:485-499: its RoPE kernel, then ``attention_bshd``).
    ``cos``/``sin`` are the ``rope_qkv`` tables. When every segment fits the short kernel
    (``fused_rope_applies``) the RoPE is fused into the attention call: q and k are read
    unrotated out of ``qkv`` and no rotated copy is written, with the same bits as the two
    steps. Otherwise the RoPE kernel writes q and k and ``attention_bshd`` follows. Returns
    ``[B, S, h*d]``."""
    if backend != "hip":
        raise ValueError(f"BSHD attention runs on the HIP kernels only (backend={backend!r})")
    b, s = qkv.shape[:2]
    view = qkv.view(b, s, 3, h, d)
    if cu_seqlens is not None and b != 1:
        raise ValueError("packed attention takes a batch of one flat sequence")
    seq = s if cu_seqlens is None else int(max_seqlen)
    if not fused_rope_applies(qkv, d, seq):
        q, k = rope_qkv(qkv, h, d, cos, sin)
        return attention_bshd(q, k, view[:, :, 2], window=window, scaling=scaling, cu_seqlens=cu_seqlens,
                              max_seqlen=max_seqlen, backend=backend)
    varlen_attention = _load_hip_attention()
    floor = None  # packed: the enclosing shared_plans scope's host bound
    if cu_seqlens is None:
        cu_seqlens = torch.arange(0, (b + 1) * s, s, dtype=torch.int32, device=qkv.device)
        max_seqlen = floor = s
    q, k, v = (view[:, :, i].reshape(b * s, h, d) for i in range(3))
    out = varlen_attention(q, k, v, cu_seqlens, int(max_seqlen), softmax_scale=scaling, window=tuple(window),
                           min_seqlen=floor, rope=(cos.reshape(-1, d), sin.reshape(-1, d)))
    return out.reshape(b, s, h * d)


def attention(q: Tensor, k: Tensor, v: Tensor, *, mask: Tensor | None, window: tuple[int, int], scaling: float,
              backend: str, cu_seqlens: Tensor | None = None, max_seqlen: int | None = None) -> Tensor:
    """BHSD attention dispatch (ops.py:541-555): ``"sdpa"`` uses the additive ``mask``, ``"hip"``
    the ``window`` and ``cu_seqlens``. An unresolved ``"auto"`` (no host-visible statistics, e.g.
    inside a capture) stays on SDPA, as in the reference."""
    if backend == "hip":
        return attention_bshd(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), window=window,
                              scaling=scaling, cu_seqlens=cu_seqlens, max_seqlen=max_seqlen)
    return sdpa_attention(q, k, v, mask, scaling)
