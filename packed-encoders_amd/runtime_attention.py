"""Choose a varlen attention kernel for one head geometry by probing it
(packed_encoders/runtime/attention.py:40-315).

Engines with grouped-query, causal or windowed attention (the reference's Qwen3.5, LFM and
EmbeddingGemma engines) ask ``select_attention`` once per attention kind. Each candidate must
build, run and match fp32 per-segment SDPA (max-abs < 2e-2) on a probe that holds an empty
segment and grouped KV heads, in both layouts the engines use:

- packed: tokens back to back with ``cu_seqlens`` (eager forward);
- padded: ``(rows, S)`` rectangles whose rows are ``[real | pad]`` segments (graphs), described
  by ``PaddedStatic.seg_cu32`` with ``2 * rows + 1`` boundaries.

Candidates, in order: ``"hip"`` (this library's kernels: packed and padded forms are one varlen
call each, GQA, causal and window handled in-kernel) and ``"sdpa"`` (always passes, so
selection never fails). A causal engine also gets the *prefixed* form, where a query segment is
the tail of a longer key segment (mask aligned to the segment end): one varlen call with
separate key segments (``cu_seqlens_k``). Rejections keep their reason.
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass, field
from typing import Callable

import torch
import torch.nn.functional as F
from torch import Tensor

from .errors import ValidationError

PROBE_TOLERANCE = 2e-2  # max abs error vs fp32 SDPA on unit-variance bf16 inputs


@dataclass
class PaddedStatic:
    """A ``(rows, seq)`` rectangle: row r holds ``lens[r]`` real tokens then padding.
    ``seg_cu32`` splits it into ``[real | pad]`` segments (packed_encoders/runtime/graphs.py:65-74)."""

    rows: int
    seq: int
    ids: Tensor
    seg_cu32: Tensor
    lens: Tensor


@dataclass
class AttentionChoice:
    """``packed(q, k, v, cu32, max_len, lengths, causal)`` and ``padded(q, k, v, static, causal)``
    take ``[tokens, heads, head_dim]`` (k/v may have fewer heads) and return q's shape;
    ``prefixed(q, k, v, cu_q, cu_k, max_q, max_k, lengths_q, lengths_k, causal)`` for causal
    engines. Every form applies ``window`` and ``scale``."""

    name: str
    packed: Callable[..., Tensor]
    padded: Callable[..., Tensor]
    max_abs_err: float = 0.0
    rejected: dict[str, str] = field(default_factory=dict)
    prefixed: Callable[..., Tensor] | None = None
    prefixed_name: str | None = None
    prefixed_max_abs_err: float | None = None
    window: tuple[int, int] = (-1, -1)
    scale: float | None = None


# ----------------------------------------------------------------------------- candidates


def _hip(window, scale) -> tuple[Callable, ...]:
    from . import ops

    varlen_attention = ops._load_hip_attention()  # ImportError when the library is unavailable

    def packed(q, k, v, cu32, max_len, lengths, causal):
        return varlen_attention(q, k, v, cu32, max_len, softmax_scale=scale, window=window, causal=causal)

    def padded(q, k, v, static: PaddedStatic, causal):
        # [real | pad] segments: pads attend among themselves (their rows are discarded)
        return varlen_attention(q, k, v, static.seg_cu32, static.seq, softmax_scale=scale, window=window,
                                causal=causal)

    def prefixed(q, k, v, cu_q, cu_k, max_q, max_k, lengths_q, lengths_k, causal):
        # query segment s is the tail of key segment s: the kernels' separate key segments
        return varlen_attention(q, k, v, cu_q, max_q, softmax_scale=scale, window=window, causal=causal,
                                cu_seqlens_k=cu_k, max_seqlen_k=max_k)

    return packed, padded, prefixed


def _repeat_kv(q: Tensor, k: Tensor, v: Tensor, dim: int) -> tuple[Tensor, Tensor]:
    r = q.shape[dim] // k.shape[dim]
    return (k, v) if r == 1 else (k.repeat_interleave(r, dim), v.repeat_interleave(r, dim))


def band(n_q: int, n_k: int, causal: bool, window, device) -> Tensor | None:
    """Keys each query may read, the queries being the last ``n_q`` of ``n_k`` positions; None
    when every key is allowed."""
    left, right = window
    right = 0 if causal else right
    if left < 0 and right < 0:
        return None
    delta = torch.arange(n_k - n_q, n_k, device=device)[:, None] - torch.arange(n_k, device=device)[None, :]
    allowed = torch.ones(n_q, n_k, dtype=torch.bool, device=device)
    if left >= 0:
        allowed &= delta <= left
    if right >= 0:
        allowed &= delta >= -right
    return allowed


def segments(q, k, v, lengths_q, lengths_k, causal, window=(-1, -1), scale=None) -> Tensor:
    """One SDPA per segment (host lengths); query segment i is the tail of key segment i."""
    k, v = _repeat_kv(q, k, v, 1)
    outs = []
    for qs, ks, vs in zip(q.split(list(lengths_q)), k.split(list(lengths_k)), v.split(list(lengths_k))):
        if not qs.shape[0]:
            continue
        mask = band(qs.shape[0], ks.shape[0], causal, window, q.device)
        qb, kb, vb = (x.transpose(0, 1).unsqueeze(0) for x in (qs, ks, vs))
        outs.append(F.scaled_dot_product_attention(qb, kb, vb, attn_mask=mask, scale=scale).squeeze(0).transpose(0, 1))
    return torch.cat(outs) if outs else torch.empty_like(q)


def _sdpa(window, scale) -> tuple[Callable, ...]:
    def packed(q, k, v, cu32, max_len, lengths, causal):
        return segments(q, k, v, list(lengths), list(lengths), causal, window, scale)

    def padded(q, k, v, static: PaddedStatic, causal):
        rows, seq = static.rows, static.seq
        k, v = _repeat_kv(q, k, v, 1)
        qb, kb, vb = (t.view(rows, seq, t.shape[1], t.shape[2]).transpose(1, 2) for t in (q, k, v))
        pad = torch.arange(seq, device=q.device)[None, :] >= static.lens[:, None]
        allowed = pad[:, :, None] == pad[:, None, :]
        b = band(seq, seq, causal, window, q.device)
        if b is not None:
            allowed = allowed & b
        out = F.scaled_dot_product_attention(qb, kb, vb, attn_mask=allowed[:, None], scale=scale)
        return out.transpose(1, 2).reshape(rows * seq, q.shape[1], q.shape[2])

    def prefixed(q, k, v, cu_q, cu_k, max_q, max_k, lengths_q, lengths_k, causal):
        return segments(q, k, v, list(lengths_q), list(lengths_k), causal, window, scale)

    return packed, padded, prefixed


_CANDIDATES: dict[str, Callable[..., tuple[Callable, ...]]] = {"hip": _hip, "sdpa": _sdpa}


def default_order(device: torch.device) -> tuple[str, ...]:
    return ("hip", "sdpa") if device.type == "cuda" else ("sdpa",)


# ----------------------------------------------------------------------------- probes


def reference(q, k, v, lengths, causal, window=(-1, -1), scale=None) -> Tensor:
    """fp32 per-segment SDPA."""
    return segments(q.float(), k.float(), v.float(), list(lengths), list(lengths), causal, window, scale)


def reference_prefixed(q, k, v, lengths_q, lengths_k, causal, window=(-1, -1), scale=None) -> Tensor:
    return segments(q.float(), k.float(), v.float(), list(lengths_q), list(lengths_k), causal, window, scale)


def _cu(lengths, device) -> Tensor:
    out = [0]
    for n in lengths:
        out.append(out[-1] + int(n))
    return torch.tensor(out, dtype=torch.int32, device=device)


def probe(packed, padded, *, n_heads, n_kv_heads, head_dim, causal, device, dtype, window, scale) -> float:
    """Max-abs error of both forms against fp32 SDPA (runtime/attention.py:207-239): packed
    lengths ``[5, max(64, 2*max(window)+3), 0, 37]``; padded rows ``[5, S, 0]`` of
    ``S = max(48, 2*max(window)+3)``, only real rows compared."""
    gen = torch.Generator(device=device).manual_seed(0)
    span = 2 * max(window) + 3

    def rnd(t, h):
        return torch.randn(t, h, head_dim, device=device, dtype=dtype, generator=gen)

    lengths = [5, max(64, span), 0, 37]
    total = sum(lengths)
    q, k, v = rnd(total, n_heads), rnd(total, n_kv_heads), rnd(total, n_kv_heads)
    ref = reference(q, k, v, lengths, causal, window, scale)
    err = (packed(q, k, v, _cu(lengths, device), max(lengths), lengths, causal).float() - ref).abs().max().item()

    rows, seq = 3, max(48, span)
    lens = [5, seq, 0]
    seg = []
    for n in lens:
        seg += [n, seq - n]
    static = PaddedStatic(rows=rows, seq=seq, ids=torch.zeros(rows, seq, dtype=torch.long, device=device),
                          seg_cu32=_cu(seg, device), lens=torch.tensor(lens, dtype=torch.int32, device=device))
    q, k, v = rnd(rows * seq, n_heads), rnd(rows * seq, n_kv_heads), rnd(rows * seq, n_kv_heads)
    out = padded(q, k, v, static, causal).float()
    keep = torch.cat([torch.arange(r * seq, r * seq + n) for r, n in enumerate(lens)]).to(device)
    ref = reference(q.index_select(0, keep), k.index_select(0, keep), v.index_select(0, keep), lens, causal, window,
                    scale)
    return max(err, (out.index_select(0, keep) - ref).abs().max().item())


def probe_prefixed(prefixed, *, n_heads, n_kv_heads, head_dim, device, dtype, window, scale, causal=True) -> float:
    gen = torch.Generator(device=device).manual_seed(1)
    lengths_q, lengths_k = [5, 1, 37, 16], [40, 64, 37, 80]

    def rnd(t, h):
        return torch.randn(t, h, head_dim, device=device, dtype=dtype, generator=gen)

    q, k, v = rnd(sum(lengths_q), n_heads), rnd(sum(lengths_k), n_kv_heads), rnd(sum(lengths_k), n_kv_heads)
    got = prefixed(q, k, v, _cu(lengths_q, device), _cu(lengths_k, device), max(lengths_q), max(lengths_k),
                   lengths_q, lengths_k, causal)
    return (got.float() - reference_prefixed(q, k, v, lengths_q, lengths_k, causal, window, scale)).abs().max().item()


def select_attention(*, n_heads: int, n_kv_heads: int, head_dim: int, causal: bool, device: torch.device,
                     dtype: torch.dtype = torch.bfloat16, order: Sequence[str] | None = None,
                     window: tuple[int, int] = (-1, -1), scale: float | None = None,
                     bidirectional_prefixed: bool = False) -> AttentionChoice:
    """The first candidate of ``order`` that builds, runs and matches fp32 SDPA; for a causal
    kind also its prefixed form (or SDPA's). ``window`` and ``scale`` (None: ``head_dim**-0.5``)
    are bound into the kernels and probed."""
    device = torch.device(device)
    rejected: dict[str, str] = {}
    window = tuple(int(w) for w in window)
    geometry = dict(n_heads=n_heads, n_kv_heads=n_kv_heads, head_dim=head_dim, device=device, dtype=dtype,
                    window=window, scale=scale)
    for name in order or default_order(device):
        try:
            packed, padded, prefixed = _CANDIDATES[name](window, scale)
            err = probe(packed, padded, causal=causal, **geometry)
        except Exception as exc:  # noqa: BLE001 - any build or launch failure rejects the candidate
            rejected[name] = _reason(exc)
            continue
        if not err < PROBE_TOLERANCE:
            rejected[name] = f"mismatch vs fp32 SDPA: max abs err {err:.3g}"
            continue
        choice = AttentionChoice(name=name, packed=packed, padded=padded, max_abs_err=err, rejected=rejected,
                                 window=window, scale=scale)
        if causal:
            for pname, fn in ((name, prefixed), ("sdpa", _sdpa(window, scale)[2])):
                try:
                    perr = max(probe_prefixed(fn, causal=c, **geometry)
                               for c in ((True, False) if bidirectional_prefixed else (True,)))
                except Exception as exc:  # noqa: BLE001
                    rejected[f"{pname}:prefixed"] = _reason(exc)
                    continue
                if perr < PROBE_TOLERANCE:
                    choice.prefixed, choice.prefixed_name, choice.prefixed_max_abs_err = fn, pname, perr
                    break
                rejected[f"{pname}:prefixed"] = f"mismatch vs fp32 SDPA: max abs err {perr:.3g}"
        return choice
    raise ValidationError(f"no attention candidate passed: {rejected}")


def _reason(exc: Exception) -> str:
    text = str(exc).splitlines()[0][:160] if str(exc) else ""
    return f"{type(exc).__name__}: {text}"


def sigmoid_gate(o: Tensor, gate: Tensor) -> Tensor:
    """``bf16(o * bf16(sigmoid(gate)))`` (packed_encoders/_kernels/hybrid.py:197-219) for callers
    that gate outside the attention call; ``varlen_attention(..., gate=)`` fuses the same
    rounding sequence into the kernels' epilogue."""
    s = torch.sigmoid(gate.float()).to(o.dtype)
    return (o.float() * s.float()).to(o.dtype)
