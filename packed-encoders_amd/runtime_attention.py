"""Pick the varlen attention implementation for one attention kind by measuring it.

Engines with grouped-query, causal or windowed attention (the reference's Qwen3.5, LFM and
EmbeddingGemma engines) ask ``select_attention`` once per attention kind (head geometry,
causality, window, scale) and keep the answer; the reference's counterpart is
packed_encoders/runtime/attention.py:40-315, whose public surface this module keeps:
``select_attention`` with its keyword arguments, ``AttentionChoice`` with its fields, and the
candidate registry ``_CANDIDATES[name] = factory(window, scale) -> (packed, padded, prefixed)``.

How a candidate is judged here: it is built for the kind, run on three small layouts, and
compared with a float64 oracle computed on the device from segment ids (``oracle_attention``),
a formulation that shares no code with either candidate. The layouts:

- packed: segments back to back with int32 ``cu_seqlens``, including an empty segment, a
  single token and a segment longer than the window span (so the window binds on both sides);
- padded: a ``(rows, seq)`` rectangle whose rows are ``[real | pad]`` segment pairs
  (``PaddedStatic.seg_cu32``: ``2 * rows + 1`` boundaries), the graph-friendly layout;
- prefixed (causal kinds): query segments that are the tails of longer key segments, the mask
  aligned to the segment end (rows continuing a shared prefix).

The first candidate of the order whose error stays under ``PROBE_TOLERANCE`` on every layout
wins; ``"sdpa"`` always passes, so selection never fails, and every rejection keeps its reason.
Candidates: ``"hip"`` (this library's kernels: each form is one ``varlen_attention`` call, GQA,
causal and window in-kernel) and ``"sdpa"`` (torch SDPA over length-bucketed padded batches).
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass, field
from typing import Callable

import torch
import torch.nn.functional as F
from torch import Tensor

from .errors import ValidationError

PROBE_TOLERANCE = 2e-2  # max abs error vs the float64 oracle on unit-variance bf16 inputs

# Padded-batch SDPA runs segments of similar length together; a bucket holds at most this many
# (segment x query x key x head) score elements, so its attention weights stay a few MB.
_SDPA_BUCKET_ELEMENTS = 1 << 25


@dataclass
class PaddedStatic:
    """A ``(rows, seq)`` rectangle: row r holds ``lens[r]`` real tokens then padding.
    ``seg_cu32`` splits it into ``[real | pad]`` segments, ``2 * rows + 1`` int32 boundaries
    (packed_encoders/runtime/graphs.py:65-74)."""

    rows: int
    seq: int
    ids: Tensor
    seg_cu32: Tensor
    lens: Tensor


@dataclass
class AttentionChoice:
    """The selected kernels of one attention kind (packed_encoders/runtime/attention.py:43-60).

    ``packed(q, k, v, cu32, max_len, lengths, causal)`` and ``padded(q, k, v, static, causal)``
    take ``[tokens, heads, head_dim]`` (k/v may have fewer heads) and return q's shape;
    ``prefixed(q, k, v, cu_q, cu_k, max_q, max_k, lengths_q, lengths_k, causal)`` serves causal
    kinds, query segment i being the last ``lengths_q[i]`` positions of key segment i. Every
    form applies ``window`` and ``scale``."""

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


# ----------------------------------------------------------------------------- masks and oracle


def allowed_keys(q_pos: Tensor, k_pos: Tensor, causal: bool, window: tuple[int, int]) -> Tensor:
    """Bool ``[..., n_q, n_k]``: a query at key position ``q_pos`` may read the key at ``k_pos``
    (``left`` keys back, ``right`` ahead, -1 unbounded; causal caps ``right`` at 0)."""
    left, right = window
    if causal:
        right = 0
    ahead = k_pos.unsqueeze(-2) - q_pos.unsqueeze(-1)  # key position minus query position
    ok = torch.ones_like(ahead, dtype=torch.bool)
    if left >= 0:
        ok &= ahead >= -left
    if right >= 0:
        ok &= ahead <= right
    return ok


def _segment_positions(lengths_q: Sequence[int], lengths_k: Sequence[int], device) -> tuple[Tensor, ...]:
    """Segment id and key position of every query and key token (queries end-aligned)."""
    lq = torch.tensor([int(n) for n in lengths_q], dtype=torch.long, device=device)
    lk = torch.tensor([int(n) for n in lengths_k], dtype=torch.long, device=device)
    seg_q = torch.repeat_interleave(torch.arange(lq.numel(), device=device), lq)
    seg_k = torch.repeat_interleave(torch.arange(lk.numel(), device=device), lk)
    start_q = torch.cumsum(lq, 0) - lq
    start_k = torch.cumsum(lk, 0) - lk
    pos_q = torch.arange(seg_q.numel(), device=device) - start_q[seg_q] + (lk - lq)[seg_q]
    pos_k = torch.arange(seg_k.numel(), device=device) - start_k[seg_k]
    return seg_q, pos_q, seg_k, pos_k


def oracle_attention(q: Tensor, k: Tensor, v: Tensor, lengths_q: Sequence[int], lengths_k: Sequence[int],
                     causal: bool, window: tuple[int, int] = (-1, -1), scale: float | None = None) -> Tensor:
    """Float64 attention over the whole packed batch at once: one score matrix, masked to each
    query's own segment and window (key positions from segment ids, queries the tail of their
    key segment); kv head ``h // (Hq / Hkv)`` serves query head h. A query that reaches no key
    gets zeros. For probe-sized inputs (the score matrix is ``[Hq, Tq, Tk]``)."""
    hq, d = q.shape[1], q.shape[2]
    group = hq // k.shape[1]
    scale = d ** -0.5 if scale is None else scale
    seg_q, pos_q, seg_k, pos_k = _segment_positions(lengths_q, lengths_k, q.device)
    mask = (seg_q[:, None] == seg_k[None, :]) & allowed_keys(pos_q, pos_k, causal, window)
    kk = k.double().repeat_interleave(group, dim=1)
    vv = v.double().repeat_interleave(group, dim=1)
    scores = torch.einsum("qhd,khd->hqk", q.double(), kk) * scale
    scores = scores.masked_fill(~mask, float("-inf"))
    top = scores.amax(dim=-1, keepdim=True)
    top = torch.where(torch.isfinite(top), top, torch.zeros_like(top))
    weights = torch.exp(scores - top)
    total = weights.sum(dim=-1, keepdim=True)
    weights = weights / torch.where(total > 0, total, torch.ones_like(total))
    return torch.einsum("hqk,khd->qhd", weights, vv)


def reference(q, k, v, lengths, causal, window=(-1, -1), scale=None) -> Tensor:
    """The float64 oracle for a packed batch (query and key segments shared)."""
    return oracle_attention(q, k, v, lengths, lengths, causal, window, scale)


def reference_prefixed(q, k, v, lengths_q, lengths_k, causal, window=(-1, -1), scale=None) -> Tensor:
    """The float64 oracle with query segment i the tail of key segment i."""
    return oracle_attention(q, k, v, lengths_q, lengths_k, causal, window, scale)


# ----------------------------------------------------------------------------- candidates


def _hip(window, scale) -> tuple[Callable, ...]:
    """This library's kernels: every form is one varlen call."""
    from . import ops

    varlen_attention = ops._load_hip_attention()  # ImportError when the library is unavailable

    def packed(q, k, v, cu32, max_len, lengths, causal):
        shortest = min((int(n) for n in lengths), default=0)  # host lengths: no short pass when none is short
        return varlen_attention(q, k, v, cu32, max_len, softmax_scale=scale, window=window, causal=causal,
                                min_seqlen=min(shortest, int(max_len)))

    def padded(q, k, v, static: PaddedStatic, causal):
        # [real | pad] segments: pads attend among themselves and their rows are discarded
        return varlen_attention(q, k, v, static.seg_cu32, static.seq, softmax_scale=scale, window=window,
                                causal=causal)

    def prefixed(q, k, v, cu_q, cu_k, max_q, max_k, lengths_q, lengths_k, causal):
        # query segment s is the tail of key segment s: the kernels' separate key segments
        shortest = min((int(n) for n in lengths_q), default=0)
        return varlen_attention(q, k, v, cu_q, max_q, softmax_scale=scale, window=window, causal=causal,
                                cu_seqlens_k=cu_k, max_seqlen_k=max_k, min_seqlen=min(shortest, int(max_q)))

    return packed, padded, prefixed


def bucketed_sdpa(q: Tensor, k: Tensor, v: Tensor, lengths_q: Sequence[int], lengths_k: Sequence[int],
                  causal: bool, window: tuple[int, int] = (-1, -1), scale: float | None = None) -> Tensor:
    """Varlen attention with torch SDPA on host-known lengths: segments sorted by length are cut
    into buckets, each gathered into a padded ``[n, H, S, D]`` batch with a per-segment mask
    (key validity, window, end-aligned causality) and run as one SDPA call, and the real rows
    are scattered back. GQA heads are expanded for SDPA."""
    lengths_q = [int(n) for n in lengths_q]
    lengths_k = [int(n) for n in lengths_k]
    out = torch.zeros_like(q)
    group = q.shape[1] // k.shape[1]
    if group > 1:
        k, v = k.repeat_interleave(group, dim=1), v.repeat_interleave(group, dim=1)
    h, dev = q.shape[1], q.device
    starts_q = [0]
    starts_k = [0]
    for a, b in zip(lengths_q, lengths_k):
        starts_q.append(starts_q[-1] + a)
        starts_k.append(starts_k[-1] + b)
    order = sorted((i for i, n in enumerate(lengths_q) if n > 0), key=lambda i: (lengths_k[i], lengths_q[i]))
    while order:
        # grow the bucket while its padded score block stays under the budget
        take = 1
        while take < len(order):
            sq = max(lengths_q[i] for i in order[:take + 1])
            sk = max(lengths_k[i] for i in order[:take + 1])
            if (take + 1) * sq * sk * h > _SDPA_BUCKET_ELEMENTS:
                break
            take += 1
        bucket, order = order[:take], order[take:]
        sq = max(lengths_q[i] for i in bucket)
        sk = max(lengths_k[i] for i in bucket)
        rows_q = torch.tensor([starts_q[i] + r if r < lengths_q[i] else 0 for i in bucket for r in range(sq)],
                              dtype=torch.long, device=dev)
        rows_k = torch.tensor([starts_k[i] + r if r < lengths_k[i] else 0 for i in bucket for r in range(sk)],
                              dtype=torch.long, device=dev)
        n = len(bucket)
        qb = q.index_select(0, rows_q).view(n, sq, h, -1).transpose(1, 2)
        kb = k.index_select(0, rows_k).view(n, sk, h, -1).transpose(1, 2)
        vb = v.index_select(0, rows_k).view(n, sk, h, -1).transpose(1, 2)
        lq = torch.tensor([lengths_q[i] for i in bucket], device=dev)
        lk = torch.tensor([lengths_k[i] for i in bucket], device=dev)
        r_q = torch.arange(sq, device=dev)
        r_k = torch.arange(sk, device=dev)
        q_pos = r_q[None, :] + (lk - lq)[:, None]  # queries end-aligned to their keys
        k_pos = r_k[None, :].expand(n, sk)
        mask = allowed_keys(q_pos, k_pos, causal, window) & (r_k[None, None, :] < lk[:, None, None])
        # a padded query row or a real row that reaches no key reads one key, discarded below
        empty = ~mask.any(dim=-1, keepdim=True)
        mask = mask | (empty & (r_k == 0)[None, None, :])
        ob = F.scaled_dot_product_attention(qb, kb, vb, attn_mask=mask[:, None], scale=scale)
        ob = ob.masked_fill(empty[:, None], 0.0)
        ob = ob.transpose(1, 2).reshape(n * sq, h, -1)
        real = torch.tensor([r < lengths_q[i] for i in bucket for r in range(sq)], device=dev)
        out.index_copy_(0, rows_q[real], ob[real])
    return out


def _sdpa(window, scale) -> tuple[Callable, ...]:
    """torch SDPA: the packed and prefixed forms read host lengths (eager only); the padded form
    builds its ``[real | pad]`` mask on the device from ``lens`` (capture-safe)."""

    def packed(q, k, v, cu32, max_len, lengths, causal):
        return bucketed_sdpa(q, k, v, lengths, lengths, causal, window, scale)

    def padded(q, k, v, static: PaddedStatic, causal):
        rows, seq = static.rows, static.seq
        group = q.shape[1] // k.shape[1]
        if group > 1:
            k, v = k.repeat_interleave(group, dim=1), v.repeat_interleave(group, dim=1)
        qb, kb, vb = (t.view(rows, seq, t.shape[1], t.shape[2]).transpose(1, 2) for t in (q, k, v))
        pos = torch.arange(seq, device=q.device)
        is_pad = pos[None, :] >= static.lens[:, None]
        # real and pad halves of a row are separate segments; a window compares positions
        # within the row, which serves both halves
        same_half = is_pad[:, :, None] == is_pad[:, None, :]
        mask = same_half & allowed_keys(pos, pos, causal, window)[None]
        out = F.scaled_dot_product_attention(qb, kb, vb, attn_mask=mask[:, None], scale=scale)
        return out.transpose(1, 2).reshape(rows * seq, q.shape[1], q.shape[2])

    def prefixed(q, k, v, cu_q, cu_k, max_q, max_k, lengths_q, lengths_k, causal):
        return bucketed_sdpa(q, k, v, lengths_q, lengths_k, causal, window, scale)

    return packed, padded, prefixed


_CANDIDATES: dict[str, Callable[..., tuple[Callable, ...]]] = {"hip": _hip, "sdpa": _sdpa}


def default_order(device: torch.device) -> tuple[str, ...]:
    return ("hip", "sdpa") if torch.device(device).type == "cuda" else ("sdpa",)


# ----------------------------------------------------------------------------- probes


def _cu(lengths: Sequence[int], device) -> Tensor:
    bounds = [0]
    for n in lengths:
        bounds.append(bounds[-1] + int(n))
    return torch.tensor(bounds, dtype=torch.int32, device=device)


class _Inputs:
    """Seeded unit-variance q / k / v of one probe geometry."""

    def __init__(self, seed: int, *, n_heads: int, n_kv_heads: int, head_dim: int, device, dtype):
        self.gen = torch.Generator(device=device).manual_seed(seed)
        self.h, self.hkv, self.d, self.device, self.dtype = n_heads, n_kv_heads, head_dim, device, dtype

    def __call__(self, tokens_q: int, tokens_k: int | None = None) -> tuple[Tensor, Tensor, Tensor]:
        tokens_k = tokens_q if tokens_k is None else tokens_k

        def draw(t, h):
            return torch.randn(t, h, self.d, device=self.device, dtype=self.dtype, generator=self.gen)

        return draw(tokens_q, self.h), draw(tokens_k, self.hkv), draw(tokens_k, self.hkv)


def probe(packed, padded, *, n_heads, n_kv_heads, head_dim, causal, device, dtype, window, scale) -> float:
    """Worst max-abs error of the packed and padded forms against the float64 oracle. Packed
    lengths ``[1, 0, max(96, span + 7), 45, 3]`` (span = the window's reach, so the window binds
    on both sides of some token); a padded rectangle of rows ``[seq, 7, 0]`` real tokens, only
    real rows compared."""
    draw = _Inputs(23 + n_heads + 5 * n_kv_heads, n_heads=n_heads, n_kv_heads=n_kv_heads, head_dim=head_dim,
                   device=device, dtype=dtype)
    span = 2 * max(window) + 3
    lengths = [1, 0, max(96, span + 7), 45, 3]
    q, k, v = draw(sum(lengths))
    got = packed(q, k, v, _cu(lengths, device), max(lengths), lengths, causal)
    worst = (got.double() - reference(q, k, v, lengths, causal, window, scale)).abs().max().item()

    seq = max(40, span + 3)
    lens = [seq, 7, 0]
    halves = [part for n in lens for part in (n, seq - n)]
    static = PaddedStatic(rows=len(lens), seq=seq, ids=torch.zeros(len(lens), seq, dtype=torch.long, device=device),
                          seg_cu32=_cu(halves, device), lens=torch.tensor(lens, dtype=torch.int32, device=device))
    q, k, v = draw(len(lens) * seq)
    got = padded(q, k, v, static, causal)
    real = torch.cat([torch.arange(r * seq, r * seq + n, device=device) for r, n in enumerate(lens)])
    want = reference(q[real], k[real], v[real], lens, causal, window, scale)
    return max(worst, (got[real].double() - want).abs().max().item())


def probe_prefixed(prefixed, *, n_heads, n_kv_heads, head_dim, device, dtype, window, scale, causal=True) -> float:
    """Max-abs error of the prefixed form: query segments ``[9, 1, 30, 2]`` as the tails of key
    segments ``[31, 48, 30, 70]`` (a short tail, a single token, a square, a long prefix)."""
    draw = _Inputs(71 + n_heads + 5 * n_kv_heads, n_heads=n_heads, n_kv_heads=n_kv_heads, head_dim=head_dim,
                   device=device, dtype=dtype)
    lengths_q, lengths_k = [9, 1, 30, 2], [31, 48, 30, 70]
    q, k, v = draw(sum(lengths_q), sum(lengths_k))
    got = prefixed(q, k, v, _cu(lengths_q, device), _cu(lengths_k, device), max(lengths_q), max(lengths_k),
                   lengths_q, lengths_k, causal)
    want = reference_prefixed(q, k, v, lengths_q, lengths_k, causal, window, scale)
    return (got.double() - want).abs().max().item()


def _why(exc: BaseException) -> str:
    """One line naming why a candidate was rejected: the exception's type and the start of its
    message."""
    message = next(iter(str(exc).splitlines()), "")
    return type(exc).__name__ + (f": {message[:160]}" if message else "")


def _measure(fn: Callable[[], float]) -> tuple[float | None, str | None]:
    """(error, None) when the probe runs and passes, (None, reason) otherwise."""
    try:
        err = fn()
    except Exception as exc:  # noqa: BLE001 - a failure to build or launch rejects the candidate
        return None, _why(exc)
    if not err < PROBE_TOLERANCE:
        return None, f"mismatch vs the float64 oracle: max abs err {err:.3g}"
    return err, None


def _first_passing(tries: Sequence[tuple[str, Callable[[], float]]],
                   rejected: dict[str, str]) -> tuple[str, float] | None:
    """The first (label, probe) whose probe passes, as (label, error); every failure is recorded
    in ``rejected`` under its label."""
    for label, run in tries:
        err, why = _measure(run)
        if why is None:
            return label, err
        rejected[label] = why
    return None


def select_attention(*, n_heads: int, n_kv_heads: int, head_dim: int, causal: bool, device: torch.device,
                     dtype: torch.dtype = torch.bfloat16, order: Sequence[str] | None = None,
                     window: tuple[int, int] = (-1, -1), scale: float | None = None,
                     bidirectional_prefixed: bool = False) -> AttentionChoice:
    """The first candidate of ``order`` (default: ``"hip"`` then ``"sdpa"`` on a GPU) that builds,
    runs and matches the oracle on the packed and padded probes; for a causal kind also its
    prefixed form (or SDPA's when the winner's fails; ``bidirectional_prefixed`` also probes it
    without the causal mask). ``window`` and ``scale`` (None: ``head_dim ** -0.5``) are bound into
    the kernels and probed. ``ValidationError`` if no candidate passes."""
    device = torch.device(device)
    window = (int(window[0]), int(window[1]))
    geometry = dict(n_heads=n_heads, n_kv_heads=n_kv_heads, head_dim=head_dim, device=device, dtype=dtype,
                    window=window, scale=scale)
    rejected: dict[str, str] = {}
    built: dict[str, tuple[Callable, ...]] = {}

    def build(name: str) -> float:  # the candidate's forms, then its packed/padded probe
        built[name] = _CANDIDATES[name](window, scale)
        packed, padded, _ = built[name]
        return probe(packed, padded, causal=causal, **geometry)

    winner = _first_passing([(name, lambda name=name: build(name)) for name in (order or default_order(device))],
                            rejected)
    if winner is None:
        raise ValidationError(f"no attention candidate passed: {rejected}")
    name, err = winner
    packed, padded, prefixed = built[name]
    choice = AttentionChoice(name=name, packed=packed, padded=padded, max_abs_err=err, rejected=rejected,
                             window=window, scale=scale)
    if causal:
        masks = (True, False) if bidirectional_prefixed else (True,)
        fallbacks = {f"{name}:prefixed": prefixed, "sdpa:prefixed": _sdpa(window, scale)[2]}
        found = _first_passing([(label, lambda fn=fn: max(probe_prefixed(fn, causal=c, **geometry) for c in masks))
                                for label, fn in fallbacks.items()], rejected)
        if found is not None:
            label, perr = found
            choice.prefixed, choice.prefixed_name = fallbacks[label], label.split(":")[0]
            choice.prefixed_max_abs_err = perr
    return choice


def sigmoid_gate(o: Tensor, gate: Tensor) -> Tensor:
    """``bf16(o * bf16(sigmoid(gate)))`` (packed_encoders/_kernels/hybrid.py:197-219) for callers
    that gate outside the attention call; ``varlen_attention(..., gate=)`` fuses the same
    rounding sequence into the kernels' epilogue."""
    s = torch.sigmoid(gate.float()).to(o.dtype)
    return (o.float() * s.float()).to(o.dtype)
