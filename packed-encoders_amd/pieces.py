"""Operation pieces of the packed ModernBERT path: a callable, the contract it serves and an
oracle it is checked against.

The reference's plug-in slot for the attention hot path is a *piece*: an operation the engine
binds once (packed_encoders/pieces/base.py:17-69), with ``pieces/attention.py:11-73`` and
``arch/modernbert_pieces.py:18-128`` holding the attention pieces and the ModernBERT selection.
The names and meanings a caller relies on are kept here: ``Contract``, ``PieceValidation``,
``Piece(name, contract, execute, reference, check, rtol, atol)`` with ``validate``, and
``ModernBertPieces`` with its slots, ``bind()``, ``all()`` and ``validate(model)``; a slot is
substituted with ``dataclasses.replace(pieces, attention_bshd=...)`` and ``bind()`` refuses a
piece whose contract differs from the slot's.

How a piece is checked: ``Piece.validate`` runs the fixture through ``check``, the piece and
its oracle, and accepts the outputs element by element within ``atol + rtol * |oracle|``
(0.02 and 0.02 by default), reporting the worst absolute error; anything else raises
``ValidationError``. The attention oracle (``attention_reference``) is a float64 score matrix
masked by segment ids and the window, independent of every attention kernel of the package; it
reads ``cu_seqlens`` on the host, which is why it serves validation fixtures only.
"""

from __future__ import annotations

from dataclasses import dataclass, fields
from functools import lru_cache
from typing import Callable

import torch

from . import ops
from .errors import UnsupportedTargetError, ValidationError


@dataclass(frozen=True)
class Contract:
    """What a slot requires: the operation, its tensor layout, its semantics, and whether it
    must support autograd and graph capture. Two pieces fit the same slot iff equal."""

    operation: str
    layout: str
    semantics: str
    autograd: bool = True
    capture: bool = True


@dataclass(frozen=True)
class PieceValidation:
    """One slot's validation outcome: worst absolute error (None when skipped, with the reason)."""

    name: str
    max_abs_error: float | None
    rtol: float
    atol: float
    skipped_reason: str | None = None


def _outputs(value) -> tuple:
    return value if isinstance(value, tuple) else (value,)


def _within(got: torch.Tensor, want: torch.Tensor, rtol: float, atol: float) -> tuple[float, str | None]:
    """(worst absolute error, None) when every element of ``got`` lies within
    ``atol + rtol * |want|`` of ``want`` (equal non-finite values accepted), else a reason."""
    if got.shape != want.shape:
        return float("inf"), f"shape {tuple(got.shape)} instead of {tuple(want.shape)}"
    a, b = got.detach().double(), want.detach().double()
    finite = torch.isfinite(a) & torch.isfinite(b)
    same_special = ~finite & ((a == b) | (torch.isnan(a) & torch.isnan(b)))
    err = torch.where(finite, (a - b).abs(), torch.zeros_like(a))
    outside = (finite & (err > atol + rtol * b.abs())) | (~finite & ~same_special)
    worst = float(err.max()) if err.numel() else 0.0
    n_out = int(outside.sum())
    if n_out:
        return worst, f"{n_out} of {a.numel()} elements outside atol {atol} + rtol {rtol} * |reference|"
    return worst, None


@dataclass(frozen=True)
class Piece:
    """A callable operation with its contract and oracle. ``execute`` and ``reference`` take the
    same arguments; ``check`` rejects fixtures outside the contract (``UnsupportedTargetError``).
    Inputs are not mutated, and outputs own their storage."""

    name: str
    contract: Contract
    execute: Callable
    reference: Callable
    check: Callable
    rtol: float = 0.02
    atol: float = 0.02

    def validate(self, *args, **kwargs) -> PieceValidation:
        self.check(*args, **kwargs)
        with torch.no_grad():
            got = _outputs(self.execute(*args, **kwargs))
            want = _outputs(self.reference(*args, **kwargs))
        if len(got) != len(want):
            raise ValidationError(f"piece {self.name}: {len(got)} outputs where its reference has {len(want)}")
        worst = 0.0
        for i, (g, w) in enumerate(zip(got, want)):
            err, why = _within(g, w, self.rtol, self.atol)
            if why is not None:
                raise ValidationError(f"piece {self.name} failed reference validation on output {i}: {why} "
                                      f"(max abs error {err:.4g})")
            worst = max(worst, err)
        return PieceValidation(self.name, worst, self.rtol, self.atol)


# ----------------------------------------------------------------------------- contracts

LN = Contract("layer_norm", "x [.., H], w [H] -> [.., H]", "bias-free LayerNorm")
ADD_LN = Contract("add_layer_norm", "x, r [.., H], w [H] -> (x + r, LN(x + r))", "fused residual + LayerNorm")
LINEAR = Contract("linear", "x [.., K], w [N, K] -> [.., N]", "bias-free projection")
GEGLU = Contract("geglu", "proj [.., 2I] -> [.., I]", "gelu(first half) * second half")
ROPE_BHSD = Contract("rope", "q, k [B, H, S, D], cos, sin [B|1, S, D] -> q, k", "split-half RoPE in fp32")
ROPE_QKV = Contract("rope_qkv", "qkv [B, S, 3HD] -> q, k [B, S, H, D] contiguous", "split-half RoPE in fp32",
                    autograd=False)
BHSD = Contract("attention", "BHSD q,k,v -> BS(HD)",
                "noncausal; no dropout; SDPA additive mask or HIP local window; packed int32 boundaries")
BSHD = Contract("attention", "BSHD q,k,v -> BS(HD)",
                "noncausal; no dropout; HIP local window; packed int32 boundaries", autograd=False)


# ----------------------------------------------------------------------------- attention oracle


def _segment_ids(cu_seqlens: torch.Tensor, length: int) -> torch.Tensor:
    """Segment index of each of ``length`` token rows; rows past the last boundary get -1."""
    bounds = torch.as_tensor(cu_seqlens.detach().to("cpu", torch.long))  # host read: validation only
    rows = torch.arange(length)
    seg = torch.bucketize(rows, bounds[1:], right=True)
    seg = torch.where(rows < bounds[-1], seg, torch.full_like(seg, -1))
    return seg.to(cu_seqlens.device)


def _fp64_attention(q, k, v, *, scaling: float, additive=None, allowed=None) -> torch.Tensor:
    """``softmax(q k^T * scaling + additive, masked to allowed) v`` over ``[B, H, S, D]`` in
    float64; a row with no allowed key comes out as zeros."""
    scores = torch.matmul(q.double(), k.double().transpose(-1, -2)) * scaling
    if additive is not None:
        scores = scores + additive.double()
    if allowed is not None:
        scores = scores.masked_fill(~allowed, float("-inf"))
    top = scores.amax(dim=-1, keepdim=True)
    top = torch.where(torch.isfinite(top), top, torch.zeros_like(top))
    weights = torch.exp(scores - top)
    total = weights.sum(dim=-1, keepdim=True)
    return torch.matmul(weights / torch.where(total > 0, total, torch.ones_like(total)), v.double())


def _band(length: int, window: tuple[int, int], device) -> torch.Tensor | None:
    """Bool ``[S, S]``: key j within ``(left, right)`` of query i (-1 unbounded); None if unbounded."""
    left, right = window
    if left < 0 and right < 0:
        return None
    ahead = torch.arange(length, device=device)[None, :] - torch.arange(length, device=device)[:, None]
    ok = torch.ones(length, length, dtype=torch.bool, device=device)
    if left >= 0:
        ok &= ahead >= -left
    if right >= 0:
        ok &= ahead <= right
    return ok


def attention_reference(q, k, v, *, mask, window, scaling, backend, cu_seqlens=None, max_seqlen=None):
    """Oracle of the BHSD attention slot: ``[B, H, S, D]`` in, ``[B, S, H * D]`` out in q's dtype.
    The dense SDPA backend takes the additive mask as given; the HIP backend applies the window
    and, with ``cu_seqlens`` (B = 1), keeps every query inside its own segment (rows past the
    last boundary come out as zeros)."""
    s = q.shape[2]
    if backend != "hip":
        out = _fp64_attention(q, k, v, scaling=scaling, additive=mask)
    else:
        allowed = _band(s, window, q.device)
        if cu_seqlens is not None:
            seg = _segment_ids(cu_seqlens, s)
            same = (seg[:, None] == seg[None, :]) & (seg[:, None] >= 0)
            allowed = same if allowed is None else allowed & same
        out = _fp64_attention(q, k, v, scaling=scaling, allowed=allowed)
    return out.to(q.dtype).transpose(1, 2).reshape(q.shape[0], s, -1)


def attention_bshd_reference(q, k, v, *, window, scaling, backend="hip", cu_seqlens=None, max_seqlen=None):
    """Oracle of the BSHD attention slot (``[B, S, H, D]`` in; the BHSD oracle on a transposed view)."""
    return attention_reference(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), mask=None, window=window,
                               scaling=scaling, backend=backend, cu_seqlens=cu_seqlens, max_seqlen=max_seqlen)


def check_attention(q, k, v, *, mask, window, scaling, backend, cu_seqlens=None, max_seqlen=None):
    if q.ndim != 4 or q.shape != k.shape or q.shape != v.shape:
        raise UnsupportedTargetError("attention piece requires equal Q/K/V shapes")
    if backend not in ops.BACKENDS or not scaling > 0:
        raise UnsupportedTargetError("unsupported attention backend or scale")
    if cu_seqlens is not None and (q.shape[0] != 1 or cu_seqlens.dtype != torch.int32 or max_seqlen is None):
        raise UnsupportedTargetError("packed attention requires B=1, int32 boundaries and max_seqlen")


def check_attention_bshd(q, k, v, *, window, scaling, backend="hip", cu_seqlens=None, max_seqlen=None):
    if backend != "hip":
        raise UnsupportedTargetError("BSHD attention requires the HIP backend")
    check_attention(q, k, v, mask=None, window=window, scaling=scaling, backend=backend, cu_seqlens=cu_seqlens,
                    max_seqlen=max_seqlen)


def attention_piece() -> Piece:
    return Piece("attention-bhsd", BHSD, ops.attention, attention_reference, check_attention)


def attention_bshd_piece() -> Piece:
    return Piece("attention-bshd", BSHD, ops.attention_bshd, attention_bshd_reference, check_attention_bshd)


# ----------------------------------------------------------------------------- other oracles


def _accept(*args, **kwargs):
    return None


def _in_fp32(fn):
    """The oracle of an elementwise / normalisation / projection piece: the same torch expression
    evaluated in fp32 on fp32 copies of the inputs, rounded back to the inputs' dtype."""

    def run(*args, **kwargs):
        dtype = next(a.dtype for a in args if isinstance(a, torch.Tensor) and a.is_floating_point())
        promoted = [a.float() if isinstance(a, torch.Tensor) and a.is_floating_point() else a for a in args]
        out = fn(*promoted, **kwargs)
        return tuple(o.to(dtype) for o in out) if isinstance(out, tuple) else out.to(dtype)

    return run


@dataclass(frozen=True)
class RoPEPiece(Piece):
    """A RoPE piece also carries its table builder ``prepare(seq, head_dim, theta, device, dtype)``."""

    prepare: Callable = ops.rope_tables


# ----------------------------------------------------------------------------- selection


@dataclass(frozen=True)
class ModernBertOps:
    """The bound callables the packed forward runs (one per slot, plus the RoPE table builder)."""

    layer_norm: Callable
    add_layer_norm: Callable
    linear: Callable
    dense_linear: Callable
    rope: Callable
    rope_qkv: Callable
    attention: Callable
    attention_bshd: Callable
    geglu: Callable
    rope_tables: Callable


_SLOT_CONTRACTS = {"layer_norm": LN, "add_layer_norm": ADD_LN, "linear": LINEAR, "dense_linear": LINEAR,
                   "rope": ROPE_BHSD, "rope_qkv": ROPE_QKV, "attention": BHSD, "attention_bshd": BSHD,
                   "geglu": GEGLU}


@dataclass(frozen=True)
class ModernBertPieces:
    """The ModernBERT selection: one piece per slot. Immutable; substitute with ``replace``."""

    layer_norm: Piece
    add_layer_norm: Piece
    linear: Piece
    dense_linear: Piece
    rope: RoPEPiece
    rope_qkv: RoPEPiece
    attention: Piece
    attention_bshd: Piece
    geglu: Piece

    def all(self) -> tuple[Piece, ...]:
        return tuple(getattr(self, f.name) for f in fields(self))

    def bind(self) -> ModernBertOps:
        """Check every slot's contract once and return the direct callables."""
        bound = {}
        for slot in fields(self):
            piece = getattr(self, slot.name)
            required = _SLOT_CONTRACTS[slot.name]
            if piece.contract != required:
                raise UnsupportedTargetError(
                    f"piece {piece.name} cannot fill slot {slot.name}: it serves {piece.contract}, the slot needs {required}")
            bound[slot.name] = piece.execute
        return ModernBertOps(**bound, rope_tables=self.rope.prepare)

    def validate(self, model) -> dict[str, PieceValidation]:
        """Validate every slot on ``model``'s own last-layer weights. The attention fixture holds
        two segments, the second longer than the model's local window span (so the band binds on
        both sides of some token), and the BSHD slot takes v as a strided view, as the packed
        forward hands it over."""
        from .config import ModernBertParams

        params = ModernBertParams.from_hf_config(model.config)
        device = next(model.parameters()).device
        gen = torch.Generator(device=device).manual_seed(29)
        bf16 = torch.bfloat16

        def draw(*shape):
            return torch.randn(shape, device=device, dtype=bf16, generator=gen)

        h, d, w = params.num_attention_heads, params.head_dim, params.sliding_half_window
        s = 11 + max(29, 2 * w + 5)
        layer = model.layers[-1]
        norm_w = layer.mlp_norm.weight.detach().to(bf16)
        eps = layer.mlp_norm.eps
        wqkv = layer.attn.Wqkv.weight.detach().to(bf16)
        x = draw(1, s, params.hidden_size)
        reports = {
            "layer_norm": self.layer_norm.validate(x, norm_w, eps),
            "add_layer_norm": self.add_layer_norm.validate(x, draw(*x.shape), norm_w, eps),
            "linear": self.linear.validate(x, wqkv),
            "dense_linear": self.dense_linear.validate(x, wqkv),
            "geglu": self.geglu.validate(draw(1, s, layer.mlp.Wi.weight.shape[0])),
        }
        q, k, v = draw(1, h, s, d), draw(1, h, s, d), draw(1, h, s, d)
        cos, sin = self.rope.prepare(s, d, params.global_rope_theta, device, bf16)
        reports["rope"] = self.rope.validate(q, k, cos, sin)
        reports["attention"] = self.attention.validate(q, k, v, mask=None, window=(-1, -1), scaling=params.scaling,
                                                       backend="sdpa")
        if device.type == "cuda" and ops.hip_available() and d in (64, 128, 256):
            qkv = draw(1, s, 3 * h * d)
            reports["rope_qkv"] = self.rope_qkv.validate(qkv, h, d, cos, sin)
            packed = torch.stack((q, k, v), dim=2).transpose(1, 3).reshape(1, s, 3, h, d)  # [1, S, 3, H, D]
            cu = torch.tensor([0, 11, s], dtype=torch.int32, device=device)
            reports["attention_bshd"] = self.attention_bshd.validate(
                packed[:, :, 0].contiguous(), packed[:, :, 1].contiguous(), packed[:, :, 2], window=(w, w),
                scaling=params.scaling, backend="hip", cu_seqlens=cu, max_seqlen=s - 11)
        else:
            for slot in ("rope_qkv", "attention_bshd"):
                piece = getattr(self, slot)
                reports[slot] = PieceValidation(piece.name, None, piece.rtol, piece.atol,
                                                "no HIP device or head dim outside the HIP kernels")
        return reports


def _rope_reference(q, k, cos, sin):
    qr, kr = ops.rope(q.float(), k.float(), cos.float(), sin.float())
    return qr.to(q.dtype), kr.to(k.dtype)


def _rope_qkv_reference(qkv, h, d, cos, sin):
    q, k = ops.rope_qkv(qkv.float(), h, d, cos.float(), sin.float())
    return q.to(qkv.dtype), k.to(qkv.dtype)


@lru_cache(maxsize=1)
def default_pieces() -> ModernBertPieces:
    return ModernBertPieces(
        layer_norm=Piece("layer-norm", LN, ops.layer_norm, _in_fp32(ops.layer_norm), _accept),
        add_layer_norm=Piece("add-layer-norm", ADD_LN, ops.add_layer_norm, _in_fp32(ops.add_layer_norm), _accept),
        linear=Piece("linear", LINEAR, ops.linear, _in_fp32(ops.linear), _accept),
        dense_linear=Piece("dense-linear", LINEAR, ops.dense_linear, _in_fp32(ops.dense_linear), _accept),
        rope=RoPEPiece("split-half-rope", ROPE_BHSD, ops.rope, _rope_reference, _accept),
        rope_qkv=RoPEPiece("split-half-rope-qkv", ROPE_QKV, ops.rope_qkv, _rope_qkv_reference, _accept),
        attention=attention_piece(),
        attention_bshd=attention_bshd_piece(),
        geglu=Piece("geglu", GEGLU, ops.geglu, _in_fp32(ops.geglu), _accept),
    )


@lru_cache(maxsize=1)
def default_execution() -> ModernBertOps:
    return default_pieces().bind()
