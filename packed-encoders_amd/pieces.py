"""Operation pieces: a callable, its contract and an independent fp32 oracle
(packed_encoders/pieces/base.py:17-69, pieces/attention.py:11-73,
arch/modernbert_pieces.py:18-128).

An engine binds each piece's ``execute`` once; ``Piece.validate`` checks a fixture, runs the
oracle and the piece, and compares them at ``rtol = atol = 0.02``, raising ``ValidationError``.
The attention pieces' oracle is a per-segment fp32 dense attention of its own (segment bounds
read on the host: validation only), so a substituted kernel is checked against something it
does not share code with. ``ModernBertPieces`` is the immutable selection the packed forward
runs; replacing a slot (``dataclasses.replace(pieces, attention_bshd=...)``) substitutes a
piece, after a contract check in ``bind()``.
"""

from __future__ import annotations

from dataclasses import dataclass, fields
from functools import lru_cache
from typing import Callable

import torch
import torch.nn.functional as F

from . import ops
from .errors import UnsupportedTargetError, ValidationError


@dataclass(frozen=True)
class Contract:
    operation: str
    layout: str
    semantics: str
    autograd: bool = True
    capture: bool = True


@dataclass(frozen=True)
class PieceValidation:
    name: str
    max_abs_error: float | None
    rtol: float
    atol: float
    skipped_reason: str | None = None


@dataclass(frozen=True)
class Piece:
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
            expected = self.reference(*args, **kwargs)
            actual = self.execute(*args, **kwargs)
        expected = expected if isinstance(expected, tuple) else (expected,)
        actual = actual if isinstance(actual, tuple) else (actual,)
        if len(actual) != len(expected):
            raise ValidationError(f"piece {self.name}: output arity differs from its reference")
        worst = 0.0
        for got, ref in zip(actual, expected):
            try:
                torch.testing.assert_close(got, ref, rtol=self.rtol, atol=self.atol)
            except AssertionError as exc:
                raise ValidationError(f"piece {self.name} failed reference validation: {exc}") from exc
            worst = max(worst, float((got.float() - ref.float()).abs().max()))
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


# ----------------------------------------------------------------------------- oracles


def _dense_fp32(q, k, v, mask, window, scaling):
    """fp32 SDPA over ``[B, H, S, D]`` with an optional additive mask and ``(left, right)`` band."""
    if window != (-1, -1):
        pos = torch.arange(q.shape[-2], device=q.device)
        delta = pos[:, None] - pos[None, :]
        outside = torch.zeros(delta.shape, device=q.device)
        if window[0] >= 0:
            outside = outside.masked_fill(delta > window[0], float("-inf"))
        if window[1] >= 0:
            outside = outside.masked_fill(delta < -window[1], float("-inf"))
        mask = outside if mask is None else mask.float() + outside
    return F.scaled_dot_product_attention(q.float(), k.float(), v.float(),
                                         attn_mask=None if mask is None else mask.float(), scale=scaling)


def attention_reference(q, k, v, *, mask, window, scaling, backend, cu_seqlens=None, max_seqlen=None):
    if backend != "hip":
        out = _dense_fp32(q, k, v, mask, (-1, -1), scaling)
    elif cu_seqlens is None:
        out = _dense_fp32(q, k, v, None, window, scaling)
    else:
        bounds = cu_seqlens.tolist()  # host read: validation only
        out = torch.zeros(q.shape, dtype=torch.float32, device=q.device)
        for a, b in zip(bounds, bounds[1:]):
            if b > a:
                out[:, :, a:b] = _dense_fp32(q[:, :, a:b], k[:, :, a:b], v[:, :, a:b], None, window, scaling)
    return out.to(q.dtype).transpose(1, 2).reshape(q.shape[0], q.shape[2], -1)


def attention_bshd_reference(q, k, v, *, window, scaling, backend="hip", cu_seqlens=None, max_seqlen=None):
    return attention_reference(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), mask=None, window=window,
                               scaling=scaling, backend=backend, cu_seqlens=cu_seqlens, max_seqlen=max_seqlen)


def check_attention(q, k, v, *, mask, window, scaling, backend, cu_seqlens=None, max_seqlen=None):
    if q.ndim != 4 or q.shape != k.shape or q.shape != v.shape:
        raise UnsupportedTargetError("attention piece requires equal Q/K/V shapes")
    if backend not in ops.BACKENDS or scaling <= 0:
        raise UnsupportedTargetError("unsupported attention backend or scale")
    if cu_seqlens is not None and (q.shape[0] != 1 or cu_seqlens.dtype != torch.int32 or max_seqlen is None):
        raise UnsupportedTargetError("packed attention requires B=1, int32 boundaries and max_seqlen")


def check_attention_bshd(q, k, v, *, window, scaling, backend="hip", cu_seqlens=None, max_seqlen=None):
    check_attention(q, k, v, mask=None, window=window, scaling=scaling, backend=backend, cu_seqlens=cu_seqlens,
                    max_seqlen=max_seqlen)
    if backend != "hip":
        raise UnsupportedTargetError("BSHD attention requires the HIP backend")


def _no_check(*args, **kwargs):
    return None


def _fp32(fn):
    def run(*args, **kwargs):
        cast = [a.float() if isinstance(a, torch.Tensor) and a.is_floating_point() else a for a in args]
        out = fn(*cast, **kwargs)
        dtype = next(a.dtype for a in args if isinstance(a, torch.Tensor) and a.is_floating_point())
        return tuple(o.to(dtype) for o in out) if isinstance(out, tuple) else out.to(dtype)
    return run


def attention_piece() -> Piece:
    return Piece("attention-bhsd", BHSD, ops.attention, attention_reference, check_attention)


def attention_bshd_piece() -> Piece:
    return Piece("attention-bshd", BSHD, ops.attention_bshd, attention_bshd_reference, check_attention_bshd)


@dataclass(frozen=True)
class RoPEPiece(Piece):
    prepare: Callable = ops.rope_tables


# ----------------------------------------------------------------------------- selection


@dataclass(frozen=True)
class ModernBertOps:
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


_REQUIRED = (LN, ADD_LN, LINEAR, LINEAR, ROPE_BHSD, ROPE_QKV, BHSD, BSHD, GEGLU)


@dataclass(frozen=True)
class ModernBertPieces:
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
        """Check each slot's contract once and return the direct callables."""
        for slot, piece, contract in zip(fields(self), self.all(), _REQUIRED):
            if piece.contract != contract:
                raise UnsupportedTargetError(f"incompatible {slot.name} piece {piece.name}: expected {contract}")
        return ModernBertOps(*(p.execute for p in self.all()), rope_tables=self.rope.prepare)

    def validate(self, model) -> dict[str, PieceValidation]:
        """Probe every slot on real weights of ``model``'s last layer (attention_bshd with the
        reference's probe: two segments ``[0, 7, 17]`` and the model's local window)."""
        from .config import ModernBertParams

        params = ModernBertParams.from_hf_config(model.config)
        device = next(model.parameters()).device
        gen = torch.Generator(device=device).manual_seed(17)

        def rand(*shape):
            return torch.randn(shape, device=device, dtype=torch.bfloat16, generator=gen)

        layer = model.layers[-1]
        x = rand(1, 17, params.hidden_size)
        w = layer.mlp_norm.weight.detach().to(torch.bfloat16)
        wi = layer.attn.Wqkv.weight.detach().to(torch.bfloat16)
        reports = {}
        reports["layer_norm"] = self.layer_norm.validate(x, w, layer.mlp_norm.eps)
        reports["add_layer_norm"] = self.add_layer_norm.validate(x, rand(*x.shape), w, layer.mlp_norm.eps)
        reports["linear"] = self.linear.validate(x, wi)
        reports["dense_linear"] = self.dense_linear.validate(x, wi)
        reports["geglu"] = self.geglu.validate(rand(1, 17, layer.mlp.Wi.weight.shape[0]))
        h, d = params.num_attention_heads, params.head_dim
        q, k, v = rand(1, h, 17, d), rand(1, h, 17, d), rand(1, h, 17, d)
        cos, sin = self.rope.prepare(17, d, params.global_rope_theta, device, q.dtype)
        reports["rope"] = self.rope.validate(q, k, cos, sin)
        reports["attention"] = self.attention.validate(q, k, v, mask=None, window=(-1, -1), scaling=params.scaling,
                                                       backend="sdpa")
        if device.type == "cuda" and ops.hip_available() and d in (64, 128, 256):
            qkv = rand(1, 17, 3 * h * d)
            reports["rope_qkv"] = self.rope_qkv.validate(qkv, h, d, cos, sin)
            cu = torch.tensor([0, 7, 17], dtype=torch.int32, device=device)
            reports["attention_bshd"] = self.attention_bshd.validate(
                q.transpose(1, 2).contiguous(), k.transpose(1, 2).contiguous(), v.transpose(1, 2),
                window=(params.sliding_half_window,) * 2, scaling=params.scaling, backend="hip", cu_seqlens=cu,
                max_seqlen=10)
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
        layer_norm=Piece("layer-norm", LN, ops.layer_norm, _fp32(ops.layer_norm), _no_check),
        add_layer_norm=Piece("add-layer-norm", ADD_LN, ops.add_layer_norm, _fp32(ops.add_layer_norm), _no_check),
        linear=Piece("linear", LINEAR, ops.linear, _fp32(ops.linear), _no_check),
        dense_linear=Piece("dense-linear", LINEAR, ops.dense_linear, _fp32(ops.dense_linear), _no_check),
        rope=RoPEPiece("split-half-rope", ROPE_BHSD, ops.rope, _rope_reference, _no_check),
        rope_qkv=RoPEPiece("split-half-rope-qkv", ROPE_QKV, ops.rope_qkv, _rope_qkv_reference, _no_check),
        attention=attention_piece(),
        attention_bshd=attention_bshd_piece(),
        geglu=Piece("geglu", GEGLU, ops.geglu, _fp32(ops.geglu), _no_check),
    )


@lru_cache(maxsize=1)
def default_execution() -> ModernBertOps:
    return default_pieces().bind()
