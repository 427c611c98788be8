"""HIP packed varlen attention for MI355X (gfx950), registered as torch ops.

The operator surface of the reference's packed attention kernel module
(packed_encoders/_kernels/triton_packed_attention.py): ``packed_short_attention``,
``packed_short_attention_supported`` and ``select_packed_short_attention_config`` keep their
names, argument meaning and error behaviour (``ValueError`` outside the envelope), and
``varlen_attention`` is the general form (long segments, GQA, causal, windows, fused sigmoid
gate) that replaces the reference's FlashAttention varlen calls.

All compute goes through ``libpe_attn.so`` (include/pe_attn.h) on the current HIP stream via
the ``pe_hip::varlen_attention`` / ``pe_hip::packed_short_attention`` torch ops, and the
producer of their q/k layout, ``rope_qkv`` (``pe_hip::rope_qkv``: RoPE straight from the packed
QKV projection). There is no CPU or eager-PyTorch fallback: if the library is missing, the
loader raises ``ImportError``.
"""

from __future__ import annotations

import contextlib
import contextvars
import ctypes

import torch
from torch import Tensor

from . import _lib

_BF16 = torch.bfloat16


def _row_aligned(t: Tensor) -> bool:
    # 16-byte rows: base pointer and token/head strides (elements) on 8-element boundaries.
    return t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and t.stride(0) % 8 == 0 and t.stride(1) % 8 == 0


def _aligned(t: Tensor) -> Tensor:
    return t if _row_aligned(t) else t.contiguous()


def _args(q: Tensor, k: Tensor, v: Tensor, o: Tensor, cu: Tensor, max_seqlen: int, scale: float,
          window_left: int, window_right: int, causal: bool, gate: Tensor | None,
          short_max: int, strip: int = 0, cu_k: Tensor | None = None,
          max_seqlen_k: int = 0, band_kernel: int = 0, min_seqlen: int = 0,
          rope: tuple[Tensor, Tensor] | None = None) -> _lib.AttnArgs:
    a = _lib.AttnArgs()
    a.struct_size = ctypes.sizeof(_lib.AttnArgs)
    a.dtype = _lib.DTYPE_BF16
    a.q, a.k, a.v, a.o = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr()
    a.gate = gate.data_ptr() if gate is not None else None
    a.cu_seqlens = cu.data_ptr()
    a.q_stride_token, a.q_stride_head = q.stride(0), q.stride(1)
    a.k_stride_token, a.k_stride_head = k.stride(0), k.stride(1)
    a.v_stride_token, a.v_stride_head = v.stride(0), v.stride(1)
    a.o_stride_token, a.o_stride_head = o.stride(0), o.stride(1)
    if gate is not None:
        a.gate_stride_token, a.gate_stride_head = gate.stride(0), gate.stride(1)
    a.n_seq = cu.numel() - 1
    a.total_tokens = q.shape[0]
    a.max_seqlen = int(max_seqlen)
    a.n_heads_q, a.n_heads_kv, a.head_dim = q.shape[1], k.shape[1], q.shape[2]
    a.softmax_scale = float(scale)
    a.window_left, a.window_right = int(window_left), int(window_right)
    a.causal = 1 if causal else 0
    a.short_max = int(short_max)
    a.strip = int(strip)
    a.band_kernel = int(band_kernel)
    a.min_seqlen = int(min_seqlen)
    if cu_k is not None:
        a.cu_seqlens_k = cu_k.data_ptr()
        a.total_tokens_k = k.shape[0]
        a.max_seqlen_k = int(max_seqlen_k)
    if rope is not None:
        cos, sin = rope
        a.rope_cos, a.rope_sin = cos.data_ptr(), sin.data_ptr()
        a.rope_table_stride, a.rope_table_rows = cos.stride(0), cos.shape[0]
    return a


def _check_tensors(q: Tensor, k: Tensor, v: Tensor, cu: Tensor, gate: Tensor | None,
                   cu_k: Tensor | None = None) -> None:
    if q.ndim != 3 or k.ndim != 3 or v.ndim != 3:
        raise ValueError("varlen attention expects [tokens, heads, head_dim] q/k/v")
    same_rows = cu_k is not None or q.shape[0] == k.shape[0]
    if k.shape != v.shape or not same_rows or q.shape[2] != k.shape[2]:
        raise ValueError(f"q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)} do not match")
    if cu_k is not None:
        if cu_k.dtype != torch.int32 or cu_k.ndim != 1 or cu_k.numel() != cu.numel():
            raise ValueError("cu_seqlens_k must be a 1-D int32 tensor with cu_seqlens' length")
        if cu_k.device != q.device:
            raise ValueError("cu_seqlens_k must be on q's device")
    if q.shape[1] % k.shape[1]:
        raise ValueError("query heads must be a multiple of kv heads")
    if q.dtype != _BF16 or k.dtype != _BF16 or v.dtype != _BF16:
        raise ValueError("varlen attention computes in bf16")
    if cu.dtype != torch.int32 or cu.ndim != 1 or cu.numel() < 1:
        raise ValueError("cu_seqlens must be a 1-D int32 tensor [n_seq + 1]")
    devices = {q.device, k.device, v.device, cu.device}
    if gate is not None:
        if gate.shape != q.shape or gate.dtype != _BF16:
            raise ValueError("gate must be bf16 with q's shape")
        devices.add(gate.device)
    if len(devices) != 1 or q.device.type != "cuda":
        raise ValueError("q, k, v, cu_seqlens (and gate) must be on one HIP device")


# Tile plans shared within a scope (one packed forward): key -> (cu_seqlens, workspace, bytes).
_PLANS: contextvars.ContextVar[dict | None] = contextvars.ContextVar("pe_hip_shared_plans", default=None)
_FLOOR: contextvars.ContextVar[int] = contextvars.ContextVar("pe_hip_min_seqlen", default=0)


@contextlib.contextmanager
def shared_plans(min_seqlen: int = 0):
    """Within this scope, varlen attention calls that share a ``cu_seqlens`` tensor, head
    geometry, window, causality and routing boundary build the tiled kernel's plan once and
    reuse it: a packed forward's 22 layers then run 2 plan kernels (global and local) instead
    of 22. The scope keeps each plan's workspace (and its ``cu_seqlens``) alive until it exits;
    the caller must not change ``cu_seqlens`` values inside the scope.

    ``min_seqlen`` is the host's lower bound on the shared batch's segment lengths (a collator
    knows them; 0 when unknown). Calls in the scope that pass no ``min_seqlen`` of their own use
    it, so a batch with no short segment skips the short kernel's launch in every layer. A
    wrong bound changes which kernel serves a segment, never the result's correctness."""
    token = _PLANS.set({})
    floor = _FLOOR.set(max(0, int(min_seqlen)))
    try:
        yield
    finally:
        _FLOOR.reset(floor)
        _PLANS.reset(token)


def _plan_key(args: _lib.AttnArgs, cu: Tensor, cu_k: Tensor | None = None) -> tuple:
    kv = (None,) if cu_k is None else (id(cu_k), cu_k.data_ptr(), args.total_tokens_k, args.max_seqlen_k)
    return (id(cu), cu.data_ptr(), cu.numel(), args.total_tokens, args.max_seqlen, args.n_heads_q,
            args.n_heads_kv, args.head_dim, args.window_left, args.window_right, args.causal, args.short_max,
            args.strip, args.band_kernel, args.min_seqlen, *kv)


def _table_rows(t: Tensor) -> Tensor:
    """A RoPE table as [rows, D] with 16-byte rows (a copy only when its layout needs one)."""
    return t if (t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and t.stride(0) % 8 == 0) else t.contiguous()


def _varlen_impl(q: Tensor, k: Tensor, v: Tensor, cu_seqlens: Tensor, max_seqlen: int,
                 softmax_scale: float, window_left: int, window_right: int, causal: bool,
                 gate: Tensor | None, short_max: int, cu_seqlens_k: Tensor | None = None,
                 max_seqlen_k: int = 0, band_kernel: int = 0, min_seqlen: int = 0,
                 rope_cos: Tensor | None = None, rope_sin: Tensor | None = None) -> Tensor:
    _check_tensors(q, k, v, cu_seqlens, gate, cu_seqlens_k)
    q, k, v = _aligned(q), _aligned(k), _aligned(v)
    gate = _aligned(gate) if gate is not None else None
    rope = None
    if (rope_cos is None) != (rope_sin is None):
        raise ValueError("RoPE needs both cos and sin tables")
    if rope_cos is not None:
        if rope_cos.dtype != _BF16 or rope_sin.dtype != _BF16 or rope_cos.device != q.device:
            raise ValueError("RoPE tables must be bf16 on q's device")
        rope_cos, rope_sin = _rope_tables(rope_cos, rope_sin, q.shape[2])
        rope = (_table_rows(rope_cos), _table_rows(rope_sin))
        if rope[0].stride(0) != rope[1].stride(0):
            rope = (rope[0].contiguous(), rope[1].contiguous())
    out = torch.empty(q.shape, dtype=_BF16, device=q.device)
    if q.shape[0] == 0 or cu_seqlens.numel() < 2:
        return out
    lib = _lib.library()
    args = _args(q, k, v, out, cu_seqlens, max_seqlen, softmax_scale, window_left, window_right,
                 causal, gate, short_max, cu_k=cu_seqlens_k, max_seqlen_k=max_seqlen_k, band_kernel=band_kernel,
                 min_seqlen=min_seqlen, rope=rope)
    stream = torch.cuda.current_stream(q.device).cuda_stream
    plans = _PLANS.get()
    if plans is None:
        size = ctypes.c_size_t(0)
        _lib.check(lib.pe_attn_workspace_size(ctypes.byref(args), ctypes.byref(size)), "pe_attn_workspace_size")
        workspace = torch.empty(size.value, dtype=torch.uint8, device=q.device) if size.value else None
        status = lib.pe_varlen_attn_fwd(ctypes.byref(args), workspace.data_ptr() if workspace is not None else None,
                                        size.value, stream)
        _lib.check(status, "pe_varlen_attn_fwd")
        return out
    key = _plan_key(args, cu_seqlens, cu_seqlens_k)
    entry = plans.get(key)
    if entry is None:
        size = ctypes.c_size_t(0)
        _lib.check(lib.pe_attn_workspace_size(ctypes.byref(args), ctypes.byref(size)), "pe_attn_workspace_size")
        workspace = torch.empty(size.value, dtype=torch.uint8, device=q.device) if size.value else None
        ptr = workspace.data_ptr() if workspace is not None else None
        _lib.check(lib.pe_attn_plan(ctypes.byref(args), ptr, size.value, stream), "pe_attn_plan")
        entry = plans[key] = ((cu_seqlens, cu_seqlens_k), workspace, size.value)
    _, workspace, nbytes = entry
    ptr = workspace.data_ptr() if workspace is not None else None
    _lib.check(lib.pe_attn_short_fwd(ctypes.byref(args), stream), "pe_attn_short_fwd")
    _lib.check(lib.pe_attn_tiled_fwd(ctypes.byref(args), ptr, nbytes, stream), "pe_attn_tiled_fwd")
    return out


def _short_impl(q: Tensor, k: Tensor, v: Tensor, cu_seqlens: Tensor, max_seqlen: int,
                softmax_scale: float, window_left: int, window_right: int) -> Tensor:
    _check_tensors(q, k, v, cu_seqlens, None)
    q, k, v = _aligned(q), _aligned(k), _aligned(v)
    out = torch.empty(q.shape, dtype=_BF16, device=q.device)
    if q.shape[0] == 0 or cu_seqlens.numel() < 2:
        return out
    lib = _lib.library()
    args = _args(q, k, v, out, cu_seqlens, max_seqlen, softmax_scale, window_left, window_right,
                 False, None, 0)
    stream = torch.cuda.current_stream(q.device).cuda_stream
    _lib.check(lib.pe_packed_short_attn_fwd(ctypes.byref(args), stream), "pe_packed_short_attn_fwd")
    return out


def _varlen_op_impl(q: Tensor, k: Tensor, v: Tensor, cu_seqlens: Tensor, max_seqlen: int, softmax_scale: float,
                    window_left: int, window_right: int, causal: bool, gate: Tensor | None, short_max: int,
                    band_kernel: int = 0, min_seqlen: int = 0, rope_cos: Tensor | None = None,
                    rope_sin: Tensor | None = None) -> Tensor:
    return _varlen_impl(q, k, v, cu_seqlens, max_seqlen, softmax_scale, window_left, window_right, causal, gate,
                        short_max, band_kernel=band_kernel, min_seqlen=min_seqlen, rope_cos=rope_cos,
                        rope_sin=rope_sin)


def _varlen_kv_impl(q: Tensor, k: Tensor, v: Tensor, cu_seqlens_q: Tensor, cu_seqlens_k: Tensor,
                    max_seqlen_q: int, max_seqlen_k: int, softmax_scale: float, window_left: int,
                    window_right: int, causal: bool, gate: Tensor | None, short_max: int,
                    band_kernel: int = 0, min_seqlen: int = 0) -> Tensor:
    return _varlen_impl(q, k, v, cu_seqlens_q, max_seqlen_q, softmax_scale, window_left, window_right, causal,
                        gate, short_max, cu_seqlens_k, max_seqlen_k, band_kernel, min_seqlen)


def _meta(q: Tensor, *args, **kwargs) -> Tensor:
    return torch.empty(q.shape, dtype=_BF16, device=q.device)


def _rope_tables(cos: Tensor, sin: Tensor, d: int) -> tuple[Tensor, Tensor]:
    if cos.ndim == 3:  # [1, rows, D] or per-row [B, S, D]
        cos, sin = cos.reshape(-1, d), sin.reshape(-1, d)
    if cos.ndim != 2 or cos.shape[-1] != d or sin.shape != cos.shape:
        raise ValueError(f"cos/sin must be [rows, {d}] (or [1, rows, {d}]), got {tuple(cos.shape)}")
    return cos, sin


def _rope_impl(qkv: Tensor, cos: Tensor, sin: Tensor, h: int, d: int) -> list[Tensor]:
    if qkv.dtype != _BF16 or cos.dtype != _BF16 or sin.dtype != _BF16:
        raise ValueError("rope_qkv computes in bf16")
    if qkv.shape[-1] != 3 * h * d:
        raise ValueError(f"qkv last dim {qkv.shape[-1]} != 3*{h}*{d}")
    cos, sin = _rope_tables(cos, sin, d)
    flat = qkv.reshape(-1, 3 * h * d)
    if flat.stride(-1) != 1 or flat.data_ptr() % 16 or flat.stride(0) % 8:
        flat = flat.contiguous()
    cos = cos if (cos.stride(-1) == 1 and cos.data_ptr() % 16 == 0 and cos.stride(0) % 8 == 0) else cos.contiguous()
    sin = sin if (sin.stride(-1) == 1 and sin.data_ptr() % 16 == 0 and sin.stride(0) % 8 == 0) else sin.contiguous()
    n = flat.shape[0]
    q = torch.empty(n, h, d, dtype=_BF16, device=qkv.device)
    k = torch.empty(n, h, d, dtype=_BF16, device=qkv.device)
    if n:
        a = _lib.RopeArgs()
        a.struct_size = ctypes.sizeof(_lib.RopeArgs)
        a.dtype = _lib.DTYPE_BF16
        a.qkv, a.cos, a.sin, a.q_out, a.k_out = flat.data_ptr(), cos.data_ptr(), sin.data_ptr(), q.data_ptr(), k.data_ptr()
        a.qkv_stride_row, a.table_stride_row = flat.stride(0), cos.stride(0)
        a.table_rows, a.n_rows, a.n_heads, a.head_dim = cos.shape[0], n, h, d
        stream = torch.cuda.current_stream(qkv.device).cuda_stream
        _lib.check(_lib.library().pe_rope_qkv_fwd(ctypes.byref(a), stream), "pe_rope_qkv_fwd")
    shape = tuple(qkv.shape[:-1]) + (h, d)
    return [q.view(shape), k.view(shape)]


def _rope_meta(qkv: Tensor, cos: Tensor, sin: Tensor, h: int, d: int) -> list[Tensor]:
    shape = tuple(qkv.shape[:-1]) + (h, d)
    return [torch.empty(shape, dtype=_BF16, device=qkv.device), torch.empty(shape, dtype=_BF16, device=qkv.device)]


def _register() -> None:
    """Define ``pe_hip::varlen_attention`` and ``pe_hip::packed_short_attention`` once per process."""
    lib = torch.library.Library("pe_hip", "FRAGMENT")
    try:
        lib.define("varlen_attention(Tensor q, Tensor k, Tensor v, Tensor cu_seqlens, int max_seqlen, "
                   "float softmax_scale, int window_left, int window_right, bool causal, Tensor? gate, "
                   "int short_max, int band_kernel=0, int min_seqlen=0, Tensor? rope_cos=None, "
                   "Tensor? rope_sin=None) -> Tensor")
        lib.define("packed_short_attention(Tensor q, Tensor k, Tensor v, Tensor cu_seqlens, int max_seqlen, "
                   "float softmax_scale, int window_left, int window_right) -> Tensor")
        lib.define("rope_qkv(Tensor qkv, Tensor cos, Tensor sin, int h, int d) -> Tensor[]")
        lib.define("varlen_attention_kv(Tensor q, Tensor k, Tensor v, Tensor cu_seqlens_q, Tensor cu_seqlens_k, "
                   "int max_seqlen_q, int max_seqlen_k, float softmax_scale, int window_left, int window_right, "
                   "bool causal, Tensor? gate, int short_max, int band_kernel=0, int min_seqlen=0) -> Tensor")
    except RuntimeError:
        return  # already defined by an earlier import in this process
    lib.impl("varlen_attention", _varlen_op_impl, "CUDA")
    lib.impl("varlen_attention", _meta, "Meta")
    lib.impl("packed_short_attention", _short_impl, "CUDA")
    lib.impl("packed_short_attention", _meta, "Meta")
    lib.impl("varlen_attention_kv", _varlen_kv_impl, "CUDA")
    lib.impl("varlen_attention_kv", _meta, "Meta")
    lib.impl("rope_qkv", _rope_impl, "CUDA")
    lib.impl("rope_qkv", _rope_meta, "Meta")
    globals()["_TORCH_LIBRARY"] = lib


_register()


def varlen_attention(q: Tensor, k: Tensor, v: Tensor, cu_seqlens: Tensor, max_seqlen: int, *,
                     softmax_scale: float | None = None, window: tuple[int, int] = (-1, -1),
                     causal: bool = False, gate: Tensor | None = None,
                     short_max: int | None = None, cu_seqlens_k: Tensor | None = None,
                     max_seqlen_k: int | None = None, band_kernel: int = 0,
                     min_seqlen: int | None = None, rope: tuple[Tensor, Tensor] | None = None) -> Tensor:
    """Packed varlen attention: q ``[T, Hq, D]``, k/v ``[T, Hkv, D]`` bf16, int32 ``cu_seqlens``.

    ``window=(left, right)`` bounds ``i - j <= left`` and ``j - i <= right`` (-1 unbounded,
    the FlashAttention convention of packed_encoders/ops.py:404-461); ``causal`` forbids
    ``j > i``; ``gate`` multiplies the output by ``bf16(sigmoid(gate))``. ``short_max`` routes
    segments of at most that length to the LDS-resident short kernel (None: the gfx950 policy
    default). Returns a new contiguous ``[T, Hq, D]``; rows beyond ``cu_seqlens[-1]`` are not
    written. Forward only.

    ``cu_seqlens_k`` / ``max_seqlen_k`` give k/v ``[Tk, Hkv, D]`` segments of their own
    (FlashAttention's varlen form): query segment s is the tail of key segment s, its row r at
    key position ``r + Lk - Lq``, which ``causal`` and ``window`` are measured from (the
    reference's prefixed form, packed_encoders/runtime/attention.py:15-19,236-245). A row that
    reaches no key comes out as zero.

    ``band_kernel`` picks the kernel of a +-64-shaped band call's long segments (see
    ``pe_attn_args.band_kernel``): 0 the library's choice by call size, 1 the streaming band
    kernel, 2 the tiled kernel; results agree within bf16 rounding, not bit for bit.

    ``rope=(cos, sin)`` fuses the RoPE producer into the call: q and k are then the
    projection's unrotated rows (e.g. strided views into ``qkv``), and each packed row ``r``
    is rotated with row ``r % rows`` of the bf16 ``[rows, D]`` (or ``[1, rows, D]``) tables,
    bit for bit as ``rope_qkv`` would (packed_encoders/ops.py:485-499,
    _kernels/rope.py:302-349). The short kernel applies it, so every segment must be short
    (``max_seqlen`` within the routing boundary; head_dim 64 or 128; no ``cu_seqlens_k``):
    ``ValueError`` otherwise.

    ``min_seqlen`` is an optional host lower bound on the query segment lengths (a collator
    that packs host-known lengths has it beside ``max_seqlen``; None takes the enclosing
    ``shared_plans`` scope's bound, 0 outside one). When it exceeds the routing
    boundary no segment can be short, and the call skips the short kernel's launch: every
    segment goes to the tiled kernels, which serve any length, so a wrong bound costs time,
    never results.
    """
    if band_kernel not in (0, 1, 2):
        raise ValueError("band_kernel must be 0 (library choice), 1 (streaming band) or 2 (tiled)")
    min_seqlen = min(_FLOOR.get(), int(max_seqlen)) if min_seqlen is None else int(min_seqlen)
    if not 0 <= min_seqlen <= int(max_seqlen):
        raise ValueError(f"min_seqlen must lie in [0, max_seqlen], got {min_seqlen} (max_seqlen {max_seqlen})")
    if torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v)):
        raise ValueError("the HIP packed attention is forward-only; call it under torch.no_grad()")
    scale = q.shape[-1] ** -0.5 if softmax_scale is None else float(softmax_scale)
    if short_max is None:
        short_max = -1
    if cu_seqlens_k is not None:
        if rope is not None:
            raise ValueError("the fused RoPE prologue takes shared key segments (no cu_seqlens_k)")
        if max_seqlen_k is None:
            raise ValueError("cu_seqlens_k needs max_seqlen_k")
        return torch.ops.pe_hip.varlen_attention_kv(q, k, v, cu_seqlens, cu_seqlens_k, int(max_seqlen),
                                                    int(max_seqlen_k), scale, int(window[0]), int(window[1]),
                                                    bool(causal), gate, int(short_max), int(band_kernel),
                                                    min_seqlen)
    return torch.ops.pe_hip.varlen_attention(q, k, v, cu_seqlens, int(max_seqlen), scale,
                                             int(window[0]), int(window[1]), bool(causal), gate,
                                             int(short_max), int(band_kernel), min_seqlen,
                                             *(rope if rope is not None else (None, None)))


def packed_short_attention_supported(q: Tensor, k: Tensor, v: Tensor, cu_seqlens: Tensor,
                                     max_seqlen: int, *, half_window: int | None) -> bool:
    """Pure capability predicate (host metadata only; the reference's
    triton_packed_attention.py:146-172). Wider than the reference's envelope: any head count,
    head_dim 64 or 128 and any non-negative half window; still bf16, Smax <= 128, no grad."""
    return (
        q.is_cuda and k.is_cuda and v.is_cuda and cu_seqlens.is_cuda
        and q.ndim == k.ndim == v.ndim == 3
        and q.shape == k.shape == v.shape
        and q.shape[2] in (64, 128)
        and q.dtype == k.dtype == v.dtype == _BF16
        and q.stride(-1) == k.stride(-1) == v.stride(-1) == 1
        and cu_seqlens.dtype == torch.int32
        and cu_seqlens.ndim == 1
        and cu_seqlens.numel() >= 2
        and 0 < int(max_seqlen) <= 128
        and (half_window is None or int(half_window) >= 0)
        and not torch.is_grad_enabled()
    )


def packed_short_attention(q: Tensor, k: Tensor, v: Tensor, cu_seqlens: Tensor, max_seqlen: int, *,
                           half_window: int | None, softmax_scale: float) -> Tensor:
    """Packed non-causal self attention over short segments; returns contiguous ``[M, H, D]``.

    Same contract as the reference's ``packed_short_attention``
    (triton_packed_attention.py:175-196): ``half_window`` None is global attention within each
    segment, an int ``w`` the symmetric band ``|i - j| <= w``; ``ValueError`` outside the
    envelope."""
    if not packed_short_attention_supported(q, k, v, cu_seqlens, max_seqlen, half_window=half_window):
        raise ValueError(
            "packed short attention requires no-grad HIP bf16 [M,H,64|128] Q/K/V, int32 "
            "cu_seqlens, Smax<=128, and global or non-negative half-window attention"
        )
    w = -1 if half_window is None else int(half_window)
    return torch.ops.pe_hip.packed_short_attention(q, k, v, cu_seqlens, int(max_seqlen),
                                                   float(softmax_scale), w, w)


def select_packed_short_attention_config(max_seqlen: int, head_dim: int = 64) -> dict[str, int]:
    """The short kernel's static launch choice for ``max_seqlen`` in JSON-friendly form.

    Same keys as the reference's table (triton_packed_attention.py:22-42): ``block_m`` query
    rows per wave, ``block_n`` keys staged per pass (the whole segment: the kernel holds up to
    ``key_capacity`` keys in LDS at once), ``num_warps`` waves per workgroup (64 lanes each) and
    ``num_stages`` staging passes (one: every load is issued before a single wait). The extra
    keys describe this kernel's tiles. Like the reference, any ``max_seqlen`` gets an answer:
    lengths past 128 report the 128-key shape, the largest the short kernel has (such batches
    run the tiled kernel for their longer segments)."""
    smax = min(max(int(max_seqlen), 1), 128)
    out = (ctypes.c_int32 * 4)()
    _lib.check(_lib.library().pe_attn_short_config(smax, int(head_dim), out), "pe_attn_short_config")
    return {"block_m": out[0], "block_n": out[1], "num_warps": out[3], "num_stages": 1,
            "key_capacity": out[1], "heads_per_workgroup": out[2], "num_waves": out[3]}


def useful_flops(lengths, n_heads_q: int, head_dim: int, *, window: tuple[int, int] = (-1, -1),
                 causal: bool = False) -> int:
    """``4 * D * Hq * sum(allowed (query, key) pairs)`` over live tokens only."""
    return 4 * head_dim * n_heads_q * sum(allowed_pairs(int(n), window, causal) for n in lengths)


def allowed_pairs(n: int, window: tuple[int, int] = (-1, -1), causal: bool = False) -> int:
    """Number of (i, j) in [0, n)^2 with ``i - j <= left`` and ``j - i <= right`` (causal: right 0)."""
    left, right = window
    right = 0 if causal else right
    left = n if left < 0 else min(left, n)
    right = n if right < 0 else min(right, n)
    # pairs with j <= i and i - j <= left, plus pairs with j > i and j - i <= right
    below = sum(n - d for d in range(0, left + 1) if d < n)
    above = sum(n - d for d in range(1, right + 1) if d < n)
    return below + above


__all__ = [
    "shared_plans",
    "packed_short_attention",
    "packed_short_attention_supported",
    "select_packed_short_attention_config",
    "varlen_attention",
    "useful_flops",
    "allowed_pairs",
]


def rope_qkv(qkv: Tensor, h: int, d: int, cos: Tensor, sin: Tensor) -> tuple[Tensor, Tensor]:
    """Split-half RoPE'd q, k read straight from the packed projection ``qkv [..., 3*h*d]``
    (bf16, on the GPU), returned contiguous ``[..., h, d]`` — the layout ``varlen_attention``
    reads, with v left as a strided view of ``qkv``. ``cos``/``sin`` are ``[rows, d]`` (or
    ``[B or 1, S, d]``, flattened to rows): row ``r`` of ``qkv`` (leading dims flattened) uses
    table row ``r % rows``, so per-token gathered tables (rows = tokens) and dense ``[S, d]``
    tables of a ``[B, S]`` batch both work. Same contract as the reference's ``apply_rope_bshd``
    (packed_encoders/_kernels/rope.py:302-349); ``ValueError`` for bad shapes or dtypes."""
    if not qkv.is_cuda:
        raise ValueError("rope_qkv runs on the HIP device")
    q, k = torch.ops.pe_hip.rope_qkv(qkv, cos, sin, int(h), int(d))
    return q, k

