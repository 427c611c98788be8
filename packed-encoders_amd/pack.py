"""``pack()``: install the packed forward onto a live ModernBERT, in place
(packed_encoders/dispatch.py:13-114, pack.py:25-344, arch/modernbert.py:30-180).

``pack(model)`` finds the backbone (a Hugging Face ``ModernBertModel``, or a task /
SentenceTransformer / PyLate model wrapping one), prepares the packed state and replaces the
encoder's bound ``forward``; weights, ``state_dict`` and ``save_pretrained`` stay Hugging Face's.
``unpack(model)`` restores the original forward.

``attention_backend``:
- ``None`` (default): ``"auto"`` when the HIP library loads, else ``"sdpa"`` with a warning;
- ``"hip"``: this build's MI355X kernels; raises ``PackedEncodersError`` if the library is missing;
- ``"auto"``: ``"hip"`` for every call inside its invariants (no autograd, bf16, HIP device);
- ``"sdpa"``: the dependency-free dense path;
- ``"flash"`` / ``"triton"``: the reference's NVIDIA kernels, not part of this build; they raise
  ``PackedEncodersError`` as the reference does when their dependency is missing.
"""

from __future__ import annotations

import warnings
from dataclasses import dataclass, field
from typing import Any

import torch
from torch import Tensor, nn

from . import forward, ops
from .batch import PackedBatch
from .config import ModernBertParams
from .errors import PackedEncodersError, UnsupportedTargetError, ValidationError
from .graph import GraphConfig, build_packed_runner
from .locate import find_encoder
from .pieces import ModernBertPieces, default_pieces
from .state import ATTR, PatchState, find_state, get_state

INSTALL_ATTR = "_packed_encoders_installation"
_NUMERIC_LENGTHS = (128, 512, 2048)
_NUMERIC_MIN_COSINE = 0.98


@dataclass
class ValidationReport:
    """What the validation gate measured (packed_encoders/validate.py:44-49)."""

    pieces: dict[str, Any] = field(default_factory=dict)
    cosine_by_seq_len: dict[int, float] = field(default_factory=dict)
    backend: str = ""


def _resolve_attention_backend(backend: str | None) -> str:
    if backend is None:
        if ops.hip_available():
            return "auto"
        warnings.warn("the HIP attention library is unavailable; packed-encoders runs the 'sdpa' attention path",
                      stacklevel=3)
        return "sdpa"
    if backend in ("flash", "triton"):
        raise PackedEncodersError(f"attention_backend={backend!r} is unavailable: this MI355X build runs the HIP "
                                  "kernels ('hip' or 'auto') or the dense 'sdpa' path")
    if backend not in ops.BACKENDS:
        raise PackedEncodersError(f"attention_backend must be 'hip', 'auto', 'sdpa' or None, got {backend!r}")
    if backend == "hip":
        try:
            ops._load_hip_attention()
        except ImportError as exc:
            raise PackedEncodersError(f"attention_backend='hip' is unavailable: {exc}") from exc
    return backend


def _device_of(encoder: nn.Module) -> torch.device:
    try:
        return next(encoder.parameters()).device
    except StopIteration as exc:
        raise PackedEncodersError("the model has no parameters") from exc


def _check_numerics(encoder: nn.Module, params: ModernBertParams, state: PatchState) -> dict[int, float]:
    """The packed forward against the original forward on random token ids: mean per-token
    cosine must reach 0.98 at every length (validate.py:129-170)."""
    device = _device_of(encoder)
    gen = torch.Generator(device="cpu").manual_seed(0)
    vocab = encoder.embeddings.tok_embeddings.num_embeddings
    out = {}
    for s in _NUMERIC_LENGTHS:
        ids = torch.randint(0, vocab, (2, s), generator=gen).to(device)
        mask = torch.ones_like(ids)
        mask[1, s // 2:] = 0
        with torch.no_grad():
            want = state.original_forward(input_ids=ids, attention_mask=mask).last_hidden_state.float()
            got = forward.fused_forward(encoder, params, ids, mask, backend=state.attention_backend,
                                        execution=state.execution).float()
        live = mask.bool()
        cos = torch.nn.functional.cosine_similarity(got[live], want[live], dim=-1).mean().item()
        out[s] = cos
        if not cos >= _NUMERIC_MIN_COSINE:
            raise ValidationError(f"packed forward cosine {cos:.4f} < {_NUMERIC_MIN_COSINE} vs the original forward "
                                  f"at S={s}")
    return out


def _make_forward(encoder: nn.Module, state: PatchState):
    """The patched ``forward(input_ids, attention_mask, ...)`` (pack.py:257-321)."""
    from transformers.modeling_outputs import BaseModelOutput

    def patched(input_ids: Tensor | None = None, attention_mask: Tensor | None = None, *, return_dict: bool = True,
                **kwargs):
        if input_ids is None:
            raise NotImplementedError("packed-encoders requires input_ids (inputs_embeds is unsupported)")
        _reject_unsupported(kwargs)
        hidden = forward.fused_forward(encoder, state.params, input_ids, attention_mask,
                                       backend=state.attention_backend, execution=state.execution)
        return BaseModelOutput(last_hidden_state=hidden) if return_dict else (hidden,)

    return patched


# Hugging Face forward arguments the packed path does not serve: (argument, whether a value
# uses it, what the error names). The messages are the reference's, which callers may match.
_UNSERVED = (
    ("inputs_embeds", lambda value: value is not None, "inputs_embeds"),
    ("output_attentions", bool, "output_attentions"),
    ("output_hidden_states", bool, "output_hidden_states"),
    ("token_type_ids", lambda value: value is not None and bool(value.any()), "non-zero token_type_ids"),
)


def _reject_unsupported(kwargs: dict) -> None:
    for argument, used, what in _UNSERVED:
        if used(kwargs.get(argument)):
            raise NotImplementedError(f"packed-encoders does not support {what}")


def _enable_graphs(encoder: nn.Module, state: PatchState, cuda_graph, seq_cutoff: int | None) -> None:
    config = cuda_graph if isinstance(cuda_graph, GraphConfig) else GraphConfig(max_seq=seq_cutoff)
    state.packed_graph_runner = build_packed_runner(encoder, state.params, config, backend=state.attention_backend,
                                                    execution=state.execution)
    state.graph_enabled = True


class PackedModernBert:
    """The installed engine (arch/modernbert.py:96-180): ``forward_packed`` for pre-packed
    batches, graph toggles and ``close``."""

    def __init__(self, encoder: nn.Module, state: PatchState):
        self.encoder = encoder
        self.state = state

    @property
    def graph_enabled(self) -> bool:
        return self.state.graph_enabled

    @graph_enabled.setter
    def graph_enabled(self, enabled: bool) -> None:
        self.state.graph_enabled = enabled

    def forward_packed(self, batch: PackedBatch) -> Tensor:
        """``[T, hidden]`` for a packed batch. Metadata checks read shapes, dtypes and devices
        only (no device-to-host transfer); value consistency belongs to the collator."""
        ids, cu, positions = batch.input_ids, batch.cu_seqlens, batch.position_ids
        if cu is None or positions is None or batch.max_seqlen is None:
            raise PackedEncodersError("ModernBERT requires cu_seqlens, max_seqlen and position_ids")
        if ids.ndim != 1 or positions.shape != ids.shape or cu.ndim != 1 or cu.numel() < 2:
            raise PackedEncodersError("expected flat ids/positions and sequence boundaries of shape [N+1]")
        if cu.dtype != torch.int32 or ids.dtype != torch.int64 or positions.dtype != torch.int64:
            raise PackedEncodersError("ModernBERT requires int64 ids/positions and int32 cu_seqlens")
        if ids.device != cu.device or ids.device != positions.device:
            raise PackedEncodersError("packed metadata must be on the token device")
        if ids.numel() == 0 or batch.max_seqlen <= 0:
            raise PackedEncodersError("empty packed batches are unsupported")
        # host lengths, when the collator gives them, bound the shortest segment (no device read)
        shortest = min(batch.host_lengths, default=0) if batch.host_lengths else 0
        return forward.packed_forward(self.encoder, self.state.params, ids, cu, batch.max_seqlen, positions,
                                      backend=self.state.attention_backend,
                                      min_seqlen=max(0, min(int(shortest), int(batch.max_seqlen))))

    def set_cuda_graph(self, enabled: bool, config: GraphConfig | None = None) -> None:
        if enabled and self.state.packed_graph_runner is None:
            _enable_graphs(self.encoder, self.state, config or GraphConfig(), None)
        self.state.graph_enabled = enabled

    def close(self) -> None:
        self.state.packed_graph_runner = None
        self.state.graph_enabled = False


def pack(target: object, *, cuda_graph: bool | GraphConfig | None = None, cuda_graph_seq_cutoff: int | None = 64,
         attention_backend: str | None = None, pieces: ModernBertPieces | None = None,
         validate: bool = True) -> object:
    """Install the packed forward on ``target``'s ModernBERT backbone and return ``target``.

    ``cuda_graph``: ``True`` or a ``GraphConfig`` enables the bucketed packed graph runner (it
    engages when the config bounds both ``max_batch`` and ``max_seq``). ``validate`` runs every
    piece's probe and the numerics gate against the original forward. Packing an already
    packed model only enables graphs; switching the backend requires ``unpack`` first.
    """
    encoder = find_encoder(target)
    state = find_state(encoder)
    if state is not None:
        if attention_backend is not None and attention_backend != state.attention_backend:
            raise PackedEncodersError("unpack the model before changing its attention backend")
        if cuda_graph and state.packed_graph_runner is None:
            _enable_graphs(encoder, state, cuda_graph, cuda_graph_seq_cutoff)
        return target
    backend = _resolve_attention_backend(attention_backend)
    device = _device_of(encoder)
    if device.type != "cuda" and backend != "sdpa":
        raise PackedEncodersError(f"the HIP attention path needs the model on a HIP device; it is on {device}")
    params = ModernBertParams.from_hf_config(encoder.config)
    pieces = pieces if pieces is not None else default_pieces()
    state = PatchState(params=params, original_forward=encoder.forward, attention_backend=backend, pieces=pieces,
                       execution=pieces.bind())
    if validate:
        report = ValidationReport(pieces=pieces.validate(encoder), backend=backend)
        report.cosine_by_seq_len = _check_numerics(encoder, params, state)
        state.validation_report = report
    if cuda_graph:
        _enable_graphs(encoder, state, cuda_graph, cuda_graph_seq_cutoff)
    had_forward = "forward" in encoder.__dict__
    try:
        setattr(encoder, ATTR, state)
        encoder.forward = _make_forward(encoder, state)
        setattr(encoder, INSTALL_ATTR, (PackedModernBert(encoder, state), had_forward))
    except BaseException:
        _restore(encoder, state, had_forward)
        raise
    return target


def _restore(encoder: nn.Module, state: PatchState, had_forward: bool) -> None:
    if had_forward:
        encoder.forward = state.original_forward
    else:
        encoder.__dict__.pop("forward", None)
    encoder.__dict__.pop(ATTR, None)
    encoder.__dict__.pop(INSTALL_ATTR, None)


def unpack(target: object) -> object:
    """Restore the original forward; trained weights stay as they are."""
    encoder = find_encoder(target)
    installed = encoder.__dict__.get(INSTALL_ATTR)
    if installed is not None:
        engine, had_forward = installed
        engine.close()
        _restore(encoder, engine.state, had_forward)
    return target


def get_engine(target: object) -> PackedModernBert:
    encoder = find_encoder(target)
    installed = encoder.__dict__.get(INSTALL_ATTR)
    if installed is None:
        raise PackedEncodersError("this model has not been packed with packed_encoders_amd.pack()")
    return installed[0]


def validate(target: object) -> ValidationReport:
    """Run the validation gate on a packed model (or prepare one temporarily to run it)."""
    encoder = find_encoder(target)
    state = find_state(encoder)
    if state is None:
        pack(target, validate=False)
        try:
            return validate(target)
        finally:
            unpack(target)
    report = ValidationReport(pieces=state.pieces.validate(encoder), backend=state.attention_backend)
    report.cosine_by_seq_len = _check_numerics(encoder, state.params, state)
    return report


def set_cuda_graph(model: object, enabled: bool, *, config: GraphConfig | None = None) -> None:
    get_engine(model).set_cuda_graph(enabled, config)


class _NoCudaGraph:
    def __init__(self, model: object):
        self._state = get_state(find_encoder(model))

    def __enter__(self):
        self._previous = self._state.graph_enabled
        self._state.graph_enabled = False
        return self

    def __exit__(self, *exc):
        self._state.graph_enabled = self._previous
        return False


def no_cuda_graph(model: object) -> _NoCudaGraph:
    """Temporarily bypass captured graphs (a one-off odd shape), restoring the setting on exit."""
    return _NoCudaGraph(model)


__all__ = ["pack", "unpack", "get_engine", "validate", "set_cuda_graph", "no_cuda_graph", "PackedModernBert",
           "ValidationReport", "UnsupportedTargetError"]
