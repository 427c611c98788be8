"""The ModernBERT configuration slice the packed forward reads (packed_encoders/config.py:19-99).

Built once from a Hugging Face config when a model is packed. It absorbs both config schemas
transformers has used: the 4.x fields (``global_rope_theta``, ``local_rope_theta``,
``global_attn_every_n_layers``) and the 5.x ones (``rope_parameters`` keyed by layer kind and the
``layer_types`` list). The attention path takes three things from it: the softmax scale
``head_dim ** -0.5``, the local half window ``local_attention // 2`` and which layers are global.
"""

from __future__ import annotations

from dataclasses import dataclass

# ``config.model_type`` values that share ModernBERT's weight layout and split-half RoPE.
SUPPORTED_MODEL_TYPES = frozenset({"modernbert", "mmbert"})


@dataclass(frozen=True)
class ModernBertParams:
    hidden_size: int
    num_attention_heads: int
    num_hidden_layers: int
    norm_eps: float
    global_rope_theta: float
    local_rope_theta: float
    local_attention: int
    global_attn_every_n_layers: int

    @property
    def head_dim(self) -> int:
        if self.hidden_size % self.num_attention_heads:
            raise ValueError(f"hidden_size={self.hidden_size} is not a multiple of "
                             f"num_attention_heads={self.num_attention_heads}")
        return self.hidden_size // self.num_attention_heads

    @property
    def scaling(self) -> float:
        return self.head_dim ** -0.5

    @property
    def sliding_half_window(self) -> int:
        """Local layers attend to keys with ``|i - j| <= local_attention // 2``."""
        return self.local_attention // 2

    def is_global_layer(self, layer_idx: int) -> bool:
        return layer_idx % self.global_attn_every_n_layers == 0

    def window(self, layer_idx: int) -> tuple[int, int]:
        """``(left, right)`` key window of a layer: ``(-1, -1)`` global, else the half window."""
        if self.is_global_layer(layer_idx):
            return (-1, -1)
        return (self.sliding_half_window, self.sliding_half_window)

    @classmethod
    def from_hf_config(cls, config) -> "ModernBertParams":
        model_type = getattr(config, "model_type", None)
        if model_type not in SUPPORTED_MODEL_TYPES:
            raise ValueError(f"only ModernBERT-architecture models {sorted(SUPPORTED_MODEL_TYPES)} are supported; "
                             f"got model_type={model_type!r}")
        global_theta, local_theta = rope_thetas(config)
        return cls(
            hidden_size=int(config.hidden_size),
            num_attention_heads=int(config.num_attention_heads),
            num_hidden_layers=int(config.num_hidden_layers),
            norm_eps=float(config.norm_eps),
            global_rope_theta=global_theta,
            local_rope_theta=local_theta,
            local_attention=int(config.local_attention),
            global_attn_every_n_layers=global_every(config),
        )


def global_every(config) -> int:
    """The global-layer period. transformers 5 stores the schedule as ``layer_types``; the
    period is recovered from it and must describe "global at layers 0, n, 2n, ..."."""
    kinds = getattr(config, "layer_types", None)
    if not kinds:
        return int(config.global_attn_every_n_layers)
    kinds = list(kinds)
    if set(kinds) <= {"full_attention", "sliding_attention"}:
        for period in range(1, len(kinds) + 1):
            if all((kind == "full_attention") == (i % period == 0) for i, kind in enumerate(kinds)):
                return period
    raise ValueError(f"global attention must recur every n layers from layer 0; got layer_types={kinds}")


def rope_thetas(config) -> tuple[float, float]:
    """(global, local) RoPE base for either config schema."""
    global_theta = getattr(config, "global_rope_theta", None)
    local_theta = getattr(config, "local_rope_theta", None)
    if global_theta is None or local_theta is None:
        params = getattr(config, "rope_parameters", None)
        params = params if isinstance(params, dict) else {}
        fallback = getattr(config, "rope_theta", None) or 160_000.0
        global_theta = global_theta or params.get("full_attention", {}).get("rope_theta") or fallback
        local_theta = local_theta or params.get("sliding_attention", {}).get("rope_theta") or fallback
    return float(global_theta), float(local_theta)
