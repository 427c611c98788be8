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
    """The global-layer period n: layers 0, n, 2n, ... are global. transformers 5 keeps only
    the ``layer_types`` list; n is then the position of the second global layer (the layer
    count when layer 0 is the only one), and the list must be exactly that pattern."""
    kinds = getattr(config, "layer_types", None)
    if not kinds:
        return int(config.global_attn_every_n_layers)
    kinds = list(kinds)
    at = [i for i, kind in enumerate(kinds) if kind == "full_attention"]
    known = set(kinds) <= {"full_attention", "sliding_attention"}
    if known and at and at[0] == 0:
        n = at[1] if len(at) > 1 else len(kinds)
        if at == list(range(0, len(kinds), n)):
            return n
    raise ValueError(f"global attention must recur every n layers from layer 0; got layer_types={kinds}")


def rope_thetas(config) -> tuple[float, float]:
    """(global, local) RoPE bases. Each is the 4.x field (``global_rope_theta``,
    ``local_rope_theta``) when the config has it, else the ``rope_theta`` of its layer kind in
    the 5.x ``rope_parameters``, else ``rope_theta``, else ModernBERT's 160,000."""
    per_kind = getattr(config, "rope_parameters", None)
    per_kind = per_kind if isinstance(per_kind, dict) else {}
    default = getattr(config, "rope_theta", None) or 160_000.0

    def base(field: str, kind: str) -> float:
        value = getattr(config, field, None)
        if value is None:
            value = (per_kind.get(kind) or {}).get("rope_theta") or default
        return float(value)

    return base("global_rope_theta", "full_attention"), base("local_rope_theta", "sliding_attention")
