"""Find the ModernBERT backbone inside what ``pack()`` is given (packed_encoders/locate.py:38-107).

A Hugging Face ``ModernBertModel``, a task model holding one under ``.model``, or a
SentenceTransformer / PyLate model holding one under ``[0].auto_model``. The known wrapper
attributes are walked breadth-first a few levels deep; an unknown container raises rather than
guessing, since a wrong guess would patch the wrong weights.
"""

from __future__ import annotations

from torch import nn

from .config import SUPPORTED_MODEL_TYPES
from .errors import UnsupportedTargetError

_WRAPPER_ATTRS = ("auto_model", "model", "modernbert", "bert", "encoder", "backbone", "language_model")


def is_modernbert_encoder(module: object) -> bool:
    """A ``ModernBertModel``-shaped backbone: a supported ``model_type`` and the embeddings,
    layers and final_norm the packed forward reads."""
    if not isinstance(module, nn.Module):
        return False
    if getattr(getattr(module, "config", None), "model_type", None) not in SUPPORTED_MODEL_TYPES:
        return False
    return all(hasattr(module, name) for name in ("embeddings", "layers", "final_norm"))


def walk_targets(target: object, max_depth: int = 4):
    """The target, then what its wrapper attributes (and ``target[0]``) hold, depth-first."""
    seen: set[int] = set()

    def walk(node, depth):
        if id(node) in seen:
            return
        seen.add(id(node))
        yield node
        if depth >= max_depth:
            return
        if hasattr(node, "__getitem__") and isinstance(node, nn.Module):
            try:
                first = node[0]
            except (KeyError, IndexError, TypeError, NotImplementedError):
                first = None
            if isinstance(first, nn.Module):
                yield from walk(first, depth + 1)
        for attr in _WRAPPER_ATTRS:
            sub = getattr(node, attr, None)
            if isinstance(sub, nn.Module):
                yield from walk(sub, depth + 1)

    yield from walk(target, 0)


def find_encoder(target: object) -> nn.Module:
    for module in walk_targets(target):
        if is_modernbert_encoder(module):
            return module
    raise UnsupportedTargetError(
        f"could not locate a ModernBERT backbone in {type(target).__name__!r}: pass a Hugging Face "
        "ModernBertModel, a task model exposing it as .model, or a SentenceTransformer / PyLate model "
        "wrapping one")
