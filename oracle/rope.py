"""CPU oracle of split-half RoPE read from a packed QKV projection — TEST INFRASTRUCTURE ONLY
(see oracle/__init__.py).

Restates the reference's rotary embedding on the packed-attention path:
``packed_encoders/_kernels/rope.py:142-199`` (``_build_bshd_for_hd``: q at column 0 and k at
column H*D of a qkv row, table row ``bs % s_mod``, ``x * cos + sign * partner * sin`` in fp32
with sign -1 on the low half) and its fp32 reference ``rotate_half`` formula
(``x * cos + rotate_half(x) * sin``), with the rounding this build fixes for it: each product
rounded to fp32, then the sum, then one rounding to bf16.

Tables follow the reference's construction (``rope.py`` cos/sin caches): angles
``pos * theta ** (-2i / D)`` in fp32, duplicated over the two halves, cos/sin rounded to bf16.

Pins (tests/test_oracle.py): position 0 is the identity; a quarter turn maps (a, b) to (-b, a)
exactly; pair norms are preserved to fp32 rounding; rotating by p then q equals rotating by
p + q; and bit-exact agreement with the torch fp32 formula on random inputs.
"""

from __future__ import annotations

import numpy as np

from .attention import to_bf16


def rope_tables(n_pos: int, d: int, theta: float) -> tuple[np.ndarray, np.ndarray]:
    """cos, sin ``[n_pos, d]`` as bf16 values (float32 arrays)."""
    inv = (1.0 / (np.float32(theta) ** (np.arange(0, d, 2, dtype=np.float32) / np.float32(d)))).astype(np.float32)
    ang = np.outer(np.arange(n_pos, dtype=np.float32), inv).astype(np.float32)
    emb = np.concatenate([ang, ang], axis=1)
    return to_bf16(np.cos(emb)), to_bf16(np.sin(emb))


def rotate(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Split-half rotation of bf16-valued ``x [..., d]`` by tables broadcast to it; bf16 out."""
    x = np.asarray(x, dtype=np.float32)
    c = np.asarray(cos, dtype=np.float32)
    s = np.asarray(sin, dtype=np.float32)
    h = x.shape[-1] // 2
    lo, hi = x[..., :h], x[..., h:]
    out_lo = (lo * c[..., :h]).astype(np.float32) - (hi * s[..., :h]).astype(np.float32)
    out_hi = (hi * c[..., h:]).astype(np.float32) + (lo * s[..., h:]).astype(np.float32)
    return to_bf16(np.concatenate([out_lo, out_hi], axis=-1))


def rope_qkv(qkv: np.ndarray, h: int, d: int, cos: np.ndarray, sin: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """q, k ``[rows, h, d]`` from ``qkv [rows, >= 3*h*d]``; row r uses table row r % len(cos)."""
    qkv = np.asarray(qkv, dtype=np.float32)
    rows = qkv.shape[0]
    t = np.arange(rows) % cos.shape[0]
    c, s = cos[t][:, None, :], sin[t][:, None, :]
    q = qkv[:, : h * d].reshape(rows, h, d)
    k = qkv[:, h * d: 2 * h * d].reshape(rows, h, d)
    return rotate(q, c, s), rotate(k, c, s)
