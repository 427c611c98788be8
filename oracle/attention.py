"""CPU oracle of packed varlen attention — TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Restates, in numpy float64, the semantics every reference oracle and kernel of the path shares:
fp32/fp64 per-segment dense softmax attention, confined to each segment's
``[cu[s], cu[s+1])`` range:

- ``packed_encoders/pieces/attention.py:15-39`` (``_dense``/``reference``: per segment, the
  ``(left, right)`` band ``delta > left | delta < -right`` masked, SDPA with ``scale``);
- ``packed_encoders/runtime/attention.py:157-204`` (``_band``/``_segments``/``_reference``: GQA by
  ``repeat_interleave`` of kv heads, causal as right window 0, empty segments skipped);
- ``tests/test_packed_short_attention.py:35-48`` (the kernel test's fp32 reference);
- ``packed_encoders/_kernels/hybrid.py:197-206`` (gate: ``bf16(o * bf16(sigmoid(g)))`` on the
  bf16 attention output).

Parity pins (tests/test_oracle.py): the brute-force loop form below on tiny inputs, closed
forms (L = 1 and half = 0 give v; q = 0 gives the window mean of v; Hkv = Hq GQA equals MHA;
half >= L - 1 equals global), bf16 rounding against torch's, and the reference's own compiled
CPU kernel (oracle/_ref) at fp32 tolerance. Separate key segments (queries the tail of their
keys) are pinned by the brute-force form and by the tail identity: they must equal the last
rows of self-attention over the whole key segment.
"""

from __future__ import annotations

import math

import numpy as np


def to_bf16(x) -> np.ndarray:
    """Round to the nearest bf16 (ties to even), returned as float32 values. NaN stays NaN."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    out = rounded.view(np.float32).copy()
    nan = np.isnan(a)
    if nan.any():
        out[nan] = np.nan
    return out


def allowed_mask(n_q: int, n_k: int, window=(-1, -1), causal: bool = False) -> np.ndarray:
    """Bool ``[n_q, n_k]``: query i (the last ``n_q`` of ``n_k`` positions) may read key j.

    ``i - j <= left`` and ``j - i <= right`` (-1 unbounded); causal forces ``right = 0``
    (runtime/attention.py:157-170)."""
    left, right = window
    right = 0 if causal else right
    qpos = np.arange(n_k - n_q, n_k)[:, None]
    kpos = np.arange(n_k)[None, :]
    delta = qpos - kpos
    ok = np.ones((n_q, n_k), dtype=bool)
    if left >= 0:
        ok &= delta <= left
    if right >= 0:
        ok &= delta >= -right
    return ok


def segment_attention(q, k, v, *, scale: float, window=(-1, -1), causal: bool = False) -> np.ndarray:
    """One segment: q ``[Lq, Hq, D]``, k/v ``[Lk, Hkv, D]`` → float64 ``[Lq, Hq, D]``. With
    ``Lk != Lq`` the queries are the last ``Lq`` of the ``Lk`` key positions (the reference's
    prefixed form, runtime/attention.py:157-170,236-245); a query that may read no key gets
    zeros (FlashAttention's convention; SDPA would give NaN)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    n, hq, _ = q.shape
    nk, hkv = k.shape[0], k.shape[1]
    if n == 0:
        return np.zeros_like(q)
    if nk == 0:
        return np.zeros_like(q)
    group = hq // hkv
    kr = np.repeat(k, group, axis=1)  # kv head h // group serves query head h
    vr = np.repeat(v, group, axis=1)
    scores = np.einsum("qhd,khd->hqk", q, kr) * scale
    mask = allowed_mask(n, nk, window, causal)
    scores = np.where(mask[None], scores, -np.inf)
    mx = scores.max(axis=-1, keepdims=True)
    empty = ~np.isfinite(mx)
    p = np.exp(scores - np.where(empty, 0.0, mx))
    total = p.sum(axis=-1, keepdims=True)
    p = p / np.where(empty, 1.0, total)
    return np.einsum("hqk,khd->qhd", p, vr)


def packed_attention(q, k, v, cu_seqlens, *, scale: float, window=(-1, -1), causal: bool = False,
                     gate=None, cu_seqlens_k=None) -> np.ndarray:
    """Packed varlen attention over ``[T, H, D]`` arrays; rows outside every segment are NaN.

    ``cu_seqlens_k`` gives k/v segments of their own (query segment s reads key segment s, its
    queries the tail of those positions); by default the query segments. With ``gate`` the
    result is the gated output computed from the bf16-rounded attention output, exactly as
    the reference's separate gate kernel consumes it."""
    cu = [int(x) for x in np.asarray(cu_seqlens).tolist()]
    cuk = cu if cu_seqlens_k is None else [int(x) for x in np.asarray(cu_seqlens_k).tolist()]
    q = np.asarray(q)
    out = np.full(q.shape, np.nan, dtype=np.float64)
    for (a, b), (ka, kb) in zip(zip(cu, cu[1:]), zip(cuk, cuk[1:])):
        if b > a:
            out[a:b] = segment_attention(q[a:b], k[ka:kb], v[ka:kb], scale=scale, window=window, causal=causal)
    if gate is not None:
        out = sigmoid_gate(to_bf16(out), gate)
    return out


def sigmoid_gate(o, g) -> np.ndarray:
    """``bf16(o * bf16(sigmoid(g)))`` with o already bf16 (hybrid.py:197-206)."""
    g = np.asarray(g, dtype=np.float64)
    s = to_bf16((1.0 / (1.0 + np.exp(-g))).astype(np.float32)).astype(np.float64)
    return to_bf16((np.asarray(o, dtype=np.float64) * s).astype(np.float32)).astype(np.float64)


def sampled_rows_attention(q, k, v, cu_seqlens, rows, *, scale: float, window=(-1, -1),
                           causal: bool = False) -> np.ndarray:
    """The oracle for selected token rows only (every head), float64 ``[len(rows), Hq, D]``.

    Each row needs only its own query against its segment's keys, so full-size outputs can be
    checked on a sample at O(rows * L * D) cost. The sampled rows of one segment are scored
    together against the keys their windows span (kv head h // (Hq / Hkv) serves query head h)."""
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    rows = np.asarray(rows, dtype=np.int64)
    q = np.asarray(q)
    hq, hkv, d = q.shape[1], k.shape[1], q.shape[2]
    group = hq // hkv
    out = np.empty((len(rows), hq, d), dtype=np.float64)
    seg_of = np.searchsorted(cu, rows, side="right") - 1
    left, right = window
    right = 0 if causal else right
    bounded = left >= 0 and right >= 0
    for s in np.unique(seg_of):
        a, b = int(cu[s]), int(cu[s + 1])
        members = np.nonzero(seg_of == s)[0]
        members = members[np.argsort(rows[members], kind="stable")]
        # rows of a bounded window are scored in clusters, so a cluster spans few keys
        if bounded:
            cut = np.nonzero(np.diff(rows[members]) > 64)[0] + 1
            chunks = np.split(members, cut)
        else:
            chunks = [members]
        for sel in chunks:
            pos = rows[sel] - a
            lo = 0 if left < 0 else max(0, int(pos.min()) - left)
            hi = b - a if right < 0 else min(b - a, int(pos.max()) + right + 1)
            # [hkv, keys, d] operands; queries [hkv, rows * group, d]
            kk = np.asarray(k[a + lo:a + hi], dtype=np.float64).transpose(1, 0, 2)
            vv = np.asarray(v[a + lo:a + hi], dtype=np.float64).transpose(1, 0, 2)
            qq = np.asarray(q[rows[sel]], dtype=np.float64).reshape(len(sel), hkv, group, d)
            qq = qq.transpose(1, 0, 2, 3).reshape(hkv, len(sel) * group, d)
            sc = (qq @ kk.transpose(0, 2, 1)).reshape(hkv, len(sel), group, hi - lo) * scale
            delta = pos[:, None] - np.arange(lo, hi)[None, :]
            ok = np.ones(delta.shape, dtype=bool)
            if left >= 0:
                ok &= delta <= left
            if right >= 0:
                ok &= delta >= -right
            sc = np.where(ok[None, :, None, :], sc, -np.inf)
            sc -= sc.max(axis=-1, keepdims=True)
            p = np.exp(sc)
            p /= p.sum(axis=-1, keepdims=True)
            o = p.reshape(hkv, len(sel) * group, hi - lo) @ vv  # [hkv, rows * group, d]
            out[sel] = o.reshape(hkv, len(sel), group, d).transpose(1, 0, 2, 3).reshape(len(sel), hq, d)
    return out


def brute_force_attention(q, k, v, cu_seqlens, *, scale: float, window=(-1, -1), causal: bool = False,
                          cu_seqlens_k=None):
    """Scalar-loop float64 form of the same semantics, for tiny inputs only: every score, max,
    exponential and weighted sum written out, with no vectorised masking or broadcasting. A
    query of segment [a, b) with key segment [ka, kb) sits at key position
    (i - a) + (kb - ka) - (b - a); a query that reaches no key gets zeros."""
    cu = [int(x) for x in np.asarray(cu_seqlens).tolist()]
    cuk = cu if cu_seqlens_k is None else [int(x) for x in np.asarray(cu_seqlens_k).tolist()]
    T, hq, d = np.asarray(q).shape
    hkv = np.asarray(k).shape[1]
    left, right = window
    if causal:
        right = 0
    out = [[[math.nan] * d for _ in range(hq)] for _ in range(T)]
    for (a, b), (ka, kb) in zip(zip(cu, cu[1:]), zip(cuk, cuk[1:])):
        shift = (kb - ka) - (b - a)
        for h in range(hq):
            kvh = h // (hq // hkv)
            for i in range(a, b):
                pos = (i - a) + shift
                keys = [j for j in range(ka, kb)
                        if (left < 0 or pos - (j - ka) <= left) and (right < 0 or (j - ka) - pos <= right)]
                if not keys:
                    for x in range(d):
                        out[i][h][x] = 0.0
                    continue
                scores = []
                for j in keys:
                    acc = 0.0
                    for x in range(d):
                        acc += float(q[i][h][x]) * float(k[j][kvh][x])
                    scores.append(acc * scale)
                m = max(scores)
                w = [math.exp(s - m) for s in scores]
                total = sum(w)
                for x in range(d):
                    out[i][h][x] = sum(wj * float(v[j][kvh][x]) for wj, j in zip(w, keys)) / total
    return np.asarray(out, dtype=np.float64)


def cosine_per_token(a, b) -> np.ndarray:
    """Cosine similarity of each ``[H*D]`` token row of a and b (float64)."""
    a = np.asarray(a, dtype=np.float64).reshape(a.shape[0], -1)
    b = np.asarray(b, dtype=np.float64).reshape(b.shape[0], -1)
    num = (a * b).sum(-1)
    den = np.linalg.norm(a, axis=-1) * np.linalg.norm(b, axis=-1)
    return num / np.maximum(den, 1e-300)
