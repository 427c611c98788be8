"""Pins the CPU oracle (oracle/attention.py) before any GPU result is compared with it.

Each check is chosen so that a plausible mistake in the oracle fails it: a dropped scale, a
transposed operand, an off-by-one band edge, a wrong GQA head mapping or a wrong bf16 rounding.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as oa


def _rand(rng, *shape):
    return rng.standard_normal(shape).astype(np.float32)


def _cu(lengths):
    return np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)


def test_to_bf16_matches_torch_rounding():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0,
        # exact ties between two bf16 neighbours (low 16 bits = 0x8000), both parities
        (np.arange(1, 2000, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
        np.array([0.0, -0.0, 1e-40, -1e-40, 3.3895e38, np.inf, -np.inf], dtype=np.float32),
    ])
    ours = oa.to_bf16(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ours.view(np.uint32), theirs.view(np.uint32))
    assert np.isnan(oa.to_bf16(np.array([np.nan], dtype=np.float32))).all()


@pytest.mark.parametrize("window,causal", [((-1, -1), False), ((2, 2), False), ((0, 3), False),
                                           ((-1, -1), True), ((1, -1), False)])
def test_vectorised_oracle_matches_brute_force(window, causal):
    rng = np.random.default_rng(1)
    lengths = [1, 5, 0, 7, 3]
    T = sum(lengths)
    q, k, v = _rand(rng, T, 4, 8), _rand(rng, T, 2, 8), _rand(rng, T, 2, 8)
    cu = _cu(lengths)
    fast = oa.packed_attention(q, k, v, cu, scale=0.3, window=window, causal=causal)
    slow = oa.brute_force_attention(q, k, v, cu, scale=0.3, window=window, causal=causal)
    np.testing.assert_allclose(fast, slow, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("window,causal", [((-1, -1), False), ((-1, -1), True), ((4, 2), False), ((3, -1), True),
                                           ((0, 0), False)])
def test_prefixed_oracle_matches_brute_force(window, causal):
    """Separate key segments: the vectorised oracle against the scalar loop, on short tails, a
    single query, a square pair and a long prefix, plus an empty query segment and an empty key
    segment (its queries reach nothing: zeros)."""
    rng = np.random.default_rng(11)
    lq, lk = [2, 1, 3, 4, 0, 2], [5, 4, 3, 9, 2, 0]
    q = _rand(rng, sum(lq), 2, 4)
    k, v = _rand(rng, sum(lk), 1, 4), _rand(rng, sum(lk), 1, 4)
    got = oa.packed_attention(q, k, v, _cu(lq), scale=0.5, window=window, causal=causal, cu_seqlens_k=_cu(lk))
    want = oa.brute_force_attention(q, k, v, _cu(lq), scale=0.5, window=window, causal=causal, cu_seqlens_k=_cu(lk))
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    assert np.all(got[-2:] == 0.0)  # the last query segment has no keys


@pytest.mark.parametrize("window,causal", [((-1, -1), False), ((-1, -1), True), ((6, 3), False), ((9, -1), True)])
def test_prefixed_queries_are_the_tail_of_full_attention(window, causal):
    """A query segment aligned to the end of its key segment reads exactly what the last rows
    of self-attention over the whole key segment read: giving the full segment queries whose
    tail is the prefixed queries, the full result's tail must equal the prefixed result. An
    alignment to the segment start, or an off-by-one shift, breaks this."""
    rng = np.random.default_rng(12)
    lq, lk = [3, 1, 20, 11], [17, 9, 20, 40]
    hq, hkv, d = 4, 2, 8
    kk, vv = _rand(rng, sum(lk), hkv, d), _rand(rng, sum(lk), hkv, d)
    q_full = _rand(rng, sum(lk), hq, d)
    cuk = _cu(lk)
    tails = np.concatenate([np.arange(cuk[i + 1] - n, cuk[i + 1]) for i, n in enumerate(lq)])
    prefixed = oa.packed_attention(q_full[tails], kk, vv, _cu(lq), scale=0.3, window=window, causal=causal,
                                   cu_seqlens_k=cuk)
    full = oa.packed_attention(q_full, kk, vv, cuk, scale=0.3, window=window, causal=causal)
    np.testing.assert_allclose(prefixed, full[tails], rtol=1e-12, atol=1e-12)


def test_prefixed_with_equal_segments_is_self_attention():
    rng = np.random.default_rng(13)
    lengths = [4, 9, 1]
    q, k, v = _rand(rng, 14, 2, 8), _rand(rng, 14, 2, 8), _rand(rng, 14, 2, 8)
    a = oa.packed_attention(q, k, v, _cu(lengths), scale=0.4, window=(2, 1), cu_seqlens_k=_cu(lengths))
    b = oa.packed_attention(q, k, v, _cu(lengths), scale=0.4, window=(2, 1))
    assert np.array_equal(a, b)


def test_single_token_segments_return_v():
    rng = np.random.default_rng(2)
    q, k, v = _rand(rng, 6, 3, 16), _rand(rng, 6, 3, 16), _rand(rng, 6, 3, 16)
    out = oa.packed_attention(q, k, v, _cu([1] * 6), scale=0.125)
    np.testing.assert_allclose(out, v, rtol=0, atol=1e-12)


def test_zero_half_window_and_causal_first_row_return_v():
    rng = np.random.default_rng(3)
    q, k, v = _rand(rng, 20, 2, 8), _rand(rng, 20, 2, 8), _rand(rng, 20, 2, 8)
    cu = _cu([9, 11])
    out = oa.packed_attention(q, k, v, cu, scale=0.125, window=(0, 0))
    np.testing.assert_allclose(out, v, atol=1e-12)
    causal = oa.packed_attention(q, k, v, cu, scale=0.125, causal=True)
    np.testing.assert_allclose(causal[[0, 9]], v[[0, 9]], atol=1e-12)


def test_zero_query_gives_window_mean_of_v():
    rng = np.random.default_rng(4)
    L, w = 13, 3
    q = np.zeros((L, 1, 8), np.float32)
    k, v = _rand(rng, L, 1, 8), _rand(rng, L, 1, 8)
    out = oa.packed_attention(q, k, v, _cu([L]), scale=0.125, window=(w, w))
    for i in range(L):
        lo, hi = max(0, i - w), min(L, i + w + 1)
        np.testing.assert_allclose(out[i, 0], v[lo:hi, 0].astype(np.float64).mean(0), atol=1e-12)


def test_wide_window_equals_global():
    rng = np.random.default_rng(5)
    lengths = [17, 30]
    T = sum(lengths)
    q, k, v = _rand(rng, T, 2, 8), _rand(rng, T, 2, 8), _rand(rng, T, 2, 8)
    cu = _cu(lengths)
    g = oa.packed_attention(q, k, v, cu, scale=0.2)
    wide = oa.packed_attention(q, k, v, cu, scale=0.2, window=(29, 29))
    narrow = oa.packed_attention(q, k, v, cu, scale=0.2, window=(28, 28))
    np.testing.assert_allclose(wide, g, atol=1e-12)
    assert np.abs(narrow - g).max() > 1e-6  # the band edge is real


def test_gqa_equals_mha_on_repeated_kv_heads():
    rng = np.random.default_rng(6)
    lengths = [7, 12]
    T = sum(lengths)
    q, k, v = _rand(rng, T, 8, 16), _rand(rng, T, 2, 16), _rand(rng, T, 2, 16)
    cu = _cu(lengths)
    gqa = oa.packed_attention(q, k, v, cu, scale=0.25, causal=True)
    mha = oa.packed_attention(q, np.repeat(k, 4, axis=1), np.repeat(v, 4, axis=1), cu, scale=0.25, causal=True)
    np.testing.assert_allclose(gqa, mha, atol=1e-12)
    # head h reads kv head h // 4, not h % 2
    wrong = oa.packed_attention(q, np.tile(k, (1, 4, 1)), np.tile(v, (1, 4, 1)), cu, scale=0.25, causal=True)
    assert np.abs(wrong - gqa).max() > 1e-3


def test_oracle_matches_torch_sdpa_per_segment():
    # torch's fp64 SDPA as an independent library routine for the same closed form.
    rng = np.random.default_rng(7)
    lengths = [5, 64, 37]
    T = sum(lengths)
    q, k, v = _rand(rng, T, 3, 32), _rand(rng, T, 3, 32), _rand(rng, T, 3, 32)
    cu = _cu(lengths)
    out = oa.packed_attention(q, k, v, cu, scale=0.17, window=(10, 4))
    for a, b in zip(cu, cu[1:]):
        n = b - a
        qt, kt, vt = (torch.from_numpy(x[a:b]).double().transpose(0, 1) for x in (q, k, v))
        pos = torch.arange(n)
        delta = pos[:, None] - pos[None, :]
        mask = (delta <= 10) & (delta >= -4)
        ref = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask, scale=0.17)
        np.testing.assert_allclose(out[a:b], ref.transpose(0, 1).numpy(), atol=1e-12)


def test_sampled_rows_match_full_oracle():
    """Sampled rows (unsorted, repeated, in clusters further apart than a window) equal the
    full oracle's rows for global, banded, asymmetric and causal attention with GQA."""
    rng = np.random.default_rng(8)
    lengths = [40, 3, 90, 300]
    T = sum(lengths)
    q, k, v = _rand(rng, T, 4, 16), _rand(rng, T, 2, 16), _rand(rng, T, 2, 16)
    cu = _cu(lengths)
    rows = [132, 0, 39, 40, 42, 43, 100, 133, 140, 431, 300, 299, 200, 140]
    for window, causal in (((-1, -1), False), ((5, 5), False), ((64, 64), False), ((3, 70), False),
                           ((-1, -1), True), ((20, -1), True)):
        full = oa.packed_attention(q, k, v, cu, scale=0.25, window=window, causal=causal)
        part = oa.sampled_rows_attention(q, k, v, cu, rows, scale=0.25, window=window, causal=causal)
        np.testing.assert_allclose(part, full[rows], atol=1e-12)


def test_gate_closed_forms():
    rng = np.random.default_rng(9)
    o = oa.to_bf16(_rand(rng, 50, 2, 8))
    half = oa.sigmoid_gate(o, np.zeros_like(o))  # sigmoid(0) = 0.5 exactly, bf16(o/2) = o/2
    np.testing.assert_array_equal(half, o.astype(np.float64) / 2)
    big = oa.sigmoid_gate(o, np.full_like(o, 40.0))  # sigmoid(40) rounds to 1 in bf16
    np.testing.assert_array_equal(big, o.astype(np.float64))
    # matches torch's bf16 pipeline: bf16(sigmoid(g)) then bf16(o * s)
    g = _rand(rng, 50, 2, 8)
    ot, gt = torch.from_numpy(o).bfloat16(), torch.from_numpy(g)
    ref = (ot.float() * torch.sigmoid(gt).bfloat16().float()).bfloat16().float().numpy()
    np.testing.assert_array_equal(oa.sigmoid_gate(o, g).astype(np.float32), ref)


def test_allowed_pairs_closed_form(pe):
    from packed_encoders_amd.hip_attention import allowed_pairs

    for L in (1, 2, 50, 65, 66, 200, 2048):
        w = 64
        expected = L * (2 * w + 1) - w * (w + 1) if L > w + 1 else L * L
        assert allowed_pairs(L, (w, w)) == expected
        assert allowed_pairs(L) == L * L
        assert allowed_pairs(L, causal=True) == L * (L + 1) // 2
        mask = oa.allowed_mask(L, L, (w, w))
        assert allowed_pairs(L, (w, w)) == int(mask.sum())


def test_rope_oracle_closed_forms():
    from oracle import rope

    rng = np.random.default_rng(5)
    d = 64
    x = oa.to_bf16(rng.standard_normal((7, d)))
    cos, sin = rope.rope_tables(8, d, 10000.0)
    # position 0: cos = 1, sin = 0 -> identity
    assert np.array_equal(rope.rotate(x, cos[0], sin[0]), x)
    # a quarter turn on every pair: (a, b) -> (-b, a) exactly
    quarter_c, quarter_s = np.zeros(d, np.float32), np.ones(d, np.float32)
    turned = rope.rotate(x, quarter_c, quarter_s)
    assert np.array_equal(turned[:, : d // 2], -x[:, d // 2:])
    assert np.array_equal(turned[:, d // 2:], x[:, : d // 2])
    # norms of (x_i, x_{i + d/2}) pairs are kept up to the rounding of the tables and outputs
    r = rope.rotate(x, cos[5], sin[5])
    n0 = x[:, : d // 2] ** 2 + x[:, d // 2:] ** 2
    n1 = r[:, : d // 2] ** 2 + r[:, d // 2:] ** 2
    assert np.allclose(n1, n0, rtol=2e-2, atol=1e-3)


def test_rope_oracle_composes_rotations():
    from oracle import rope

    rng = np.random.default_rng(6)
    d = 64
    x = rng.standard_normal((5, d)).astype(np.float32)
    inv = 1.0 / (10000.0 ** (np.arange(0, d, 2) / d))
    def exact(v, pos):  # float64 rotation, no rounding
        a = np.concatenate([pos * inv, pos * inv])
        h = d // 2
        return np.concatenate([v[:, :h] * np.cos(a[:h]) - v[:, h:] * np.sin(a[:h]),
                               v[:, h:] * np.cos(a[h:]) + v[:, :h] * np.sin(a[h:])], axis=1)
    # the bf16 pipeline at position p + q stays close to rotating by p, then by q
    cos, sin = rope.rope_tables(64, d, 10000.0)
    direct = rope.rotate(oa.to_bf16(x), cos[30], sin[30])
    assert np.allclose(direct, exact(exact(x, 10), 20), atol=5e-2)


def test_rope_oracle_matches_torch_fp32_formula_bit_exactly():
    import torch

    from oracle import rope

    rng = np.random.default_rng(7)
    h, d, rows = 3, 64, 11
    qkv = oa.to_bf16(rng.standard_normal((rows, 3 * h * d)))
    cos, sin = rope.rope_tables(rows, d, 160000.0)
    q, k = rope.rope_qkv(qkv, h, d, cos, sin)
    t = torch.from_numpy(qkv).view(rows, 3, h, d)
    c = torch.from_numpy(cos)[:, None, :]
    s = torch.from_numpy(sin)[:, None, :]

    def rot(x):
        half = d // 2
        rotated = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
        return (x * c + rotated * s).bfloat16().float().numpy()

    assert np.array_equal(q, rot(t[:, 0]))
    assert np.array_equal(k, rot(t[:, 1]))
