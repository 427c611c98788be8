"""The fused RoPE prologue of the short kernel (pe_attn_args.rope_cos / rope_sin,
varlen_attention(rope=...), ops.flash_attention_qkv_bshd) against the two-step path it
replaces: the RoPE kernel (pe_rope_qkv_fwd) writing q and k, then the attention call. Both
round every product as the reference's apply_rope_bshd does (packed_encoders/_kernels/rope.py:
302-349), so the fused call must give the same bits; it is also checked against the CPU
oracles (oracle/rope.py, then oracle/attention.py).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce
from oracle import attention as oa

pytestmark = pytest.mark.gpu


def _tables(rows, d, seed):
    from oracle import rope

    cos_np, sin_np = rope.rope_tables(4096, d, 10000.0)
    pos = np.random.default_rng(seed).integers(0, 4096, rows)
    return (torch.from_numpy(cos_np[pos]).bfloat16().cuda(), torch.from_numpy(sin_np[pos]).bfloat16().cuda())


def _batch(lengths, h, d, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    T = sum(lengths)
    qkv = torch.randn(T, 3 * h * d, device="cuda", generator=g, dtype=torch.bfloat16)
    cu = torch.tensor([0, *np.cumsum(lengths).tolist()], dtype=torch.int32, device="cuda")
    return qkv, cu


# (head_dim, heads, n_seq): 12 x 64 with 32, 400 and 700 segments takes the short kernel with
# 1, 2 and 4 heads per workgroup; 6 x 128 with 40 and 700 segments, 1 and 2.
SHAPES = [(64, 12, 32), (64, 12, 400), (64, 12, 700), (128, 6, 40), (128, 6, 700)]


@pytest.mark.parametrize("d,h,n_seq", SHAPES, ids=[f"d{s[0]}_{s[2]}seg" for s in SHAPES])
@pytest.mark.parametrize("tables", ["per-token", "dense-modulo", "strided"])
@pytest.mark.parametrize("window,gate", [((-1, -1), False), ((16, 16), True)], ids=["global", "band16-gate"])
def test_fused_rope_is_bit_identical_to_rope_then_attention(pe, d, h, n_seq, tables, window, gate):
    from packed_encoders_amd.hip_attention import rope_qkv, varlen_attention

    announce(f"fused rope d={d} h={h} n_seq={n_seq} tables={tables} window={window} gate={gate}")
    rng = np.random.default_rng(n_seq + d)
    lengths = rng.integers(1, 129 if n_seq < 100 else 65, size=n_seq).tolist()
    qkv, cu = _batch(lengths, h, d, seed=n_seq)
    T, max_len = sum(lengths), max(lengths)
    cos, sin = _tables(T if tables != "dense-modulo" else 97, d, seed=d)  # 97 rows: row r % 97
    if tables == "strided":  # column views of one [T, 2 * D] table: row stride 2 * D
        both = torch.cat([cos, sin], dim=1)
        cos, sin = both[:, :d], both[:, d:]
    gt = torch.randn(T, h, d, device="cuda", dtype=torch.bfloat16) if gate else None
    view = qkv.view(T, 3, h, d)
    with torch.inference_mode():
        q, k = rope_qkv(qkv, h, d, cos, sin)
        want = varlen_attention(q, k, view[:, 2], cu, max_len, window=window, gate=gt)
        got = varlen_attention(view[:, 0], view[:, 1], view[:, 2], cu, max_len, window=window, gate=gt,
                               rope=(cos, sin))
    assert torch.equal(got, want)


def test_fused_rope_matches_the_oracles(pe):
    from oracle import rope

    from packed_encoders_amd.hip_attention import varlen_attention

    announce("fused rope vs oracles")
    h, d = 4, 64
    lengths = [1, 17, 64, 100, 128, 33]
    qkv, cu = _batch(lengths, h, d, seed=5)
    T = sum(lengths)
    cos, sin = _tables(T, d, seed=6)
    view = qkv.view(T, 3, h, d)
    with torch.inference_mode():
        got = varlen_attention(view[:, 0], view[:, 1], view[:, 2], cu, max(lengths), softmax_scale=0.125,
                               rope=(cos, sin))
    f = lambda t: t.float().cpu().numpy()
    q, k = rope.rope_qkv(f(qkv), h, d, f(cos), f(sin))
    want = oa.packed_attention(q, k, f(view[:, 2]), cu.cpu().numpy(), scale=0.125)
    got = got.float().cpu().numpy().astype(np.float64)
    assert np.abs(got - want).max() <= 2e-2
    assert oa.cosine_per_token(got, want).min() >= 0.9999


@pytest.mark.parametrize("packed", [True, False], ids=["packed", "dense"])
@pytest.mark.parametrize("s", [40, 128, 300], ids=["S40", "S128", "S300-two-steps"])
def test_flash_attention_qkv_bshd_fuses_where_it_can(pe, packed, s):
    """The reference-named entry point: fused on segments of at most 128 tokens, RoPE kernel then
    attention past that, the same bits as the two steps either way (packed [1, T] with
    cu_seqlens, or a dense [B, S] batch with [S, D] tables)."""
    from packed_encoders_amd import ops

    announce(f"flash_attention_qkv_bshd packed={packed} S={s}")
    h, d = 12, 64
    if packed:
        lengths = np.random.default_rng(s).integers(1, s + 1, size=24).tolist()
        qkv2, cu = _batch(lengths, h, d, seed=s)
        qkv, seq = qkv2[None], max(lengths)
        cos, sin = _tables(qkv2.shape[0], d, seed=1)
        cos, sin = cos[None], sin[None]
    else:
        qkv2, _ = _batch([s] * 5, h, d, seed=s)
        qkv, cu, seq = qkv2.view(5, s, 3 * h * d), None, None
        cos, sin = _tables(s, d, seed=2)
        cos, sin = cos[None], sin[None]
    assert ops.fused_rope_applies(qkv, d, seq if packed else s) == (s <= 128)
    with torch.inference_mode():
        got = ops.flash_attention_qkv_bshd(qkv, h, d, cos=cos, sin=sin, window=(64, 64), scaling=0.125,
                                           cu_seqlens=cu, max_seqlen=seq)
        q, k = ops.rope_qkv(qkv, h, d, cos, sin)
        v = qkv.view(*qkv.shape[:2], 3, h, d)[:, :, 2]
        want = ops.attention_bshd(q, k, v, window=(64, 64), scaling=0.125, cu_seqlens=cu, max_seqlen=seq)
    assert got.shape == want.shape and torch.equal(got, want)


def test_fused_rope_outside_the_short_kernel_is_refused(pe):
    from packed_encoders_amd.hip_attention import varlen_attention

    announce("fused rope refusals")
    h, d = 4, 64
    qkv, cu = _batch([200, 30], h, d, seed=9)
    view = qkv.view(230, 3, h, d)
    cos, sin = _tables(230, d, seed=9)
    with torch.inference_mode():
        with pytest.raises(ValueError):  # a segment past the short kernel's reach
            varlen_attention(view[:, 0], view[:, 1], view[:, 2], cu, 200, rope=(cos, sin))
        with pytest.raises(ValueError):  # separate key segments
            varlen_attention(view[:, 0], view[:, 1], view[:, 2], cu, 200, cu_seqlens_k=cu, max_seqlen_k=200,
                             rope=(cos, sin))
        q256 = torch.randn(230, 2, 256, device="cuda", dtype=torch.bfloat16)
        c256, s256 = _tables(230, 256, seed=3)
        with pytest.raises(ValueError):  # head_dim 256 runs no short kernel
            varlen_attention(q256, q256, q256, cu, 200, rope=(c256, s256))
        with pytest.raises(ValueError):  # one table only
            varlen_attention(view[:, 0], view[:, 1], view[:, 2], cu, 200, rope=(cos, None))


@pytest.mark.parametrize("d", [64, 128])
def test_fused_rope_with_gqa(pe, d):
    """Eight query heads on two kv heads, q / k / v as column views of one projection
    [T, (8 + 2 + 2) * D]: the fused call equals, bit for bit, attention over q and k rotated by
    the oracle (oracle/rope.rotate, the kernel's rounding: each product to fp32, their sum to
    bf16) and uploaded, and matches the attention oracle at the reference's bar. Each query head
    of a workgroup rotates its kv head's keys in its own LDS slot."""
    from oracle import rope

    from packed_encoders_amd.hip_attention import varlen_attention

    hq, hkv = 8, 2
    announce(f"fused rope gqa d={d}")
    lengths = np.random.default_rng(d).integers(1, 65, size=60).tolist()
    T = sum(lengths)
    g = torch.Generator(device="cuda").manual_seed(d)
    proj = torch.randn(T, (hq + 2 * hkv) * d, device="cuda", generator=g, dtype=torch.bfloat16)
    q = proj[:, : hq * d].view(T, hq, d)
    k = proj[:, hq * d:(hq + hkv) * d].view(T, hkv, d)
    v = proj[:, (hq + hkv) * d:].view(T, hkv, d)
    cos, sin = _tables(T, d, seed=d + 1)
    cu = torch.tensor([0, *np.cumsum(lengths).tolist()], dtype=torch.int32, device="cuda")
    f = lambda t: t.float().cpu().numpy()
    qr = rope.rotate(f(q), f(cos)[:, None, :], f(sin)[:, None, :])
    kr = rope.rotate(f(k), f(cos)[:, None, :], f(sin)[:, None, :])
    with torch.inference_mode():
        got = varlen_attention(q, k, v, cu, max(lengths), softmax_scale=d ** -0.5, rope=(cos, sin))
        two_step = varlen_attention(torch.from_numpy(qr).bfloat16().cuda(), torch.from_numpy(kr).bfloat16().cuda(),
                                    v.contiguous(), cu, max(lengths), softmax_scale=d ** -0.5)
    assert torch.equal(got, two_step)
    want = oa.packed_attention(qr, kr, f(v), cu.cpu().numpy(), scale=d ** -0.5)
    got64 = got.float().cpu().numpy().astype(np.float64)
    assert np.abs(got64 - want).max() <= 2e-2
    assert oa.cosine_per_token(got64, want).min() >= 0.9999


def _draw_rope_case(seed: int) -> dict:
    rng = np.random.default_rng(1000 + seed)
    d = int(rng.choice([64, 128]))
    hq, hkv = [(12, 12), (8, 2), (6, 3), (4, 4), (4, 1)][int(rng.integers(0, 5))]
    cap = int(rng.choice([32, 64, 128]))
    lengths = rng.integers(1, cap + 1, size=int(rng.integers(1, 80))).tolist()
    window = [(-1, -1), (16, 16), (0, 40), (33, 7)][int(rng.integers(0, 4))]
    return dict(d=d, hq=hq, hkv=hkv, lengths=lengths, window=window, gate=bool(rng.integers(0, 2)),
                tables=["per-token", "modulo", "strided"][int(rng.integers(0, 3))], seed=seed)


@pytest.mark.parametrize("seed", range(24))
def test_random_fused_rope_calls(pe, seed):
    """Seeded random fused-RoPE calls (head_dim 64 / 128, MHA and GQA, capacities 32 / 64 / 128,
    windows, the gate, per-token, modulo and strided tables; q / k / v column views of one
    projection): each equals, bit for bit, attention over q and k rotated by the oracle and
    uploaded."""
    from oracle import rope

    from packed_encoders_amd.hip_attention import varlen_attention

    c = _draw_rope_case(seed)
    d, hq, hkv, lengths = c["d"], c["hq"], c["hkv"], c["lengths"]
    announce(f"random fused rope {seed}: d={d} heads={hq}/{hkv} n={len(lengths)} max={max(lengths)} "
             f"window={c['window']} gate={c['gate']} tables={c['tables']}")
    T = sum(lengths)
    g = torch.Generator(device="cuda").manual_seed(seed)
    proj = torch.randn(T, (hq + 2 * hkv) * d, device="cuda", generator=g, dtype=torch.bfloat16)
    q = proj[:, : hq * d].view(T, hq, d)
    k = proj[:, hq * d:(hq + hkv) * d].view(T, hkv, d)
    v = proj[:, (hq + hkv) * d:].view(T, hkv, d)
    gt = torch.randn(T, hq, d, device="cuda", generator=g, dtype=torch.bfloat16) if c["gate"] else None
    rows = 53 if c["tables"] == "modulo" else T
    cos, sin = _tables(rows, d, seed=seed + 7)
    if c["tables"] == "strided":
        both = torch.cat([cos, sin], dim=1)
        cos, sin = both[:, :d], both[:, d:]
    cu = torch.tensor([0, *np.cumsum(lengths).tolist()], dtype=torch.int32, device="cuda")
    f = lambda t: t.float().cpu().numpy()
    idx = np.arange(T) % rows
    cr, sr = f(cos)[idx][:, None, :], f(sin)[idx][:, None, :]
    qr = torch.from_numpy(rope.rotate(f(q), cr, sr)).bfloat16().cuda()
    kr = torch.from_numpy(rope.rotate(f(k), cr, sr)).bfloat16().cuda()
    with torch.inference_mode():
        got = varlen_attention(q, k, v, cu, max(lengths), softmax_scale=d ** -0.5, window=c["window"], gate=gt,
                               rope=(cos, sin))
        want = varlen_attention(qr, kr, v.contiguous(), cu, max(lengths), softmax_scale=d ** -0.5,
                                window=c["window"], gate=gt)
    assert torch.isfinite(got).all()
    assert torch.equal(got, want), f"random fused rope case {seed} differs from attention over rotated q, k"
