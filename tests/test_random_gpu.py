"""Seeded random calls over the whole argument space of varlen_attention against the oracle.

The other GPU tests pin each feature on chosen shapes; these cases draw the features together,
as a caller combines them: head_dim 64 / 128 / 256, MHA and GQA, global, +-64, asymmetric and
one-sided windows, causal with and without a left window, the sigmoid gate, separate key
segments (longer, equal or shorter than their queries), empty segments, every routing boundary,
a host lower bound on the lengths, the band kernel forced on or off, logits at 1x, 2x and 4x
N(0,1), and contiguous tensors or strided views into packed projection rows. Each case is a pure function of its seed (numpy's PCG64), so a failure names a
reproducible call. Bar: the reference's tolerances (max-abs 2e-2, per-token cosine 0.9999),
except where 2e-2 is less than the output's own rounding step: an output of magnitude 2 or
more (peaked rows at 2x and 4x logits) has a bf16 step of 2^-6 and above, and a kernel output a
hair from the exact value can round to the other side of a step boundary, which the gate's
second rounding, bf16(bf16(o) * bf16(sigmoid(g))), can widen to 1.5 steps. Such an element must
then equal what one of the two bf16 neighbours of the exact output gives (gated, when the
call has a gate): the output was correctly rounded or off by the one step the boundary allows.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from conftest import announce
from oracle import attention as oa

MAX_ABS = 2e-2
MIN_COS = 0.9999
HEADS = [(4, 4), (8, 2), (6, 3), (8, 8), (4, 1), (12, 12)]
# Seeds [FIRST, FIRST + N_CASES): 96 from 0 by default; PE_RANDOM_FIRST / PE_RANDOM_CASES widen a
# sweep without changing what a default run checks.
FIRST = int(os.environ.get("PE_RANDOM_FIRST", "0"))
N_CASES = int(os.environ.get("PE_RANDOM_CASES", "96"))


def _lengths(rng, kind: str) -> list[int]:
    n = int(rng.integers(1, 20))
    if kind == "short":
        out = rng.integers(0, 65, size=n)
    elif kind == "mixed":
        out = np.where(rng.random(n) < 0.6, rng.integers(0, 129, size=n), rng.integers(129, 701, size=n))
    else:
        out = rng.integers(200, 901, size=max(1, n // 3))
    out = [int(x) for x in out]
    if max(out) == 0:
        out[0] = 1
    return out


def _bf16_neighbours(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """The bf16 values just below and just above |x| in magnitude (both equal to x when x is a
    bf16 value), as float64: the upper 16 bits of x's float32, and the next bf16 away from 0."""
    bits = np.ascontiguousarray(np.asarray(x, dtype=np.float32)).view(np.uint32)
    low = bits & np.uint32(0xFFFF0000)
    high = np.where(low == bits, low, low + np.uint32(0x10000)).astype(np.uint32)
    return low.view(np.float32).astype(np.float64), high.view(np.float32).astype(np.float64)


def test_bf16_neighbours_bracket_the_value():
    x = np.array([1.0, 1.0078125, -2.7, 3.0e-3, 0.0, 65504.0, -1.0e-30, 1.00390625])
    lo, hi = _bf16_neighbours(x)
    assert np.all(np.minimum(np.abs(lo), np.abs(hi)) <= np.abs(x)) and np.all(np.abs(x) <= np.maximum(np.abs(lo), np.abs(hi)))
    assert np.array_equal(oa.to_bf16(lo), lo) and np.array_equal(oa.to_bf16(hi), hi)
    assert np.all((oa.to_bf16(x) == lo) | (oa.to_bf16(x) == hi))  # round to nearest picks one of them
    assert lo[0] == hi[0] == 1.0 and lo[1] == hi[1] == 1.0078125  # bf16 values are their own neighbours
    assert lo[2] == -2.6875 and hi[2] == -2.703125
    assert lo[7] == 1.0 and hi[7] == 1.0078125  # a tie between two bf16 values


def draw_case(seed: int) -> dict:
    """The call of case `seed`: every argument of varlen_attention and the inputs' shapes."""
    rng = np.random.default_rng(seed)
    d = int(rng.choice([64, 64, 64, 128, 256]))
    hq, hkv = HEADS[int(rng.integers(len(HEADS)))]
    if d == 256:
        hq, hkv = min(hq, 8), min(hkv, 8)
        hq -= hq % hkv
    lengths = _lengths(rng, str(rng.choice(["short", "mixed", "long"])))
    causal = bool(rng.random() < 0.3)
    kind = str(rng.choice(["global", "band64", "asym", "one-sided"], p=[0.3, 0.4, 0.15, 0.15]))
    if kind == "global":
        window = (-1, -1)
    elif kind == "band64":
        window = (64, 64)
    elif kind == "asym":
        window = (int(rng.integers(0, 200)), int(rng.integers(0, 200)))
    else:
        window = (int(rng.integers(0, 300)), -1) if rng.random() < 0.5 else (-1, int(rng.integers(0, 300)))
    if causal:
        window = (window[0], -1)
    keys = None
    if rng.random() < 0.2:
        keys = [max(0, n + int(rng.integers(-20, 200))) for n in lengths]
        keys[0] = max(keys[0], 1)
    short_max = [None, 0, 32, 64, 128][int(rng.integers(5))] if d <= 128 else [None, 0][int(rng.integers(2))]
    band_kernel = int(rng.integers(3))  # calls the band kernel cannot serve ignore it
    if seed % 8 == 7:  # every eighth case a shape the streaming band kernel serves
        d, window, causal, keys = 64, (64, 64), False, None
        hq, hkv = [(4, 4), (12, 12), (6, 2)][int(rng.integers(3))]
    return {"seed": seed, "d": d, "hq": hq, "hkv": hkv, "lengths": lengths, "keys": keys,
            "window": window, "causal": causal, "gate": bool(rng.random() < 0.3), "short_max": short_max,
            "band_kernel": band_kernel, "bound": bool(rng.random() < 0.3),
            "logit_scale": float(rng.choice([1.0, 1.0, 2.0, 4.0])),
            "packed": bool(rng.random() < 0.35)}


def _device_inputs(c, q, k, v, gt):
    """The call's device tensors: contiguous copies, or (c["packed"]) strided views into packed
    projection rows, as callers hand them over: per head [q | gate] interleaved when there is
    a gate (packed_encoders/arch/qwen3_5/engine.py:556-558: head stride 2 d), then k and v in
    the same rows (keys shared with the queries) or in packed rows of their own, each row
    padded by 64 elements."""
    if not c["packed"]:
        return [None if t is None else t.cuda() for t in (q, k, v, gt)]
    T, hq, d = q.shape
    Tk, hkv = k.shape[0], k.shape[1]
    qg = torch.stack([q, gt], dim=2).reshape(T, hq * 2 * d) if gt is not None else q.reshape(T, hq * d)
    kv = torch.cat([k.reshape(Tk, hkv * d), v.reshape(Tk, hkv * d)], dim=1)
    if c["keys"] is None:
        rows = torch.cat([qg, kv, torch.zeros(T, 64, dtype=q.dtype)], dim=1).cuda()
        qg_d, kv_d = rows[:, :qg.shape[1]], rows[:, qg.shape[1]:qg.shape[1] + kv.shape[1]]
    else:
        qg_d = torch.cat([qg, torch.zeros(T, 64, dtype=q.dtype)], dim=1).cuda()[:, :qg.shape[1]]
        kv_d = torch.cat([kv, torch.zeros(Tk, 64, dtype=q.dtype)], dim=1).cuda()[:, :kv.shape[1]]
    if gt is not None:
        heads = qg_d.view(T, hq, 2 * d)
        qd, gd = heads[..., :d], heads[..., d:]
    else:
        qd, gd = qg_d.view(T, hq, d), None
    kd = kv_d[:, :hkv * d].view(Tk, hkv, d)
    vd = kv_d[:, hkv * d:].view(Tk, hkv, d)
    return qd, kd, vd, gd


def test_draws_cover_the_argument_space():
    """The drawn cases reach every head dim, window kind, causal, the gate, separate keys, empty
    segments, every routing boundary and the forced band kernel (a CPU check of the generator,
    so the GPU cases below cannot silently narrow)."""
    cases = [draw_case(s) for s in range(N_CASES)]
    assert {c["d"] for c in cases} == {64, 128, 256}
    assert {c["window"] == (-1, -1) for c in cases} == {True, False}
    assert any(c["window"] == (64, 64) for c in cases)
    assert any(c["causal"] for c in cases) and any(c["gate"] for c in cases)
    assert any(c["keys"] is not None for c in cases)
    assert any(0 in c["lengths"] for c in cases)
    assert {c["short_max"] for c in cases} == {None, 0, 32, 64, 128}
    assert any(c["hq"] != c["hkv"] for c in cases)
    band = [c for c in cases if c["d"] == 64 and c["window"] == (64, 64) and not c["causal"]
            and c["keys"] is None and (c["hq"] // c["hkv"]) % 2 == 1]  # shapes the band kernel serves
    assert {c["band_kernel"] for c in band} == {0, 1, 2}
    assert any(c["bound"] for c in cases) and {c["logit_scale"] for c in cases} == {1.0, 2.0, 4.0}
    assert {(c["packed"], c["gate"]) for c in cases} == {(False, False), (False, True), (True, False), (True, True)}
    assert any(c["packed"] and c["keys"] is not None for c in cases)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(FIRST, FIRST + N_CASES))
def test_random_call_matches_oracle(pe, seed):
    c = draw_case(seed)
    announce(f"random case {c}")
    g = torch.Generator().manual_seed(1000 + seed)
    lengths, keys = c["lengths"], c["keys"] if c["keys"] is not None else c["lengths"]
    T, Tk = sum(lengths), sum(keys)
    q = (torch.randn(T, c["hq"], c["d"], generator=g) * c["logit_scale"]).bfloat16()
    k = (torch.randn(Tk, c["hkv"], c["d"], generator=g) * c["logit_scale"]).bfloat16()
    v = torch.randn(Tk, c["hkv"], c["d"], generator=g).bfloat16()
    gt = torch.randn(T, c["hq"], c["d"], generator=g).bfloat16() if c["gate"] else None
    cu = torch.tensor([0, *np.cumsum(lengths).tolist()], dtype=torch.int32)
    cuk = torch.tensor([0, *np.cumsum(keys).tolist()], dtype=torch.int32) if c["keys"] is not None else None
    scale = c["d"] ** -0.5
    qd, kd, vd, gd = _device_inputs(c, q, k, v, gt)
    if c["packed"]:
        assert not qd.is_contiguous() and not kd.is_contiguous()
    with torch.inference_mode():
        got = pe.varlen_attention(
            qd, kd, vd, cu.cuda(), max(lengths), softmax_scale=scale, window=c["window"],
            causal=c["causal"], gate=gd, short_max=c["short_max"],
            cu_seqlens_k=None if cuk is None else cuk.cuda(), max_seqlen_k=max(keys) if cuk is not None else None,
            band_kernel=c["band_kernel"], min_seqlen=min(lengths) if c["bound"] else None)
    f = lambda t: t.float().numpy()
    exact = oa.packed_attention(f(q), f(k), f(v), cu.numpy(), scale=scale, window=c["window"], causal=c["causal"],
                                cu_seqlens_k=None if cuk is None else cuk.numpy())[:T]
    want = exact if gt is None else oa.sigmoid_gate(oa.to_bf16(exact), f(gt))
    got = got.float().cpu().numpy().astype(np.float64)[:T]
    assert np.isfinite(got).all()
    err = np.abs(got - want)
    over = err > MAX_ABS
    if over.any():
        down, up = _bf16_neighbours(exact[over])
        if gt is not None:
            down, up = (oa.sigmoid_gate(x, f(gt)[over]) for x in (down, up))
        stray = (got[over] != down) & (got[over] != up)
        assert not stray.any(), (f"case {seed}: {int(stray.sum())} of {int(over.sum())} elements past {MAX_ABS} are not "
                                 f"a rounding of the exact output's bf16 neighbours; max abs {err.max():.4g}")
    zero = ~np.any(want.reshape(T, -1), axis=1)  # rows that reach no key
    assert not np.any(got.reshape(T, -1)[zero]), f"case {seed}: rows that reach no key must be zero"
    cos = oa.cosine_per_token(got[~zero], want[~zero])
    assert cos.size == 0 or cos.min() >= MIN_COS, f"case {seed}: min cosine {cos.min():.6f}"
