"""GPU parity and invariants of the streaming band kernel (band64_attn_kernel), forced with
``band_kernel=1`` at sizes the library would otherwise give the tiled kernel.

It serves head_dim 64 windows whose rows each span five 32-key blocks, one query head per kv
head group: left and right bounds whose block counts ceil(left / 32) + ceil(right / 32) sum to
four — (33..64, 33..64) such as ModernBERT's +-64, (1..32, 65..96), (65..96, 1..32),
(0, 97..128), (97..128, 0), and causal with a left window of 97..128 (causal is a right bound
of 0). Checked: the oracle on segment lengths straddling every block and tile edge for the
extreme shapes of every such class, MHA and GQA 3:1, the fused gate, strips of 1..8 tiles
bit-identical to each other, a stale running maximum past the overflow guard, zero
cross-segment leakage and independence from batch composition (bit for bit), agreement with
the tiled kernel within the bf16 tolerance, and a segment whose kernel changes with the size
of the call it is packed in (the library's size rule) within the same tolerance.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce
from test_hip_attention import WINDOW_LENGTHS, _assert_parity, _dev, _inputs, _oracle

pytestmark = pytest.mark.gpu

BAND_WINDOWS = [(64, 64), (33, 33), (40, 60), (64, 33)]
# The extreme (left, right) of every block-count class the band kernel admits besides
# (33..64, 33..64), and causal with a left window (window, causal).
CLASS_EXTREMES = [((0, 97), False), ((0, 128), False), ((97, 0), False), ((128, 0), False),
                  ((1, 65), False), ((1, 96), False), ((32, 65), False), ((32, 96), False),
                  ((65, 1), False), ((65, 32), False), ((96, 1), False), ((96, 32), False),
                  ((33, 64), False), ((97, -1), True), ((128, -1), True)]


def _kernel_of(q, k, cu, max_seqlen, window, band_kernel, causal=False):
    import ctypes

    from packed_encoders_amd import _lib, hip_attention as hip

    out = torch.empty_like(q)
    a = hip._args(q, k, k, out, cu, max_seqlen, 0.125, window[0], window[1], causal, None, 0,
                  band_kernel=band_kernel)
    res = (ctypes.c_int32 * 6)()
    assert _lib.library().pe_attn_kernels(ctypes.byref(a), res) == 0
    return res[1], res[2]


def _run(pe, q, k, v, cu, mx, window, band_kernel=1, gate=None, strip=None, causal=False):
    if strip is None:
        with torch.inference_mode():
            return pe.varlen_attention(q, k, v, cu, mx, softmax_scale=0.125, window=window, short_max=0,
                                       gate=gate, band_kernel=band_kernel, causal=causal)
    import ctypes

    from packed_encoders_amd import _lib, hip_attention as hip

    lib = _lib.library()
    out = torch.empty_like(q)
    a = hip._args(q, k, v, out, cu, mx, 0.125, window[0], window[1], causal, gate, 0, strip=strip,
                  band_kernel=band_kernel)
    size = ctypes.c_size_t()
    assert lib.pe_attn_workspace_size(ctypes.byref(a), ctypes.byref(size)) == 0
    ws = torch.empty(max(size.value, 1), dtype=torch.uint8, device="cuda")
    assert lib.pe_varlen_attn_fwd(ctypes.byref(a), ws.data_ptr(), size.value,
                                  torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("hq,hkv", [(4, 4), (6, 2)], ids=["mha", "gqa3"])
@pytest.mark.parametrize("window", BAND_WINDOWS, ids=[f"{w[0]}_{w[1]}" for w in BAND_WINDOWS])
def test_band_kernel_matches_oracle_and_strips_agree(pe, window, hq, hkv):
    from packed_encoders_amd import _lib

    announce(f"band kernel window={window} heads={hq}/{hkv}")
    q, k, v, cu, _ = _inputs(WINDOW_LENGTHS, hq=hq, hkv=hkv, seed=61)
    qd, kd, vd, cud = _dev(q, k, v, cu)
    mx = max(WINDOW_LENGTHS)
    assert _kernel_of(qd, kd, cud, mx, window, 1)[0] == _lib.KERNEL_BAND64
    got = _run(pe, qd, kd, vd, cud, mx, window)
    torch.cuda.synchronize()
    want = _oracle(q, k, v, cu, scale=0.125, window=window)
    _assert_parity(got, want, cu)
    for strip in (1, 2, 3, 8):
        assert torch.equal(_run(pe, qd, kd, vd, cud, mx, window, strip=strip), got), strip


@pytest.mark.parametrize("window,causal", CLASS_EXTREMES,
                         ids=[f"{w[0]}_{w[1]}{'c' if c else ''}" for w, c in CLASS_EXTREMES])
def test_band_kernel_every_admitted_window_class(pe, window, causal):
    """Every window shape the band kernel accepts, at the extremes of its block-count class,
    forced onto the band kernel: the oracle, and strips of 1 and 3 tiles bit-identical."""
    from packed_encoders_amd import _lib

    announce(f"band kernel window class {window} causal={causal}")
    q, k, v, cu, _ = _inputs(WINDOW_LENGTHS, hq=4, seed=67)
    qd, kd, vd, cud = _dev(q, k, v, cu)
    mx = max(WINDOW_LENGTHS)
    assert _kernel_of(qd, kd, cud, mx, window, 1, causal)[0] == _lib.KERNEL_BAND64
    got = _run(pe, qd, kd, vd, cud, mx, window, causal=causal)
    torch.cuda.synchronize()
    want = _oracle(q, k, v, cu, scale=0.125, window=window, causal=causal)
    _assert_parity(got, want, cu)
    for strip in (1, 3):
        assert torch.equal(_run(pe, qd, kd, vd, cud, mx, window, strip=strip, causal=causal), got), strip


def test_segment_across_the_size_rule(pe):
    """A +-64 segment alone (a small call: the tiled kernel) and the same segment packed into a
    call of at least 17,667 query tiles (the band kernel) agree within the parity bar, not bit
    for bit: besides the short-kernel boundary, the library's size rule is the one way a
    segment's bits depend on its batch."""
    from packed_encoders_amd import _lib

    announce("segment alone (tiled) vs in a large call (band)")
    lengths = [1000] + [8192] * 24  # 18,432 query tiles at 12 heads
    q, k, v, cu, _ = _inputs(lengths, hq=12, seed=68)
    qd, kd, vd, cud = _dev(q, k, v, cu)
    mx = max(lengths)
    assert _kernel_of(qd, kd, cud, mx, (64, 64), 0)[0] == _lib.KERNEL_BAND64
    big = _run(pe, qd, kd, vd, cud, mx, (64, 64), band_kernel=0)
    one = torch.tensor([0, 1000], dtype=torch.int32, device="cuda")
    assert _kernel_of(qd[:1000], kd[:1000], one, 1000, (64, 64), 0)[0] == _lib.KERNEL_TILED
    alone = _run(pe, qd[:1000].contiguous(), kd[:1000].contiguous(), vd[:1000].contiguous(), one, 1000, (64, 64),
                 band_kernel=0)
    torch.cuda.synchronize()
    want = _oracle(q[:1000], k[:1000], v[:1000], cu[:2], scale=0.125, window=(64, 64))
    _assert_parity(alone, want, cu[:2])
    _assert_parity(big[:1000], want, cu[:2])
    assert (alone.float() - big[:1000].float()).abs().max().item() <= 2e-2


def test_band_kernel_gate_and_agreement_with_tiled(pe):
    from packed_encoders_amd import _lib

    lengths = [2000, 129, 1, 640, 3000, 77]
    announce("band kernel gate vs tiled")
    q, k, v, cu, gt = _inputs(lengths, hq=12, seed=62, gate=True)
    qd, kd, vd, cud, gd = _dev(q, k, v, cu, gt)
    mx = max(lengths)
    assert _kernel_of(qd, kd, cud, mx, (64, 64), 2)[0] == _lib.KERNEL_TILED
    band = _run(pe, qd, kd, vd, cud, mx, (64, 64), gate=gd)
    tiled = _run(pe, qd, kd, vd, cud, mx, (64, 64), band_kernel=2, gate=gd)
    torch.cuda.synchronize()
    want = _oracle(q, k, v, cu, scale=0.125, window=(64, 64), gate=gt)
    _assert_parity(band, want, cu)
    _assert_parity(tiled, want, cu)
    assert (band.float() - tiled.float()).abs().max().item() <= 2e-2


@pytest.mark.parametrize("jump", [4.0, 10.0], ids=["below-guard", "past-guard"])
def test_band_kernel_scores_jumping_past_a_stale_maximum(pe, jump):
    lengths = [700, 300, 129]
    announce(f"band kernel score jump={jump}")
    q, k, v, cu, _ = _inputs(lengths, hq=4, seed=63)
    q = q.float().abs().bfloat16()
    k = k.float()
    for a in (0, 700):
        k[a + 200:a + 264] = jump
    k = k.bfloat16()
    qd, kd, vd, cud = _dev(q, k, v, cu)
    got = _run(pe, qd, kd, vd, cud, max(lengths), (64, 64))
    torch.cuda.synchronize()
    want = _oracle(q, k, v, cu, scale=0.125, window=(64, 64))
    _assert_parity(got, want, cu)


def test_band_kernel_no_leakage_and_batch_independence(pe):
    """Scaling one segment's q/k/v leaves every other segment's bits unchanged; each segment run
    alone (the band kernel pinned) gives the bits it has inside the batch."""
    lengths = [300, 1, 257, 1024, 96, 513]
    announce("band kernel leakage / independence")
    q, k, v, cu, gt = _inputs(lengths, hq=6, hkv=2, seed=64, gate=True)
    qd, kd, vd, cud, gd = _dev(q, k, v, cu, gt)
    mx = max(lengths)
    base = _run(pe, qd, kd, vd, cud, mx, (64, 64), gate=gd)
    c = cu.tolist()
    s = 3
    q2, k2, v2, g2 = qd.clone(), kd.clone(), vd.clone(), gd.clone()
    q2[c[s]:c[s + 1]] *= 7
    k2[c[s]:c[s + 1]] *= 100
    v2[c[s]:c[s + 1]] *= -100
    g2[c[s]:c[s + 1]] *= -3
    changed = _run(pe, q2, k2, v2, cud, mx, (64, 64), gate=g2)
    torch.cuda.synchronize()
    assert torch.isfinite(base).all()
    assert torch.equal(base[:c[s]], changed[:c[s]]) and torch.equal(base[c[s + 1]:], changed[c[s + 1]:])
    assert not torch.equal(base[c[s]:c[s + 1]], changed[c[s]:c[s + 1]])
    for i, (a, b) in enumerate(zip(c, c[1:])):
        cu1 = torch.tensor([0, b - a], dtype=torch.int32, device="cuda")
        alone = _run(pe, qd[a:b].contiguous(), kd[a:b].contiguous(), vd[a:b].contiguous(), cu1, b - a, (64, 64),
                     gate=gd[a:b].contiguous())
        torch.cuda.synchronize()
        assert torch.equal(alone, base[a:b]), f"segment {i} ({b - a} rows) differs alone"


def test_library_choice_by_call_size(pe):
    """band_kernel=0 keeps the tiled kernel on a small call and takes the band kernel (strip 8)
    on a large one; the large call matches the oracle on sampled rows."""
    from oracle import attention as oa
    from packed_encoders_amd import _lib

    announce("band kernel size rule")
    small = [512] * 8
    q, k, v, cu, _ = _inputs(small, hq=12, seed=65)
    qd, kd, vd, cud = _dev(q, k, v, cu)
    assert _kernel_of(qd, kd, cud, 512, (64, 64), 0)[0] == _lib.KERNEL_TILED
    big = [8192] * 24  # 1,536 query tiles x 12 heads = 18,432
    q, k, v, cu, _ = _inputs(big, hq=12, seed=66)
    qd, kd, vd, cud = _dev(q, k, v, cu)
    assert _kernel_of(qd, kd, cud, 8192, (64, 64), 0) == (_lib.KERNEL_BAND64, 8)
    got = _run(pe, qd, kd, vd, cud, 8192, (64, 64), band_kernel=0)
    torch.cuda.synchronize()
    rows = np.linspace(0, sum(big) - 1, 96).astype(np.int64)
    f = lambda t: t.float().numpy()
    want = oa.sampled_rows_attention(f(q), f(k), f(v), cu.numpy(), rows, scale=0.125, window=(64, 64), causal=False)
    err = np.abs(got.float().cpu().numpy()[rows] - want).max()
    assert err <= 2e-2, err
