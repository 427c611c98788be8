"""GPU parity of the HIP packed attention kernels against the CPU oracle (oracle/attention.py).

Bar (the reference's tolerances): max-abs <= 2e-2 (runtime/attention.py:40), per-token cosine
>= 0.9999, mean-abs close to what bf16 inputs and outputs allow, and bit-exact invariants:
zero cross-segment leakage, determinism, independence from batch composition
(tests/test_packed_short_attention.py:97-147 and tests/test_cpu_short_attention.py:72-77).
Inputs are drawn in fp32 on the CPU, rounded to bf16 for the GPU; the oracle reads the same
bf16 values in float64.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from conftest import announce
from oracle import attention as oa

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MIN_COS = 0.9999


def _inputs(lengths, hq=12, hkv=None, d=64, seed=0, logit_scale=1.0, gate=False):
    hkv = hq if hkv is None else hkv
    g = torch.Generator().manual_seed(seed)
    T = sum(lengths)
    q = (torch.randn(T, hq, d, generator=g) * logit_scale).bfloat16()
    k = (torch.randn(T, hkv, d, generator=g) * logit_scale).bfloat16()
    v = torch.randn(T, hkv, d, generator=g).bfloat16()
    gt = torch.randn(T, hq, d, generator=g).bfloat16() if gate else None
    cu = torch.tensor([0, *np.cumsum(lengths).tolist()], dtype=torch.int32)
    return q, k, v, cu, gt


def _dev(*ts):
    return [None if t is None else t.cuda() for t in ts]


def _oracle(q, k, v, cu, *, scale, window=(-1, -1), causal=False, gate=None):
    f = lambda t: t.float().numpy()
    return oa.packed_attention(f(q), f(k), f(v), cu.numpy(), scale=scale, window=window, causal=causal,
                               gate=None if gate is None else f(gate))


def _assert_parity(got, want, cu, *, max_abs=MAX_ABS, min_cos=MIN_COS):
    got = got.float().cpu().numpy().astype(np.float64)
    live = np.zeros(got.shape[0], dtype=bool)
    c = cu.tolist()
    for a, b in zip(c, c[1:]):
        live[a:b] = True
    g, w = got[live], want[live]
    assert np.isfinite(g).all()
    err = np.abs(g - w)
    assert err.max() <= max_abs, f"max abs {err.max():.4g}"
    # rows that reach no key (separate key segments) are exactly zero in both; cosine elsewhere
    zero = ~np.any(w.reshape(w.shape[0], -1), axis=1)
    assert not np.any(g.reshape(g.shape[0], -1)[zero]), "rows that reach no key must be zero"
    cos = oa.cosine_per_token(g[~zero], w[~zero])
    assert cos.size == 0 or cos.min() >= min_cos, f"min cosine {cos.min():.6f}"
    return float(err.max()), float(err.mean())


SHORT_LENGTHS = [
    [1, 2, 31, 32, 33, 63, 64, 65, 127, 128],
    [128] * 8,
    [128, 64, 16, 16, 16, 16, 16, 16],
    [46, 46, 45, 45, 45, 44, 43, 42],
]


@pytest.mark.parametrize("half_window", [None, 64])
@pytest.mark.parametrize("lengths", SHORT_LENGTHS, ids=["ragged", "128x8", "mixed", "agentir"])
def test_packed_short_attention_matches_oracle(pe, lengths, half_window):
    announce(f"packed_short lengths={lengths[:4]} half={half_window}")
    q, k, v, cu, _ = _inputs(lengths, seed=17)
    qd, kd, vd, cud = _dev(q, k, v, cu)
    with torch.inference_mode():
        got = pe.packed_short_attention(qd, kd, vd, cud, max(lengths), half_window=half_window,
                                        softmax_scale=0.125)
    window = (-1, -1) if half_window is None else (half_window, half_window)
    want = _oracle(q, k, v, cu, scale=0.125, window=window)
    _, mean = _assert_parity(got, want, cu)
    # bf16 output rounding alone gives ~1e-3 mean error on these magnitudes
    assert mean < 4e-3


SHORT_HEADS = [(64, 12, 32, 1), (64, 12, 400, 2), (64, 12, 700, 4), (128, 6, 40, 1), (128, 6, 700, 2)]


@pytest.mark.parametrize("d,hq,n_seq,heads", SHORT_HEADS, ids=[f"d{c[0]}_{c[2]}seg" for c in SHORT_HEADS])
def test_short_kernel_heads_per_workgroup(pe, d, hq, n_seq, heads):
    """A small batch runs the short kernel with fewer query heads per workgroup (the library
    reports the choice, pe_attn_kernels out[4]): every choice matches the oracle with the gate
    and a +-16 window over lengths 1..64, and the first 32 segments run alone (one head per
    workgroup) are bit-identical to the same segments inside the larger batch."""
    from packed_encoders_amd import _lib
    from packed_encoders_amd.hip_attention import _args

    announce(f"short kernel d={d} hq={hq} n_seq={n_seq} heads={heads}")
    rng = np.random.default_rng(n_seq + d)
    lengths = rng.integers(1, 65, size=n_seq).tolist()
    q, k, v, cu, gt = _inputs(lengths, hq=hq, d=d, seed=n_seq, gate=True)
    qd, kd, vd, cud, gd = _dev(q, k, v, cu, gt)
    lib = _lib.library()
    out = (ctypes.c_int32 * 6)()
    a = _args(qd, kd, vd, qd, cud, 64, 0.125, 16, 16, False, gd, 64, 0)
    assert lib.pe_attn_kernels(ctypes.byref(a), out) == 0
    assert (out[0], out[1], out[4], out[5]) == (64, _lib.KERNEL_NONE, heads, n_seq * -(-hq // heads))
    got = _launch(lib, qd, kd, vd, cud, 64, (16, 16), False, gate=gd, short_max=64)
    want = _oracle(q, k, v, cu, scale=0.125, window=(16, 16), gate=gt)
    _assert_parity(got, want, cu)
    t32 = int(cu[32])
    alone = _launch(lib, qd[:t32], kd[:t32], vd[:t32], cud[:33], 64, (16, 16), False, gate=gd[:t32], short_max=64)
    assert torch.equal(alone, got[:t32])


LONG_CASES = [
    ([1, 300, 1000, 129, 2048, 64, 7], (-1, -1), False),
    ([1, 300, 1000, 129, 2048, 64, 7], (64, 64), False),
    ([1, 300, 1000, 129, 513, 64, 7], (-1, -1), True),
    ([700, 33, 0, 250], (10, 3), False),
    ([4096], (-1, -1), False),
]


@pytest.mark.parametrize("short_max", [0, 64, 128])
@pytest.mark.parametrize("lengths,window,causal", LONG_CASES, ids=["global", "band64", "causal", "asym", "4k"])
def test_varlen_attention_matches_oracle(pe, lengths, window, causal, short_max):
    announce(f"varlen lengths={lengths} window={window} causal={causal} short_max={short_max}")
    q, k, v, cu, _ = _inputs(lengths, hq=4, seed=3)
    qd, kd, vd, cud = _dev(q, k, v, cu)
    with torch.inference_mode():
        got = pe.varlen_attention(qd, kd, vd, cud, max(lengths), softmax_scale=0.125, window=window,
                                  causal=causal, short_max=short_max)
    want = _oracle(q, k, v, cu, scale=0.125, window=window, causal=causal)
    _assert_parity(got, want, cu)


@pytest.mark.parametrize("d,hq,hkv", [(64, 8, 2), (128, 6, 3), (128, 4, 4), (256, 8, 2), (256, 8, 1), (64, 16, 2),
                                      (256, 4, 4), (256, 6, 3)])
@pytest.mark.parametrize("causal", [False, True])
def test_gqa_head_dims(pe, d, hq, hkv, causal):
    lengths = [16, 200, 5, 77, 512]
    announce(f"gqa d={d} hq={hq} hkv={hkv} causal={causal}")
    q, k, v, cu, _ = _inputs(lengths, hq=hq, hkv=hkv, d=d, seed=11)
    qd, kd, vd, cud = _dev(q, k, v, cu)
    with torch.inference_mode():
        got = pe.varlen_attention(qd, kd, vd, cud, max(lengths), causal=causal)
    want = _oracle(q, k, v, cu, scale=d ** -0.5, causal=causal)
    _assert_parity(got, want, cu)


# Segments of more than 128 tokens whose last query tile holds rows for at most half of a
# head's waves (1..128 rows past a multiple of 256 with one query head per workgroup, 1..64
# past a multiple of 128 with two): the global kernel splits such a tile's key blocks between
# two waves and merges their maxima, sums and accumulators. 257 and 321 leave the second wave
# no key in the last key tile, 300 a masked partial block; the segments of at most 128 tokens
# do not split.
SPLIT_LENGTHS = [1, 20, 33, 64, 100, 128, 129, 160, 200, 257, 300, 321, 384, 385, 640, 700]


@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 4), (8, 2)], ids=["mha", "gqa2", "gqa4"])
@pytest.mark.parametrize("gate", [False, True], ids=["plain", "gate"])
def test_split_query_tiles_match_oracle(pe, hq, hkv, gate):
    announce(f"split query tiles hq={hq} hkv={hkv} gate={gate}")
    q, k, v, cu, gt = _inputs(SPLIT_LENGTHS, hq=hq, hkv=hkv, seed=53, gate=gate)
    qd, kd, vd, cud, gd = _dev(q, k, v, cu, gt)
    with torch.inference_mode():
        got = pe.varlen_attention(qd, kd, vd, cud, max(SPLIT_LENGTHS), softmax_scale=0.125, gate=gd, short_max=0)
        alone = [pe.varlen_attention(qd[a:b], kd[a:b], vd[a:b], cud.new_tensor([0, b - a]), b - a,
                                     softmax_scale=0.125, gate=None if gd is None else gd[a:b], short_max=0)
                 for a, b in zip(cu.tolist(), cu.tolist()[1:])]
    _assert_parity(got, _oracle(q, k, v, cu, scale=0.125, gate=gt), cu)
    # a tile splits by its segment's length alone: each segment's bits are its own
    assert torch.equal(got, torch.cat(alone))


@pytest.mark.parametrize("d,short_max", [(256, 0), (64, 64), (128, 32)])
def test_fused_sigmoid_gate(pe, d, short_max):
    lengths = [16, 300, 40, 129]
    announce(f"gate d={d}")
    q, k, v, cu, g = _inputs(lengths, hq=8, hkv=2, d=d, seed=13, gate=True)
    qd, kd, vd, cud, gd = _dev(q, k, v, cu, g)
    with torch.inference_mode():
        got = pe.varlen_attention(qd, kd, vd, cud, max(lengths), causal=True, gate=gd, short_max=short_max)
    want = _oracle(q, k, v, cu, scale=d ** -0.5, causal=True, gate=g)
    _assert_parity(got, want, cu)


@pytest.mark.parametrize("logit_scale", [0.01, 1.0, 8.0])
@pytest.mark.parametrize("short_max", [0, 128])
def test_softmax_stability_and_determinism(pe, logit_scale, short_max):
    lengths = [33, 65, 127]
    announce(f"stability scale={logit_scale} short_max={short_max}")
    q, k, v, cu, _ = _inputs(lengths, seed=11, logit_scale=logit_scale)
    qd, kd, vd, cud = _dev(q, k, v, cu)
    with torch.inference_mode():
        first = pe.varlen_attention(qd, kd, vd, cud, 127, softmax_scale=0.125, window=(64, 64), short_max=short_max)
        second = pe.varlen_attention(qd, kd, vd, cud, 127, softmax_scale=0.125, window=(64, 64), short_max=short_max)
    assert torch.isfinite(first).all()
    assert torch.equal(first, second)


LARGE_LOGIT_LONG = [700, 300, 129, 65, 40, 16]
LARGE_LOGIT_CASES = {
    # id: (lengths, head_dim, kv heads, window, causal, short_max, band_kernel)
    "global": (LARGE_LOGIT_LONG, 64, 4, (-1, -1), False, 0, 0),
    "global-short": (LARGE_LOGIT_LONG, 64, 4, (-1, -1), False, 128, 0),
    "band64": (LARGE_LOGIT_LONG, 64, 4, (64, 64), False, 0, 0),
    "band64-stream": (LARGE_LOGIT_LONG, 64, 4, (64, 64), False, 0, 1),
    "causal": (LARGE_LOGIT_LONG, 64, 4, (-1, -1), True, 0, 0),
    "d128": (LARGE_LOGIT_LONG, 128, 4, (-1, -1), False, 0, 0),
    "d256-causal": (LARGE_LOGIT_LONG, 256, 2, (-1, -1), True, 0, 0),
    # 2,080 segments of 1..64 tokens: the short kernel with four heads per workgroup (it keeps
    # four while segments x head groups fill eight workgroups per CU)
    "short-4heads": ([1 + (7 * i) % 64 for i in range(2080)], 64, 4, (-1, -1), False, 64, 0),
}


@pytest.mark.parametrize("logit_scale", [2.0, 4.0])
@pytest.mark.parametrize("case", list(LARGE_LOGIT_CASES))
def test_large_logits_match_oracle(pe, logit_scale, case):
    """Q and K drawn at 2x and 4x N(0,1): logits of about 10 and 40 natural units, rows whose
    near-tied top scores magnify any rounding of the scores themselves. Every kernel scales
    the fp32 Q.K product, as the reference does (triton_packed_attention.py:114), which keeps
    them inside the parity bar; a query operand rounded to bf16 after multiplying by the scale
    does not: a build of the global kernel that did so failed the two global cases here with
    max-abs 0.029 (2x) and 0.114 (4x), while passing every N(0,1) test."""
    lengths, d, hkv, window, causal, short_max, band_kernel = LARGE_LOGIT_CASES[case]
    announce(f"large logits x{logit_scale} {case}")
    q, k, v, cu, _ = _inputs(lengths, hq=4, hkv=hkv, d=d, seed=29, logit_scale=logit_scale)
    qd, kd, vd, cud = _dev(q, k, v, cu)
    with torch.inference_mode():
        got = pe.varlen_attention(qd, kd, vd, cud, max(lengths), softmax_scale=d ** -0.5, window=window,
                                  causal=causal, short_max=short_max, band_kernel=band_kernel)
    want = _oracle(q, k, v, cu, scale=d ** -0.5, window=window, causal=causal)
    _assert_parity(got, want, cu)


@pytest.mark.parametrize("short_max", [0, 128])
def test_no_cross_sequence_leakage(pe, short_max):
    lengths = [31, 65, 300]
    announce(f"leakage short_max={short_max}")
    q, k, v, cu, _ = _inputs(lengths, seed=7)
    qd, kd, vd, cud = _dev(q, k, v, cu)
    with torch.inference_mode():
        base = pe.varlen_attention(qd, kd, vd, cud, 300, softmax_scale=0.125, short_max=short_max)
        k2, v2 = kd.clone(), vd.clone()
        k2[31:96] *= 100
        v2[31:96] *= -100
        changed = pe.varlen_attention(qd, k2, v2, cud, 300, softmax_scale=0.125, short_max=short_max)
    assert torch.equal(base[:31], changed[:31])
    assert torch.equal(base[96:], changed[96:])


def test_segment_alone_equals_segment_in_batch(pe):
    lengths = [50, 700, 20]
    announce("batch independence")
    q, k, v, cu, _ = _inputs(lengths, seed=9)
    qd, kd, vd, cud = _dev(q, k, v, cu)
    with torch.inference_mode():
        batch = pe.varlen_attention(qd, kd, vd, cud, 700, window=(64, 64), short_max=64)
        for a, b in ((0, 50), (50, 750), (750, 770)):
            one = torch.tensor([0, b - a], dtype=torch.int32, device="cuda")
            alone = pe.varlen_attention(qd[a:b].contiguous(), kd[a:b].contiguous(), vd[a:b].contiguous(), one, b - a,
                                        window=(64, 64), short_max=64)
            assert torch.equal(alone, batch[a:b])


def test_strided_v_view_of_packed_qkv(pe):
    # v as the reference passes it: a view into qkv [T, 3*H*D] (token stride 3*H*D)
    lengths = [40, 200]
    T, h, d = sum(lengths), 12, 64
    announce("strided v")
    g = torch.Generator().manual_seed(21)
    qkv = torch.randn(T, 3 * h * d, generator=g).bfloat16()
    cu = torch.tensor([0, 40, 240], dtype=torch.int32)
    q = qkv.view(T, 3, h, d)[:, 0].contiguous()
    k = qkv.view(T, 3, h, d)[:, 1].contiguous()
    qkvd = qkv.cuda()
    v_view = qkvd.view(T, 3, h, d)[:, 2]
    assert v_view.stride(0) == 3 * h * d
    with torch.inference_mode():
        got = pe.varlen_attention(q.cuda(), k.cuda(), v_view, cu.cuda(), 200, softmax_scale=0.125)
    want = _oracle(q, k, qkv.view(T, 3, h, d)[:, 2], cu, scale=0.125)
    _assert_parity(got, want, cu)


def test_rows_beyond_last_boundary_and_empty_segments_untouched(pe):
    from packed_encoders_amd import _lib
    from packed_encoders_amd.hip_attention import _args

    lengths = [0, 20, 0, 130, 0]
    T = sum(lengths) + 24  # 24 padding rows beyond cu[-1]
    announce("untouched rows")
    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(T, 4, 64, generator=g).bfloat16().cuda() for _ in range(3))
    cu = torch.tensor([0, *np.cumsum(lengths).tolist()], dtype=torch.int32, device="cuda")
    out = torch.full((T, 4, 64), 7.0, dtype=torch.bfloat16, device="cuda")
    lib = _lib.library()
    for short_max in (0, 64):
        a = _args(q, k, v, out, cu, 130, 0.125, -1, -1, False, None, short_max)
        size = ctypes.c_size_t()
        assert lib.pe_attn_workspace_size(ctypes.byref(a), ctypes.byref(size)) == 0
        ws = torch.empty(max(size.value, 1), dtype=torch.uint8, device="cuda")
        rc = lib.pe_varlen_attn_fwd(ctypes.byref(a), ws.data_ptr(), size.value, torch.cuda.current_stream().cuda_stream)
        assert rc == 0
        torch.cuda.synchronize()
        assert torch.all(out[150:] == 7.0)
        want = _oracle(q.cpu(), k.cpu(), v.cpu(), cu.cpu(), scale=0.125)
        _assert_parity(out, want, cu.cpu())


@pytest.mark.parametrize("lengths,max_seqlen,skipped", [([100, 300, 150], 200, (100, 400)),
                                                         ([300, 129, 129], 200, (0, 300))],
                         ids=["middle", "evicts"])
@pytest.mark.parametrize("d", [64, 128, 256])
def test_segment_longer_than_max_seqlen_is_skipped(pe, d, lengths, max_seqlen, skipped):
    """max_seqlen sizes the kernels' 32-bit offsets and the plan's list; a segment longer than
    the caller's bound breaches that contract and is left unwritten instead of being
    addressed, while the other segments of the call are computed as usual. In the "evicts"
    case the list is sized from max_seqlen (for head_dim 128: 6 entries of 128-row tiles, for
    head_dim 64's 256-row tiles: 3) and the over-long segment's tiles alone would fill it: it
    must take none, so no tile of a valid segment is dropped."""
    from packed_encoders_amd import _lib

    announce(f"segment longer than max_seqlen d={d} lengths={lengths}")
    q, k, v, cu, _ = _inputs(lengths, hq=4, hkv=1 if d == 256 else 4, d=d, seed=61)
    qd, kd, vd, cud = _dev(q, k, v, cu)
    out = _launch(_lib.library(), qd, kd, vd, cud, max_seqlen, (-1, -1), False)
    a, b = skipped
    assert torch.all(out[a:b] == 3.0)
    want = _oracle(q, k, v, cu, scale=0.125)
    keep = torch.ones(sum(lengths), dtype=torch.bool)
    keep[a:b] = False
    idx = keep.nonzero().flatten()
    got = out.float().cpu()[idx]
    kept = [n for n in lengths if n <= max_seqlen]
    sub_cu = torch.tensor([0, *np.cumsum(kept).tolist()], dtype=torch.int32)
    _assert_parity(got, want[idx.numpy()], sub_cu)


def test_plan_reports_entries_written_and_needed(pe):
    """The plan's header holds the entries it wrote and the entries it needed; with arguments
    inside the contract (here an over-long segment that takes no entry) the two are equal."""
    from packed_encoders_amd import _lib
    from packed_encoders_amd.hip_attention import _args

    announce("plan header counts")
    lengths = [300, 129, 129, 40]
    q, k, v, cu, _ = _inputs(lengths, hq=4, d=64, seed=62)
    qd, kd, vd, cud = _dev(q, k, v, cu)
    out = torch.empty_like(qd)
    a = _args(qd, kd, vd, out, cud, 200, 0.125, -1, -1, False, None, 64)
    lib = _lib.library()
    size = ctypes.c_size_t()
    assert lib.pe_attn_workspace_size(ctypes.byref(a), ctypes.byref(size)) == 0
    ws = torch.zeros(size.value, dtype=torch.uint8, device="cuda")
    assert lib.pe_attn_plan(ctypes.byref(a), ws.data_ptr(), size.value, torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    written, needed = ws[:8].view(torch.int32).tolist()
    assert written == needed == 2  # two 129-row segments of one 256-row tile; 300 and 40 take none


def test_workspace_too_small_is_reported(pe):
    from packed_encoders_amd import _lib
    from packed_encoders_amd.hip_attention import _args

    q = torch.zeros(300, 2, 64, dtype=torch.bfloat16, device="cuda")
    cu = torch.tensor([0, 300], dtype=torch.int32, device="cuda")
    a = _args(q, q, q, q.clone(), cu, 300, 0.125, -1, -1, False, None, 0)
    ws = torch.empty(16, dtype=torch.uint8, device="cuda")
    assert _lib.library().pe_varlen_attn_fwd(ctypes.byref(a), ws.data_ptr(), 16, None) == -3


def test_out_of_envelope_raises_value_error(pe):
    q, k, v, cu, _ = _dev(*_inputs([32, 17], seed=1))
    with torch.inference_mode():
        assert pe.packed_short_attention_supported(q, k, v, cu, 32, half_window=None)
        assert not pe.packed_short_attention_supported(q, k, v, cu, 129, half_window=None)
        with pytest.raises(ValueError):
            pe.packed_short_attention(q, k, v, cu, 129, half_window=None, softmax_scale=0.125)
        with pytest.raises(ValueError):
            pe.varlen_attention(q.float(), k, v, cu, 32)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("window,causal", [((-1, -1), False), ((64, 64), False), ((-1, -1), True), ((5, 130), False)],
                         ids=["global", "band64", "causal", "asym"])
def test_strips_are_bit_identical_and_match_oracle(pe, window, causal, d):
    """A workgroup walking a strip of query tiles computes every row exactly as a one-tile
    workgroup does: outputs are bit-identical for every strip length (including strips that
    cross into a segment's last, partial tile) and match the oracle (head_dim 64 and the
    head_dim 128 kernel)."""
    from packed_encoders_amd import _lib
    from packed_encoders_amd.hip_attention import _args

    lengths = [700, 65, 1500, 129, 5, 1024]
    announce(f"strips window={window} causal={causal} d={d}")
    q, k, v, cu, _ = _inputs(lengths, hq=4, hkv=2, d=d, seed=31)
    qd, kd, vd, cud = _dev(q, k, v, cu)
    lib = _lib.library()
    outs = {}
    for strip in (1, 2, 3, 8, 64):
        out = torch.full(qd.shape, 3.0, dtype=torch.bfloat16, device="cuda")
        a = _args(qd, kd, vd, out, cud, max(lengths), 0.125, window[0], window[1], causal, None, 64, strip)
        size = ctypes.c_size_t()
        assert lib.pe_attn_workspace_size(ctypes.byref(a), ctypes.byref(size)) == 0
        ws = torch.empty(max(size.value, 1), dtype=torch.uint8, device="cuda")
        assert lib.pe_varlen_attn_fwd(ctypes.byref(a), ws.data_ptr(), size.value,
                                      torch.cuda.current_stream().cuda_stream) == 0
        torch.cuda.synchronize()
        outs[strip] = out
    for strip, out in outs.items():
        assert torch.equal(out, outs[1]), f"strip {strip} differs from strip 1"
    want = _oracle(q, k, v, cu, scale=0.125, window=window, causal=causal)
    _assert_parity(outs[1], want, cu)


def _launch(lib, qd, kd, vd, cud, max_seqlen, window, causal, *, gate=None, strip=0, short_max=0):
    """One pe_varlen_attn_fwd call through the C-ABI into a fresh output (3.0 everywhere)."""
    from packed_encoders_amd.hip_attention import _args

    out = torch.full(qd.shape, 3.0, dtype=torch.bfloat16, device="cuda")
    a = _args(qd, kd, vd, out, cud, max_seqlen, 0.125, window[0], window[1], causal, gate, short_max, strip)
    size = ctypes.c_size_t()
    assert lib.pe_attn_workspace_size(ctypes.byref(a), ctypes.byref(size)) == 0
    ws = torch.empty(max(size.value, 1), dtype=torch.uint8, device="cuda")
    assert lib.pe_varlen_attn_fwd(ctypes.byref(a), ws.data_ptr(), size.value,
                                  torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    return out


WINDOW_LENGTHS = [1, 31, 32, 33, 127, 128, 129, 255, 256, 257, 700, 1500, 64, 2]
WINDOW_CASES = [((64, 64), False), ((0, 0), False), ((1, 0), False), ((127, -1), True), ((63, 65), False),
                ((100, 28), False), ((0, 128), False), ((31, 33), False), ((128, 0), False), ((5, 3), True)]


@pytest.mark.parametrize("hq,hkv", [(4, 4), (6, 2)], ids=["mha", "gqa3"])
@pytest.mark.parametrize("window,causal", WINDOW_CASES, ids=[f"{w[0]}_{w[1]}{'c' if c else ''}" for w, c in WINDOW_CASES])
def test_bounded_windows_match_oracle(pe, window, causal, hq, hkv):
    """Bounded windows of every alignment against the 32-key blocks and 128-row query tiles
    (segment lengths straddle both edges), with one and three query heads per kv head: the
    tiled kernel matches the oracle, and a strip of three query tiles per workgroup is
    bit-identical to one-tile workgroups."""
    from packed_encoders_amd import _lib

    announce(f"bounded window={window} causal={causal} heads={hq}/{hkv}")
    q, k, v, cu, _ = _inputs(WINDOW_LENGTHS, hq=hq, hkv=hkv, seed=53)
    qd, kd, vd, cud = _dev(q, k, v, cu)
    lib = _lib.library()
    mx = max(WINDOW_LENGTHS)
    got = _launch(lib, qd, kd, vd, cud, mx, window, causal)
    want = _oracle(q, k, v, cu, scale=0.125, window=window, causal=causal)
    _assert_parity(got, want, cu)
    assert torch.equal(_launch(lib, qd, kd, vd, cud, mx, window, causal, strip=3), got)


@pytest.mark.parametrize("window,causal", [((64, 64), False), ((100, -1), True)], ids=["band64", "causal100"])
def test_window_gate_and_short_routing(pe, window, causal):
    """A windowed call with the fused sigmoid gate, short segments routed to the short kernel in
    the same call, against the oracle."""
    from packed_encoders_amd import _lib

    announce(f"window gate window={window} causal={causal}")
    lengths = [300, 17, 129, 64, 1000, 3]
    q, k, v, cu, gt = _inputs(lengths, hq=4, seed=59, gate=True)
    qd, kd, vd, cud, gd = _dev(q, k, v, cu, gt)
    got = _launch(_lib.library(), qd, kd, vd, cud, max(lengths), window, causal, gate=gd, short_max=64)
    want = _oracle(q, k, v, cu, scale=0.125, window=window, causal=causal, gate=gt)
    _assert_parity(got, want, cu)


@pytest.mark.parametrize("window", [(-1, -1), (64, 64)], ids=["global", "band64"])
def test_min_seqlen_bound_skips_the_short_pass_only(pe, window):
    """A lower bound on the lengths above the boundary: with no short segment the output is
    bit-identical to the unbounded call (same plan, same kernel); with short segments present
    (a bound that is wrong) the tiled kernel serves them and the output still matches the
    oracle."""
    announce(f"min_seqlen bound window={window}")
    long_only = [98, 300, 129, 1000, 65]
    q, k, v, cu, gt = _inputs(long_only, hq=4, seed=71, gate=True)
    qd, kd, vd, cud, gd = _dev(q, k, v, cu, gt)
    mx = max(long_only)
    with torch.inference_mode():
        plain = pe.varlen_attention(qd, kd, vd, cud, mx, softmax_scale=0.125, window=window, gate=gd)
        bounded = pe.varlen_attention(qd, kd, vd, cud, mx, softmax_scale=0.125, window=window, gate=gd,
                                      min_seqlen=min(long_only))
    torch.cuda.synchronize()
    assert torch.equal(plain, bounded)
    _assert_parity(bounded, _oracle(q, k, v, cu, scale=0.125, window=window, gate=gt), cu)
    mixed = [5, 300, 64, 1, 129, 33]
    q, k, v, cu, _ = _inputs(mixed, hq=4, seed=72)
    qd, kd, vd, cud = _dev(q, k, v, cu)
    with torch.inference_mode():
        wrong = pe.varlen_attention(qd, kd, vd, cud, max(mixed), softmax_scale=0.125, window=window, min_seqlen=65)
    torch.cuda.synchronize()
    _assert_parity(wrong, _oracle(q, k, v, cu, scale=0.125, window=window), cu)
    with pytest.raises(ValueError):
        pe.varlen_attention(qd, kd, vd, cud, max(mixed), min_seqlen=max(mixed) + 1)


@pytest.mark.parametrize("window,causal", [((-1, -1), False), ((64, 64), False), ((-1, -1), True), ((200, 7), False)],
                         ids=["global", "band64", "causal", "asym"])
def test_long_segments_planned_by_waves(pe, window, causal):
    """Segments of more than 32 strips are planned by a whole wave (lanes over strips, runs of
    equal cost buckets found per 64-strip chunk): 9,000 and 4,500 tokens give 71 and 36
    query tiles of 128 rows, whose band-edge and causal costs split runs inside and across the
    chunks. Every row must be written exactly once (the output starts as 3.0 everywhere) and
    sampled rows, including every tile edge of the long segment, match the oracle."""
    from packed_encoders_amd import _lib

    lengths = [3, 9000, 4500, 200]
    announce(f"wave-planned long segments window={window} causal={causal}")
    q, k, v, cu, _ = _inputs(lengths, hq=2, seed=79)
    qd, kd, vd, cud = _dev(q, k, v, cu)
    got = _launch(_lib.library(), qd, kd, vd, cud, max(lengths), window, causal)
    live = int(cu[-1])
    written = ~(got[:live].float() == 3.0).all(dim=-1).all(dim=-1)
    assert bool(written.all()), f"{int((~written).sum())} rows never written"
    edges = [3 + 128 * t + d for t in range(71) for d in (0, 127) if 128 * t + d < 9000]
    rows = np.unique(np.array(edges + [0, 1, 2] + list(range(9003, live, 97)) + [live - 1]))
    f = lambda t: t.float().numpy()
    want = oa.sampled_rows_attention(f(q), f(k), f(v), cu.numpy(), rows, scale=0.125, window=window, causal=causal)
    err = np.abs(got.float().cpu().numpy()[rows] - want)
    assert err.max() <= MAX_ABS, f"max abs {err.max():.4g}"
    cos = oa.cosine_per_token(got.float().cpu().numpy()[rows].astype(np.float64), want)
    assert cos.min() >= MIN_COS, f"min cosine {cos.min():.6f}"


WIDE_LENGTHS = [1, 15, 16, 17, 31, 32, 33, 100, 255, 257, 513, 0, 2]
WIDE_CASES = [((-1, -1), False), ((-1, -1), True), ((64, 64), False), ((0, 0), False), ((15, 17), False),
              ((100, -1), True), ((33, 0), False)]


@pytest.mark.parametrize("window,causal", WIDE_CASES, ids=[f"{w[0]}_{w[1]}{'c' if c else ''}" for w, c in WIDE_CASES])
def test_head_dim_256_windows_strips_and_gate(pe, window, causal):
    """head_dim 256 (16-row query blocks, four heads per kv head, 32-key steps): windows and
    causal bounds of every alignment against the 16-row blocks and 32-key steps (lengths
    straddle both edges, an empty segment included), with the fused gate; strips of three and
    of eight query tiles per workgroup are bit-identical to one-tile workgroups."""
    from packed_encoders_amd import _lib

    announce(f"head_dim 256 window={window} causal={causal}")
    q, k, v, cu, gt = _inputs(WIDE_LENGTHS, hq=8, hkv=2, d=256, seed=71, gate=True)
    qd, kd, vd, cud, gd = _dev(q, k, v, cu, gt)
    lib = _lib.library()
    mx = max(WIDE_LENGTHS)
    got = _launch(lib, qd, kd, vd, cud, mx, window, causal, gate=gd)
    want = _oracle(q, k, v, cu, scale=0.125, window=window, causal=causal, gate=gt)
    _assert_parity(got, want, cu)
    for strip in (3, 8):
        assert torch.equal(_launch(lib, qd, kd, vd, cud, mx, window, causal, gate=gd, strip=strip), got)


@pytest.mark.parametrize("jump", [0.25, 1.0, 10.0], ids=["below-lazy", "rescale", "far"])
@pytest.mark.parametrize("causal", [False, True])
def test_head_dim_256_rescales_on_rising_scores(pe, jump, causal):
    """head_dim 256 keeps the exact running maximum of every key tile and rescales lazily (only
    when a tile's maximum exceeds it by more than 8 in log2 units): keys 40..109 of a segment
    score about 18 * jump log2 units above the rest (|q| . jump over 256 dims at scale 1/16),
    so jump 0.25 stays under the threshold (unnormalised probabilities up to ~2^5 kept), 1.0
    rescales mid-segment at a block edge, and 10.0 underflows every earlier probability; all
    must match the oracle."""
    lengths = [300, 129, 64]
    announce(f"head_dim 256 score jump={jump} causal={causal}")
    q, k, v, cu, _ = _inputs(lengths, hq=8, hkv=2, d=256, seed=73)
    q = q.float().abs().bfloat16()
    k = k.float()
    for a in (0, 300):
        k[a + 40:a + 110] = jump
    k = k.bfloat16()
    qd, kd, vd, cud = _dev(q, k, v, cu)
    with torch.inference_mode():
        got = pe.varlen_attention(qd, kd, vd, cud, max(lengths), softmax_scale=1.0 / 16, causal=causal,
                                  short_max=0)
    want = _oracle(q, k, v, cu, scale=1.0 / 16, causal=causal)
    _assert_parity(got, want, cu)


PREFIX_Q = [5, 1, 37, 16, 130, 300, 64, 20, 0, 7, 260]
PREFIX_K = [40, 64, 37, 80, 700, 300, 200, 5, 50, 7, 1000]  # the reference's probe pairs, then longer


@pytest.mark.parametrize("short_max", [0, 64])
@pytest.mark.parametrize("d,hq,hkv", [(64, 4, 4), (64, 6, 2), (128, 4, 2), (256, 8, 2)])
@pytest.mark.parametrize("window,causal", [((-1, -1), True), ((-1, -1), False), ((48, -1), True), ((20, 9), False)],
                         ids=["causal", "bidir", "causal-window", "window"])
def test_separate_key_segments_match_oracle(pe, window, causal, d, hq, hkv, short_max):
    """Query segments that are the tails of longer (or equal, or shorter) key segments
    (FlashAttention's cu_seqlens_k; the reference's prefixed form): causal bound and window
    measured from each query's key position, every kernel (short, tiled, wide), GQA. The
    reference's own probe pairs come first; a 20-query segment over 5 keys leaves its first
    causal rows with no key (zeros), and empty query or key segments are included."""
    announce(f"separate key segments window={window} causal={causal} d={d} heads={hq}/{hkv} short_max={short_max}")
    g = torch.Generator().manual_seed(67)
    q = torch.randn(sum(PREFIX_Q), hq, d, generator=g).bfloat16()
    k = torch.randn(sum(PREFIX_K), hkv, d, generator=g).bfloat16()
    v = torch.randn(sum(PREFIX_K), hkv, d, generator=g).bfloat16()
    cu_q = torch.tensor([0, *np.cumsum(PREFIX_Q).tolist()], dtype=torch.int32)
    cu_k = torch.tensor([0, *np.cumsum(PREFIX_K).tolist()], dtype=torch.int32)
    qd, kd, vd, cqd, ckd = _dev(q, k, v, cu_q, cu_k)
    with torch.inference_mode():
        got = pe.varlen_attention(qd, kd, vd, cqd, max(PREFIX_Q), softmax_scale=0.125, window=window, causal=causal,
                                  short_max=short_max, cu_seqlens_k=ckd, max_seqlen_k=max(PREFIX_K))
    f = lambda t: t.float().numpy()
    want = oa.packed_attention(f(q), f(k), f(v), cu_q.numpy(), scale=0.125, window=window, causal=causal,
                               cu_seqlens_k=cu_k.numpy())
    _assert_parity(got, want, cu_q)


@pytest.mark.parametrize("d,hq,hkv,short_max", [(64, 4, 4, 64), (128, 4, 2, 0), (256, 8, 2, 0)])
def test_separate_key_segments_with_gate(pe, d, hq, hkv, short_max):
    """The prefixed form with the fused sigmoid gate (the gated hybrid layers continuing a
    shared prefix): causal rows at their key positions, gate applied per query row, rows with
    no key written as zero (the gate of a zero output is still zero)."""
    announce(f"separate key segments with gate d={d} heads={hq}/{hkv} short_max={short_max}")
    g = torch.Generator().manual_seed(83)
    q = torch.randn(sum(PREFIX_Q), hq, d, generator=g).bfloat16()
    k = torch.randn(sum(PREFIX_K), hkv, d, generator=g).bfloat16()
    v = torch.randn(sum(PREFIX_K), hkv, d, generator=g).bfloat16()
    gt = torch.randn(sum(PREFIX_Q), hq, d, generator=g).bfloat16()
    cu_q = torch.tensor([0, *np.cumsum(PREFIX_Q).tolist()], dtype=torch.int32)
    cu_k = torch.tensor([0, *np.cumsum(PREFIX_K).tolist()], dtype=torch.int32)
    qd, kd, vd, cqd, ckd, gd = _dev(q, k, v, cu_q, cu_k, gt)
    with torch.inference_mode():
        got = pe.varlen_attention(qd, kd, vd, cqd, max(PREFIX_Q), softmax_scale=0.125, causal=True, gate=gd,
                                  short_max=short_max, cu_seqlens_k=ckd, max_seqlen_k=max(PREFIX_K))
    f = lambda t: t.float().numpy()
    want = oa.packed_attention(f(q), f(k), f(v), cu_q.numpy(), scale=0.125, causal=True, gate=f(gt),
                               cu_seqlens_k=cu_k.numpy())
    _assert_parity(got, want, cu_q)


@pytest.mark.parametrize("jump", [4.0, 10.0], ids=["below-guard", "past-guard"])
@pytest.mark.parametrize("window,causal", [((-1, -1), False), ((64, 64), False), ((-1, -1), True)],
                         ids=["global", "band64", "causal"])
def test_scores_jumping_past_a_stale_maximum(pe, jump, window, causal):
    """Keys far into a segment whose scores exceed every earlier score by ~9 * jump (log2
    units): the tiled kernel's running maximum, taken on a query tile's first key tile, is
    then far too small. Below the overflow guard (jump 4: probabilities up to ~2^37) the
    stale maximum is kept; past it (jump 10: ~2^92) the block is re-scored exactly. Both must
    match the oracle."""
    lengths = [700, 300, 129]
    announce(f"score jump={jump} window={window} causal={causal}")
    q, k, v, cu, _ = _inputs(lengths, hq=4, seed=41)
    q = q.float().abs().bfloat16()
    k = k.float()
    for a in (0, 700):  # keys 200..263 of the first two segments
        k[a + 200:a + 264] = jump
    k = k.bfloat16()
    qd, kd, vd, cud = _dev(q, k, v, cu)
    with torch.inference_mode():
        got = pe.varlen_attention(qd, kd, vd, cud, max(lengths), softmax_scale=0.125, window=window,
                                  causal=causal, short_max=0)
    want = _oracle(q, k, v, cu, scale=0.125, window=window, causal=causal)
    _assert_parity(got, want, cu)


def test_score_jump_in_a_tiles_last_half_block(pe):
    """A jump that only the second 32 rows of each 64-row group see (their first 32 rows'
    queries scaled down 64x), in the second 32-key block of a key tile (keys 224..255): only the
    tile's last half block overflows the stale maximum. The global kernel runs that half block
    under the next key tile's first products; here it is re-scored exactly there (segment of
    700: tile 4 follows) and before a partial last key tile (segment of 300: tile 4 is partial),
    and must match the oracle."""
    lengths = [700, 300, 129]
    announce("score jump in a tile's last half block")
    q, k, v, cu, _ = _inputs(lengths, hq=4, seed=43)
    q = q.float().abs()
    k = k.float()
    for a, n in ((0, 700), (700, 300), (1000, 129)):
        rows = torch.arange(n)
        q[a + rows[rows % 64 < 32]] /= 64.0
    for a in (0, 700):
        k[a + 224:a + 256] = 10.0
    q, k = q.bfloat16(), k.bfloat16()
    qd, kd, vd, cud = _dev(q, k, v, cu)
    with torch.inference_mode():
        got = pe.varlen_attention(qd, kd, vd, cud, max(lengths), softmax_scale=0.125, short_max=0)
    want = _oracle(q, k, v, cu, scale=0.125)
    _assert_parity(got, want, cu)


@pytest.mark.parametrize("d,h", [(64, 12), (128, 6), (256, 8), (64, 1)])
@pytest.mark.parametrize("tables", ["per-token", "dense-modulo", "batched"])
def test_rope_qkv_is_bit_exact_against_the_oracle(pe, d, h, tables):
    """pe_rope_qkv_fwd through the torch op: q, k bit-identical to the CPU oracle
    (oracle/rope.py), v untouched, for per-token gathered tables, dense [S, D] tables reused
    across a batch (row % S), and per-row [B, S, D] tables; qkv rows wider than 3HD (a
    strided slice) included."""
    from oracle import rope
    from packed_encoders_amd import hip_attention

    announce(f"rope_qkv d={d} h={h} tables={tables}")
    rng = np.random.default_rng(d + h)
    B, S = 3, 37
    wide = oa.to_bf16(rng.standard_normal((B, S, 3 * h * d + 64)))
    cos_np, sin_np = rope.rope_tables(4096, d, 10000.0)
    if tables == "per-token":
        pos = rng.integers(0, 4096, B * S)
        cos, sin = cos_np[pos][None], sin_np[pos][None]
        shape = (1, B * S)
    elif tables == "dense-modulo":
        cos, sin = cos_np[:S][None], sin_np[:S][None]
        shape = (B, S)
    else:
        pos = rng.integers(0, 4096, (B, S))
        cos, sin = cos_np[pos], sin_np[pos]
        shape = (B, S)
    rows = B * S
    want_q, want_k = rope.rope_qkv(wide.reshape(rows, -1), h, d, cos.reshape(-1, d), sin.reshape(-1, d))
    xd = torch.from_numpy(wide).bfloat16().cuda()[..., : 3 * h * d].reshape(*shape, 3 * h * d)
    before = xd.clone()
    cd, sd = torch.from_numpy(cos).bfloat16().cuda(), torch.from_numpy(sin).bfloat16().cuda()
    with torch.inference_mode():
        got_q, got_k = hip_attention.rope_qkv(xd, h, d, cd, sd)
    assert got_q.shape == (*shape, h, d) and got_q.is_contiguous() and got_k.is_contiguous()
    assert np.array_equal(got_q.float().cpu().numpy().reshape(rows, h, d), want_q)
    assert np.array_equal(got_k.float().cpu().numpy().reshape(rows, h, d), want_k)
    assert torch.equal(xd, before)  # qkv (v included) is read only
