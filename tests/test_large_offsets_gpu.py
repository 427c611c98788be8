"""Batches whose tensors pass 2 GiB: the largest inputs a packed call meets in practice.

Every kernel addresses a segment through a 64-bit base (segment start x token stride) and
32-bit offsets inside the segment. These calls put segments past byte 2^31 of Q, K, V, O (and
the gate) for each kernel family: the global kernel, the streaming band kernel and the tiled
kernel on +-64, the short kernel, head_dim 128 causal GQA, head_dim 256 causal GQA with the
gate, and the RoPE producer over a 6.5 GB projection. The first segment, the one straddling
byte 2^31 of Q, and the last two are checked against the oracle at the reference's bar (the
RoPE rows bit for bit); the tensors are drawn on the device, the checked rows copied back.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce
from oracle import attention as oa

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MIN_COS = 0.9999
GIB2 = 2 ** 31

# name: head_dim, hq, hkv, segment length, window, causal, gate, short_max, band_kernel
CASES = {
    "global64": (64, 12, 12, 1000, (-1, -1), False, False, 0, 0),
    "band64-stream": (64, 12, 12, 1000, (64, 64), False, False, 0, 1),
    "band64-tiled": (64, 12, 12, 1000, (64, 64), False, False, 0, 2),
    "short": (64, 12, 12, 48, (-1, -1), False, False, 64, 0),
    "d128-causal-gqa": (128, 8, 2, 1000, (-1, -1), True, False, 0, 0),
    "d256-causal-gqa-gate": (256, 8, 2, 700, (-1, -1), True, True, 0, 0),
}


@pytest.mark.parametrize("case", list(CASES))
def test_segments_past_two_gib_match_oracle(pe, case):
    d, hq, hkv, seg, window, causal, gate, short_max, band_kernel = CASES[case]
    row_bytes = hq * d * 2  # Q (and O, gate) bytes per token
    n_seg = (GIB2 // row_bytes) // seg + 8  # a few segments wholly past byte 2^31 of Q
    T = n_seg * seg
    announce(f"large offsets {case}: {n_seg} segments x {seg} tokens, Q {T * row_bytes / 2**30:.2f} GiB")
    g = torch.Generator(device="cuda").manual_seed(100 + list(CASES).index(case))
    q = torch.randn(T, hq, d, device="cuda", generator=g, dtype=torch.bfloat16)
    k = torch.randn(T, hkv, d, device="cuda", generator=g, dtype=torch.bfloat16)
    v = torch.randn(T, hkv, d, device="cuda", generator=g, dtype=torch.bfloat16)
    gt = torch.randn(T, hq, d, device="cuda", generator=g, dtype=torch.bfloat16) if gate else None
    cu = torch.arange(0, T + 1, seg, dtype=torch.int32, device="cuda")
    scale = d ** -0.5
    with torch.inference_mode():
        out = pe.varlen_attention(q, k, v, cu, seg, softmax_scale=scale, window=window, causal=causal, gate=gt,
                                  short_max=short_max, band_kernel=band_kernel)
    torch.cuda.synchronize()
    straddle = GIB2 // row_bytes // seg  # the segment holding byte 2^31 of Q
    assert (straddle + 1) * seg * row_bytes > GIB2 >= straddle * seg * row_bytes
    for s in (0, straddle, n_seg - 2, n_seg - 1):
        a, b = s * seg, (s + 1) * seg
        f = lambda t: t[a:b].float().cpu().numpy()
        want = oa.packed_attention(f(q), f(k), f(v), np.array([0, seg]), scale=scale, window=window, causal=causal,
                                   gate=None if gt is None else f(gt))
        got = out[a:b].float().cpu().numpy().astype(np.float64)
        err = np.abs(got - want).max()
        assert np.isfinite(got).all() and err <= MAX_ABS, f"segment {s} (rows {a}..{b}): max abs {err:.4g}"
        assert oa.cosine_per_token(got, want).min() >= MIN_COS, f"segment {s}: cosine"
    del q, k, v, gt, out
    torch.cuda.empty_cache()


def test_rope_producer_past_two_gib(pe):
    """rope_qkv over a [T, 3*H*D] projection of 6.5 GB: rows past byte 2^31 of its q and k
    outputs (and past 4 GiB of the projection) bit-identical to the CPU oracle."""
    from oracle import rope
    from packed_encoders_amd import hip_attention

    h, d = 12, 64
    T = GIB2 // (h * d * 2) + 4096  # q_out past 2^31 bytes; qkv past 4 GiB
    announce(f"large offsets rope: {T} rows, qkv {T * 3 * h * d * 2 / 2**30:.2f} GiB")
    g = torch.Generator(device="cuda").manual_seed(77)
    qkv = torch.randn(T, 3 * h * d, device="cuda", generator=g, dtype=torch.bfloat16)
    cos_np, sin_np = rope.rope_tables(8192, d, 10000.0)
    pos = torch.arange(T, device="cuda") % 8192
    cos = torch.from_numpy(cos_np).bfloat16().cuda()[pos]
    sin = torch.from_numpy(sin_np).bfloat16().cuda()[pos]
    with torch.inference_mode():
        got_q, got_k = hip_attention.rope_qkv(qkv, h, d, cos, sin)
    torch.cuda.synchronize()
    for a in (0, T - 4096, T - 64):
        rows = slice(a, a + 64)
        want_q, want_k = rope.rope_qkv(qkv[rows].float().cpu().numpy(), h, d, cos[rows].float().cpu().numpy(),
                                       sin[rows].float().cpu().numpy())
        assert np.array_equal(got_q[rows].float().cpu().numpy().reshape(want_q.shape), want_q), f"q rows {a}.."
        assert np.array_equal(got_k[rows].float().cpu().numpy().reshape(want_k.shape), want_k), f"k rows {a}.."
    del qkv, cos, sin, got_q, got_k
    torch.cuda.empty_cache()
