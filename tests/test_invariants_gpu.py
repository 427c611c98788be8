"""Bit-exact invariants on every kernel path: zero cross-segment leakage and independence from
batch composition (tests/test_packed_short_attention.py:112-126 and
tests/test_cpu_short_attention.py:72-77 of the reference), for head_dim 64, 128 and 256, global,
+-64 band, causal, the fused gate and separate key segments (``cu_seqlens_k``).

Leakage: scaling another segment's keys by 100, its values by -100, its queries by 7 and its
gate by -3 leaves every other segment's output bits unchanged. Independence: a segment run
alone (its own tensors, a one-segment ``cu_seqlens``) gives the same bits as inside the batch
under the same routing boundary (``short_max`` 64: a segment's kernel follows its own length).
The library's default boundary is keyed on the batch's longest segment (every segment short
when it is at most 128 tokens), so with the default a 65-128-token segment may take the short
kernel alone and the tiled kernel in a longer batch: both within tolerance, not the same bits,
as the reference's per-batch Triton / FlashAttention choice. The one other exception is the
+-64-shaped band's size rule: a call of at least 17,667 query tiles (128 rows x heads) runs its
long segments in the streaming band kernel, a smaller one in the tiled kernel, so such a segment
alone and inside a large call agree within tolerance, not bit for bit
(tests/test_band_kernel_gpu.py::test_segment_across_the_size_rule checks that bound).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce

pytestmark = pytest.mark.gpu

# (head_dim, query heads, kv heads, window, causal, gate)
CASES = [
    (64, 4, 4, (64, 64), False, False),
    (64, 6, 2, (-1, -1), True, False),
    (128, 4, 2, (-1, -1), False, False),
    (128, 4, 4, (64, 64), False, True),
    (256, 8, 2, (-1, -1), True, True),
    (256, 8, 2, (-1, -1), False, False),
]
IDS = [f"d{d}_{hq}:{hkv}_{w[0]}_{w[1]}{'_causal' if c else ''}{'_gate' if g else ''}" for d, hq, hkv, w, c, g in CASES]

Q_LENGTHS = [31, 65, 300, 129, 1]
K_EXTRA = [5, 0, 40, 200, 3]  # key segments longer than their queries (queries are the tail)


def _tensors(d, hq, hkv, gate, separate_keys, seed):
    g = torch.Generator().manual_seed(seed)
    T = sum(Q_LENGTHS)
    k_lengths = [a + b for a, b in zip(Q_LENGTHS, K_EXTRA)] if separate_keys else Q_LENGTHS
    Tk = sum(k_lengths)
    q = torch.randn(T, hq, d, generator=g).bfloat16().cuda()
    k = torch.randn(Tk, hkv, d, generator=g).bfloat16().cuda()
    v = torch.randn(Tk, hkv, d, generator=g).bfloat16().cuda()
    gt = torch.randn(T, hq, d, generator=g).bfloat16().cuda() if gate else None
    cu = [0, *np.cumsum(Q_LENGTHS).tolist()]
    cuk = [0, *np.cumsum(k_lengths).tolist()]
    return q, k, v, gt, cu, cuk, k_lengths


def _run(pe, q, k, v, gt, cu, cuk, window, causal, short_max, separate_keys):
    cud = torch.tensor(cu, dtype=torch.int32, device="cuda")
    kw = dict(softmax_scale=q.shape[-1] ** -0.5, window=window, causal=causal, gate=gt, short_max=short_max)
    max_q = max(b - a for a, b in zip(cu, cu[1:]))
    if separate_keys:
        cukd = torch.tensor(cuk, dtype=torch.int32, device="cuda")
        max_k = max(b - a for a, b in zip(cuk, cuk[1:]))
        kw.update(cu_seqlens_k=cukd, max_seqlen_k=max_k)
    with torch.inference_mode():
        return pe.varlen_attention(q, k, v, cud, max_q, **kw)


@pytest.mark.parametrize("separate_keys", [False, True], ids=["shared", "cu_k"])
@pytest.mark.parametrize("short_max", [0, -1], ids=["tiled", "routed"])
@pytest.mark.parametrize("d,hq,hkv,window,causal,gate", CASES, ids=IDS)
def test_no_cross_segment_leakage(pe, d, hq, hkv, window, causal, gate, short_max, separate_keys):
    announce(f"leakage d={d} {hq}:{hkv} window={window} causal={causal} gate={gate} short_max={short_max} "
             f"separate_keys={separate_keys}")
    q, k, v, gt, cu, cuk, _ = _tensors(d, hq, hkv, gate, separate_keys, seed=d + hq)
    base = _run(pe, q, k, v, gt, cu, cuk, window, causal, short_max, separate_keys)
    s = 2  # perturb the 300-row segment
    q2, k2, v2 = q.clone(), k.clone(), v.clone()
    q2[cu[s]:cu[s + 1]] *= 7
    k2[cuk[s]:cuk[s + 1]] *= 100
    v2[cuk[s]:cuk[s + 1]] *= -100
    g2 = None
    if gt is not None:
        g2 = gt.clone()
        g2[cu[s]:cu[s + 1]] *= -3
    changed = _run(pe, q2, k2, v2, g2, cu, cuk, window, causal, short_max, separate_keys)
    torch.cuda.synchronize()
    assert torch.isfinite(base).all()
    assert torch.equal(base[:cu[s]], changed[:cu[s]])
    assert torch.equal(base[cu[s + 1]:], changed[cu[s + 1]:])
    assert not torch.equal(base[cu[s]:cu[s + 1]], changed[cu[s]:cu[s + 1]])  # the perturbation took


@pytest.mark.parametrize("separate_keys", [False, True], ids=["shared", "cu_k"])
@pytest.mark.parametrize("d,hq,hkv,window,causal,gate", CASES, ids=IDS)
def test_segment_alone_equals_segment_in_batch(pe, d, hq, hkv, window, causal, gate, separate_keys):
    announce(f"batch independence d={d} {hq}:{hkv} window={window} causal={causal} gate={gate} "
             f"separate_keys={separate_keys}")
    q, k, v, gt, cu, cuk, _ = _tensors(d, hq, hkv, gate, separate_keys, seed=3 * d + hkv)
    batch = _run(pe, q, k, v, gt, cu, cuk, window, causal, 64, separate_keys)
    for s in range(len(Q_LENGTHS)):
        a, b, ka, kb = cu[s], cu[s + 1], cuk[s], cuk[s + 1]
        alone = _run(pe, q[a:b].contiguous(), k[ka:kb].contiguous(), v[ka:kb].contiguous(),
                     None if gt is None else gt[a:b].contiguous(), [0, b - a], [0, kb - ka], window, causal, 64,
                     separate_keys)
        torch.cuda.synchronize()
        assert torch.equal(alone, batch[a:b]), f"segment {s} ({b - a} rows) differs alone"
