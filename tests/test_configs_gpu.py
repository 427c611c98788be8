"""Full-size parity on the benchmark configurations, as the benchmark generates them.

Every workload of ``packed_encoders_amd.workloads`` (C1, the two layer kinds of C2, C3, C4 global
and +-64, C5 with its gate) runs through ``varlen_attention`` at its real size, lengths and head
geometry, on bf16 Q/K/V drawn on the device. The oracle then checks a sample of rows covering
every segment's first and last row, the rows on either side of every 32-row block edge and
128-row query-tile edge, and seeded random rows, at the north-star bar: max-abs <= 2e-2 and
per-token cosine >= 0.9999 (the reference's harness checks outputs on the shapes it times,
benchmarks/packed_short_attention_bench.py:96-117,243-309). Every output row must be finite.
C3's rows cover both kernels of its mixed call (segments <= 64 tokens take the short kernel), in
its generated order (queries, then documents) and shuffled (the two interleaved).
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


def _sample_rows(lengths, n_random=256, seed=0):
    """First and last row of every segment; both sides of every 32-row block edge of its first
    and last 128-row query tile (of every edge when the segment is at most 512 rows); two
    interior tile edges of longer segments; and n_random seeded rows."""
    rng = np.random.default_rng(seed)
    rows = set()
    start = 0
    for n in lengths:
        if n:
            rows.update((start, start + n - 1))
            last_tile = (n - 1) // 128 * 128
            edges = [e for e in range(32, n, 32) if n <= 512 or e <= 128 or e >= last_tile]
            if n > 512:
                edges += (rng.integers(2, n // 128, size=2) * 128).tolist()
            for e in edges:
                rows.update((start + e - 1, start + e))
        start += n
    rows.update(rng.integers(0, start, size=n_random).tolist())
    return np.array(sorted(rows), dtype=np.int64)


def _workloads():
    from packed_encoders_amd import workloads as w

    c2 = w.c2()
    return {
        "C1": (w.c1(), 0),
        "C2-global": (c2, 0),
        "C2-band": (c2, 1),
        "C3": (w.c3(), 0),
        "C3-shuffled": (w.c3(shuffled=True), 0),
        "C4": (w.c4(), 0),
        "C4-band": (w.c4(band=True), 0),
        "C5": (w.c5(), 0),
    }


@pytest.mark.parametrize("name", ["C1", "C2-global", "C2-band", "C3", "C3-shuffled", "C4", "C4-band", "C5"])
def test_benchmark_workload_matches_oracle(pe, name):
    workload, layer_index = _workloads()[name]
    layer = workload.layers[layer_index]
    T, hq, hkv, d = workload.total_tokens, workload.n_heads_q, workload.n_heads_kv, workload.head_dim
    announce(f"full-size {name}: T={T} segments={len(workload.lengths)} heads={hq}/{hkv}x{d} "
             f"window={layer.window} causal={layer.causal} gate={layer.gate}")
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev).manual_seed(4321)
    q = torch.randn(T, hq, d, device=dev, generator=gen, dtype=torch.bfloat16)
    k = torch.randn(T, hkv, d, device=dev, generator=gen, dtype=torch.bfloat16)
    v = torch.randn(T, hkv, d, device=dev, generator=gen, dtype=torch.bfloat16)
    gate = torch.randn(T, hq, d, device=dev, generator=gen, dtype=torch.bfloat16) if layer.gate else None
    cu = torch.tensor(workload.cu_seqlens(), dtype=torch.int32, device=dev)
    with torch.inference_mode():
        out = pe.varlen_attention(q, k, v, cu, workload.max_seqlen, softmax_scale=workload.scale,
                                  window=layer.window, causal=layer.causal, gate=gate)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all())

    rows = _sample_rows(workload.lengths)
    assert len(rows) >= 256
    idx = torch.from_numpy(rows).to(dev)
    f = lambda t: t.float().cpu().numpy()
    want = oa.sampled_rows_attention(f(q), f(k), f(v), cu.cpu().numpy(), rows,
                                     scale=workload.scale, window=layer.window, causal=layer.causal)
    if gate is not None:
        want = oa.sigmoid_gate(oa.to_bf16(want), f(gate[idx]))
    got = f(out[idx]).astype(np.float64)
    err = np.abs(got - want)
    assert err.max() <= MAX_ABS, f"{name}: max abs {err.max():.4g} at row {rows[err.reshape(len(rows), -1).max(1).argmax()]}"
    cos = oa.cosine_per_token(got, want)
    assert cos.min() >= MIN_COS, f"{name}: min cosine {cos.min():.6f} at row {rows[cos.argmin()]}"
