"""varlen_attention captured into a HIP graph and replayed, per kernel family.

The library makes no allocation, synchronisation or device-to-host read, and plans on the
device from cu_seqlens, so one captured call serves every batch with the captured token and
segment counts and max_seqlen: the inputs and cu_seqlens are rewritten in place between
replays. Each replay must equal the same call made eagerly, bit for bit; the replays are
interleaved with eager work and synchronisations, and repeat earlier batches, so a graph
whose state leaked from one replay to the next would show it.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce

pytestmark = pytest.mark.gpu

# name: head_dim, hq, hkv, window, causal, gate, separate key segments
CASES = {
    "short+global64": (64, 12, 12, (-1, -1), False, False, False),
    "short+band64": (64, 12, 12, (64, 64), False, False, False),
    "d128-causal-gqa": (128, 8, 2, (-1, -1), True, False, False),
    "d256-causal-gqa-gate": (256, 8, 2, (-1, -1), True, True, False),
    "prefixed-keys": (64, 4, 4, (-1, -1), True, False, True),
}
# Three batches of 6 segments and 2,400 tokens each, routed differently (short and long).
BATCHES = ([700, 40, 900, 300, 60, 400], [100, 1200, 64, 36, 300, 700], [2, 998, 1000, 0, 1, 399])
KEY_EXTRA = (0, 100, 5, 300, 0, 64)  # separate key segments: each query segment's prefix length


def _cu(lengths):
    return torch.tensor([0, *np.cumsum(lengths).tolist()], dtype=torch.int32, device="cuda")


@pytest.mark.parametrize("case", list(CASES))
def test_captured_call_replays_match_eager(pe, case):
    d, hq, hkv, window, causal, gate, prefixed = CASES[case]
    T = sum(BATCHES[0])
    assert all(sum(b) == T for b in BATCHES)
    max_q = max(max(b) for b in BATCHES)
    Tk = T + sum(KEY_EXTRA) if prefixed else T
    max_k = max(max(n + e for n, e in zip(b, KEY_EXTRA)) for b in BATCHES) if prefixed else None
    g = torch.Generator(device="cuda").manual_seed(31 + list(CASES).index(case))

    def draw():
        return (torch.randn(T, hq, d, device="cuda", generator=g, dtype=torch.bfloat16),
                torch.randn(Tk, hkv, d, device="cuda", generator=g, dtype=torch.bfloat16),
                torch.randn(Tk, hkv, d, device="cuda", generator=g, dtype=torch.bfloat16),
                torch.randn(T, hq, d, device="cuda", generator=g, dtype=torch.bfloat16) if gate else None)

    inputs = [draw() for _ in BATCHES]
    cus = [_cu(b) for b in BATCHES]
    cuks = [_cu([n + e for n, e in zip(b, KEY_EXTRA)]) for b in BATCHES] if prefixed else None
    q, k, v, gt = (None if t is None else t.clone() for t in inputs[0])
    cu = cus[0].clone()
    cuk = cuks[0].clone() if prefixed else None

    def call(q, k, v, gt, cu, cuk):
        return pe.varlen_attention(q, k, v, cu, max_q, softmax_scale=d ** -0.5, window=window, causal=causal,
                                   gate=gt, cu_seqlens_k=cuk, max_seqlen_k=max_k)

    announce(f"graph capture {case}: eager warm-up and capture")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.inference_mode():
        with torch.cuda.stream(side):
            call(q, k, v, gt, cu, cuk)  # warm-up outside the capture (library load, allocator)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = call(q, k, v, gt, cu, cuk)
        torch.cuda.synchronize()
        for i in (0, 1, 2, 0, 2, 1):
            announce(f"graph capture {case}: replay with batch {i} {BATCHES[i]}")
            for dst, src in zip((q, k, v, gt), inputs[i]):
                if dst is not None:
                    dst.copy_(src)
            cu.copy_(cus[i])
            if prefixed:
                cuk.copy_(cuks[i])
            out.fill_(7.0)
            graph.replay()
            torch.cuda.synchronize()
            got = out[:T].clone()
            noise = torch.randn(1 << 20, device="cuda").sum()  # eager work between replays
            want = call(*inputs[i], cus[i], cuks[i] if prefixed else None)
            torch.cuda.synchronize()
            assert torch.isfinite(noise)
            assert torch.equal(got, want[:T]), f"{case}: replay with batch {i} differs from the eager call"
    del graph


def test_captured_fused_rope_call_replays_match_eager(pe):
    """varlen_attention(rope=(cos, sin)) on unrotated q/k views of a packed projection, captured
    once: replays with the projection rows, the tables and cu_seqlens rewritten in place (five
    segments of at most 64 tokens, 200 tokens, routed differently each time) equal the eager
    call bit for bit."""
    from oracle import rope

    h, d, T = 12, 64, 200
    batches = ([40, 64, 8, 56, 32], [64, 64, 64, 7, 1], [50, 50, 50, 25, 25])
    assert all(sum(b) == T and len(b) == 5 for b in batches)
    cos_np, sin_np = rope.rope_tables(4096, d, 10000.0)
    g = torch.Generator(device="cuda").manual_seed(57)
    rng = np.random.default_rng(57)

    def draw():
        pos = rng.integers(0, 4096, T)
        return (torch.randn(T, 3 * h * d, device="cuda", generator=g, dtype=torch.bfloat16),
                torch.from_numpy(cos_np[pos]).bfloat16().cuda(), torch.from_numpy(sin_np[pos]).bfloat16().cuda())

    inputs = [draw() for _ in batches]
    cus = [_cu(b) for b in batches]
    qkv, cos, sin = (t.clone() for t in inputs[0])
    cu = cus[0].clone()

    def call(qkv, cos, sin, cu):
        view = qkv.view(T, 3, h, d)
        return pe.varlen_attention(view[:, 0], view[:, 1], view[:, 2], cu, 64, softmax_scale=0.125, rope=(cos, sin))

    announce("graph capture fused rope: eager warm-up and capture")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.inference_mode():
        with torch.cuda.stream(side):
            call(qkv, cos, sin, cu)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = call(qkv, cos, sin, cu)
        torch.cuda.synchronize()
        for i in (0, 1, 2, 0, 2, 1):
            announce(f"graph capture fused rope: replay with batch {i} {batches[i]}")
            for dst, src in zip((qkv, cos, sin), inputs[i]):
                dst.copy_(src)
            cu.copy_(cus[i])
            out.fill_(7.0)
            graph.replay()
            torch.cuda.synchronize()
            got = out.clone()
            want = call(*inputs[i], cus[i])
            torch.cuda.synchronize()
            assert torch.equal(got, want), f"fused rope: replay with batch {i} differs from the eager call"
    del graph


def test_calls_on_two_streams_at_once_match_calls_alone(pe):
    """Two streams issue calls back to back with no ordering between them (a short + global batch
    on one, a +-64 batch with a gate on the other, each with its own workspace from the caching
    allocator): every output equals the same call made alone on the default stream. The library
    keeps no state between calls beyond the caller's workspace."""
    g = torch.Generator(device="cuda").manual_seed(71)

    def batch(lengths, h, d, gate):
        T = sum(lengths)
        q, k, v = (torch.randn(T, h, d, device="cuda", generator=g, dtype=torch.bfloat16) for _ in range(3))
        gt = torch.randn(T, h, d, device="cuda", generator=g, dtype=torch.bfloat16) if gate else None
        return q, k, v, gt, _cu(lengths), max(lengths)

    a = batch([700, 40, 900, 30, 64, 1200], 12, 64, False)
    b = batch([300, 1000, 77, 512], 8, 64, True)

    def call_a(x):
        q, k, v, gt, cu, mx = x
        return pe.varlen_attention(q, k, v, cu, mx, softmax_scale=0.125)

    def call_b(x):
        q, k, v, gt, cu, mx = x
        return pe.varlen_attention(q, k, v, cu, mx, softmax_scale=0.125, window=(64, 64), gate=gt)

    announce("two streams: calls alone")
    with torch.inference_mode():
        want_a, want_b = call_a(a), call_b(b)
        torch.cuda.synchronize()
        s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
        s1.wait_stream(torch.cuda.current_stream())
        s2.wait_stream(torch.cuda.current_stream())
        outs_a, outs_b = [], []
        announce("two streams: interleaved calls")
        for _ in range(8):
            with torch.cuda.stream(s1):
                outs_a.append(call_a(a))
            with torch.cuda.stream(s2):
                outs_b.append(call_b(b))
        torch.cuda.synchronize()
    assert all(torch.equal(o, want_a) for o in outs_a), "a call on stream 1 differs from the call alone"
    assert all(torch.equal(o, want_b) for o in outs_b), "a call on stream 2 differs from the call alone"
