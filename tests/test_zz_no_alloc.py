"""pe_varlen_attn_fwd_noalloc, the entry point that allocates nothing, against
pe_varlen_attn_fwd on the GPU, through the C ABI.

The variant keeps the tiled kernels' plan list in the library's static device array instead
of a caller workspace. Two calls in a row, the second with a smaller input, must each give
bit-identical outputs to the workspace entry point (the second call reuses the array the
first one filled, so stale entries must not leak into it); the short kernel's segments and
all three head dims are covered.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from conftest import announce

pytestmark = pytest.mark.gpu


def _call(lib, fn, q, k, v, cu, max_seqlen, window, causal, gate):
    from packed_encoders_amd.hip_attention import _args

    out = torch.full(q.shape, 5.0, dtype=torch.bfloat16, device="cuda")
    a = _args(q, k, v, out, cu, max_seqlen, q.shape[-1] ** -0.5, window[0], window[1], causal, gate, -1)
    stream = torch.cuda.current_stream().cuda_stream
    if fn == "noalloc":
        rc = lib.pe_varlen_attn_fwd_noalloc(ctypes.byref(a), stream)
    else:
        size = ctypes.c_size_t()
        assert lib.pe_attn_workspace_size(ctypes.byref(a), ctypes.byref(size)) == 0
        ws = torch.empty(max(size.value, 1), dtype=torch.uint8, device="cuda")
        rc = lib.pe_varlen_attn_fwd(ctypes.byref(a), ws.data_ptr(), size.value, stream)
    assert rc == 0, rc
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("d,hq,hkv,window,causal,gate", [
    (64, 12, 12, (-1, -1), False, False),
    (64, 12, 12, (64, 64), False, False),
    (128, 8, 2, (-1, -1), True, False),
    (256, 8, 2, (-1, -1), True, True),
], ids=["d64_global", "d64_band", "d128_causal", "d256_gate"])
def test_noalloc_matches_workspace_entry_point_on_two_calls(pe, d, hq, hkv, window, causal, gate):
    from packed_encoders_amd import _lib

    lib = _lib.library()
    g = torch.Generator().manual_seed(d + hq)
    for call, lengths in enumerate(([700, 40, 1500, 129, 64, 300], [200, 17, 90])):  # the second is smaller
        announce(f"noalloc d={d} window={window} causal={causal} gate={gate} call={call} lengths={lengths}")
        T = sum(lengths)
        q = torch.randn(T, hq, d, generator=g).bfloat16().cuda()
        k = torch.randn(T, hkv, d, generator=g).bfloat16().cuda()
        v = torch.randn(T, hkv, d, generator=g).bfloat16().cuda()
        gt = torch.randn(T, hq, d, generator=g).bfloat16().cuda() if gate else None
        cu = torch.tensor([0, *np.cumsum(lengths).tolist()], dtype=torch.int32, device="cuda")
        want = _call(lib, "workspace", q, k, v, cu, max(lengths), window, causal, gt)
        got = _call(lib, "noalloc", q, k, v, cu, max(lengths), window, causal, gt)
        assert torch.isfinite(got).all()
        assert torch.equal(got, want), f"call {call}: noalloc output differs from the workspace entry point"


def test_noalloc_matches_workspace_entry_point_on_random_calls(pe):
    """The first 24 seeded calls of the random parity sweep (tests/test_random_gpu.py: every
    head dim, windows, causal, the gate, separate key segments, routing boundaries, host length
    bounds, forced band kernels), one after another on one device: the no-allocation entry point
    gives the workspace entry point's bits on each, whatever the previous call left in the
    static array."""
    from test_random_gpu import draw_case

    from packed_encoders_amd import _lib
    from packed_encoders_amd.hip_attention import _args

    lib = _lib.library()
    stream = torch.cuda.current_stream().cuda_stream
    for seed in range(24):
        c = draw_case(seed)
        announce(f"noalloc random case {seed}: d={c['d']} heads={c['hq']}/{c['hkv']} window={c['window']} "
                 f"causal={c['causal']} keys={c['keys'] is not None}")
        g = torch.Generator().manual_seed(500 + seed)
        lengths = c["lengths"]
        keys = c["keys"] if c["keys"] is not None else lengths
        T, Tk = sum(lengths), sum(keys)
        q = torch.randn(T, c["hq"], c["d"], generator=g).bfloat16().cuda()
        k = torch.randn(Tk, c["hkv"], c["d"], generator=g).bfloat16().cuda()
        v = torch.randn(Tk, c["hkv"], c["d"], generator=g).bfloat16().cuda()
        gt = torch.randn(T, c["hq"], c["d"], generator=g).bfloat16().cuda() if c["gate"] else None
        cu = torch.tensor([0, *np.cumsum(lengths).tolist()], dtype=torch.int32, device="cuda")
        cuk = (torch.tensor([0, *np.cumsum(keys).tolist()], dtype=torch.int32, device="cuda")
               if c["keys"] is not None else None)
        outs = []
        for fn in ("workspace", "noalloc"):
            out = torch.full(q.shape, 5.0, dtype=torch.bfloat16, device="cuda")
            a = _args(q, k, v, out, cu, max(lengths), c["d"] ** -0.5, c["window"][0], c["window"][1], c["causal"], gt,
                      -1 if c["short_max"] is None else c["short_max"], 0, cuk, max(keys) if cuk is not None else 0,
                      c["band_kernel"], min(lengths) if c["bound"] else 0)
            if fn == "noalloc":
                assert lib.pe_varlen_attn_fwd_noalloc(ctypes.byref(a), stream) == 0
            else:
                size = ctypes.c_size_t()
                assert lib.pe_attn_workspace_size(ctypes.byref(a), ctypes.byref(size)) == 0
                ws = torch.empty(max(size.value, 1), dtype=torch.uint8, device="cuda")
                assert lib.pe_varlen_attn_fwd(ctypes.byref(a), ws.data_ptr(), size.value, stream) == 0
            torch.cuda.synchronize()
            outs.append(out[:T])
        assert torch.equal(outs[0], outs[1]), f"random case {seed}: noalloc output differs from the workspace entry point"


@pytest.mark.parametrize("d,h", [(64, 12), (128, 6)], ids=["d64", "d128"])
def test_noalloc_with_fused_rope_matches_workspace_entry_point(pe, d, h):
    """The short kernel's fused RoPE (pe_attn_args.rope_cos / rope_sin, q and k unrotated views
    of a packed projection) through the no-allocation entry point: the workspace entry point's
    bits on two calls in a row, the second smaller, with the gate on the second."""
    from oracle import rope

    from packed_encoders_amd import _lib
    from packed_encoders_amd.hip_attention import _args

    lib = _lib.library()
    stream = torch.cuda.current_stream().cuda_stream
    cos_np, sin_np = rope.rope_tables(4096, d, 10000.0)
    for call, (n_seq, gate) in enumerate(((300, False), (40, True))):
        announce(f"noalloc fused rope d={d} call {call}: {n_seq} segments gate={gate}")
        rng = np.random.default_rng(70 + call)
        lengths = rng.integers(1, 65, size=n_seq).tolist()
        T = sum(lengths)
        g = torch.Generator().manual_seed(80 + call)
        qkv = torch.randn(T, 3 * h * d, generator=g).bfloat16().cuda()
        view = qkv.view(T, 3, h, d)
        gt = torch.randn(T, h, d, generator=g).bfloat16().cuda() if gate else None
        pos = rng.integers(0, 4096, T)
        cos = torch.from_numpy(cos_np[pos]).bfloat16().cuda()
        sin = torch.from_numpy(sin_np[pos]).bfloat16().cuda()
        cu = torch.tensor([0, *np.cumsum(lengths).tolist()], dtype=torch.int32, device="cuda")
        outs = []
        for fn in ("workspace", "noalloc"):
            out = torch.full((T, h, d), float("nan"), dtype=torch.bfloat16, device="cuda")
            a = _args(view[:, 0], view[:, 1], view[:, 2], out, cu, max(lengths), d ** -0.5, -1, -1, False, gt, -1,
                      rope=(cos, sin))
            if fn == "noalloc":
                assert lib.pe_varlen_attn_fwd_noalloc(ctypes.byref(a), stream) == 0
            else:
                size = ctypes.c_size_t()
                assert lib.pe_attn_workspace_size(ctypes.byref(a), ctypes.byref(size)) == 0
                ws = torch.empty(max(size.value, 1), dtype=torch.uint8, device="cuda")
                assert lib.pe_varlen_attn_fwd(ctypes.byref(a), ws.data_ptr(), size.value, stream) == 0
            torch.cuda.synchronize()
            outs.append(out)
        assert torch.isfinite(outs[1]).all(), "every output row is written"
        assert torch.equal(outs[0], outs[1]), f"call {call}: noalloc output differs from the workspace entry point"


def _inputs(T, hq, hkv, d, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(T, h, d, generator=g).bfloat16().cuda() for h in (hq, hkv, hkv)]


def test_noalloc_captured_replays_follow_rewritten_lengths(pe):
    """The no-allocation call captured once in a HIP graph (after an eager call on this device)
    and replayed while cu_seqlens is rewritten in place between replays: every replay re-plans
    from the static array and matches the workspace entry point run eagerly on the same lengths,
    bit for bit (the graph holds no memset: the plan writes every count it reads)."""
    from packed_encoders_amd import _lib
    from packed_encoders_amd.hip_attention import _args

    lib = _lib.library()
    T, max_seqlen = 2000, 1500
    q, k, v = _inputs(T, 12, 12, 64, seed=71)
    batches = ([700, 40, 900, 300, 60], [100, 1500, 64, 36, 300], [2, 998, 1000, 0, 0])
    cus = [torch.tensor([0, *np.cumsum(b).tolist()], dtype=torch.int32, device="cuda") for b in batches]
    cu = cus[0].clone()
    out = torch.zeros(T, 12, 64, dtype=torch.bfloat16, device="cuda")
    a = _args(q, k, v, out, cu, max_seqlen, 0.125, -1, -1, False, None, -1)
    announce("noalloc eager call before capture")
    assert lib.pe_varlen_attn_fwd_noalloc(ctypes.byref(a), torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    announce("noalloc capture")
    with torch.cuda.graph(graph, stream=side):
        assert lib.pe_varlen_attn_fwd_noalloc(ctypes.byref(a), torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for i in (0, 1, 2, 0, 1):
        announce(f"noalloc replay with lengths {batches[i]}")
        cu.copy_(cus[i])
        out.fill_(3.0)
        graph.replay()
        torch.cuda.synchronize()
        want = _call(lib, "workspace", q, k, v, cus[i], max_seqlen, (-1, -1), False, None)
        n = int(cus[i][-1])
        assert torch.equal(out[:n], want[:n]), f"replay with lengths {batches[i]} differs"
    del graph


_CHILD = r"""
import ctypes, sys
sys.path.insert(0, sys.argv[1])
import torch
import packed_encoders_amd as pe
from packed_encoders_amd import _lib
from packed_encoders_amd.hip_attention import _args
lib = _lib.library()
g = torch.Generator().manual_seed(5)
q, k, v = (torch.randn(900, 4, 64, generator=g).bfloat16().cuda() for _ in range(3))
cu = torch.tensor([0, 300, 340, 900], dtype=torch.int32, device="cuda")
out = torch.zeros_like(q)
a = _args(q, k, v, out, cu, 560, 0.125, -1, -1, False, None, -1)
graph = torch.cuda.CUDAGraph()
side = torch.cuda.Stream()
side.wait_stream(torch.cuda.current_stream())
with torch.cuda.graph(graph, stream=side):  # the library's first no-allocation call on this device
    rc = lib.pe_varlen_attn_fwd_noalloc(ctypes.byref(a), torch.cuda.current_stream().cuda_stream)
torch.cuda.current_stream().wait_stream(side)
print("capture rc", rc, flush=True)
assert rc == 0, rc
graph.replay()
torch.cuda.synchronize()
with torch.inference_mode():
    want = pe.varlen_attention(q, k, v, cu, 560, softmax_scale=0.125)
torch.cuda.synchronize()
assert torch.equal(out, want)
print("CHILD_OK", flush=True)
"""


def test_noalloc_first_call_inside_capture(pe):
    """In a fresh process whose first no-allocation call is made inside a graph capture (the
    static array's per-device address looked up while capturing), the captured call replays to
    the same bits as the workspace path."""
    import subprocess
    import sys

    from conftest import ROOT

    announce("noalloc first call inside capture (child process)")
    proc = subprocess.run([sys.executable, "-c", _CHILD, str(ROOT)], capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0 and "CHILD_OK" in proc.stdout, proc.stdout[-2000:] + proc.stderr[-2000:]
