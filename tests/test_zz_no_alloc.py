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
