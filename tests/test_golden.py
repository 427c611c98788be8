"""Parity against the reference's own outputs: tests/golden/ref_cpu_attention.npz, written by
tests/golden/make_golden.py from the reference's compiled CPU packed attention
(packed_encoders/cpu/local_attention_x86.c:192-234) on bf16-representable inputs.

CPU tests pin the float64 oracle and this repository's C port to the fixture at the reference
CPU test's fp32 tolerance (tests/test_cpu_short_attention.py:47, atol = rtol = 2e-5). GPU tests
run the HIP kernels on the same inputs through the torch ops and the C ABI and compare with the
reference's outputs at the bf16 bar: max-abs <= 2e-2 and per-token cosine >= 0.9999.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import attention as oa
from oracle import cpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "ref_cpu_attention.npz"


@pytest.fixture(scope="module")
def golden():
    z = np.load(GOLDEN)  # allow_pickle stays False: plain arrays only
    bits = lambda name: (z[name].astype(np.uint32) << 16).view(np.float32)
    g = {name: z[name] for name in z.files}
    g["q"], g["k"], g["v"] = bits("q_bf16"), bits("k_bf16"), bits("v_bf16")
    g["cu"] = np.concatenate([[0], np.cumsum(g["lengths"])]).astype(np.int32)
    return g


def _token_major(x):
    return np.ascontiguousarray(x.transpose(1, 0, 2))


def test_fixture_is_well_formed(golden):
    assert golden["q"].shape == golden["k"].shape == golden["v"].shape
    assert golden["q"].shape[1] == int(golden["lengths"].sum())
    assert np.array_equal(oa.to_bf16(golden["k"]), golden["k"])  # inputs are exact bf16 values
    for half in golden["halves"]:
        assert np.isfinite(golden[f"out_half{half}"]).all()


@pytest.mark.parametrize("idx", range(4))
def test_oracle_matches_reference_outputs(golden, idx):
    half = int(golden["halves"][idx])
    q, k, v = (_token_major(golden[n]) for n in ("q", "k", "v"))
    want = oa.packed_attention(q, k, v, golden["cu"], scale=float(golden["scale"]), window=(half, half))
    np.testing.assert_allclose(_token_major(golden[f"out_half{half}"]), want, atol=2e-5, rtol=2e-5)


@pytest.mark.parametrize("idx", range(4))
def test_c_port_matches_reference_outputs(golden, idx):
    cpu.build()
    half = int(golden["halves"][idx])
    got = cpu.local_attention(golden["q"], golden["k"], golden["v"], golden["lengths"], half, kind="port", tile=16)
    np.testing.assert_allclose(got, golden[f"out_half{half}"], atol=2e-5, rtol=2e-5)


def _bf16_parity(got, want):
    got = np.asarray(got, dtype=np.float64)
    err = np.abs(got - want)
    assert np.isfinite(got).all()
    assert err.max() <= 2e-2, f"max abs {err.max():.4g}"
    cos = oa.cosine_per_token(got, want)
    assert cos.min() >= 0.9999, f"min cosine {cos.min():.6f}"


@pytest.mark.gpu
@pytest.mark.parametrize("short_max", [0, 64, 128])
@pytest.mark.parametrize("idx", range(4))
def test_hip_varlen_matches_reference_outputs(pe, golden, idx, short_max):
    import torch

    from conftest import announce

    half = int(golden["halves"][idx])
    announce(f"golden varlen half={half} short_max={short_max}")
    q, k, v = (torch.from_numpy(_token_major(golden[n])).bfloat16().cuda() for n in ("q", "k", "v"))
    cu = torch.from_numpy(golden["cu"]).cuda()
    with torch.inference_mode():
        out = pe.varlen_attention(q, k, v, cu, int(golden["lengths"].max()), softmax_scale=0.125,
                                  window=(half, half), short_max=short_max)
    _bf16_parity(out.float().cpu().numpy(), _token_major(golden[f"out_half{half}"]))


@pytest.mark.gpu
@pytest.mark.parametrize("half_window", [None, 16, 64])
def test_hip_packed_short_matches_reference_outputs(pe, golden, half_window):
    import torch

    from conftest import announce

    # the segments up to 128 tokens (all but the 129- and 7-token tail)
    n_seg = 8
    cu_np = golden["cu"][: n_seg + 1]
    T = int(cu_np[-1])
    longest = int(golden["lengths"][:n_seg].max())
    half = longest if half_window is None else half_window
    if half not in golden["halves"]:
        ref_half = int(golden["halves"][-1])  # global over the whole fixture = global per segment
        assert half_window is None
        half = ref_half
    announce(f"golden packed_short half_window={half_window}")
    q, k, v = (torch.from_numpy(_token_major(golden[n])[:T]).bfloat16().cuda() for n in ("q", "k", "v"))
    cu = torch.from_numpy(cu_np).cuda()
    with torch.inference_mode():
        out = pe.packed_short_attention(q, k, v, cu, longest, half_window=half_window, softmax_scale=0.125)
    _bf16_parity(out.float().cpu().numpy(), _token_major(golden[f"out_half{half}"])[:T])
