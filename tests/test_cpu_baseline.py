"""The CPU baseline (oracle/cpu_attention.c) and the reference's own compiled CPU kernel
(oracle/_ref) against the float64 oracle, and against each other.

Restates the reference's CPU attention test (tests/test_cpu_short_attention.py:27-77): the same
lengths, half widths, a zero query row and a very sharp one, fp32 tolerance 2e-5, and bitwise
independence from the thread count.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import attention as oa
from oracle import cpu

LENGTHS = (16, 32, 1, 15, 17, 31, 33, 65)


def _inputs(seed=43, heads=3, d=64):
    rng = np.random.default_rng(seed)
    T = sum(LENGTHS)
    q, k, v = (rng.standard_normal((heads, T, d)).astype(np.float32) * 2 for _ in range(3))
    q[:, 0] = 0.0      # uniform logits: softmax ties
    q[:, 1] *= 100.0   # a very sharp row: exp underflow
    return q, k, v


def _oracle(q, k, v, half, scale=0.125):
    cu = np.concatenate([[0], np.cumsum(LENGTHS)])
    out = oa.packed_attention(q.transpose(1, 0, 2), k.transpose(1, 0, 2), v.transpose(1, 0, 2), cu,
                              scale=scale, window=(half, half))
    return out.transpose(1, 0, 2)


@pytest.fixture(scope="module", autouse=True)
def _built():
    cpu.build()


@pytest.mark.parametrize("half", [0, 14, 15, 16, 30, 31, 32, 64])
def test_port_matches_oracle(half):
    q, k, v = _inputs()
    got = cpu.local_attention(q, k, v, LENGTHS, half, kind="port", tile=4)
    np.testing.assert_allclose(got, _oracle(q, k, v, half), atol=2e-5, rtol=2e-5)


@pytest.mark.parametrize("half", [0, 16, 31, 64])
def test_reference_kernel_matches_oracle_and_port(half):
    if not cpu.available("reference"):
        pytest.skip("oracle/_ref not built (reference checkout absent when building)")
    q, k, v = _inputs()
    ref = cpu.local_attention(q, k, v, LENGTHS, half, kind="reference", tile=16)
    np.testing.assert_allclose(ref, _oracle(q, k, v, half), atol=2e-5, rtol=2e-5)
    port = cpu.local_attention(q, k, v, LENGTHS, half, kind="port", tile=16)
    np.testing.assert_allclose(port, ref, atol=2e-5, rtol=2e-5)


def test_port_general_head_dim_and_scale():
    rng = np.random.default_rng(5)
    lengths = (7, 40)
    T = sum(lengths)
    q, k, v = (rng.standard_normal((2, T, 24)).astype(np.float32) for _ in range(3))
    got = cpu.local_attention(q, k, v, lengths, 100, kind="port", scale=0.3)
    cu = np.concatenate([[0], np.cumsum(lengths)])
    want = oa.packed_attention(q.transpose(1, 0, 2), k.transpose(1, 0, 2), v.transpose(1, 0, 2), cu,
                               scale=0.3).transpose(1, 0, 2)
    np.testing.assert_allclose(got, want, atol=2e-5, rtol=2e-5)


def test_port_thread_count_and_layout_are_bitwise_stable():
    q, k, v = _inputs(seed=44)
    by_tile = {}
    for threads in (1, 4):
        for tile in (16, 64):
            for token_major in (False, True):
                got = cpu.local_attention(q, k, v, LENGTHS, 64, kind="port", threads=threads, tile=tile,
                                          token_major=token_major)
                if token_major:
                    got = got.reshape(got.shape[0], 3, 64).transpose(1, 0, 2)
                key = tile
                if key in by_tile:
                    assert np.array_equal(got, by_tile[key])
                else:
                    by_tile[key] = got.copy()


def test_port_rejects_bad_arguments():
    q, k, v = _inputs()
    with pytest.raises(RuntimeError):
        cpu.local_attention(q, k, v, (5,) * 3, 4, kind="port")  # lengths do not sum to tokens


def test_physical_cores_positive():
    assert cpu.physical_cores() >= 1


def test_cpu_leg_samples_whole_segments_past_its_flop_cap(monkeypatch):
    """bench.cpu_bench on a schedule past its caps times the whole segments at the front of the
    batch that fit them (at least one), says so in its sample, and reports the sample's own
    FLOP rate; under the caps it keeps the full schedule."""
    import bench
    from packed_encoders_amd import hip_attention as hip
    from packed_encoders_amd.workloads import GLOBAL, Workload

    lengths = (40, 60, 50, 30)
    w = Workload("T4", lengths, 2, 2, 64, (GLOBAL,), "four short documents")
    per_seg = [hip.useful_flops([n], 2, 64, window=(-1, -1)) for n in lengths]
    monkeypatch.setattr(bench, "CPU_STEP_FLOPS", per_seg[0] + per_seg[1] + 1)
    monkeypatch.setattr(bench, "CPU_ONE_THREAD_FLOPS", 1.0)
    r = bench.cpu_bench(w, repeats=1)
    assert "first 2 of 4 segments" in r["sample"] and "on the first 1 segment(s)" in r["sample"]
    assert r["value"] > 0 and r["one_thread"]["value"] > 0
    monkeypatch.setattr(bench, "CPU_STEP_FLOPS", 1e15)
    monkeypatch.setattr(bench, "CPU_ONE_THREAD_FLOPS", 1e15)
    r = bench.cpu_bench(w, repeats=1)
    assert r["sample"].startswith("full T4 schedule") and "on the first 4 segment(s)" in r["sample"]
