"""Host-side logic of the packed path, on the CPU: configuration, unpad/repad, backend
resolution, the dispatch score tables, pieces, the varlen probe's SDPA candidate, graph
staging, and pack()/unpack() with the dense 'sdpa' path against Hugging Face's own forward.

Known answers restate the reference's tests: tests/test_varlen.py:42-121 (unpad/repad),
tests/test_attention_dispatch_score.py:15-146 (policy boundaries), tests/test_engine.py and
tests/test_registry.py (install/restore). No kernel launches here.
"""

from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

import packed_encoders_amd as pe
from packed_encoders_amd import attention_dispatch, forward, graph, ops, pieces, runtime_attention
from packed_encoders_amd.config import ModernBertParams, global_every, rope_thetas
from packed_encoders_amd.errors import PackedEncodersError, UnsupportedTargetError, ValidationError

BASE = ModernBertParams(hidden_size=768, num_attention_heads=12, num_hidden_layers=22, norm_eps=1e-5,
                        global_rope_theta=160_000.0, local_rope_theta=10_000.0, local_attention=128,
                        global_attn_every_n_layers=3)


def tiny_model(layers=4, hidden=64, heads=2, local_attention=8, seed=0):
    from transformers import ModernBertConfig, ModernBertModel

    torch.manual_seed(seed)
    cfg = ModernBertConfig(vocab_size=512, hidden_size=hidden, intermediate_size=96, num_hidden_layers=layers,
                           num_attention_heads=heads, local_attention=local_attention, global_attn_every_n_layers=3,
                           pad_token_id=0, attn_implementation="sdpa")
    return ModernBertModel(cfg).eval()


# ----------------------------------------------------------------------------- config


def test_params_follow_modernbert_base_schedule():
    assert BASE.head_dim == 64 and BASE.scaling == 0.125 and BASE.sliding_half_window == 64
    globals_ = [i for i in range(22) if BASE.is_global_layer(i)]
    assert globals_ == [0, 3, 6, 9, 12, 15, 18, 21]  # 8 global, 14 local
    assert BASE.window(0) == (-1, -1) and BASE.window(1) == (64, 64)


def test_config_schema_variants():
    m = tiny_model()
    p = ModernBertParams.from_hf_config(m.config)
    assert p.global_attn_every_n_layers == 3
    assert (p.global_rope_theta, p.local_rope_theta) == (160_000.0, 10_000.0)

    class Old:  # transformers 4.x fields
        model_type = "modernbert"
        global_rope_theta, local_rope_theta, global_attn_every_n_layers = 80_000.0, 5_000.0, 2
        layer_types = None

    assert rope_thetas(Old) == (80_000.0, 5_000.0) and global_every(Old) == 2

    class Bad:
        layer_types = ["sliding_attention", "full_attention"]

    with pytest.raises(ValueError):
        global_every(Bad)

    class NotBert:
        model_type = "bert"

    with pytest.raises(ValueError):
        ModernBertParams.from_hf_config(NotBert)


def test_global_period_is_the_smallest_period_of_layer_types():
    """global_every against a brute-force search over every full/sliding pattern of up to 8
    layers: the smallest n with "layer i is global iff i % n == 0", and ValueError when none is."""
    import itertools
    from types import SimpleNamespace

    for n_layers in range(1, 9):
        for bits in itertools.product((False, True), repeat=n_layers):
            kinds = ["full_attention" if b else "sliding_attention" for b in bits]
            want = next((n for n in range(1, n_layers + 1) if all(b == (i % n == 0) for i, b in enumerate(bits))),
                        None)
            cfg = SimpleNamespace(layer_types=kinds)
            if want is None:
                with pytest.raises(ValueError):
                    global_every(cfg)
            else:
                assert global_every(cfg) == want, kinds


def test_rope_bases_per_field_and_schema():
    from types import SimpleNamespace as NS

    assert rope_thetas(NS(global_rope_theta=1.0, local_rope_theta=None,
                          rope_parameters={"sliding_attention": {"rope_theta": 2.0}})) == (1.0, 2.0)
    assert rope_thetas(NS(rope_parameters={"full_attention": {"rope_theta": 3.0}}, rope_theta=4.0)) == (3.0, 4.0)
    assert rope_thetas(NS()) == (160_000.0, 160_000.0)


# ----------------------------------------------------------------------------- unpad / repad


def test_unpad_shapes_and_positions():
    am = torch.tensor([[1, 1, 1, 1, 1], [1, 1, 0, 0, 0], [1, 1, 1, 1, 0]], dtype=torch.long)
    x = torch.arange(3 * 5 * 4, dtype=torch.float32).reshape(3, 5, 4)
    packed, indices, cu, max_seqlen, positions = forward.unpad(x, am)
    assert packed.shape == (11, 4)
    assert cu.tolist() == [0, 5, 7, 11] and cu.dtype == torch.int32
    assert max_seqlen == 5
    assert torch.equal(packed, torch.stack([x[b, s] for b in range(3) for s in range(5) if am[b, s]]))
    assert positions.tolist() == [s for b in range(3) for s in range(5) if am[b, s]]


def test_unpad_repad_roundtrip_and_identity_order():
    am = torch.tensor([[1, 1, 1, 0], [1, 0, 0, 0], [1, 1, 1, 1]], dtype=torch.long)
    x = torch.randn(3, 4, 8)
    packed, indices, *_ = forward.unpad(x, am)
    back = forward.repad(packed, indices, 3, 4)
    m = am.bool().unsqueeze(-1).expand_as(x)
    assert torch.equal(back[m], x[m]) and torch.equal(back[~m], torch.zeros_like(back[~m]))
    packed, _, cu, _, positions = forward.unpad(torch.randn(2, 3, 5), torch.ones(2, 3, dtype=torch.long))
    assert packed.shape == (6, 5) and cu.tolist() == [0, 3, 6] and positions.tolist() == [0, 1, 2, 0, 1, 2]


def test_host_layouts_match_the_device_style_unpad():
    """staging.padded_layout_host (the sync-free path's layout) equals what unpad computes from
    the same mask, for right padding, holes, left padding and empty rows; packed_layout_host
    restarts positions per sequence."""
    from packed_encoders_amd import staging

    g = torch.Generator().manual_seed(3)
    masks = [torch.tensor([[1, 1, 1, 0, 0], [1, 1, 1, 1, 1], [0, 0, 0, 0, 0], [0, 1, 1, 0, 1]]),
             (torch.rand(6, 9, generator=g) > 0.4).long()]
    for am in masks:
        x = torch.randn(*am.shape, 3, generator=g)
        _, want_idx, want_cu, want_max, want_pos = forward.unpad(x, am)
        idx, cu, pos, mx = staging.padded_layout_host(am)
        assert torch.equal(idx, want_idx) and torch.equal(cu.to(torch.int32), want_cu)
        assert torch.equal(pos, want_pos) and mx == want_max
    cu, pos = staging.packed_layout_host([3, 0, 2, 1])
    assert cu.tolist() == [0, 3, 3, 5, 6] and pos.tolist() == [0, 1, 2, 0, 1, 0]
    with pytest.raises(ValueError):
        staging.padded_layout_host(torch.ones(3, dtype=torch.long))


def test_unpad_without_a_mask_is_the_identity_layout():
    x = torch.randn(2, 5, 3)
    packed, idx, cu, mx, pos = forward.unpad(x, None)
    assert torch.equal(packed, x.reshape(10, 3)) and idx.tolist() == list(range(10))
    assert cu.tolist() == [0, 5, 10] and cu.dtype == torch.int32 and mx == 5
    assert pos.tolist() == [0, 1, 2, 3, 4] * 2


def test_packed_sdpa_fallback_repads_and_restores_packed_order(monkeypatch):
    ids = torch.tensor([11, 12, 21, 31, 32, 33])
    cu = torch.tensor([0, 2, 3, 6], dtype=torch.int32)
    positions = torch.tensor([0, 1, 0, 0, 1, 2])
    seen = {}

    def fake_fused(_model, _params, padded_ids, mask, *, backend, execution=None):
        seen.update(ids=padded_ids.clone(), mask=mask.clone(), backend=backend)
        return padded_ids.unsqueeze(-1).expand(*padded_ids.shape, 2)

    monkeypatch.setattr(forward, "fused_forward", fake_fused)
    out = forward.packed_sdpa_fallback(object(), object(), ids, cu, 3, positions)
    assert seen["backend"] == "sdpa"
    assert seen["ids"].tolist() == [[11, 12, 0], [21, 0, 0], [31, 32, 33]]
    assert seen["mask"].tolist() == [[1, 1, 0], [1, 0, 0], [1, 1, 1]]
    assert out[:, 0].tolist() == ids.tolist()


# ----------------------------------------------------------------------------- backend resolution


def test_backend_resolution_is_host_only_and_falls_back_outside_the_invariants():
    cpu = torch.device("cpu")
    assert forward.resolve_backend("sdpa", BASE, device=cpu, dtype=torch.bfloat16) == "sdpa"
    # CPU / fp32 / autograd are outside the HIP kernels' invariants
    assert forward.resolve_backend("hip", BASE, device=cpu, dtype=torch.bfloat16) == "sdpa"
    with pytest.raises(ValueError):
        forward.resolve_backend("flash", BASE, device=cpu, dtype=torch.bfloat16)


def test_attention_workload_from_mask():
    ids = torch.zeros((3, 8), dtype=torch.long)
    mask = torch.tensor([[1] * 8, [1] * 5 + [0] * 3, [1] * 2 + [0] * 6], dtype=torch.long)
    w = forward.attention_workload(BASE, ids, mask)
    assert (w.n_sequences, w.live_tokens, w.max_seqlen, w.rectangle_tokens, w.fragmentation_tokens) == (3, 15, 8, 24, 9)
    w = forward.packed_workload(total_tokens=35, n_sequences=3, max_seqlen=20)
    assert w.fragmentation_tokens == 25


def _workload(lengths):
    return attention_dispatch.AttentionWorkload.from_lengths(lengths)


def test_packed_inference_policy_is_the_gfx950_policy_and_none_elsewhere():
    """The reference's entry point answers with this architecture's calibrated policy only:
    gfx950 by its compute capability (9, 5) or its name; NVIDIA cards and other AMD parts get
    None (no crossover is borrowed from another GPU)."""
    for cc, name in (((9, 5), "AMD Instinct MI355X"), ((9, 5), ""), ((0, 0), "AMD Instinct MI350X")):
        policy = attention_dispatch.get_packed_inference_policy(cc, name)
        assert policy is not None and policy.arch == "gfx950"
        assert attention_dispatch.get_packed_inference_policy(cc, name, for_cuda_graph=True) == policy
    for cc, name in (((12, 0), "NVIDIA GeForce RTX 5090"), ((8, 0), "NVIDIA A100-SXM4-40GB"),
                     ((9, 4), "AMD Instinct MI300X")):
        assert attention_dispatch.get_packed_inference_policy(cc, name) is None
    policy = attention_dispatch.get_packed_inference_policy((9, 5), "AMD Instinct MI355X")
    # the reference's per-batch question: does the batch need the long-segment kernel?
    assert not policy.use_flash(_workload((128,) * 160)) and not policy.use_flash(_workload((5, 100)))
    assert policy.use_flash(_workload((129, 3))) and policy.use_flash(_workload((2048,)))
    assert policy.use_flash(_workload((2048,)), head_dim=128)


def test_attention_workload_statistics_and_validation():
    w = _workload((5, 0, 12))
    assert (w.n_sequences, w.live_tokens, w.max_seqlen, w.rectangle_tokens, w.fragmentation_tokens) == (3, 17, 12, 36, 19)
    assert attention_dispatch.AttentionWorkload.from_summary(n_sequences=3, live_tokens=17, max_seqlen=12) == w
    for bad in (dict(n_sequences=2, live_tokens=33, max_seqlen=16), dict(n_sequences=0, live_tokens=0, max_seqlen=1),
                dict(n_sequences=1, live_tokens=-1, max_seqlen=4)):
        with pytest.raises(ValueError):
            attention_dispatch.AttentionWorkload.from_summary(**bad)
    with pytest.raises(ValueError):
        _workload(())


def test_gfx950_routing_policy():
    policy = attention_dispatch.get_hip_dispatch_policy("gfx950:sramecc+:xnack-")
    assert policy is not None and policy.short_max(64) == 64 and policy.short_max(256) == 0
    assert policy.short_max(64, max_seqlen=100) == 100 and policy.short_max(128, max_seqlen=128) == 128
    assert policy.short_max(64, max_seqlen=129) == 64 and policy.short_max(256, max_seqlen=50) == 0
    assert policy.short_max(128, max_seqlen=129) == 32
    short, tiled = policy.route([0, 10, 64, 65, 2048], 64)
    assert short == [1, 2] and tiled == [3, 4]
    short, tiled = policy.route([0, 10, 100, 128], 64)  # every segment fits the short kernel
    assert short == [1, 2, 3] and tiled == []
    assert attention_dispatch.get_hip_dispatch_policy("gfx942") is None
    assert [attention_dispatch.capacity_for(n) for n in (1, 32, 33, 64, 65, 128, 129)] == [32, 32, 64, 64, 128, 128, 0]


def test_library_default_routing_is_the_policy():
    """The C ABI's short_max = -1 routes exactly as the Python policy: same workspace (the tiled
    kernel's share) as an explicit short_max from HipDispatchPolicy.short_max."""
    import ctypes

    from packed_encoders_amd import _lib

    lib = _lib.library()
    policy = attention_dispatch.get_hip_dispatch_policy("gfx950")

    def ws(d, max_seqlen, short_max, n=64, t=20000):
        a = _lib.AttnArgs()
        a.struct_size, a.dtype = ctypes.sizeof(_lib.AttnArgs), 1
        a.n_seq, a.total_tokens, a.max_seqlen = n, t, max_seqlen
        a.n_heads_q = a.n_heads_kv = 8
        a.head_dim, a.softmax_scale = d, 0.1
        a.window_left = a.window_right = -1
        a.short_max = short_max
        size = ctypes.c_size_t()
        assert lib.pe_attn_workspace_size(ctypes.byref(a), ctypes.byref(size)) == 0
        return size.value

    for d in (64, 128, 256):
        for max_seqlen in (20, 64, 65, 128, 129, 300, 2048):
            for n in (64, 2000):  # with 2000 segments the workspace bound depends on the boundary
                want = ws(d, max_seqlen, policy.short_max(d, max_seqlen), n=n)
                assert ws(d, max_seqlen, -1, n=n) == want, (d, max_seqlen, n)
    assert ws(64, 100, -1) == 0  # all short: no tiled work at all
    assert ws(128, 300, 32, n=2000) != ws(128, 300, 64, n=2000)


def _sweep_rows():
    """The data table of profiles/dispatch_sweep.md (the committed gfx950 sweep)."""
    import pathlib

    text = (pathlib.Path(__file__).resolve().parents[1] / "profiles" / "dispatch_sweep.md").read_text()
    lines = [ln for ln in text.splitlines() if ln.startswith("|")]
    header = next(i for i, ln in enumerate(lines) if ln.startswith("| head_dim | heads |"))
    names = [c.strip() for c in lines[header].strip("|").split("|")]
    rows = []
    for ln in lines[header + 2:]:
        rows.append(dict(zip(names, (float(c) for c in ln.strip("|").split("|")))))
    return rows


def test_gfx950_boundaries_are_the_fit_of_the_committed_sweep():
    """The policy's boundaries are what fit_boundary derives from the committed sweep, and the
    all-short rule for batches of at most 128 tokens holds in every measured row."""
    rows = _sweep_rows()
    assert len(rows) == 52 and {int(r["head_dim"]) for r in rows} == {64, 128}
    policy = attention_dispatch.get_hip_dispatch_policy("gfx950")
    for d in (64, 128):
        assert attention_dispatch.fit_boundary(rows, d) == dict(policy.boundaries)[d], d
        assert policy.short_max(d, max_seqlen=4096) == attention_dispatch.fit_boundary(rows, d)
    for r in rows:
        assert r["short_us"] < r["tiled_us"], r
    # the fit responds to the data: make the tiled kernel free and it takes every segment
    assert attention_dispatch.fit_boundary([dict(r, tiled_us=0.0) for r in rows], 64) == 0
    assert attention_dispatch.fit_boundary(rows, 64, min_segments=10 ** 6) == 0


def _band_sweep_rows():
    """The data table of profiles/band_sweep.md (the committed gfx950 band sweep)."""
    import pathlib

    text = (pathlib.Path(__file__).resolve().parents[1] / "profiles" / "band_sweep.md").read_text()
    lines = text.splitlines()
    header = next(i for i, ln in enumerate(lines) if ln.startswith("| batch | n_seq |"))
    names = [c.strip() for c in lines[header].strip("|").split("|")]
    rows = []
    for ln in lines[header + 2:]:
        if not ln.startswith("|"):
            break  # the table ends at its first non-row line
        cells = [c.strip() for c in ln.strip("|").split("|")]
        rows.append({k: (v if k == "batch" else float(v)) for k, v in zip(names, cells)})
    return rows


def test_band_size_rule_is_the_fit_of_the_committed_sweep(pe):
    """The C library's band-kernel thresholds (streaming band kernel from kBandMinTiles query
    tiles, strip 8 from kBandStrip8Tiles) are what fit_band_rule derives from the committed
    band sweep: one tile below the threshold a +-64 call runs the tiled kernel, at it the band
    kernel at the fitted strip. The fit responds to the data."""
    import ctypes

    from packed_encoders_amd import _lib

    rows = _band_sweep_rows()
    assert len(rows) == 17
    t, s8 = attention_dispatch.fit_band_rule(rows)
    assert t is not None and s8 is not None and s8 >= t

    def kernels(tiles):
        a = _lib.AttnArgs()
        a.struct_size = ctypes.sizeof(_lib.AttnArgs)
        a.dtype, a.head_dim, a.n_heads_q, a.n_heads_kv = 1, 64, 1, 1
        a.n_seq, a.total_tokens, a.max_seqlen = 1, tiles * 128, tiles * 128
        a.softmax_scale, a.window_left, a.window_right, a.short_max = 0.125, 64, 64, -1
        out = (ctypes.c_int32 * 6)()
        assert _lib.library().pe_attn_kernels(ctypes.byref(a), out) == 0
        return out[1], out[2]

    assert kernels(t - 1) == (_lib.KERNEL_TILED, 1)
    assert kernels(t) == (_lib.KERNEL_BAND64, 8 if t >= s8 else 4)
    assert kernels(s8) == (_lib.KERNEL_BAND64, 8)
    # a free band kernel takes every row; a free tiled kernel none
    assert attention_dispatch.fit_band_rule([dict(r, band8_us=0.0) for r in rows]) == (0, 0)
    assert attention_dispatch.fit_band_rule([dict(r, tiled_us=0.0) for r in rows]) == (None, None)


# ----------------------------------------------------------------------------- pieces


def test_pieces_bind_checks_contracts_and_validate_catches_a_wrong_kernel():
    sel = pieces.default_pieces()
    ops_ = sel.bind()
    assert ops_.attention_bshd is ops.attention_bshd and ops_.rope_tables is ops.rope_tables
    with pytest.raises(UnsupportedTargetError):
        dataclasses.replace(sel, attention=sel.attention_bshd).bind()  # BSHD piece in the BHSD slot
    q, k, v = (torch.randn(1, 2, 9, 8) for _ in range(3))
    ok = sel.attention.validate(q, k, v, mask=None, window=(-1, -1), scaling=0.3, backend="sdpa")
    assert ok.max_abs_error < 1e-5
    wrong = dataclasses.replace(sel.attention, execute=lambda q, k, v, **kw: ops.sdpa_attention(q, k, v, None, 0.9))
    with pytest.raises(ValidationError):
        wrong.validate(q, k, v, mask=None, window=(-1, -1), scaling=0.3, backend="sdpa")


def test_attention_piece_oracle_respects_segments_and_band():
    torch.manual_seed(0)
    q, k, v = (torch.randn(1, 2, 12, 8) for _ in range(3))
    cu = torch.tensor([0, 5, 12], dtype=torch.int32)
    got = pieces.attention_reference(q, k, v, mask=None, window=(2, 2), scaling=0.35, backend="hip", cu_seqlens=cu,
                                     max_seqlen=7)
    for a, b in ((0, 5), (5, 12)):
        n = b - a
        pos = torch.arange(n)
        allowed = (pos[:, None] - pos[None, :]).abs() <= 2
        want = torch.nn.functional.scaled_dot_product_attention(q[:, :, a:b], k[:, :, a:b], v[:, :, a:b],
                                                                attn_mask=allowed, scale=0.35)
        assert torch.allclose(got[:, a:b], want.transpose(1, 2).reshape(1, n, -1), atol=1e-6)


# ----------------------------------------------------------------------------- varlen probe


def test_select_attention_sdpa_candidate_and_rejections_on_cpu():
    choice = runtime_attention.select_attention(n_heads=4, n_kv_heads=2, head_dim=16, causal=True,
                                                device=torch.device("cpu"), dtype=torch.float32,
                                                order=("hip", "sdpa"), window=(3, -1))
    assert choice.name == "sdpa" and "hip" in choice.rejected
    assert choice.prefixed_name == "sdpa" and choice.max_abs_err < 1e-5
    # the padded [real | pad] form agrees with the packed form on real rows
    q, k, v = torch.randn(2 * 6, 4, 16), torch.randn(12, 2, 16), torch.randn(12, 2, 16)
    static = runtime_attention.PaddedStatic(rows=2, seq=6, ids=torch.zeros(2, 6, dtype=torch.long),
                                            seg_cu32=torch.tensor([0, 4, 6, 9, 12], dtype=torch.int32),
                                            lens=torch.tensor([4, 3], dtype=torch.int32))
    padded = choice.padded(q, k, v, static, True)
    keep = torch.tensor([0, 1, 2, 3, 6, 7, 8])
    packed = choice.packed(q[keep], k[keep], v[keep], torch.tensor([0, 4, 7], dtype=torch.int32), 4, [4, 3], True)
    assert torch.allclose(padded[keep], packed, atol=1e-5)


@pytest.mark.parametrize("window,causal", [((-1, -1), False), ((5, 3), False), ((-1, -1), True), ((4, -1), True),
                                           ((0, 0), False)])
def test_probe_oracle_and_bucketed_sdpa_match_the_numpy_oracle(window, causal, monkeypatch):
    """The selector's float64 oracle (one masked score matrix from segment ids) and the SDPA
    candidate (length-bucketed padded batches, several buckets forced by a small budget) against
    oracle/attention.py's per-segment loops, with GQA, empty and one-token segments, and query
    segments that are the tails of longer key segments."""
    from oracle import attention as oa

    monkeypatch.setattr(runtime_attention, "_SDPA_BUCKET_ELEMENTS", 4 * 40 * 40)
    g = torch.Generator().manual_seed(5)
    lengths_q, lengths_k = [7, 0, 1, 33, 12, 40], [7, 3, 9, 33, 30, 40]
    q = torch.randn(sum(lengths_q), 4, 8, generator=g, dtype=torch.float64)
    k = torch.randn(sum(lengths_k), 2, 8, generator=g, dtype=torch.float64)
    v = torch.randn(sum(lengths_k), 2, 8, generator=g, dtype=torch.float64)
    cu_q = np.cumsum([0] + lengths_q)
    cu_k = np.cumsum([0] + lengths_k)
    want = oa.packed_attention(q.numpy(), k.numpy(), v.numpy(), cu_q, scale=0.3, window=window, causal=causal,
                               cu_seqlens_k=cu_k)
    got = runtime_attention.oracle_attention(q, k, v, lengths_q, lengths_k, causal, window, 0.3).numpy()
    np.testing.assert_allclose(got, want, atol=1e-12)
    got = runtime_attention.bucketed_sdpa(q.float(), k.float(), v.float(), lengths_q, lengths_k, causal, window, 0.3)
    np.testing.assert_allclose(got.double().numpy(), want, atol=2e-5)


def test_sigmoid_gate_rounding():
    o = torch.randn(10, 4).bfloat16()
    g = torch.randn(10, 4)
    want = (o.float() * torch.sigmoid(g).bfloat16().float()).bfloat16()
    assert torch.equal(runtime_attention.sigmoid_gate(o, g.bfloat16()), want) or \
        (runtime_attention.sigmoid_gate(o, g.bfloat16()).float() - want.float()).abs().max() < 1e-2


# ----------------------------------------------------------------------------- graph staging


def test_packed_static_inputs_stage_fills_tails():
    s = graph.PackedStaticInputs(input_ids=torch.full((8,), 7), cu_seqlens=torch.full((4,), 9, dtype=torch.int32),
                                 position_ids=torch.full((8,), 5), max_seqlen=4)
    m = s.stage(torch.tensor([1, 2, 3, 4, 5]), torch.tensor([0, 3, 5], dtype=torch.int32), torch.tensor([0, 1, 2, 0, 1]))
    assert m == 5
    assert s.input_ids.tolist() == [1, 2, 3, 4, 5, 0, 0, 0]
    assert s.position_ids.tolist() == [0, 1, 2, 0, 1, 0, 0, 0]
    assert s.cu_seqlens.tolist() == [0, 3, 5, 5]
    assert graph.round_up(65, 64) == 128 and graph.round_up(64, 64) == 64
    # a longer batch, then a shorter one: the rows the longer one wrote are zeroed again
    s.stage(torch.arange(1, 9), torch.tensor([0, 8], dtype=torch.int32), torch.arange(8))
    assert s.written == 8 and s.cu_seqlens.tolist() == [0, 8, 8, 8]
    s.stage(torch.tensor([9, 9]), torch.tensor([0, 1, 2], dtype=torch.int32), torch.tensor([0, 0]))
    assert s.input_ids.tolist() == [9, 9, 0, 0, 0, 0, 0, 0] and s.position_ids.tolist() == [0] * 8
    assert s.cu_seqlens.tolist() == [0, 1, 2, 2]


def test_packed_layout_host_against_per_sequence_counting():
    from packed_encoders_amd import staging

    g = np.random.default_rng(5)
    for _ in range(100):
        lengths = g.choice([0, 0, 1, 2, 5, 17], size=g.integers(0, 12)).tolist()
        cu, pos = staging.packed_layout_host(lengths)
        assert cu.tolist() == [0, *np.cumsum(lengths, dtype=np.int64).tolist()]
        assert pos.tolist() == [p for n in lengths for p in range(n)]
    with pytest.raises(ValueError):
        staging.packed_layout_host([3, -1])


def test_graph_runner_needs_bounded_config():
    m = tiny_model()
    p = ModernBertParams.from_hf_config(m.config)
    assert graph.build_packed_runner(m, p, graph.GraphConfig(), backend="hip") is None
    assert graph.build_packed_runner(m, p, graph.GraphConfig(max_batch=8, max_seq=64), backend="sdpa") is None
    r = graph.build_packed_runner(m, p, graph.GraphConfig(max_batch=8, max_seq=64, pad_to=32), backend="hip")
    assert r is not None
    assert r.admits(100, 8, 64) and not r.admits(100, 9, 64) and not r.admits(100, 8, 65)
    assert r.key(65, 3, 40) == (96, 3, 40, "sdpa")  # CPU model: the key records the resolved backend


# ----------------------------------------------------------------------------- pack / unpack


def test_pack_sdpa_matches_hf_and_unpack_restores():
    m = tiny_model()
    ids = torch.randint(1, 512, (3, 20))
    mask = torch.ones_like(ids)
    mask[1, 12:] = 0
    mask[2, 5:] = 0
    with torch.no_grad():
        want = m(input_ids=ids, attention_mask=mask).last_hidden_state
    original = m.forward
    pe.pack(m, attention_backend="sdpa", validate=False)
    assert "forward" in m.__dict__
    with torch.no_grad():
        got = m(input_ids=ids, attention_mask=mask).last_hidden_state
    live = mask.bool()
    assert torch.allclose(got[live], want[live], atol=2e-4, rtol=2e-4)
    # the packed entry with the dense fallback gives the same rows
    flat, _, cu, max_seqlen, positions = forward.unpad(ids, mask)
    engine = pe.get_engine(m)
    with torch.no_grad():
        packed = engine.forward_packed(pe.PackedBatch(flat, cu, max_seqlen, positions))
    assert torch.allclose(packed, want[live], atol=2e-4, rtol=2e-4)
    pe.unpack(m)
    assert "forward" not in m.__dict__ and m.forward == original
    with pytest.raises(PackedEncodersError):
        pe.get_engine(m)


def test_pack_rejects_unavailable_backends_and_wrong_targets():
    m = tiny_model()
    for backend in ("flash", "triton", "cuda"):
        with pytest.raises(PackedEncodersError):
            pe.pack(m, attention_backend=backend, validate=False)
    with pytest.raises(PackedEncodersError):
        pe.pack(m, attention_backend="hip", validate=False)  # CPU weights (or no HIP library)
    with pytest.raises(UnsupportedTargetError):
        pe.pack(torch.nn.Linear(2, 2))
    assert "forward" not in m.__dict__


def test_pack_locates_the_backbone_in_wrappers():
    from transformers import ModernBertForMaskedLM

    m = tiny_model()
    task = ModernBertForMaskedLM(m.config).eval()
    pe.pack(task, attention_backend="sdpa", validate=False)
    assert "forward" in task.model.__dict__
    pe.unpack(task)
    assert "forward" not in task.model.__dict__


def test_pack_validation_gate_on_cpu():
    m = tiny_model(layers=3)
    pe.pack(m, attention_backend="sdpa", validate=True)
    report = m._packed_encoders.validation_report
    assert min(report.cosine_by_seq_len.values()) > 0.999
    assert report.pieces["attention"].max_abs_error is not None
    assert report.pieces["attention_bshd"].skipped_reason
    pe.unpack(m)
