"""The packed ModernBERT path on the GPU: pack(), the packed forward, shared tile plans, the
bucketed HIP-graph runner and the varlen probe, against Hugging Face's own forward.

Oracles: the model's original forward in fp32 (what the reference validates against,
validate.py:129-170, tests/test_varlen.py:146-434 with random-init weights instead of a
download), the dense SDPA path of this package, and eager execution for graph replays
(tests/test_engine.py:29-73). A spy on the C ABI proves the HIP kernels ran (no silent
fallback) and counts the plan launches the shared-plan scope saves.
"""

from __future__ import annotations

import copy

import pytest
import torch

from conftest import announce

pytestmark = pytest.mark.gpu


def make_model(layers=4, hidden=128, heads=2, local_attention=16, seed=0):
    from transformers import ModernBertConfig, ModernBertModel

    torch.manual_seed(seed)
    cfg = ModernBertConfig(vocab_size=1024, hidden_size=hidden, intermediate_size=192, num_hidden_layers=layers,
                           num_attention_heads=heads, local_attention=local_attention, global_attn_every_n_layers=3,
                           pad_token_id=0, attn_implementation="sdpa")
    return ModernBertModel(cfg).eval()


def batch(lengths, vocab=1024, seed=1, device="cuda"):
    g = torch.Generator().manual_seed(seed)
    S = max(lengths)
    ids = torch.randint(1, vocab, (len(lengths), S), generator=g)
    mask = torch.zeros_like(ids)
    for i, n in enumerate(lengths):
        mask[i, :n] = 1
    return ids.to(device), mask.to(device)


def token_cosine(a, b):
    return torch.nn.functional.cosine_similarity(a.float(), b.float(), dim=-1)


class Spy:
    """Counts C-ABI calls made through the loaded library (wraps the ctypes functions)."""

    def __init__(self, monkeypatch):
        from packed_encoders_amd import _lib

        real = _lib.library()
        self.calls = {}
        self.short_launches = 0  # pe_attn_short_fwd calls that launch a kernel (pe_attn_kernels)
        spy = self

        class Proxy:
            def __getattr__(self, name):
                fn = getattr(real, name)
                if not name.startswith("pe_"):
                    return fn

                def wrapped(*args):
                    spy.calls[name] = spy.calls.get(name, 0) + 1
                    if name == "pe_attn_short_fwd":
                        import ctypes

                        out = (ctypes.c_int32 * 6)()
                        assert real.pe_attn_kernels(args[0], out) == 0
                        spy.short_launches += out[0] > 0
                    return fn(*args)

                return wrapped

        monkeypatch.setattr(_lib, "library", lambda path=None: Proxy())


def test_pack_hip_validates_and_matches_hf_fp32(pe, monkeypatch):
    announce("pack hip vs HF fp32")
    ref = make_model().cuda()
    model = copy.deepcopy(ref).to(torch.bfloat16)
    ids, mask = batch([300, 37, 129, 5, 64])
    with torch.no_grad():
        want = ref(input_ids=ids, attention_mask=mask).last_hidden_state
    pe.pack(model, attention_backend="hip", validate=True)
    report = model._packed_encoders.validation_report
    assert min(report.cosine_by_seq_len.values()) >= 0.98
    assert report.pieces["attention_bshd"].skipped_reason is None
    assert report.pieces["attention_bshd"].max_abs_error <= 2e-2
    spy = Spy(monkeypatch)
    with torch.no_grad():
        got = model(input_ids=ids, attention_mask=mask).last_hidden_state
    live = mask.bool()
    cos = token_cosine(got[live], want[live])
    assert cos.min() >= 0.995, cos.min()
    assert cos.mean() >= 0.999, cos.mean()
    # 4 layers = 2 global + 2 local: one plan per window kind, a short and a tiled launch per layer
    assert spy.calls.get("pe_attn_plan") == 2
    assert spy.calls.get("pe_attn_tiled_fwd") == 4 and spy.calls.get("pe_attn_short_fwd") == 4
    pe.unpack(model)


def test_packed_forward_hip_matches_dense_fallback(pe):
    from packed_encoders_amd import forward

    announce("packed_forward hip vs sdpa fallback")
    model = make_model(layers=3).cuda().to(torch.bfloat16)
    params = pe.config.ModernBertParams.from_hf_config(model.config)
    ids, mask = batch([513, 1, 90, 257, 33], seed=3)
    flat, _, cu, max_seqlen, positions = forward.unpad(ids, mask)
    with torch.no_grad():
        hip = forward.packed_forward(model, params, flat, cu, max_seqlen, positions, backend="hip")
        dense = forward.packed_sdpa_fallback(model, params, flat, cu, max_seqlen, positions)
    cos = token_cosine(hip, dense)
    assert cos.min() >= 0.995 and cos.mean() >= 0.999, (cos.min(), cos.mean())


def test_packed_graph_runner_replays_match_eager(pe):
    """Graph replays equal eager execution (and each other, bit for bit), and match the
    Hugging Face forward of the same weights in fp32 at the bar of the pack() test."""
    announce("packed graph runner")
    ref = make_model().cuda()
    model = copy.deepcopy(ref).to(torch.bfloat16)
    config = pe.GraphConfig(max_batch=8, max_seq=512, pad_to=64, warmup=2)
    pe.pack(model, attention_backend="hip", cuda_graph=config, validate=False)
    engine = pe.get_engine(model)
    from packed_encoders_amd import forward

    batches, hf = [], []
    for lengths, seed in (([300, 100, 37], 5), ([37, 300, 90], 6), ([200, 200, 27], 7)):
        ids, mask = batch(lengths, seed=seed)
        flat, _, cu, max_seqlen, positions = forward.unpad(ids, mask)
        batches.append(pe.PackedBatch(flat, cu, max_seqlen, positions))
        with torch.no_grad():
            hf.append(ref(input_ids=ids, attention_mask=mask).last_hidden_state[mask.bool()])
    # same (M bucket, N) for all three; max_seqlen differs for the third
    with torch.no_grad():
        eager = []
        with pe.no_cuda_graph(model):
            for b in batches:
                eager.append(engine.forward_packed(b))
        runner = model._packed_encoders.packed_graph_runner
        first = [None] * len(batches)
        for rep in range(3):
            for i, (b, want) in enumerate(zip(batches, eager)):
                got = engine.forward_packed(b)
                torch.cuda.synchronize()
                # the graph runs the dense layers at the bucketed token count (their GEMMs may
                # round differently); attention rows are computed identically
                cos = token_cosine(got, want)
                assert cos.min() >= 0.999, (rep, i, cos.min())
                if first[i] is None:
                    first[i] = got
                    fp32 = token_cosine(got, hf[i])
                    assert fp32.min() >= 0.995 and fp32.mean() >= 0.999, (i, fp32.min(), fp32.mean())
                else:
                    assert torch.equal(got, first[i]), f"replay {rep} of batch {i} is not deterministic"
                _ = torch.randn(1000, device="cuda").sum()  # unrelated eager work between replays
    assert runner.captures == 2  # (448, 3, 300) shared by the first two batches; (448, 3, 200)
    pe.unpack(model)


def test_select_attention_picks_hip_for_gqa_causal_and_windows(pe):
    announce("select_attention")
    for kw in (dict(n_heads=8, n_kv_heads=2, head_dim=256, causal=True),
               dict(n_heads=12, n_kv_heads=12, head_dim=64, causal=False, window=(64, 64)),
               dict(n_heads=4, n_kv_heads=1, head_dim=128, causal=False, window=(10, 3))):
        choice = pe.select_attention(device=torch.device("cuda"), **kw)
        assert choice.name == "hip", choice.rejected
        assert choice.max_abs_err < 2e-2
        if kw["causal"]:
            # the prefixed form (queries the tail of longer key segments) runs the HIP kernels too
            assert choice.prefixed_name == "hip", choice.rejected
            assert choice.prefixed_max_abs_err < 2e-2
    choice = pe.select_attention(device=torch.device("cuda"), n_heads=8, n_kv_heads=2, head_dim=64, causal=True,
                                 window=(32, -1), bidirectional_prefixed=True)
    assert choice.name == "hip" and choice.prefixed_name == "hip", choice.rejected


def test_modernbert_base_shape_packed_forward(pe):
    """The C2 model shape (22 layers, hidden 768, 12 x 64, local 128) on a few documents."""
    from transformers import ModernBertConfig, ModernBertModel
    from packed_encoders_amd import forward

    announce("ModernBERT-base shape")
    torch.manual_seed(0)
    cfg = ModernBertConfig(vocab_size=50368, hidden_size=768, intermediate_size=1152, num_hidden_layers=22,
                           num_attention_heads=12, local_attention=128, global_attn_every_n_layers=3,
                           attn_implementation="sdpa")
    model = ModernBertModel(cfg).eval().cuda().to(torch.bfloat16)
    params = pe.config.ModernBertParams.from_hf_config(cfg)
    assert params.head_dim == 64 and params.sliding_half_window == 64
    ids, mask = batch([400, 1200, 35, 700, 64, 2048], vocab=50368, seed=9)
    flat, _, cu, max_seqlen, positions = forward.unpad(ids, mask)
    with torch.no_grad():
        hip = forward.packed_forward(model, params, flat, cu, max_seqlen, positions, backend="hip")
        dense = forward.packed_sdpa_fallback(model, params, flat, cu, max_seqlen, positions)
    cos = token_cosine(hip, dense)
    assert torch.isfinite(hip).all()
    assert cos.min() >= 0.99 and cos.mean() >= 0.999, (cos.min(), cos.mean())


def test_c2_full_batch_forward_matches_hf_fp32(pe, monkeypatch):
    """The headline workload end to end: ModernBERT-base (22 layers, hidden 768, 12 x 64, random
    init) on C2's full batch of 64 documents through ``pe.pack`` with the collator's host
    lengths, against Hugging Face's fp32 forward of the same weights (each document on its own,
    no padding), per token. The bf16 dense SDPA path of this package on the same packed batch
    is the control: the HIP path must be at least as close to fp32, up to a small margin. The
    C-ABI spy checks the launches are the benchmark step's: two tile plans, one tiled call per
    layer and no short pass (the shortest document, 98 tokens, is past the boundary of 64)."""
    from transformers import ModernBertConfig, ModernBertModel

    from packed_encoders_amd import forward, workloads

    announce("C2 full batch, 22 layers, vs HF fp32")
    wl = workloads.c2()
    lengths = list(wl.lengths)
    cfg = ModernBertConfig(vocab_size=50368, hidden_size=768, intermediate_size=1152, num_hidden_layers=22,
                           num_attention_heads=12, local_attention=128, global_attn_every_n_layers=3,
                           global_rope_theta=160000.0, local_rope_theta=10000.0, attn_implementation="sdpa")
    torch.manual_seed(0)
    ref = ModernBertModel(cfg).eval().cuda()
    model = copy.deepcopy(ref).to(torch.bfloat16)
    g = torch.Generator().manual_seed(77)
    ids = torch.randint(0, cfg.vocab_size, (sum(lengths),), generator=g).cuda()
    c = wl.cu_seqlens()
    cu = torch.tensor(c, dtype=torch.int32, device="cuda")
    positions = torch.cat([torch.arange(n, device="cuda") for n in lengths])
    want = torch.empty(sum(lengths), cfg.hidden_size, device="cuda")
    with torch.no_grad():
        for a, b in zip(c, c[1:]):
            want[a:b] = ref(input_ids=ids[a:b][None]).last_hidden_state[0]
    del ref
    pe.pack(model, attention_backend="hip", validate=False)
    engine = pe.get_engine(model)
    spy = Spy(monkeypatch)
    with torch.no_grad(), pe.no_cuda_graph(model):
        got = engine.forward_packed(pe.PackedBatch(ids, cu, max(lengths), positions, host_lengths=tuple(lengths)))
    assert spy.calls.get("pe_attn_plan") == 2 and spy.calls.get("pe_attn_tiled_fwd") == 22
    assert spy.short_launches == 0, spy.short_launches
    params = pe.config.ModernBertParams.from_hf_config(cfg)
    with torch.no_grad():
        dense = forward.packed_sdpa_fallback(model, params, ids, cu, max(lengths), positions)
    pe.unpack(model)
    assert torch.isfinite(got).all()
    cos, cos_dense = token_cosine(got, want), token_cosine(dense, want)
    print(f"[c2 vs fp32] hip min {cos.min():.5f} mean {cos.mean():.6f}; "
          f"bf16 sdpa min {cos_dense.min():.5f} mean {cos_dense.mean():.6f}", flush=True)
    assert cos.mean() >= 0.999 and cos.min() >= 0.99, (cos.min(), cos.mean())
    assert cos.mean() >= cos_dense.mean() - 2e-4 and cos.min() >= cos_dense.min() - 5e-3


def test_padded_forward_with_a_host_mask_never_synchronises(pe):
    """A host attention mask takes the staged layout (one pinned non-blocking copy): the padded
    forward then makes no device-to-host synchronisation (torch's sync debug mode turns one into
    an error; the device-mask path, which does synchronise, is the negative control) and
    returns exactly what the device-mask path returns. No mask at all is sync-free too."""
    announce("host-mask forward without syncs")
    model = make_model().cuda().to(torch.bfloat16)
    pe.pack(model, attention_backend="hip", validate=False)
    ids, mask = batch([300, 37, 129, 5, 64], seed=11)
    mask_host = mask.cpu()
    with torch.no_grad():
        want = model(input_ids=ids, attention_mask=mask).last_hidden_state
        model(input_ids=ids, attention_mask=mask_host)  # warm-up: allocations, library load
        torch.cuda.synchronize()
        torch.cuda.set_sync_debug_mode("error")
        try:
            got = model(input_ids=ids, attention_mask=mask_host).last_hidden_state
            dense = model(input_ids=ids).last_hidden_state
            # negative control: the device-mask path's syncs are caught by the same mode
            with pytest.raises(RuntimeError):
                model(input_ids=ids, attention_mask=mask)
        finally:
            torch.cuda.set_sync_debug_mode(0)
        torch.cuda.synchronize()
    assert torch.equal(got, want)
    with torch.no_grad():
        dense_want = model(input_ids=ids, attention_mask=torch.ones_like(ids)).last_hidden_state
    assert torch.equal(dense, dense_want)
    pe.unpack(model)
