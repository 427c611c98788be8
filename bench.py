#!/usr/bin/env python3
"""Benchmark of the packed varlen attention path on one MI355X.

Default workload (the one the baseline metric is quoted on): the attention of a ModernBERT-base
packed batch — 64 documents, lengths LogNormal(400, 0.8) clipped to [32, 2048], 12 heads x 64,
22 layers (every 3rd global, the rest a +-64 band), bf16. A step is one pass of those 22
attention calls over synthetic per-layer Q/K/V already resident in HBM, each call the full
library path through the C ABI on the current stream: the short kernel and the tiled MFMA
kernel per layer, plus one device-built tile plan per window kind (global, +-64), which every
layer of that kind shares as a packed forward does. ``value`` is useful attention TFLOP/s
(live token pairs only, ``4*D*H*pairs``); ``tokens_per_s`` is packed tokens through all 22
attention layers per second.

The dominant kernel (the tiled kernel of the global layers) is bracketed with HIP events
recorded on the stream it is launched on, inside the timed region; its algorithmic FLOPs per
launch over the average launch time give ``roofline.achieved``. The CPU baseline times the same
schedule on the host's cores with the reference's own CPU kernel (oracle/_ref) for the band and
short-global layers and per-segment fp32 torch SDPA for global layers longer than 128 (the
reference's rule).

For C2 and C1 the line also carries ``end_to_end``: the whole packed ModernBERT-base forward
(random-init weights, bf16) over the same batch through ``pe.pack``, eager and replayed from
the bucketed HIP-graph runner, in tokens/s (C1's short batch is the launch-bound case graphs
exist for).

Before the W warm-up steps the step runs untimed for ``--settle`` seconds (0.3 by default,
reported as ``settle_s``): an idle MI355X measures up to 10% slower over its first ~10 ms of
load, which a 20-step timed region of a sub-millisecond step would otherwise include.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload C2] [--no-cpu-baseline]
                       [--no-model] [--settle S]
"""

from __future__ import annotations

import argparse
import ctypes
import itertools
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "useful attn TFLOP/s & tokens/s, ModernBERT-base packed batch, 1 MI355X; % of roofline"
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def compulsory_bytes(total_tokens: int, n_seq: int, hq: int, hkv: int, d: int, gate: bool) -> int:
    """Read Q, K, V once and write O once (bf16), plus the gate and cu_seqlens."""
    b = 2 * total_tokens * d * (2 * hq + 2 * hkv) + 4 * (n_seq + 1)
    if gate:
        b += 2 * total_tokens * hq * d
    return b


class LayerCall:
    """One attention call: pre-allocated tensors and C-ABI arguments, launched stage by stage.

    Layers with the same window kind share one tile plan (workspace): the plan depends only on
    cu_seqlens, the window and the head geometry, so a packed forward builds it once per kind
    (twice for ModernBERT: global and +-64) and every layer of that kind reuses it."""

    def __init__(self, lib, hip, workload, layer, cu, q, k, v, gate, short_max, plans, strip=0, min_seqlen=True):
        import torch

        self.lib, self.layer = lib, layer
        self.out = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)
        # The host knows the batch's lengths (it built cu_seqlens from them), so it passes the
        # shortest beside max_seqlen, as a collator does.
        shortest = min(workload.lengths) if min_seqlen and workload.lengths else 0
        self.args = hip._args(q, k, v, self.out, cu, workload.max_seqlen, workload.scale, layer.window[0],
                              layer.window[1], layer.causal, gate, short_max, strip, min_seqlen=shortest)
        size = ctypes.c_size_t()
        rc = lib.pe_attn_workspace_size(ctypes.byref(self.args), ctypes.byref(size))
        assert rc == 0, rc
        self.ws_bytes = size.value
        kind = (layer.window, layer.causal)
        self.plans_here = kind not in plans  # the first layer of a kind builds the shared plan
        if self.plans_here:
            plans[kind] = torch.empty(max(1, size.value), dtype=torch.uint8, device=q.device)
        self.ws = plans[kind]
        self.keep = (q, k, v, gate, cu)

    def short(self, stream):
        rc = self.lib.pe_attn_short_fwd(ctypes.byref(self.args), stream)
        if rc:
            raise RuntimeError(f"pe_attn_short_fwd: {rc}")

    def plan(self, stream):
        rc = self.lib.pe_attn_plan(ctypes.byref(self.args), self.ws.data_ptr(), self.ws_bytes, stream)
        if rc:
            raise RuntimeError(f"pe_attn_plan: {rc}")

    def tiled(self, stream):
        rc = self.lib.pe_attn_tiled_fwd(ctypes.byref(self.args), self.ws.data_ptr(), self.ws_bytes, stream)
        if rc:
            raise RuntimeError(f"pe_attn_tiled_fwd: {rc}")


def dominant(workload, short_max):
    """(stage, bound, layer indices) of the kernel the roofline is for: the tiled kernel of the
    global layers when there are any (MFMA-bound), else the kernel of the windowed/causal
    layers (HBM-bound), or the short kernel when every segment is short."""
    long_layers = [i for i, l in enumerate(workload.layers) if l.window == (-1, -1) and not l.causal]
    if workload.max_seqlen <= short_max:
        return "short", "hbm", list(range(len(workload.layers)))
    if long_layers and not any(l.gate for l in workload.layers):
        return "tiled", "mfma", long_layers
    return "tiled", "hbm", list(range(len(workload.layers)))


def useful_flops_served(workload, short_max, kernel):
    """Useful FLOPs per launch of ``kernel`` (the short kernel or the long-segment kernel of the
    dominant layer): 4 D Hq sum(allowed pairs) over the segments it serves."""
    from packed_encoders_amd import hip_attention as hip

    _, _, timed = dominant(workload, short_max)
    layer = workload.layers[timed[0]]
    short = kernel.startswith("pe::short_attn_kernel")
    served = [n for n in workload.lengths if (n <= short_max) == short]
    return hip.useful_flops(served, workload.n_heads_q, workload.head_dim, window=layer.window, causal=layer.causal)


def kernel_instance(lib, call, workload):
    """The name rocprofv3 lists (template arguments included) for the kernels of one layer's
    call, as the library reports its choice (pe_attn_kernels): (short kernel, long kernel)."""
    from packed_encoders_amd import _lib

    out = (ctypes.c_int32 * 6)()
    rc = lib.pe_attn_kernels(ctypes.byref(call.args), out)
    if rc:
        raise RuntimeError(f"pe_attn_kernels: {rc}")
    layer, d = call.layer, workload.head_dim
    gate = str(layer.gate).lower()
    win = str(layer.window != (-1, -1) or layer.causal).lower()
    g = math.gcd(workload.n_heads_q // workload.n_heads_kv, 4)
    short = None
    if out[0]:
        short = f"pe::short_attn_kernel<{d}, {out[0]}, {out[4]}, {gate}>"
    long = {
        _lib.KERNEL_NONE: None,
        _lib.KERNEL_TILED: f"pe::tiled_attn_kernel<64, {g}, 64, 3, {gate}, {win}>",
        _lib.KERNEL_GLOBAL64: f"pe::global64_attn_kernel<{g}, {gate}>",
        _lib.KERNEL_BAND64: f"pe::band64_attn_kernel<{gate}>",
        _lib.KERNEL_WIDE: f"pe::wide_attn_kernel<128, {g}, 64, 2, {gate}, {win}>",
        _lib.KERNEL_WIDE16: f"pe::wide16_attn_kernel<256, 4, {g}, 2, {gate}, {win}>",
    }[out[1]]
    return short, long


def settle(step, seconds: float) -> float:
    """Run `step` untimed until `seconds` of wall time have passed (synchronising every few
    steps); returns the time spent. An idle MI355X reaches its sustained clock and memory
    behaviour only after some load: the first ~10 ms of a kernel stream measure up to 10% slower
    than the same kernels a few hundred milliseconds in (measured on the band kernel: 303 us
    cold against 266-273 us warm for the same launch). Settling first makes a short timed
    region report the steady state a continuously serving process sees."""
    import torch

    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(4):
            step()
        torch.cuda.synchronize()
    return time.perf_counter() - t0


def gpu_bench(args, workload):
    import torch

    import packed_encoders_amd as pe
    from packed_encoders_amd import _lib, hip_attention as hip
    from packed_encoders_amd.attention_dispatch import hip_short_max

    lib = _lib.library()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    short_max = (hip_short_max(workload.head_dim, max_seqlen=workload.max_seqlen) if args.short_max is None
                 else args.short_max)
    cu = torch.tensor(workload.cu_seqlens(), dtype=torch.int32, device=dev)
    T, hq, hkv, d = workload.total_tokens, workload.n_heads_q, workload.n_heads_kv, workload.head_dim
    log(f"{workload.name}: T={T} segments={len(workload.lengths)} max={workload.max_seqlen} heads={hq}/{hkv}x{d} "
        f"layers={len(workload.layers)} short_max={short_max}")
    gen = torch.Generator(device=dev).manual_seed(1234)
    calls, plans = [], {}
    for layer in workload.layers:
        q = torch.randn(T, hq, d, device=dev, generator=gen, dtype=torch.bfloat16)
        k = torch.randn(T, hkv, d, device=dev, generator=gen, dtype=torch.bfloat16)
        v = torch.randn(T, hkv, d, device=dev, generator=gen, dtype=torch.bfloat16)
        g = torch.randn(T, hq, d, device=dev, generator=gen, dtype=torch.bfloat16) if layer.gate else None
        calls.append(LayerCall(lib, hip, workload, layer, cu, q, k, v, g, short_max, plans, args.strip,
                               not args.no_min_seqlen))
    stage, bound, timed_layers = dominant(workload, short_max)
    stream = torch.cuda.current_stream(dev)

    timed_set = set(timed_layers)
    # Stages with no segment to serve are not called (host-known: every segment is at most
    # max_seqlen tokens long), which keeps an all-short batch at one library call per layer.
    has_short = 0 < short_max and d <= 128
    has_tiled = workload.max_seqlen > (short_max if has_short else 0)

    def bracket(fn, events, sp):
        e0, e1 = events.pop()
        e0.record(stream)
        fn(sp)
        e1.record(stream)
        timed.append((e0, e1))

    def step(events=None, sp=stream.cuda_stream):
        for i, c in enumerate(calls):
            here = events is not None and i in timed_set
            if has_short:
                bracket(c.short, events, sp) if here and stage == "short" else c.short(sp)
            if has_tiled:
                if c.plans_here:
                    c.plan(sp)
                bracket(c.tiled, events, sp) if here and stage == "tiled" else c.tiled(sp)

    timed = []
    settle_s = settle(step, args.settle)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    pool = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            for _ in range(args.steps * len(timed_layers))]
    # an event at every step boundary: per-step GPU times for the samples' median and spread
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    marks[0].record(stream)
    for i in range(args.steps):
        step(pool)
        marks[i + 1].record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    wall_ms = (t1 - t0) * 1e3 / args.steps
    gpu_ms = marks[0].elapsed_time(marks[-1]) / args.steps
    per_step = [a.elapsed_time(b) for a, b in zip(marks, marks[1:])]
    kernel_times = [a.elapsed_time(b) for a, b in timed]
    kernel_ms = statistics.mean(kernel_times)

    # The same step captured once into a HIP graph and replayed: the launch cost a serving loop
    # that captures its packed forward pays (no host work per kernel).
    graph_ms = None
    if not args.no_graph:
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream(dev)  # default priority
        side.wait_stream(stream)
        with torch.cuda.graph(graph, stream=side):
            step(sp=side.cuda_stream)
        stream.wait_stream(side)
        graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            graph.replay()
        torch.cuda.synchronize()
        graph_ms = (time.perf_counter() - t0) * 1e3 / args.steps
        del graph

    # Algorithmic work: all layers for the value; the dominant kernel's own segments for the roofline.
    flops = sum(hip.useful_flops(workload.lengths, hq, d, window=l.window, causal=l.causal) for l in workload.layers)
    if stage == "tiled":
        served = [n for n in workload.lengths if n > short_max]
    else:
        served = [n for n in workload.lengths if n <= short_max]
    layer0 = workload.layers[timed_layers[0]]
    if bound == "mfma":
        per_launch = hip.useful_flops(served, hq, d, window=layer0.window, causal=layer0.causal)
        achieved = per_launch / (kernel_ms * 1e-3) / 1e12
        peak, unit = PEAK_BF16_TFLOPS, "TFLOP/s"
    else:
        per_launch = compulsory_bytes(sum(served), len(served), hq, hkv, d, layer0.gate)
        achieved = per_launch / (kernel_ms * 1e-3) / 1e9
        peak, unit = PEAK_HBM_GBS, "GB/s"
    short_name, long_name = kernel_instance(lib, calls[timed_layers[0]], workload)
    kernel_name = short_name if stage == "short" else long_name
    roofline = {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
                "frac": round(achieved / peak, 4), "traffic": traffic_from_profiles(workload.name, kernel_name),
                "kernel": kernel_name, "kernel_ms": round(kernel_ms, 4), "algorithmic_per_launch": per_launch}
    value = flops / (wall_ms * 1e-3) / 1e12
    log(f"wall {wall_ms:.3f} ms/step (events {gpu_ms:.3f}, graph replay {graph_ms}), {value:.1f} TFLOP/s, "
        f"dominant {kernel_name} {kernel_ms * 1e3:.1f} us -> {achieved:.1f} {unit} ({achieved / peak:.1%})")
    replay = None if graph_ms is None else {
        "ms_per_step": round(graph_ms, 4), "value": round(flops / (graph_ms * 1e-3) / 1e12, 3),
        "tokens_per_s": round(workload.total_tokens / (graph_ms * 1e-3), 1)}
    roofline["kernel_ms_median"] = round(statistics.median(kernel_times), 4)
    measured = achieved_peaks()
    if measured is not None:  # this card's sustained rate (profiles/peaks.md), beside the spec peak
        # the highest sustained rate of its kind (random-data MFMA; the faster of read and copy)
        top = (measured["bf16_mfma_tflops_random"] if bound == "mfma"
               else max(measured["hbm_read_gbs"], measured["hbm_copy_gbs_read_plus_write"]))
        roofline["achieved_peak"] = top
        roofline["frac_of_achieved_peak"] = round(achieved / top, 4)
    return {
        "samples": step_samples(per_step, args.samples), "value": value, "ms_per_step": wall_ms,
        "gpu_ms_per_step": gpu_ms, "flops_per_step": flops,
        "graph_replay": replay, "settle_s": round(settle_s, 3),
        "tokens_per_s": workload.total_tokens / (wall_ms * 1e-3), "roofline": roofline, "short_max": short_max,
        "min_seqlen": int(calls[0].args.min_seqlen),
        "_outputs": (calls, cu),
    }


def step_samples(per_step: list[float], n: int) -> dict:
    """The timed steps' GPU times (HIP events at every step boundary) cut into ``n`` consecutive
    samples of equal step counts: each sample's mean ms per step, their median and their spread
    ((max - min) / median), as the reference's dispatch benchmark reports medians of repeated
    samples (benchmarks/packed_attention_dispatch_bench.py:169-229)."""
    n = max(1, min(n, len(per_step)))
    size = len(per_step) // n
    means = [statistics.mean(per_step[i * size:(i + 1) * size]) for i in range(n)]
    med = statistics.median(means)
    return {"n": n, "steps_each": size, "ms_per_step": [round(m, 4) for m in means],
            "median_ms_per_step": round(med, 4), "spread": round((max(means) - min(means)) / med, 4)}


def sanity_check(calls, workload, cu):
    """Part of the CPU leg: a sample of the timed GPU outputs' rows against the oracle."""
    import numpy as np

    from oracle import attention as oa

    c = calls[0]
    q, k, v, gate, _ = c.keep
    rows = np.linspace(0, workload.total_tokens - 1, 48).astype(np.int64)
    layer = c.layer
    want = oa.sampled_rows_attention(q.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(),
                                     cu.cpu().numpy(), rows, scale=workload.scale, window=layer.window,
                                     causal=layer.causal)
    got = c.out.float().cpu().numpy()[rows]
    if gate is not None:
        want = oa.sigmoid_gate(oa.to_bf16(want), gate.float().cpu().numpy()[rows])
    err = float(np.abs(got - want).max())
    if not err <= 2e-2:
        raise SystemExit(f"bench output check failed: max-abs {err}")


def model_bench(args, workload):
    """End-to-end ModernBERT-base (random init, bf16) over the workload's packed batch: the
    packed forward through ``pe.pack`` (embeddings, 22 layers with this library's attention,
    final norm), eager and replayed from the bucketed HIP-graph runner. Returns tokens/s and
    ms per forward of both, timed with events around K forwards after W warm-ups."""
    import torch
    from transformers import ModernBertConfig, ModernBertModel

    import packed_encoders_amd as pe
    from packed_encoders_amd import forward

    dev = torch.device("cuda", 0)
    torch.manual_seed(0)
    cfg = ModernBertConfig(vocab_size=50368, hidden_size=768, intermediate_size=1152, num_hidden_layers=22,
                           num_attention_heads=12, local_attention=128, global_attn_every_n_layers=3,
                           global_rope_theta=160000.0, local_rope_theta=10000.0, attn_implementation="sdpa")
    model = ModernBertModel(cfg).eval().to(dev, torch.bfloat16)
    lengths = workload.lengths
    g = torch.Generator(device=dev).manual_seed(77)
    ids = torch.randint(0, cfg.vocab_size, (sum(lengths),), device=dev, generator=g)
    cu = torch.tensor(workload.cu_seqlens(), dtype=torch.int32, device=dev)
    positions = torch.cat([torch.arange(n, device=dev) for n in lengths])
    batch = pe.PackedBatch(ids, cu, max(lengths), positions, host_lengths=tuple(lengths))  # as a collator gives
    gcfg = pe.GraphConfig(max_batch=len(lengths), max_seq=max(lengths), pad_to=256, warmup=2)
    pe.pack(model, attention_backend="hip", cuda_graph=gcfg, validate=False)
    engine = pe.get_engine(model)
    stream = torch.cuda.current_stream(dev)

    def timed(fn):
        settle(fn, args.settle)
        for _ in range(max(args.warmup, 2)):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for _ in range(args.steps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) * 1e3 / args.steps
        return wall, e0.elapsed_time(e1) / args.steps

    res = {"model": "ModernBERT-base, 22 layers, hidden 768, 12x64, GeGLU 1152, vocab 50368, random init, bf16",
           "tokens": workload.total_tokens}
    with torch.no_grad():
        with pe.no_cuda_graph(model):
            wall, gpu = timed(lambda: engine.forward_packed(batch))
            eager_out = engine.forward_packed(batch)
        res["eager_ms"] = round(wall, 3)
        res["eager_tokens_per_s"] = round(workload.total_tokens / (wall * 1e-3), 1)
        wall, gpu = timed(lambda: engine.forward_packed(batch))
        graph_out = engine.forward_packed(batch)
        res["graph_ms"] = round(wall, 3)
        res["graph_tokens_per_s"] = round(workload.total_tokens / (wall * 1e-3), 1)
        cos = torch.nn.functional.cosine_similarity(graph_out.float(), eager_out.float(), dim=-1)
        res["graph_vs_eager_min_cosine"] = round(float(cos.min()), 5)
    log(f"model: eager {res['eager_ms']:.2f} ms ({res['eager_tokens_per_s'] / 1e6:.2f} M tokens/s), "
        f"graph {res['graph_ms']:.2f} ms ({res['graph_tokens_per_s'] / 1e6:.2f} M tokens/s)")
    pe.unpack(model)
    return res


def traffic_from_profiles(workload_name: str, kernel: str):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary (profiles/traffic.json),
    or None when there is none for this kernel or it was measured on other kernel sources (the
    table carries the source digest it was measured at)."""
    from packed_encoders_amd._build import source_digest

    path = ROOT / "profiles" / "traffic.json"
    try:
        table = json.loads(path.read_text())
    except (OSError, ValueError):
        return None
    if table.get("source_digest") != source_digest():
        log(f"profiles/traffic.json was measured at sources {table.get('source_digest')}, "
            f"not {source_digest()}: traffic not reported")
        return None
    entry = table.get("kernels", {}).get(f"{workload_name}:{kernel}")
    return None if entry is None else entry.get("hbm_bytes_per_launch")


def cpu_threads() -> int:
    from oracle import cpu

    cores = cpu.physical_cores()
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        cores = min(cores, int(env))
    return max(1, cores)


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or the platform's processor string."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


# FLOPs the CPU leg's timed step may take (the whole schedule up to this, else whole segments
# from the front of the batch), and the 1-thread run's sample: about 1 s and 1-3 s of CPU work
# per repeat on the GPU boxes' 16 threads, so the default run stays within minutes.
CPU_STEP_FLOPS = 1.0e12
CPU_ONE_THREAD_FLOPS = 1.0e11


def cpu_bench(workload, repeats: int = 7):
    """The same attention schedule on the host CPU (fp32): one warm-up, then the median of
    ``repeats`` timed steps on all physical cores (benchmarks/cpu/README.md:27-31), and a
    1-thread run on a bounded sample (the first global and the first banded layer, median of
    3) scaled to the same unit. A schedule past CPU_STEP_FLOPS (C4's global layer: 4.4e12) is
    timed on the whole segments at the front of the batch that fit it, the 1-thread run on
    those that fit CPU_ONE_THREAD_FLOPS (at least one); TFLOP/s is a rate, so a sample of whole
    segments measures it without scaling."""
    import numpy as np
    import torch
    import torch.nn.functional as F

    from oracle import cpu
    from packed_encoders_amd import hip_attention as hip

    cpu.build()
    kind = "reference" if cpu.available("reference") and workload.head_dim == 64 else "port"
    threads = cpu_threads()
    T, hq, d = workload.total_tokens, workload.n_heads_q, workload.head_dim
    if workload.n_heads_kv != hq:
        return None
    gen = torch.Generator().manual_seed(99)
    q_all, k_all, v_all = (torch.randn(hq, T, d, generator=gen) for _ in range(3))
    all_lengths = list(workload.lengths)

    def front(layers, cap: float) -> int:
        """Whole segments from the front of the batch whose FLOPs over `layers` fit `cap`."""
        n, acc = 0, 0.0
        for length in all_lengths:
            f = sum(hip.useful_flops([length], hq, d, window=l.window) for l in layers)
            if n and acc + f > cap:
                break
            n, acc = n + 1, acc + f
        return n

    q = k = v = qn = kn = vn = out = lengths = longest = offsets = None

    def use(n_seg: int):
        """Time the first n_seg segments from here on (contiguous fp32 copies of their rows)."""
        nonlocal q, k, v, qn, kn, vn, out, lengths, longest, offsets
        lengths = all_lengths[:n_seg]
        t = sum(lengths)
        q, k, v = (x[:, :t].contiguous() for x in (q_all, k_all, v_all))
        qn, kn, vn = (x.numpy() for x in (q, k, v))
        out = np.empty((hq, t, d), dtype=np.float32)
        longest = max(lengths)
        offsets = np.concatenate([[0], np.cumsum(lengths)])

    def layer_call(layer, n_threads):
        if layer.causal or layer.gate or layer.window[0] != layer.window[1]:
            raise ValueError("CPU baseline covers symmetric bands and global attention")
        if layer.window != (-1, -1):
            cpu.local_attention(qn, kn, vn, lengths, layer.window[0], kind=kind, threads=n_threads, out=out,
                                scale=workload.scale)
        elif longest <= 128:
            cpu.local_attention(qn, kn, vn, lengths, longest, kind=kind, threads=n_threads, out=out,
                                scale=workload.scale)
        else:  # per-segment fp32 SDPA, as the reference's CPU engine does for long global layers
            with torch.inference_mode():
                for a, b in zip(offsets, offsets[1:]):
                    F.scaled_dot_product_attention(q[None, :, a:b], k[None, :, a:b], v[None, :, a:b],
                                                   scale=workload.scale)

    def timed(layers, n_threads, n):
        torch.set_num_threads(n_threads)
        for layer in layers:  # warm-up
            layer_call(layer, n_threads)
        times = []
        for _ in range(n):
            t0 = time.perf_counter()
            for layer in layers:
                layer_call(layer, n_threads)
            times.append(time.perf_counter() - t0)
        return statistics.median(times)

    n_step = front(workload.layers, CPU_STEP_FLOPS)
    use(n_step)
    seconds = timed(workload.layers, threads, repeats)
    flops = sum(hip.useful_flops(lengths, hq, d, window=l.window) for l in workload.layers)
    step_t = sum(lengths)
    # 1 thread: one layer of each kind present, on the segments that fit its cap
    kinds = []
    for layer in workload.layers:
        if layer not in kinds:
            kinds.append(layer)
    n_one = min(n_step, front(kinds, CPU_ONE_THREAD_FLOPS))
    use(n_one)
    one_flops = sum(hip.useful_flops(lengths, hq, d, window=l.window) for l in kinds)
    one_seconds = timed(kinds, 1, 3)
    one_tflops = one_flops / one_seconds / 1e12
    model = cpu_model()
    whole = n_step == len(all_lengths)
    what = (f"full {workload.name} schedule ({len(workload.layers)} attention layers, T={T})" if whole else
            f"{workload.name} schedule ({len(workload.layers)} attention layers) on its first {n_step} of "
            f"{len(all_lengths)} segments (T={step_t} of {T}, {flops:.3g} of the step's FLOPs)")
    sample = (f"{what} in fp32 on {threads} threads (physical cores of the affinity mask), median of {repeats} "
              f"after 1 warm-up; band/short layers: "
              f"{'reference pe_local_attention (oracle/_ref)' if kind == 'reference' else 'oracle C port'}; "
              f"global layers longer than 128: per-segment torch SDPA. 1-thread: one layer of each kind "
              f"({len(kinds)}) on the first {n_one} segment(s), median of 3")
    log(f"cpu baseline ({kind}, {threads} threads, {model}): {seconds * 1e3:.1f} ms/step -> "
        f"{flops / seconds / 1e12:.3f} TFLOP/s; 1 thread {one_tflops:.4f} TFLOP/s")
    return {"value": round(flops / seconds / 1e12, 4), "unit": "TFLOP/s", "cores": threads, "kind": kind,
            "sample": sample, "ms_per_step": round(seconds * 1e3, 2), "repeats": repeats, "cpu_model": model,
            "nproc": os.cpu_count(), "one_thread": {"value": round(one_tflops, 5), "unit": "TFLOP/s",
                                                    "ms_per_sample": round(one_seconds * 1e3, 2),
                                                    "layers": len(kinds)}}


def copy_calibration(steps: int) -> int:
    """A plain device copy of known size: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of this run,
    divided by the bytes moved, is the factor that turns those counters into HBM bytes."""
    import torch

    n = 1 << 30
    src = torch.ones(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / max(1, steps)
    print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "launches": steps,
                      "ms_per_copy": round(dt * 1e3, 4), "GBps_read_plus_write": round(2 * n / dt / 1e9, 1)}))
    return 0


def _workload(name: str):
    def make():
        from packed_encoders_amd import workloads as w

        return {"C1": w.c1, "C2": w.c2, "C3": w.c3, "C3-shuffled": lambda: w.c3(shuffled=True), "C4": w.c4,
                "C4-band": lambda: w.c4(band=True), "C5": w.c5, "Q4096": w.query_sweep}[name]()

    return make


WORKLOADS = {name: _workload(name) for name in ("C1", "C2", "C3", "C3-shuffled", "C4", "C4-band", "C5", "Q4096")}
PROFILED = ("C1", "Q4096", "C2", "C3", "C3-shuffled", "C4", "C4-band", "C5")
SQ_PASSES = {  # two counter passes of at most 8 SQ counters (plus GRBM) each
    "SQA": "SQ_WAVES SQ_BUSY_CYCLES SQ_WAVE_CYCLES SQ_INSTS_VALU SQ_INSTS_MFMA SQ_INSTS_LDS SQ_INSTS_SALU "
           "SQ_WAIT_INST_ANY GRBM_GUI_ACTIVE",
    "SQB": "SQ_VALU_MFMA_BUSY_CYCLES SQ_VALU_MFMA_COEXEC_CYCLES SQ_ACTIVE_INST_VALU SQ_ACTIVE_INST_LDS "
           "SQ_WAIT_INST_LDS SQ_LDS_BANK_CONFLICT SQ_INSTS_VALU_MFMA_MOPS_BF16 SQ_BUSY_CU_CYCLES GRBM_GUI_ACTIVE",
}
MFMA_PROFILED = ("C2", "C3", "C4", "C4-band", "C5")  # SQ counter passes (MFMA and VALU use, waits)
KERNEL_PROFILED = ("C3-shuffled",)  # kernel trace only


def profile_commands(out: str = "gpurun_out/prof") -> list[tuple[str, str]]:
    """(name, command) of every rocprofv3 run the committed summaries under profiles/ come from,
    run from the repository root with TMPDIR=/tmp. ``--summarize-profiles`` reads their output."""
    cmds = []
    for pmc in ("FETCH_SIZE", "WRITE_SIZE"):
        cmds.append((f"copy_{pmc}", f"rocprofv3 --pmc {pmc} --output-format csv -d {out}/copy_{pmc} -o p -- "
                                    f"python3 bench.py --copy-calibration --steps 3"))
    for w in PROFILED:
        run = f"python3 bench.py --workload {w} --no-cpu-baseline --no-model"
        cmds.append((f"{w}_kt", f"rocprofv3 --kernel-trace --stats --output-format csv -d {out}/{w}_kt -o k -- "
                                f"{run} --steps 10 --warmup 2"))
        if w in KERNEL_PROFILED:
            continue
        run += " --no-graph --settle 0.05"  # counter passes: eager launches, short settle
        for pmc in ("FETCH_SIZE", "WRITE_SIZE"):
            cmds.append((f"{w}_{pmc}", f"rocprofv3 --pmc {pmc} --output-format csv -d {out}/{w}_{pmc} -o p -- "
                                       f"{run} --steps 2 --warmup 1"))
        if w in MFMA_PROFILED:
            for name, counters in SQ_PASSES.items():
                cmds.append((f"{w}_{name}", f"rocprofv3 --pmc {counters} --output-format csv -d {out}/{w}_{name} "
                                            f"-o p -- {run} --steps 2 --warmup 1"))
    return cmds


def _kernel_label(name: str) -> str:
    """``void pe::x<...>(pe::AttnParams)`` -> ``pe::x<...>`` (the name kernel_instance gives)."""
    name = name.strip()
    if name.startswith("void "):
        name = name[5:]
    return name[: -len("(pe::AttnParams)")] if name.endswith("(pe::AttnParams)") else name


def _counters(path: Path) -> dict[str, dict[str, list[float]]]:
    """{kernel: {counter: [value per dispatch]}} from a rocprofv3 counter_collection CSV."""
    import csv

    per: dict[str, dict[str, dict[str, float]]] = {}
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            k = _kernel_label(r["Kernel_Name"])
            per.setdefault(k, {}).setdefault(r["Counter_Name"], {})
            per[k][r["Counter_Name"]][r["Dispatch_Id"]] = float(r["Counter_Value"])
    return {k: {c: list(v.values()) for c, v in cs.items()} for k, cs in per.items()}


def summarize_profiles(src: Path) -> int:
    """Write profiles/<W>_kernel_trace_stats.md, profiles/<W>_hbm_traffic.md,
    profiles/<W>_mfma_counters.md and profiles/traffic.json from the output of
    ``profile_commands`` under ``src`` (a missing run is skipped). HBM bytes are FETCH_SIZE and
    WRITE_SIZE (KiB per dispatch) scaled by what the same counters read for the 1 GiB copy of
    ``--copy-calibration``; traffic.json carries the source digest of the kernels measured."""
    import csv

    import packed_encoders_amd as pe
    from packed_encoders_amd._build import source_digest

    cmds = dict(profile_commands())
    digest = source_digest()
    prof = ROOT / "profiles"
    copy_bytes = 1 << 30
    scale = {}
    for pmc in ("FETCH_SIZE", "WRITE_SIZE"):
        table = _counters(src / f"copy_{pmc}" / "p_counter_collection.csv")
        per_copy = max(max(v[pmc]) for v in table.values() if pmc in v)  # the 1 GiB copies
        scale[pmc] = copy_bytes / (per_copy * 1024)
    workloads = WORKLOADS
    traffic = {"source_digest": digest,
               "calibration": {"copy_bytes": copy_bytes, "fetch_scale": round(scale["FETCH_SIZE"], 4),
                               "write_scale": round(scale["WRITE_SIZE"], 4)},
               "kernels": {}}
    header = (f"Kernel sources: digest `{digest}` (`packed_encoders_amd._build.source_digest()`). One MI355X "
              f"(gfx950); commands run from the repository root with TMPDIR=/tmp.\n")
    for w in PROFILED:
        kt_dir = src / f"{w}_kt"
        line_path = src / f"{w}_kt.json"
        if not (kt_dir / "k_kernel_stats.csv").exists() or not line_path.exists():
            continue
        wl = workloads[w]()
        bench_line = json.loads(line_path.read_text().strip().splitlines()[-1])
        roof = bench_line["roofline"]
        with open(kt_dir / "k_kernel_stats.csv", newline="") as f:
            stats = [r for r in csv.DictReader(f)]
        ours = [r for r in stats if _kernel_label(r["Name"]).startswith("pe::")]
        total_pct = sum(float(r["Percentage"]) for r in ours)
        dom = next((r for r in ours if _kernel_label(r["Name"]) == roof["kernel"]), None)
        out = [f"# {w}: kernel trace statistics (rocprofv3 --kernel-trace --stats)\n",
               f"Workload: {wl.description}; T = {wl.total_tokens} tokens, {len(wl.lengths)} segments.\n",
               header, "```", f"{cmds[f'{w}_kt']} > gpurun_out/prof/{w}_kt.json", "```\n",
               "| kernel | calls | average us | min us | max us | % of GPU time |", "|---|---|---|---|---|---|"]
        for r in ours:
            out.append(f"| `{_kernel_label(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                       f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} | {float(r['Percentage']):.1f} |")
        out.append(f"\nThe library's kernels take {total_pct:.1f}% of the profiled run's GPU time (the rest is "
                   f"input set-up: torch.randn).\n")
        out.append(f"The bench line of the same run: dominant kernel `{roof['kernel']}`, "
                   f"{roof['kernel_ms'] * 1e3:.1f} us per launch with HIP events on its stream"
                   + (f" (trace average {float(dom['AverageNs']) / 1e3:.1f} us, ratio "
                      f"{roof['kernel_ms'] * 1e6 / float(dom['AverageNs']):.3f})" if dom else "")
                   + f"; {roof['achieved']} {roof['unit']} = {roof['frac']:.1%} of {roof['peak']} {roof['unit']} "
                   f"({roof['bound']}-bound). Step: {bench_line['ms_per_step']:.4f} ms wall "
                   f"({bench_line['gpu_ms_per_step']:.4f} ms events), "
                   f"{bench_line['graph_replay']['ms_per_step']:.4f} ms replayed from a HIP graph.")
        (prof / f"{w}_kernel_trace_stats.md").write_text("\n".join(out) + "\n")

        fetch_p = src / f"{w}_FETCH_SIZE" / "p_counter_collection.csv"
        write_p = src / f"{w}_WRITE_SIZE" / "p_counter_collection.csv"
        if fetch_p.exists() and write_p.exists():
            fetch, write = _counters(fetch_p), _counters(write_p)
            out = [f"# {w}: HBM traffic per launch (rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE)\n", header,
                   "```", cmds[f"{w}_FETCH_SIZE"], cmds[f"{w}_WRITE_SIZE"], cmds["copy_FETCH_SIZE"],
                   cmds["copy_WRITE_SIZE"], "```\n",
                   f"Calibration: for the 1 GiB device copy (1,048,576 KiB read and written) FETCH_SIZE reads "
                   f"{copy_bytes / 1024 / scale['FETCH_SIZE']:,.0f} KiB and WRITE_SIZE "
                   f"{copy_bytes / 1024 / scale['WRITE_SIZE']:,.0f} KiB per copy, so HBM bytes = FETCH_SIZE x "
                   f"{scale['FETCH_SIZE']:.3f} x 1024 and WRITE_SIZE x {scale['WRITE_SIZE']:.3f} x 1024.\n",
                   "| kernel | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM read MB | HBM write MB | "
                   "HBM total MB |", "|---|---|---|---|---|---|---|"]
            for k in sorted(fetch):
                if not k.startswith("pe::") or k not in write:
                    continue
                f_kib = statistics.mean(fetch[k]["FETCH_SIZE"])
                w_kib = statistics.mean(write[k]["WRITE_SIZE"])
                rd, wr = f_kib * 1024 * scale["FETCH_SIZE"], w_kib * 1024 * scale["WRITE_SIZE"]
                traffic["kernels"][f"{w}:{k}"] = {"hbm_bytes_per_launch": round(rd + wr), "read_bytes": round(rd),
                                                  "write_bytes": round(wr)}
                out.append(f"| `{k}` | {len(fetch[k]['FETCH_SIZE'])} | {f_kib:,.1f} | {w_kib:,.1f} | "
                           f"{rd / 1e6:.2f} | {wr / 1e6:.2f} | {(rd + wr) / 1e6:.2f} |")
            entry = traffic["kernels"].get(f"{w}:{roof['kernel']}")
            if entry:
                cut = bench_line["config"]["short_max"]
                short_kernel = roof["kernel"].startswith("pe::short_attn_kernel")
                served = [n for n in wl.lengths if (n <= cut) == short_kernel]
                need = compulsory_bytes(sum(served), len(served), wl.n_heads_q, wl.n_heads_kv, wl.head_dim,
                                        any(l.gate for l in wl.layers))
                out.append(f"\nDominant kernel `{roof['kernel']}`: {entry['hbm_bytes_per_launch'] / 1e6:.2f} MB "
                           f"per launch against {need / 1e6:.2f} MB compulsory (Q, K, V read once, O written "
                           f"once{', gate read once' if any(l.gate for l in wl.layers) else ''}): "
                           f"{entry['hbm_bytes_per_launch'] / need:.2f}x; at the event-timed "
                           f"{roof['kernel_ms'] * 1e3:.1f} us that is "
                           f"{entry['hbm_bytes_per_launch'] / (roof['kernel_ms'] * 1e-3) / 1e9:,.0f} GB/s of HBM.")
            (prof / f"{w}_hbm_traffic.md").write_text("\n".join(out) + "\n")

        a_p, b_p = src / f"{w}_SQA" / "p_counter_collection.csv", src / f"{w}_SQB" / "p_counter_collection.csv"
        if a_p.exists() and b_p.exists():
            a, b = _counters(a_p).get(roof["kernel"]), _counters(b_p).get(roof["kernel"])
            if a and b:
                m = {c: statistics.mean(v) for c, v in {**a, **b}.items()}
                mfma = m["SQ_INSTS_MFMA"]
                flops = m["SQ_INSTS_VALU_MFMA_MOPS_BF16"] * 512
                xcd_cycles = m["GRBM_GUI_ACTIVE"] / 8  # GRBM_GUI_ACTIVE sums the 8 XCDs
                out = [f"# {w}: MFMA utilisation of `{roof['kernel']}` (rocprofv3 --pmc)\n", header, "```",
                       cmds[f"{w}_SQA"], cmds[f"{w}_SQB"], "```\n",
                       f"Means per dispatch over {len(a['SQ_INSTS_MFMA'])} dispatches of the dominant kernel.\n",
                       "| counter | per dispatch |", "|---|---|"]
                for c in sorted(m):
                    out.append(f"| {c} | {m[c]:,.0f} |")
                useful = useful_flops_served(wl, bench_line["config"]["short_max"], roof["kernel"])
                out += ["", "| derived | value |", "|---|---|",
                        f"| MFMA FLOPs (MOPS_BF16 x 512) | {flops:.4g} (useful {useful:.4g}) |",
                        f"| MFMA pipe busy / (4 SIMDs x SQ_BUSY_CU_CYCLES) | "
                        f"{m['SQ_VALU_MFMA_BUSY_CYCLES'] / (4 * m['SQ_BUSY_CU_CYCLES']):.3f} |",
                        f"| MFMA pipe busy / (1024 SIMDs x GRBM_GUI_ACTIVE / 8) | "
                        f"{m['SQ_VALU_MFMA_BUSY_CYCLES'] / (1024 * xcd_cycles):.3f} |",
                        f"| VALU co-issued with MFMA / MFMA busy | "
                        f"{m['SQ_VALU_MFMA_COEXEC_CYCLES'] / m['SQ_VALU_MFMA_BUSY_CYCLES']:.3f} |",
                        f"| non-MFMA VALU / SALU / LDS instructions per MFMA | "
                        f"{(m['SQ_INSTS_VALU'] - mfma) / mfma:.2f} / {m['SQ_INSTS_SALU'] / mfma:.2f} / "
                        f"{m['SQ_INSTS_LDS'] / mfma:.2f} |",
                        f"| SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES | {m['SQ_WAIT_INST_ANY'] / m['SQ_WAVE_CYCLES']:.3f} |",
                        f"| LDS bank conflicts / LDS instructions | "
                        f"{m['SQ_LDS_BANK_CONFLICT'] / m['SQ_INSTS_LDS']:.3f} |",
                        "", f"Event-timed in the bench line of the kernel-trace run: {roof['kernel_ms'] * 1e3:.1f} us, "
                        f"{useful / (roof['kernel_ms'] * 1e-3) / 1e12:.1f} useful TFLOP/s = "
                        f"{useful / (roof['kernel_ms'] * 1e-3) / 2.5e15:.1%} of the 2.5 PFLOP/s dense bf16 peak; "
                        f"its roofline ({roof['bound']}-bound): {roof['achieved']} {roof['unit']} = "
                        f"{roof['frac']:.1%} of {roof['peak']} {roof['unit']}."]
                (prof / f"{w}_mfma_counters.md").write_text("\n".join(out) + "\n")
    (prof / "traffic.json").write_text(json.dumps(traffic, indent=1, sort_keys=True) + "\n")
    return 0


def peaks(repeats: int = 7) -> int:
    """Achieved peaks of this card (libpe_peaks.so, include/pe_peaks.h), beside the spec peaks
    the roofline fractions divide by: bf16 MFMA (v_mfma_f32_32x32x16_bf16, four independent
    chains per wave, eight waves per SIMD) on random and on all-zero operands (the chip's clock
    under MFMA load depends on the bits it toggles), a streaming HBM read and an HBM copy with
    16-byte vector loads, and the direct global-to-LDS loads the attention kernels stage with.
    Each figure is the median of ``repeats`` HIP-event-timed launches after one warm-up. Prints
    one JSON line; the committed summary is profiles/peaks.md (read by the bench line)."""
    import torch

    from packed_encoders_amd import _build

    lib = ctypes.CDLL(str(_build.PEAKS_LIBRARY))
    vp, i32, sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_size_t
    lib.pe_peak_mfma_bf16.argtypes = [vp, vp, i32, i32, vp]
    lib.pe_peak_read.argtypes = [vp, sz, vp, i32, vp]
    lib.pe_peak_copy.argtypes = [vp, vp, sz, i32, vp]
    lib.pe_peak_read_lds.argtypes = [vp, sz, vp, i32, vp]
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream
    blocks = 256 * 8  # eight 4-wave workgroups per CU
    sink = torch.empty(blocks * 256, dtype=torch.float32, device=dev)

    def timed(launch) -> float:
        launch()
        times = []
        for _ in range(repeats):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            launch()
            e1.record(stream)
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1) * 1e-3)
        return statistics.median(times)

    res = {"spec": {"bf16_mfma_tflops": PEAK_BF16_TFLOPS, "hbm_gbs": PEAK_HBM_GBS}, "repeats": repeats}
    iters = 20000
    flops = blocks * 16 * iters * 32768
    g = torch.Generator(device=dev).manual_seed(5)
    for name, ops in (("random", torch.randn(8 * 4096, device=dev, generator=g, dtype=torch.bfloat16)),
                      ("zeros", torch.zeros(8 * 4096, device=dev, dtype=torch.bfloat16))):
        t = timed(lambda: lib.pe_peak_mfma_bf16(ops.data_ptr(), sink.data_ptr(), blocks, iters, sp))
        res[f"bf16_mfma_tflops_{name}"] = round(flops / t / 1e12, 1)
    n = 4 << 30
    src = torch.empty(n, dtype=torch.uint8, device=dev).random_(generator=g)
    t = timed(lambda: lib.pe_peak_read(src.data_ptr(), n, sink.data_ptr(), blocks, sp))
    res["hbm_read_gbs"] = round(n / t / 1e9, 1)
    t = timed(lambda: lib.pe_peak_read_lds(src.data_ptr(), n, sink.data_ptr(), blocks, sp))
    res["hbm_read_to_lds_gbs"] = round(n / t / 1e9, 1)
    half = n // 2
    t = timed(lambda: lib.pe_peak_copy(src.data_ptr(), src.data_ptr() + half, half, blocks, sp))
    res["hbm_copy_gbs_read_plus_write"] = round(2 * half / t / 1e9, 1)
    res["fraction_of_spec"] = {
        "bf16_mfma_random": round(res["bf16_mfma_tflops_random"] / PEAK_BF16_TFLOPS, 3),
        "bf16_mfma_zeros": round(res["bf16_mfma_tflops_zeros"] / PEAK_BF16_TFLOPS, 3),
        "hbm_read": round(res["hbm_read_gbs"] / PEAK_HBM_GBS, 3),
        "hbm_read_to_lds": round(res["hbm_read_to_lds_gbs"] / PEAK_HBM_GBS, 3),
        "hbm_copy": round(res["hbm_copy_gbs_read_plus_write"] / PEAK_HBM_GBS, 3)}
    print(json.dumps(res), flush=True)
    return 0


def achieved_peaks():
    """The achieved peaks committed in profiles/peaks.md (its JSON line), or None."""
    path = ROOT / "profiles" / "peaks.md"
    try:
        for line in path.read_text().splitlines():
            if line.startswith("{") and "bf16_mfma_tflops_random" in line:
                return json.loads(line)
    except (OSError, ValueError):
        return None
    return None


def band_sweep(reps: int = 10, replays: int = 5) -> int:
    """The streaming band kernel against the tiled kernel on +-64 calls of every size: the
    measurement the library's size rule (band kernel from a number of query tiles on, strip 8
    from a larger one) is fitted to (attention_dispatch.fit_band_rule). Batches: C2-like
    document mixes (LogNormal(400, 0.8) in [32, 2048]) of 16 to 1,024 documents and
    equal-length batches of 256 to 8,192 tokens, 12 heads x 64. Per batch the tile plan is built
    once and ``reps`` calls of the long-segment stage are graph-captured and replayed, cycling
    over enough distinct Q/K/V sets that they do not stay resident in the 256 MB Infinity Cache
    (a packed forward's layers each bring their own). Times: tiled kernel, band kernel at strips
    4 and 8. One JSON line per batch; the committed summary is profiles/band_sweep.md
    (the reference's counterpart: benchmarks/packed_attention_dispatch_bench.py:153-229)."""
    import torch

    from packed_encoders_amd import _lib, hip_attention as hip, workloads as W

    lib = _lib.library()
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(13)
    stream = torch.cuda.Stream(dev)
    h, d = 12, 64
    batches = []
    for n_docs in (16, 32, 64, 128, 256, 512, 1024):
        rng = W.SplitMix64(100 + n_docs)
        batches.append((f"mix{n_docs}", tuple(rng.lognormal_length(400, 0.8, 32, 2048) for _ in range(n_docs))))
    for L, n in ((256, 256), (512, 128), (512, 512), (1024, 64), (1024, 256), (2048, 32), (2048, 128),
                 (4096, 32), (8192, 16), (8192, 32)):
        batches.append((f"eq{L}x{n}", (L,) * n))
    for name, lengths in batches:
        T = sum(lengths)
        per_set = 2 * T * h * d * 4  # q, k, v read and o written
        n_sets = max(2, min(16, -(-600_000_000 // per_set)))
        cu = torch.tensor([0, *itertools.accumulate(lengths)], dtype=torch.int32, device=dev)
        sets = [tuple(torch.randn(T, h, d, device=dev, generator=gen, dtype=torch.bfloat16) for _ in range(3))
                for _ in range(n_sets)]
        outs = [torch.empty_like(s_[0]) for s_ in sets]
        times = {}
        for kind, band_kernel, strip in (("tiled", 2, 0), ("band4", 1, 4), ("band8", 1, 8)):
            argss = [hip._args(q, k, v, o, cu, max(lengths), 0.125, 64, 64, False, None, 0, strip,
                               band_kernel=band_kernel, min_seqlen=min(lengths)) for (q, k, v), o in zip(sets, outs)]
            size = ctypes.c_size_t()
            assert lib.pe_attn_workspace_size(ctypes.byref(argss[0]), ctypes.byref(size)) == 0
            ws = torch.empty(max(size.value, 1), dtype=torch.uint8, device=dev)
            with torch.cuda.stream(stream):
                assert lib.pe_attn_plan(ctypes.byref(argss[0]), ws.data_ptr(), size.value, stream.cuda_stream) == 0
                for a in argss:
                    assert lib.pe_attn_tiled_fwd(ctypes.byref(a), ws.data_ptr(), size.value, stream.cuda_stream) == 0
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                for i in range(reps):
                    a = argss[i % n_sets]
                    assert lib.pe_attn_tiled_fwd(ctypes.byref(a), ws.data_ptr(), size.value,
                                                 torch.cuda.current_stream(dev).cuda_stream) == 0
            graph.replay()
            torch.cuda.synchronize()
            samples = []
            for _ in range(replays):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                graph.replay()
                e1.record()
                torch.cuda.synchronize()
                samples.append(e0.elapsed_time(e1) * 1e3 / reps)
            times[kind] = statistics.median(samples)
            del graph
        print(json.dumps({"batch": name, "n_seq": len(lengths), "tokens": T, "query_tiles": T // 128 * h,
                          "tiled_us": round(times["tiled"], 2), "band4_us": round(times["band4"], 2),
                          "band8_us": round(times["band8"], 2)}), flush=True)
        del sets, outs
    return 0


def graph_overhead(repeats: int = 7) -> int:
    """What a HIP-graph replay costs beside eager launches on this stack. Nodes: the C1
    attention call (one short-kernel launch, about 7 us of kernel) and, as a control, a torch
    elementwise kernel on one element (about 2 us). For N = 1..64 nodes captured into one graph,
    the replay's time per replay (HIP events on the replaying stream, median of ``repeats``
    samples of 50 replays) against N eager launches of the same work; a least-squares line
    through the replay times separates the fixed cost of a replay from the cost of each node.
    Prints one JSON line per node kind; the committed summary is profiles/graph_overhead.md."""
    import torch

    import packed_encoders_amd as pe
    from packed_encoders_amd import _lib, hip_attention as hip

    lib = _lib.library()
    dev = torch.device("cuda", 0)
    stream = torch.cuda.Stream(dev)
    wl = pe.workloads.c1()
    T, h, d = wl.total_tokens, wl.n_heads_q, wl.head_dim
    gen = torch.Generator(device=dev).manual_seed(3)
    q, k, v = (torch.randn(T, h, d, device=dev, generator=gen, dtype=torch.bfloat16) for _ in range(3))
    out = torch.empty_like(q)
    cu = torch.tensor(wl.cu_seqlens(), dtype=torch.int32, device=dev)
    a = hip._args(q, k, v, out, cu, wl.max_seqlen, wl.scale, -1, -1, False, None, -1)
    tiny = torch.zeros(1, device=dev)

    def attention():
        assert lib.pe_attn_short_fwd(ctypes.byref(a), torch.cuda.current_stream(dev).cuda_stream) == 0

    def elementwise():
        tiny.add_(1.0)

    def per_call_us(fn, n, reps=50) -> float:
        samples = []
        for _ in range(repeats):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(torch.cuda.current_stream(dev))
            for _ in range(reps):
                fn()
            e1.record(torch.cuda.current_stream(dev))
            torch.cuda.synchronize()
            samples.append(e0.elapsed_time(e1) * 1e3 / reps)
        return statistics.median(samples)

    for kind, node in (("c1_attention", attention), ("elementwise_1", elementwise)):
        rows = []
        for n in (1, 2, 4, 8, 16, 32, 64):
            with torch.cuda.stream(stream):
                for _ in range(3):
                    node()
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                for _ in range(n):
                    node()
            graph.replay()
            torch.cuda.synchronize()
            replay = per_call_us(graph.replay, n)
            eager = per_call_us(lambda: [node() for _ in range(n)], n)
            rows.append({"nodes": n, "replay_us": round(replay, 2), "eager_us": round(eager, 2)})
            del graph
        xs, ys = [r["nodes"] for r in rows], [r["replay_us"] for r in rows]
        mx, my = statistics.mean(xs), statistics.mean(ys)
        slope = sum((x - mx) * (y - my) for x, y in zip(xs, ys)) / sum((x - mx) ** 2 for x in xs)
        ex = [r["eager_us"] for r in rows]
        me = statistics.mean(ex)
        slope_e = sum((x - mx) * (y - me) for x, y in zip(xs, ex)) / sum((x - mx) ** 2 for x in xs)
        print(json.dumps({"node": kind, "rows": rows,
                          "replay_fixed_us": round(my - slope * mx, 2), "replay_per_node_us": round(slope, 3),
                          "eager_fixed_us": round(me - slope_e * mx, 2), "eager_per_call_us": round(slope_e, 3)}),
              flush=True)
    return 0


def compare_libraries(args, paths: list[str]) -> int:
    """Interleaved medians of one layer's long-segment stage (or its short pass, or its plan)
    across library builds: the in-tree ``libpe_attn.so`` first, then each build in ``paths``
    (the same C ABI, compiled from modified sources). Every build plans and runs the same call
    on the same inputs, cycling over ``--sets`` distinct Q/K/V sets; their outputs are checked
    bit for bit against the first build's (a change that alters a result is reported). Then
    ``--samples`` rounds, each timing ``--steps`` calls of every build in turn with HIP events,
    so a build's median is never taken on a different stretch of the box's clock than
    another's. This is how keep-or-drop decisions are made."""
    import torch

    from packed_encoders_amd import _build, _lib, hip_attention as hip, workloads as W
    from packed_encoders_amd.attention_dispatch import hip_short_max

    workload = WORKLOADS[args.workload]()
    layer = workload.layers[0] if args.window is None else {"global": W.GLOBAL, "band": W.BAND64}[args.window]
    dev = torch.device("cuda", 0)
    T, hq, hkv, d = workload.total_tokens, workload.n_heads_q, workload.n_heads_kv, workload.head_dim
    gen = torch.Generator(device=dev).manual_seed(1234)
    sets = []
    for _ in range(max(1, args.sets)):
        q, k, v = (torch.randn(T, h, d, device=dev, generator=gen, dtype=torch.bfloat16) for h in (hq, hkv, hkv))
        g = torch.randn(T, hq, d, device=dev, generator=gen, dtype=torch.bfloat16) if layer.gate else None
        sets.append((q, k, v, g))
    cu = torch.tensor(workload.cu_seqlens(), dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    A = ctypes.POINTER(_lib.AttnArgs)
    stage = args.compare_stage
    short_max = (hip_short_max(d, max_seqlen=workload.max_seqlen) if args.short_max is None else args.short_max)
    builds = []
    for path in [str(_build.LIBRARY), *paths]:
        lib = ctypes.CDLL(path)
        for name in ("pe_attn_plan", "pe_attn_tiled_fwd"):
            getattr(lib, name).argtypes = [A, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        lib.pe_attn_short_fwd.argtypes = [A, ctypes.c_void_p]
        lib.pe_attn_workspace_size.argtypes = [A, ctypes.POINTER(ctypes.c_size_t)]
        outs = [torch.zeros(T, hq, d, device=dev, dtype=torch.bfloat16) for _ in sets]
        shortest = 0 if stage == "short" or args.no_min_seqlen else min(workload.lengths)
        argl = [hip._args(q, k, v, o, cu, workload.max_seqlen, workload.scale, layer.window[0], layer.window[1],
                          layer.causal, g, short_max, args.strip, min_seqlen=shortest)
                for (q, k, v, g), o in zip(sets, outs)]
        size = ctypes.c_size_t()
        assert lib.pe_attn_workspace_size(ctypes.byref(argl[0]), ctypes.byref(size)) == 0
        ws = torch.zeros(max(1, size.value), dtype=torch.uint8, device=dev)
        counter = [0]

        def call(lib=lib, argl=argl, ws=ws, n=size.value, counter=counter):
            a = ctypes.byref(argl[counter[0] % len(argl)])
            counter[0] += 1
            if stage == "short":
                rc = lib.pe_attn_short_fwd(a, stream)
            elif stage == "plan":
                rc = lib.pe_attn_plan(a, ws.data_ptr(), n, stream)
            else:
                rc = lib.pe_attn_tiled_fwd(a, ws.data_ptr(), n, stream)
            assert rc == 0, rc

        assert lib.pe_attn_plan(ctypes.byref(argl[0]), ws.data_ptr(), size.value, stream) == 0
        for _ in argl:
            call()
        builds.append((path, call, outs[0]))
    torch.cuda.synchronize()
    results = {}
    for path, _, out in builds:
        results[path] = {"bit_identical_to_first": bool(torch.equal(out, builds[0][2])), "us": []}
    settle(lambda: [b[1]() for b in builds], args.settle)
    for _ in range(args.samples):
        for path, call, _ in builds:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(args.steps):
                call()
            e1.record()
            torch.cuda.synchronize()
            results[path]["us"].append(round(e0.elapsed_time(e1) * 1e3 / args.steps, 2))
    for path, r in results.items():
        r["median_us"] = statistics.median(r["us"])
    print(json.dumps({"compare": workload.name, "layer": {"window": layer.window, "causal": layer.causal,
                                                          "gate": layer.gate},
                      "stage": stage, "sets": len(sets), "results": results}), flush=True)
    return 0


def variant_timing(args, which: str) -> int:
    """Interleaved medians of one layer call of ``--workload`` in two forms, on the in-tree
    library: ``gate`` the call with and without its sigmoid gate (what the fused gate costs);
    ``side-stream`` a mixed batch's short pass on a second stream (default priority) beside the
    plan and the long-segment kernel, joined before the call ends, against the library's
    one-stream order (outputs checked bit for bit). ``--samples`` rounds of ``--steps`` calls,
    cycling over four Q/K/V sets."""
    import torch

    from packed_encoders_amd import _lib, hip_attention as hip
    from packed_encoders_amd.attention_dispatch import hip_short_max

    workload = WORKLOADS[args.workload]()
    if which == "rope":
        return _rope_timing(args, workload)
    layer = workload.layers[0]
    dev = torch.device("cuda", 0)
    T, hq, hkv, d = workload.total_tokens, workload.n_heads_q, workload.n_heads_kv, workload.head_dim
    gen = torch.Generator(device=dev).manual_seed(1)
    sets = []
    for _ in range(4):
        q, k, v = (torch.randn(T, h, d, device=dev, generator=gen, dtype=torch.bfloat16) for h in (hq, hkv, hkv))
        sets.append((q, k, v, torch.randn(T, hq, d, device=dev, generator=gen, dtype=torch.bfloat16)))
    cu = torch.tensor(workload.cu_seqlens(), dtype=torch.int32, device=dev)
    lib = _lib.library()
    short_max = hip_short_max(d, max_seqlen=workload.max_seqlen) if args.short_max is None else args.short_max
    outs = [torch.zeros(T, hq, d, device=dev, dtype=torch.bfloat16) for _ in sets]

    def arglist(gate: bool, bound: int):
        return [hip._args(q, k, v, o, cu, workload.max_seqlen, workload.scale, layer.window[0], layer.window[1],
                          layer.causal, g if gate else None, short_max, args.strip, min_seqlen=bound)
                for (q, k, v, g), o in zip(sets, outs)]

    main = torch.cuda.current_stream(dev)
    side = torch.cuda.Stream(dev)
    counter = [0]
    if which == "gate":
        if not layer.gate:
            raise SystemExit(f"{workload.name}'s layer has no gate")
        forms = {"gate": arglist(True, min(workload.lengths)), "no_gate": arglist(False, min(workload.lengths))}
    else:
        forms = {"one_stream": arglist(layer.gate, 0), "side_stream": arglist(layer.gate, 0)}
    size = ctypes.c_size_t()
    assert lib.pe_attn_workspace_size(ctypes.byref(next(iter(forms.values()))[0]), ctypes.byref(size)) == 0
    ws = torch.zeros(max(1, size.value), dtype=torch.uint8, device=dev)

    def call(form: str):
        a = ctypes.byref(forms[form][counter[0] % len(sets)])
        counter[0] += 1
        s = main.cuda_stream
        if form == "side_stream":
            side.wait_stream(main)
            assert lib.pe_attn_short_fwd(a, side.cuda_stream) == 0
        elif which != "gate":
            assert lib.pe_attn_short_fwd(a, s) == 0
        if which != "gate" or counter[0] <= len(sets):
            assert lib.pe_attn_plan(a, ws.data_ptr(), size.value, s) == 0
        assert lib.pe_attn_tiled_fwd(a, ws.data_ptr(), size.value, s) == 0
        if form == "side_stream":
            main.wait_stream(side)

    check = {}
    for form in forms:
        for _ in sets:
            call(form)
        torch.cuda.synchronize()
        check[form] = [o.clone() for o in outs]
    same = None if which == "gate" else all(torch.equal(a, b) for a, b in zip(*check.values()))
    settle(lambda: [call(f) for f in forms], args.settle)
    res = {f: [] for f in forms}
    for _ in range(args.samples):
        for form in forms:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(args.steps):
                call(form)
            e1.record()
            torch.cuda.synchronize()
            res[form].append(round(e0.elapsed_time(e1) * 1e3 / args.steps, 2))
    print(json.dumps({"variant_timing": which, "workload": workload.name, "bit_identical": same,
                      **{f: {"median_us": statistics.median(v), "us": v} for f, v in res.items()}}), flush=True)
    return 0


def _rope_timing(args, workload) -> int:
    """``--variant-timing rope``: RoPE + attention of one layer of an all-short workload (Q4096,
    C1) from the packed projection ``qkv [T, 3*H*D]`` with per-token tables, in two forms,
    interleaved: the RoPE kernel writing q and k then the attention call, and the attention call
    with the RoPE fused into its prologue (``varlen_attention(rope=...)``). Outputs are checked
    bit for bit; compulsory bytes of each form are reported beside the times."""
    import torch

    from packed_encoders_amd import ops
    from packed_encoders_amd.hip_attention import rope_qkv, varlen_attention

    layer = workload.layers[0]
    dev = torch.device("cuda", 0)
    T, h, d = workload.total_tokens, workload.n_heads_q, workload.head_dim
    if workload.n_heads_kv != h or not ops.fused_rope_applies(torch.empty(1, dtype=torch.bfloat16, device=dev),
                                                              d, workload.max_seqlen):
        raise SystemExit(f"{workload.name}: the fused RoPE serves all-short MHA calls (head_dim 64/128, <= 128 tokens)")
    gen = torch.Generator(device=dev).manual_seed(3)
    cu = torch.tensor(workload.cu_seqlens(), dtype=torch.int32, device=dev)
    theta = torch.arange(0, d, 2, device=dev, dtype=torch.float32) / d
    pos = torch.cat([torch.arange(n, device=dev) for n in workload.lengths]).float()
    ang = pos[:, None] * (10000.0 ** -theta)[None]
    cos = torch.cat([ang.cos(), ang.cos()], dim=1).bfloat16()
    sin = torch.cat([ang.sin(), ang.sin()], dim=1).bfloat16()
    sets = [torch.randn(T, 3 * h * d, device=dev, generator=gen, dtype=torch.bfloat16) for _ in range(4)]
    counter = [0]
    kw = dict(softmax_scale=workload.scale, window=layer.window)

    def two_steps():
        qkv = sets[counter[0] % 4]
        counter[0] += 1
        q, k = rope_qkv(qkv, h, d, cos, sin)
        return varlen_attention(q, k, qkv.view(T, 3, h, d)[:, 2], cu, workload.max_seqlen, **kw)

    def fused():
        qkv = sets[counter[0] % 4]
        counter[0] += 1
        view = qkv.view(T, 3, h, d)
        return varlen_attention(view[:, 0], view[:, 1], view[:, 2], cu, workload.max_seqlen, rope=(cos, sin), **kw)

    forms = {"rope_then_attention": two_steps, "fused": fused}
    with torch.inference_mode():
        outs = {}
        for name, f in forms.items():
            counter[0] = 0
            outs[name] = f()
        torch.cuda.synchronize()
        same = torch.equal(*outs.values())
        settle(lambda: [f() for f in forms.values()], args.settle)
        res = {f: [] for f in forms}
        for _ in range(args.samples):
            for name, f in forms.items():
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(args.steps):
                    f()
                e1.record()
                torch.cuda.synchronize()
                res[name].append(round(e0.elapsed_time(e1) * 1e3 / args.steps, 2))
    row = 2 * h * d  # bytes of one head-row set of one tensor per token
    table = 2 * 2 * d  # cos and sin rows per token
    moved = {"rope_then_attention": T * (2 * row + 2 * row + table) + T * (3 * row + row),
             "fused": T * (3 * row + row + table)}
    print(json.dumps({"variant_timing": "rope", "workload": workload.name, "bit_identical": same,
                      **{f: {"median_us": statistics.median(v), "us": v, "compulsory_mb": round(moved[f] / 1e6, 1)}
                         for f, v in res.items()}}), flush=True)
    return 0


def dispatch_sweep(reps: int = 20, replays: int = 5) -> int:
    """Short kernel vs tiled kernel per segment length: the measurement the gfx950 routing
    boundary (attention_dispatch.HipDispatchPolicy) is fitted to. For head_dim 64 (12 heads)
    and 128 (8 heads), batches of N segments of exactly L tokens (a C1-sized batch of 32 and a
    query batch of about 64K tokens) run through the short kernel at its smallest key capacity
    that holds L (short_max = L), at capacities 64 and 128 (short_max = max(L, 64) and 128, as a
    batch with longer segments routes its short ones under those boundaries) and through the
    tiled kernel (short_max = 0, plan included), each call graph-captured `reps` times and replayed, so host overhead is
    not timed. Prints one JSON line per (head_dim, L, N); the committed summary is
    profiles/dispatch_sweep.md (packed_encoders/benchmarks/packed_attention_dispatch_bench.py:153-229
    is the reference's counterpart)."""
    import torch

    from packed_encoders_amd import _lib, hip_attention as hip

    lib = _lib.library()
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(11)
    stream = torch.cuda.Stream(dev)
    for d, h in ((64, 12), (128, 8)):
        for n_target in (32, 65536):
            for L in (8, 16, 24, 32, 40, 48, 56, 64, 72, 80, 96, 112, 128):
                n = 32 if n_target == 32 else max(32, n_target // L)
                T = n * L
                q, k, v = (torch.randn(T, h, d, device=dev, generator=gen, dtype=torch.bfloat16) for _ in range(3))
                cu = torch.arange(0, T + 1, L, dtype=torch.int32, device=dev)
                times = {}
                for kind, short_max in (("short", L), ("short64", max(L, 64)), ("short128", 128), ("tiled", 0)):
                    out = torch.empty_like(q)
                    a = hip._args(q, k, v, out, cu, L, d ** -0.5, -1, -1, False, None, short_max)
                    size = ctypes.c_size_t()
                    assert lib.pe_attn_workspace_size(ctypes.byref(a), ctypes.byref(size)) == 0
                    ws = torch.empty(max(size.value, 1), dtype=torch.uint8, device=dev)

                    def call():
                        rc = lib.pe_varlen_attn_fwd(ctypes.byref(a), ws.data_ptr(), size.value,
                                                    torch.cuda.current_stream(dev).cuda_stream)
                        assert rc == 0, rc

                    with torch.cuda.stream(stream):
                        call()
                    torch.cuda.synchronize()
                    graph = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(graph, stream=stream):
                        for _ in range(reps):
                            call()
                    graph.replay()
                    torch.cuda.synchronize()
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record()
                    for _ in range(replays):
                        graph.replay()
                    e1.record()
                    torch.cuda.synchronize()
                    times[kind] = e0.elapsed_time(e1) * 1e3 / (reps * replays)
                    del graph
                print(json.dumps({"head_dim": d, "heads": h, "L": L, "n_seq": n, "tokens": T,
                                  "short_us": round(times["short"], 3), "short64_us": round(times["short64"], 3),
                                  "short128_us": round(times["short128"], 3), "tiled_us": round(times["tiled"], 3)}),
                      flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="C2", help="C1 C2 C3 C3-shuffled C4 C4-band C5 Q4096 (default C2)")
    ap.add_argument("--samples", type=int, default=5,
                    help="consecutive samples the timed steps are cut into for the median and spread (default 5)")
    ap.add_argument("--short-max", type=int, default=None, help="routing boundary (default: gfx950 policy)")
    ap.add_argument("--strip", type=int, default=0, help="query tiles per tiled-kernel workgroup (0: library default)")
    ap.add_argument("--no-min-seqlen", action="store_true",
                    help="pass no lower bound on the segment lengths (the short pass then always launches)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="skip the graph-replayed timing of the step")
    ap.add_argument("--settle", type=float, default=0.3,
                    help="seconds of untimed steps before the warm-up, to reach the sustained clock (default 0.3)")
    ap.add_argument("--no-model", action="store_true",
                    help="skip the end-to-end packed ModernBERT forward (C2 only)")
    ap.add_argument("--dispatch-sweep", action="store_true",
                    help="only time the short kernel against the tiled kernel per segment length")
    ap.add_argument("--band-sweep", action="store_true",
                    help="only time the streaming band kernel against the tiled kernel on +-64 calls of every size")
    ap.add_argument("--compare", nargs="+", metavar="LIB",
                    help="only time one layer call of --workload across library builds (the in-tree one first), "
                         "interleaved, --samples rounds of --steps calls each")
    ap.add_argument("--compare-stage", choices=("long", "short", "plan"), default="long",
                    help="which stage --compare times (default: the long-segment kernel)")
    ap.add_argument("--window", choices=("global", "band"), default=None,
                    help="--compare: the layer's window (default: the workload's first layer)")
    ap.add_argument("--sets", type=int, default=4, help="--compare: distinct Q/K/V sets cycled over (default 4)")
    ap.add_argument("--variant-timing", choices=("gate", "side-stream", "rope"), default=None,
                    help="only time one layer call of --workload in two forms, interleaved: with and without its "
                         "gate, a mixed batch's short pass on a second stream against one stream, or RoPE kernel + "
                         "attention against the fused RoPE prologue (all-short workloads)")
    ap.add_argument("--graph-overhead", action="store_true",
                    help="only measure a HIP-graph replay's fixed and per-node cost against eager launches")
    ap.add_argument("--peaks", action="store_true",
                    help="only measure this card's achieved bf16 MFMA, HBM read/copy and global-to-LDS rates")
    ap.add_argument("--profile-commands", action="store_true",
                    help="only print the rocprofv3 commands behind the committed profiles (name<TAB>command)")
    ap.add_argument("--summarize-profiles", metavar="DIR",
                    help="only write the profiles/ summaries from the output of --profile-commands under DIR")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only copy a 1 GiB buffer --steps times (scale for rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}): this build runs one MI355X; "
              "packed segments would shard across GPUs by segment, with no exchange between them",
              file=sys.stderr)
        return 2

    if args.profile_commands:
        for name, cmd in profile_commands():
            print(f"{name}\t{cmd}")
        return 0
    if args.summarize_profiles:
        return summarize_profiles(Path(args.summarize_profiles))
    if args.copy_calibration:
        return copy_calibration(args.steps)
    if args.dispatch_sweep:
        return dispatch_sweep()
    if args.band_sweep:
        return band_sweep()
    if args.peaks:
        return peaks()
    if args.graph_overhead:
        return graph_overhead()
    if args.compare:
        return compare_libraries(args, args.compare)
    if args.variant_timing:
        return variant_timing(args, args.variant_timing)

    import packed_encoders_amd as pe

    w = args.workload
    workload = WORKLOADS[w]()
    res = gpu_bench(args, workload)
    model_res = None
    if w in ("C1", "C2") and not args.no_model:
        try:
            model_res = model_bench(args, workload)
        except Exception as exc:  # reported, never required
            model_res = {"error": f"{type(exc).__name__}: {exc}"}
            log(f"model leg skipped: {model_res['error']}")
    cpu_res = None
    if not args.no_cpu_baseline:
        calls, cu = res.pop("_outputs")
        sanity_check(calls, workload, cu)
        try:
            cpu_res = cpu_bench(workload)
        except Exception as exc:  # the baseline is reported, never required
            log(f"cpu baseline skipped: {type(exc).__name__}: {exc}")
    n_global = sum(1 for l in workload.layers if l.window == (-1, -1))
    line = {
        "metric": METRIC,
        "value": round(res["value"], 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": workload.name + ": " + workload.description,
            "n_segments": len(workload.lengths),
            "total_tokens": workload.total_tokens,
            "max_seqlen": workload.max_seqlen,
            "heads_q": workload.n_heads_q,
            "heads_kv": workload.n_heads_kv,
            "head_dim": workload.head_dim,
            "attention_layers": len(workload.layers),
            "global_layers": n_global,
            "short_max": res["short_max"],
            "min_seqlen": res["min_seqlen"],
            "parallelism": "single GPU",
        },
        "tokens_per_s": round(res["tokens_per_s"], 1),
        "gpu_ms_per_step": round(res["gpu_ms_per_step"], 4),
        "samples": res["samples"],
        "graph_replay": res["graph_replay"],
        "settle_s": res["settle_s"],
        "roofline": res["roofline"],
        "cpu_baseline": cpu_res,
    }
    if model_res is not None:
        line["end_to_end"] = model_res
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
