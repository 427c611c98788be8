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

For C2 the line also carries ``end_to_end``: the whole packed ModernBERT-base forward
(random-init weights, bf16) over the same batch through ``pe.pack``, eager and replayed from
the bucketed HIP-graph runner, in tokens/s.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload C2] [--no-cpu-baseline]
                       [--no-model]
"""

from __future__ import annotations

import argparse
import ctypes
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

    def __init__(self, lib, hip, workload, layer, cu, q, k, v, gate, short_max, plans, strip=0):
        import torch

        self.lib, self.layer = lib, layer
        self.out = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)
        self.args = hip._args(q, k, v, self.out, cu, workload.max_seqlen, workload.scale, layer.window[0],
                              layer.window[1], layer.causal, gate, short_max, strip)
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


def kernel_instance(stage, workload, layer, short_max):
    """The kernel's name as rocprofv3 lists it (template arguments included)."""
    d = workload.head_dim
    if stage == "short":
        sk = 32 if short_max <= 32 else (64 if short_max <= 64 else 128)
        hpw = (2 if sk == 128 else 4) if d == 64 else (4 if sk == 32 else (2 if sk == 64 else 1))
        return f"pe::short_attn_kernel<{d}, {sk}, {hpw}, {str(layer.gate).lower()}>"
    g = math.gcd(workload.n_heads_q // workload.n_heads_kv, 4)
    bn = 32 if d >= 256 else 64
    ns = 3 if d == 64 else 2
    win = layer.window != (-1, -1) or layer.causal
    flags = f"{str(layer.gate).lower()}, {str(win).lower()}"
    if d == 256:
        return f"pe::wide16_attn_kernel<{d}, 4, {g}, {ns}, {flags}>"  # four waves per workgroup
    if d == 64 and not win:
        return f"pe::global64_attn_kernel<{g}, {str(layer.gate).lower()}>"
    name = "tiled_attn_kernel" if d == 64 else "wide_attn_kernel"
    return f"pe::{name}<{d}, {g}, {bn}, {ns}, {flags}>"


def gpu_bench(args, workload):
    import torch

    import packed_encoders_amd as pe
    from packed_encoders_amd import _lib, hip_attention as hip
    from packed_encoders_amd.attention_dispatch import hip_short_max

    lib = _lib.library()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    short_max = hip_short_max(workload.head_dim) if args.short_max is None else args.short_max
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
        calls.append(LayerCall(lib, hip, workload, layer, cu, q, k, v, g, short_max, plans, args.strip))
    stage, bound, timed_layers = dominant(workload, short_max)
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream

    timed_set = set(timed_layers)

    def bracket(fn, events):
        e0, e1 = events.pop()
        e0.record(stream)
        fn(sp)
        e1.record(stream)
        timed.append((e0, e1))

    def step(events=None):
        for i, c in enumerate(calls):
            here = events is not None and i in timed_set
            bracket(c.short, events) if here and stage == "short" else c.short(sp)
            if c.plans_here:
                c.plan(sp)
            bracket(c.tiled, events) if here and stage == "tiled" else c.tiled(sp)

    timed = []
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    pool = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            for _ in range(args.steps * len(timed_layers))]
    g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g0.record(stream)
    for _ in range(args.steps):
        step(pool)
    g1.record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    wall_ms = (t1 - t0) * 1e3 / args.steps
    gpu_ms = g0.elapsed_time(g1) / args.steps
    kernel_ms = statistics.mean(a.elapsed_time(b) for a, b in timed)

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
    kernel_name = kernel_instance(stage, workload, layer0, short_max)
    roofline = {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
                "frac": round(achieved / peak, 4), "traffic": traffic_from_profiles(workload.name, kernel_name),
                "kernel": kernel_name, "kernel_ms": round(kernel_ms, 4), "algorithmic_per_launch": per_launch}
    value = flops / (wall_ms * 1e-3) / 1e12
    log(f"wall {wall_ms:.3f} ms/step (events {gpu_ms:.3f}), {value:.1f} TFLOP/s, dominant {kernel_name} "
        f"{kernel_ms * 1e3:.1f} us -> {achieved:.1f} {unit} ({achieved / peak:.1%})")
    return {
        "value": value, "ms_per_step": wall_ms, "gpu_ms_per_step": gpu_ms, "flops_per_step": flops,
        "tokens_per_s": workload.total_tokens / (wall_ms * 1e-3), "roofline": roofline, "short_max": short_max,
        "_outputs": (calls, cu),
    }


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
    batch = pe.PackedBatch(ids, cu, max(lengths), positions)
    gcfg = pe.GraphConfig(max_batch=len(lengths), max_seq=max(lengths), pad_to=256, warmup=2)
    pe.pack(model, attention_backend="hip", cuda_graph=gcfg, validate=False)
    engine = pe.get_engine(model)
    stream = torch.cuda.current_stream(dev)

    def timed(fn):
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
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if one exists."""
    path = ROOT / "profiles" / "traffic.json"
    try:
        table = json.loads(path.read_text())
    except (OSError, ValueError):
        return None
    entry = table.get(f"{workload_name}:{kernel}")
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


def cpu_bench(workload, repeats: int = 7):
    """The same attention schedule on the host CPU (fp32): one warm-up, then the median of
    ``repeats`` timed steps on all physical cores (benchmarks/cpu/README.md:27-31), and a
    1-thread run on a bounded sample (the first global and the first banded layer, median of
    3) scaled to the same unit."""
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
    q, k, v = (torch.randn(hq, T, d, generator=gen) for _ in range(3))
    qn, kn, vn = (t.numpy() for t in (q, k, v))
    out = np.empty((hq, T, d), dtype=np.float32)
    lengths = list(workload.lengths)
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

    seconds = timed(workload.layers, threads, repeats)
    flops = sum(hip.useful_flops(lengths, hq, d, window=l.window) for l in workload.layers)
    # 1 thread: one layer of each kind present, scaled by its share of the schedule's FLOPs
    kinds = []
    for layer in workload.layers:
        if layer not in kinds:
            kinds.append(layer)
    one_flops = sum(hip.useful_flops(lengths, hq, d, window=l.window) for l in kinds)
    one_seconds = timed(kinds, 1, 3)
    one_tflops = one_flops / one_seconds / 1e12
    model = cpu_model()
    sample = (f"full {workload.name} schedule ({len(workload.layers)} attention layers, T={T}) in fp32 on {threads} "
              f"threads (physical cores of the affinity mask), median of {repeats} after 1 warm-up; band/short "
              f"layers: {'reference pe_local_attention (oracle/_ref)' if kind == 'reference' else 'oracle C port'}; "
              f"global layers longer than 128: per-segment torch SDPA. 1-thread: one layer of each kind "
              f"({len(kinds)}), median of 3")
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


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="C2", help="C1 C2 C3 C4 C4-band C5 Q4096 (default C2)")
    ap.add_argument("--short-max", type=int, default=None, help="routing boundary (default: gfx950 policy)")
    ap.add_argument("--strip", type=int, default=0, help="query tiles per tiled-kernel workgroup (0: library default)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-model", action="store_true",
                    help="skip the end-to-end packed ModernBERT forward (C2 only)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only copy a 1 GiB buffer --steps times (scale for rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}): this build runs one MI355X; "
              "segments shard across GPUs with no exchange, see DESIGN.md", file=sys.stderr)
        return 2

    if args.copy_calibration:
        return copy_calibration(args.steps)

    import packed_encoders_amd as pe

    w = args.workload
    workload = {"C1": pe.workloads.c1, "C2": pe.workloads.c2, "C3": pe.workloads.c3, "C4": pe.workloads.c4,
                "C4-band": lambda: pe.workloads.c4(band=True), "C5": pe.workloads.c5,
                "Q4096": pe.workloads.query_sweep}[w]()
    res = gpu_bench(args, workload)
    model_res = None
    if w == "C2" and not args.no_model:
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
            "parallelism": "single GPU",
        },
        "tokens_per_s": round(res["tokens_per_s"], 1),
        "gpu_ms_per_step": round(res["gpu_ms_per_step"], 4),
        "roofline": res["roofline"],
        "cpu_baseline": cpu_res,
    }
    if model_res is not None:
        line["end_to_end"] = model_res
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
