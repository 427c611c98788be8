"""Bucketed HIP-graph capture of the packed forward (packed_encoders/graph.py:45-74,212-412).

One graph per ``(M_bucket, N, Smax, backend)``: ``M_bucket = ceil(M / pad_to) * pad_to`` live
tokens, the real sequence count N and the real ``max_seqlen``. The captured region is the whole
packed forward read from static buffers, so a replay costs three small device copies (ids,
positions, ``cu_seqlens``) plus the replay itself. Tokens between the real M and the bucket
run through the dense layers but lie outside ``cu_seqlens[N]``, so no attention reads them and
their rows are dropped from the output.

What makes the capture valid on PyTorch-ROCm:
- every HIP attention launch takes torch's current stream (the capture stream) and the library
  allocates nothing, synchronises nothing and never reads ``cu_seqlens`` on the host; the
  tile plan is built on the device inside the graph, so a replay with new boundaries in the
  same bucket re-plans itself;
- the static buffers are refilled with copies and a fill kernel (``zero_`` / ``fill_``), never a
  memset node inside the graph;
- a graph replays against fixed addresses, so it is used only without autograd and without
  autocast (the packed forward checks both).
"""

from __future__ import annotations

import os
from collections import OrderedDict
from dataclasses import dataclass

import torch
from torch import Tensor, nn

from . import forward
from .config import ModernBertParams

GRAPH_ENV_VAR = forward.GRAPH_ENV


def graphs_globally_disabled() -> bool:
    """The ``PACKED_ENCODERS_GRAPH=0`` kill switch."""
    return os.environ.get(GRAPH_ENV_VAR, "1") == "0"


@dataclass(frozen=True)
class GraphConfig:
    """Bucketing policy. ``pad_to`` rounds the token count; ``max_batch`` / ``max_seq`` /
    ``max_tokens`` bound which calls are graphed (larger ones run eagerly); ``max_graphs`` bounds
    the cache by LRU; ``warmup`` eager runs precede each capture."""

    pad_to: int = 64
    max_batch: int | None = None
    seq_buckets: tuple[int, ...] | None = None
    max_graphs: int = 32
    max_tokens: int = 2 ** 20
    max_seq: int | None = None
    warmup: int = 3


def round_up(value: int, multiple: int) -> int:
    return (value + multiple - 1) // multiple * multiple


@dataclass
class PackedStaticInputs:
    """Fixed-address inputs of one packed graph."""

    input_ids: Tensor
    cu_seqlens: Tensor
    position_ids: Tensor
    max_seqlen: int

    def stage(self, packed_ids: Tensor, cu_seqlens: Tensor, position_ids: Tensor) -> int:
        """Copy a real batch in: the bucket tail gets id 0 / position 0, and ``cu_seqlens`` past
        the real sequences (none when N matches the key) is filled with M."""
        m = packed_ids.shape[0]
        n = cu_seqlens.shape[0] - 1
        self.input_ids[:m].copy_(packed_ids)
        self.input_ids[m:].zero_()
        self.position_ids[:m].copy_(position_ids)
        self.position_ids[m:].zero_()
        self.cu_seqlens[: n + 1].copy_(cu_seqlens)
        if n + 1 < self.cu_seqlens.shape[0]:
            self.cu_seqlens[n + 1:].fill_(m)
        return m


@dataclass
class PackedCaptured:
    graph: "torch.cuda.CUDAGraph"
    inputs: PackedStaticInputs
    out: Tensor


class PackedGraphRunner:
    """Captures ``packed_forward`` per ``(M_bucket, N, Smax, backend)`` and replays it
    (graph.py:241-400)."""

    def __init__(self, model: nn.Module, params: ModernBertParams, config: GraphConfig, backend: str = "hip", *,
                 execution=None):
        self.model = model
        self.params = params
        self.config = config
        self.backend = backend
        self.execution = forward._execution_for(model, execution)
        self.device = next(model.parameters()).device
        self.cache: "OrderedDict[tuple[int, int, int, str], PackedCaptured]" = OrderedDict()
        self.captures = 0  # number of graphs captured so far (observability and tests)

    def key(self, m: int, n: int, max_seqlen: int) -> tuple[int, int, int, str]:
        dtype = self.model.embeddings.tok_embeddings.weight.dtype
        resolved = forward.resolve_backend(self.backend, self.params, device=self.device, dtype=dtype)
        return (round_up(m, self.config.pad_to), n, int(max_seqlen), resolved)

    def admits(self, m: int, n: int, max_seqlen: int) -> bool:
        c = self.config
        return not ((c.max_seq is not None and max_seqlen > c.max_seq) or (c.max_batch is not None and n > c.max_batch)
                    or m > c.max_tokens)

    def __call__(self, packed_ids: Tensor, cu_seqlens: Tensor, max_seqlen: int, position_ids: Tensor) -> Tensor:
        m, n = packed_ids.shape[0], cu_seqlens.numel() - 1
        if not self.admits(m, n, max_seqlen):
            return self.eager(packed_ids, cu_seqlens, max_seqlen, position_ids)
        key = self.key(m, n, max_seqlen)
        if key[3] != "hip":
            return self.eager(packed_ids, cu_seqlens, max_seqlen, position_ids)
        captured = self.cache.get(key)
        if captured is None:
            captured = self.capture(*key)
            while len(self.cache) >= self.config.max_graphs:
                self.cache.popitem(last=False)
            self.cache[key] = captured
        else:
            self.cache.move_to_end(key)
        m_real = captured.inputs.stage(packed_ids, cu_seqlens, position_ids)
        captured.graph.replay()
        return captured.out[:m_real].clone()

    def eager(self, packed_ids, cu_seqlens, max_seqlen, position_ids) -> Tensor:
        return forward.packed_forward(self.model, self.params, packed_ids, cu_seqlens, max_seqlen, position_ids,
                                      backend=self.backend, execution=self.execution, _allow_graph=False)

    def capture(self, mb: int, n: int, max_seqlen: int, backend: str) -> PackedCaptured:
        dev = self.device
        static = PackedStaticInputs(input_ids=torch.zeros(mb, dtype=torch.long, device=dev),
                                    cu_seqlens=torch.zeros(n + 1, dtype=torch.int32, device=dev),
                                    position_ids=torch.zeros(mb, dtype=torch.long, device=dev),
                                    max_seqlen=max_seqlen)
        # A valid synthetic distribution for warm-up and capture: N sequences of up to max_seqlen
        # tokens; a bucket larger than N * max_seqlen leaves its tail outside cu_seqlens.
        lengths, remaining = [], min(mb, n * max_seqlen)
        for _ in range(n):
            lengths.append(min(max_seqlen, remaining))
            remaining -= lengths[-1]
        cu = torch.tensor([0, *torch.tensor(lengths).cumsum(0).tolist()], dtype=torch.int32)
        static.cu_seqlens.copy_(cu.to(dev))
        pos = torch.cat([torch.arange(x) for x in lengths]) if lengths else torch.zeros(0, dtype=torch.long)
        static.position_ids[: pos.numel()].copy_(pos.to(dev))
        with torch.no_grad():
            side = torch.cuda.Stream(device=dev)
            side.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(side):
                for _ in range(self.config.warmup):
                    self.run(static)
            torch.cuda.current_stream(dev).wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                out = self.run(static)
        self.captures += 1
        return PackedCaptured(graph=graph, inputs=static, out=out)

    def run(self, static: PackedStaticInputs) -> Tensor:
        """The captured region: embeddings, RoPE gather, the layer loop and the final norm."""
        model, ex = self.model, self.execution
        norm = model.embeddings.norm
        x = ex.layer_norm(model.embeddings.tok_embeddings(static.input_ids), norm.weight, norm.eps)
        return forward.packed_core(model, self.params, x, static.cu_seqlens, static.max_seqlen, static.position_ids,
                                   execution=ex)


def build_packed_runner(model: nn.Module, params: ModernBertParams, config: GraphConfig, backend: str = "hip", *,
                        execution=None) -> PackedGraphRunner | None:
    """A runner when the backend can be captured (the HIP kernels) and the config bounds both
    the sequence count and the length (graph.py:403-412)."""
    if backend == "sdpa" or config.max_batch is None or config.max_seq is None:
        return None
    return PackedGraphRunner(model, params, config, backend=backend, execution=execution)
