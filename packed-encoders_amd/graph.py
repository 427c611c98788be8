"""HIP-graph replay of the packed forward, one graph per token bucket.

The reference's packed graph runner (packed_encoders/graph.py:212-412) captures the packed
forward per ``(M_bucket, N, Smax, backend)``; the same key and the same public names are kept
here (``GraphConfig``, ``PackedStaticInputs.stage``, ``build_packed_runner``,
``graphs_globally_disabled``). The runner itself is organised around what a replay costs on
MI355X, where the forward of a short batch is a few hundred microseconds of kernels and the
host work around a replay is what is left to trim:

- a ``_Bucket`` owns its fixed-address inputs, the graph and the graph's output;
- staging a batch is two device copies of the real rows plus ``cu_seqlens``; the rows past the
  real token count are zeroed only when they may hold rows of an earlier, longer batch (the
  bucket tracks how far its inputs were written), so a stream of equal-length batches stages
  with no fill kernel at all;
- the backend resolution a key needs is computed once per autograd state, not per call.

What makes the capture valid: every attention launch takes torch's current stream (the capture
stream) and the HIP library allocates nothing, synchronises nothing and never reads
``cu_seqlens`` on the host (its tile plan is built on the device inside the graph, so a replay
with new boundaries in the same bucket re-plans itself); inputs are refilled with copies and
fill kernels, never with a memset node; and a graph replays against fixed addresses, so the
packed forward uses it only without autograd and without autocast. Rows between the real token
count and the bucket run through the dense layers but lie outside ``cu_seqlens[N]``: no
attention reads them and their outputs are dropped.
"""

from __future__ import annotations

import os
from collections import OrderedDict
from dataclasses import dataclass

import torch
from torch import Tensor, nn

from . import forward, staging
from .config import ModernBertParams

GRAPH_ENV_VAR = forward.GRAPH_ENV


def graphs_globally_disabled() -> bool:
    """True when ``PACKED_ENCODERS_GRAPH=0`` switches every graph runner off."""
    return os.environ.get(GRAPH_ENV_VAR, "1") == "0"


@dataclass(frozen=True)
class GraphConfig:
    """Which packed calls are graphed, and how graphs are cached.

    ``pad_to``: token counts are rounded up to a multiple of it (one graph serves the bucket).
    ``max_batch`` / ``max_seq`` / ``max_tokens``: calls with more sequences, a longer sequence or
    more tokens run eagerly; the packed runner needs the first two set. ``max_graphs``: the
    least recently replayed graph is dropped beyond this many. ``warmup``: eager runs before a
    capture. ``seq_buckets`` belongs to the padded-batch runner's pre-capture list; packed
    graphs are captured on first use."""

    pad_to: int = 64
    max_batch: int | None = None
    seq_buckets: tuple[int, ...] | None = None
    max_graphs: int = 32
    max_tokens: int = 2 ** 20
    max_seq: int | None = None
    warmup: int = 3


def round_up(value: int, multiple: int) -> int:
    return -(-value // multiple) * multiple


@dataclass
class PackedStaticInputs:
    """The fixed-address inputs one packed graph reads. ``written`` is how many leading rows of
    ``input_ids`` / ``position_ids`` may be non-zero (-1: unknown, the whole buffer)."""

    input_ids: Tensor
    cu_seqlens: Tensor
    position_ids: Tensor
    max_seqlen: int
    written: int = -1

    def stage(self, packed_ids: Tensor, cu_seqlens: Tensor, position_ids: Tensor) -> int:
        """Copy one batch in and return its token count M. Rows past M hold id 0 and position
        0; entries of ``cu_seqlens`` past the batch's own hold M (empty trailing sequences)."""
        m, bounds = packed_ids.shape[0], cu_seqlens.shape[0]
        self.input_ids[:m].copy_(packed_ids)
        self.position_ids[:m].copy_(position_ids)
        stale = self.input_ids.shape[0] if self.written < 0 else self.written
        if stale > m:
            self.input_ids[m:stale].zero_()
            self.position_ids[m:stale].zero_()
        self.written = m
        self.cu_seqlens[:bounds].copy_(cu_seqlens)
        if bounds < self.cu_seqlens.shape[0]:
            self.cu_seqlens[bounds:].fill_(m)
        return m


@dataclass
class _Bucket:
    graph: "torch.cuda.CUDAGraph"
    inputs: PackedStaticInputs
    out: Tensor


def _synthetic_lengths(tokens: int, n: int, max_seqlen: int) -> list[int]:
    """A valid batch for warm-up and capture: ``n`` sequences filled greedily up to
    ``max_seqlen`` from ``tokens`` (a bucket above ``n * max_seqlen`` keeps its tail outside)."""
    lengths, left = [], min(tokens, n * max_seqlen)
    for _ in range(n):
        lengths.append(min(max_seqlen, left))
        left -= lengths[-1]
    return lengths


class PackedGraphRunner:
    """Replays ``packed_forward`` from graphs keyed ``(round_up(M, pad_to), N, Smax, backend)``.
    ``captures`` counts the graphs captured so far."""

    def __init__(self, model: nn.Module, params: ModernBertParams, config: GraphConfig, backend: str = "hip", *,
                 execution=None):
        self.model = model
        self.params = params
        self.config = config
        self.backend = backend
        self.execution = forward._execution_for(model, execution)
        self.device = next(model.parameters()).device
        self.cache: "OrderedDict[tuple[int, int, int, str], _Bucket]" = OrderedDict()
        self.captures = 0
        self._resolved: dict[bool, str] = {}

    def _backend_now(self) -> str:
        grad = torch.is_grad_enabled()
        if grad not in self._resolved:
            dtype = self.model.embeddings.tok_embeddings.weight.dtype
            self._resolved[grad] = forward.resolve_backend(self.backend, self.params, device=self.device,
                                                           dtype=dtype)
        return self._resolved[grad]

    def key(self, m: int, n: int, max_seqlen: int) -> tuple[int, int, int, str]:
        return (round_up(m, self.config.pad_to), n, int(max_seqlen), self._backend_now())

    def admits(self, m: int, n: int, max_seqlen: int) -> bool:
        c = self.config
        return (m <= c.max_tokens and (c.max_seq is None or max_seqlen <= c.max_seq)
                and (c.max_batch is None or n <= c.max_batch))

    def __call__(self, packed_ids: Tensor, cu_seqlens: Tensor, max_seqlen: int, position_ids: Tensor) -> Tensor:
        m, n = packed_ids.shape[0], cu_seqlens.numel() - 1
        key = self.key(m, n, max_seqlen) if self.admits(m, n, max_seqlen) else None
        if key is None or key[3] != "hip":
            return self.eager(packed_ids, cu_seqlens, max_seqlen, position_ids)
        bucket = self.cache.get(key)
        if bucket is None:
            bucket = self.capture(*key)
            while len(self.cache) >= self.config.max_graphs:
                self.cache.popitem(last=False)
            self.cache[key] = bucket
        else:
            self.cache.move_to_end(key)
        rows = bucket.inputs.stage(packed_ids, cu_seqlens, position_ids)
        bucket.graph.replay()
        return bucket.out[:rows].clone()

    def eager(self, packed_ids, cu_seqlens, max_seqlen, position_ids) -> Tensor:
        return forward.packed_forward(self.model, self.params, packed_ids, cu_seqlens, max_seqlen, position_ids,
                                      backend=self.backend, execution=self.execution, _allow_graph=False)

    def capture(self, tokens: int, n: int, max_seqlen: int, backend: str) -> _Bucket:
        dev = self.device
        inputs = PackedStaticInputs(input_ids=torch.zeros(tokens, dtype=torch.long, device=dev),
                                    cu_seqlens=torch.zeros(n + 1, dtype=torch.int32, device=dev),
                                    position_ids=torch.zeros(tokens, dtype=torch.long, device=dev),
                                    max_seqlen=max_seqlen, written=0)
        cu, positions = staging.packed_layout_host(_synthetic_lengths(tokens, n, max_seqlen))
        inputs.stage(torch.zeros(positions.numel(), dtype=torch.long, device=dev), cu.to(dev, torch.int32),
                     positions.to(dev))
        current = torch.cuda.current_stream(dev)
        with torch.no_grad():
            side = torch.cuda.Stream(device=dev)  # default priority
            side.wait_stream(current)
            with torch.cuda.stream(side):
                for _ in range(self.config.warmup):
                    self.run(inputs)
            current.wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                out = self.run(inputs)
        self.captures += 1
        return _Bucket(graph=graph, inputs=inputs, out=out)

    def run(self, inputs: PackedStaticInputs) -> Tensor:
        """The captured region: embeddings and their norm, then the packed layer stack."""
        model, ex = self.model, self.execution
        norm = model.embeddings.norm
        x = ex.layer_norm(model.embeddings.tok_embeddings(inputs.input_ids), norm.weight, norm.eps)
        return forward.packed_core(model, self.params, x, inputs.cu_seqlens, inputs.max_seqlen, inputs.position_ids,
                                   execution=ex)


def build_packed_runner(model: nn.Module, params: ModernBertParams, config: GraphConfig, backend: str = "hip", *,
                        execution=None) -> PackedGraphRunner | None:
    """A runner when the backend can be captured (not ``"sdpa"``) and ``config`` bounds both the
    sequence count and the longest sequence (the reference's rule, graph.py:403-412); else None."""
    if backend == "sdpa" or config.max_batch is None or config.max_seq is None:
        return None
    return PackedGraphRunner(model, params, config, backend=backend, execution=execution)
