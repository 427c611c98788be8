"""Which kernel serves which packed segment on gfx950, and why.

The reference decides per batch, with an integer score calibrated per NVIDIA card, whether its
Triton short-segment kernel or FlashAttention serves the whole batch
(packed_encoders/attention_dispatch.py:17-205, fitted by benchmarks/fit_packed_attention_dispatch.py).
Here both legs are kernels of one library call and the decision is per segment, on the device:
a segment of at most ``short_max`` tokens runs the LDS-resident short kernel, a longer one the
tiled MFMA kernel, with no host read of ``cu_seqlens``. The one host decision is ``short_max``,
from host-known sizes only (head dim and ``max_seqlen``), so it is the same eagerly and while a
graph is captured; the C ABI takes the same default when called with ``short_max = -1``.

The rule, fitted to the short-vs-tiled sweep (``python bench.py --dispatch-sweep``, committed as
profiles/dispatch_sweep.md and re-derived by ``fit_boundary`` in the tests):

- ``max_seqlen <= 128``: every segment takes the short kernel, at its smallest key capacity
  (32, 64 or 128) that holds ``max_seqlen`` — faster than the tiled kernel at every measured
  length, both head dims and both batch scales (the reference's Triton kernel likewise keys its
  tile choice on ``Smax``, triton_packed_attention.py:29-42);
- longer batches: segments up to the fitted boundary (64 for head_dim 64, 32 for head_dim 128)
  take the short kernel at that capacity, the rest the tiled kernel. A larger capacity makes
  the short kernel slower on the shortest segments (fewer heads per workgroup, more staged
  keys), so the boundary is the capacity with the least sweep time summed over the measured
  lengths, per token.
- head_dim 256 always runs the tiled kernel (the short kernel serves head_dim <= 128).

The long segments of a call with a +-64-shaped band go to the tiled kernel or, on large calls,
the streaming band kernel; that size rule is fitted by ``fit_band_rule`` to the band sweep
(``python bench.py --band-sweep``, profiles/band_sweep.md) and is the C library's
``kBandMinTiles`` / ``kBandStrip8Tiles``.

Names the reference's callers consult are kept: ``AttentionWorkload`` (capture-safe batch
statistics) and ``get_packed_inference_policy`` (the current device's calibrated policy, None
where none is calibrated; crossovers are never borrowed from another GPU).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Iterable, Mapping, Sequence

import torch

SHORT_CAPACITIES = (32, 64, 128)  # key capacities of the short kernel's LDS tiles
SHORT_HEAD_DIMS = (64, 128)       # head dims the short kernel serves


def capacity_for(length: int) -> int:
    """The short kernel's smallest key capacity holding ``length`` keys (0 past the largest)."""
    for c in SHORT_CAPACITIES:
        if length <= c:
            return c
    return 0


@dataclass(frozen=True)
class AttentionWorkload:
    """Capture-safe statistics of a packed batch: segment count, live tokens, longest segment.
    Derived: the padded rectangle ``n_sequences * max_seqlen`` and the padding it would hold."""

    n_sequences: int
    live_tokens: int
    max_seqlen: int

    def __post_init__(self):
        n, m, s = self.n_sequences, self.live_tokens, self.max_seqlen
        if n < 1 or s < 1 or m < 0 or m > n * s:
            raise ValueError(f"invalid packed workload: {n} segments, {m} live tokens, longest {s}")

    @property
    def rectangle_tokens(self) -> int:
        return self.n_sequences * self.max_seqlen

    @property
    def fragmentation_tokens(self) -> int:
        return self.rectangle_tokens - self.live_tokens

    @property
    def mean_length(self) -> float:
        return self.live_tokens / self.n_sequences

    @classmethod
    def from_lengths(cls, lengths: Iterable[int]) -> "AttentionWorkload":
        values = [int(n) for n in lengths]
        if not values or min(values) < 0:
            raise ValueError("segment lengths must be a non-empty list of non-negative integers")
        return cls(len(values), sum(values), max(values))

    @classmethod
    def from_summary(cls, *, n_sequences: int, live_tokens: int, max_seqlen: int) -> "AttentionWorkload":
        return cls(int(n_sequences), int(live_tokens), int(max_seqlen))


@dataclass(frozen=True)
class HipDispatchPolicy:
    """Per-segment routing between the short and the tiled kernel on one GPU architecture.
    ``boundaries`` maps head dim to the short kernel's share of a batch whose longest segment
    exceeds its largest capacity (0: every segment to the tiled kernel)."""

    arch: str
    boundaries: tuple[tuple[int, int], ...]

    def short_max(self, head_dim: int, max_seqlen: int | None = None) -> int:
        """The routing boundary for a call: ``max_seqlen`` itself when the short kernel holds
        it, else the fitted boundary for ``head_dim``."""
        if int(head_dim) not in SHORT_HEAD_DIMS:
            return 0
        if max_seqlen is not None and 0 < int(max_seqlen) <= SHORT_CAPACITIES[-1]:
            return int(max_seqlen)
        return dict(self.boundaries).get(int(head_dim), 0)

    def route(self, lengths: Sequence[int], head_dim: int) -> tuple[list[int], list[int]]:
        """Indices of the segments each kernel serves, (short, tiled); empty ones in neither."""
        cut = self.short_max(head_dim, max(lengths) if lengths else None)
        short = [i for i, n in enumerate(lengths) if 0 < n <= cut]
        tiled = [i for i, n in enumerate(lengths) if n > cut]
        return short, tiled

    def use_flash(self, workload: AttentionWorkload, head_dim: int = 64) -> bool:
        """The reference's per-batch question on this architecture: whether the batch needs the
        long-segment (tiled) kernel at all."""
        return workload.max_seqlen > self.short_max(head_dim, workload.max_seqlen)


def fit_boundary(rows: Iterable[Mapping], head_dim: int, *, min_segments: int = 512) -> int:
    """The boundary (0, 32, 64 or 128) with the least total time over the sweep's query-batch
    rows for ``head_dim``: every measured length L is weighted by its tokens' time, a segment of
    length L <= c costing the short kernel's time at capacity c (columns ``short_us`` at L's own
    capacity, ``short64_us``, ``short128_us``), a longer one the tiled kernel's (``tiled_us``).
    Rows of small batches (fewer than ``min_segments`` segments) are launch-bound and ignored.
    Returns 0 when no row qualifies."""
    rows = [r for r in rows if int(r["head_dim"]) == int(head_dim) and int(r["n_seq"]) >= min_segments]
    if not rows:
        return 0

    def per_token(r, key):
        return float(r[key]) / float(r["tokens"])

    def cost(c: int) -> float:
        total = 0.0
        for r in rows:
            length = int(r["L"])
            if length > c:
                total += per_token(r, "tiled_us")
            elif c == capacity_for(length):
                total += per_token(r, "short_us")
            else:
                total += per_token(r, f"short{c}_us")
        return total

    return min((0, *SHORT_CAPACITIES), key=lambda c: (cost(c), c))


def fit_band_rule(rows: Iterable[Mapping]) -> tuple[int | None, int | None]:
    """The library's size rule for +-64-shaped band calls, fitted to the band sweep
    (``python bench.py --band-sweep``, profiles/band_sweep.md): ``(min_tiles, strip8_tiles)``,
    the streaming band kernel from ``min_tiles`` query tiles (128 rows x heads) on, at strip 8
    from ``strip8_tiles`` on and strip 4 below, the tiled kernel under ``min_tiles`` (None:
    never). The pair has the least total time over the rows (columns ``query_tiles``,
    ``tiled_us``, ``band4_us``, ``band8_us``); on equal totals the tiled kernel keeps more rows.
    Each threshold is placed halfway (geometric mean, rounded) between the two measured tile
    counts it separates, 0 when it precedes every row."""
    rows = [dict(r) for r in rows]
    counts = sorted({int(r["query_tiles"]) for r in rows})
    if not counts:
        return None, None
    n = len(counts)

    def cost(k: int, j: int) -> float:  # band from counts[k], strip 8 from counts[j] (n: never)
        total = 0.0
        for r in rows:
            i = counts.index(int(r["query_tiles"]))
            total += float(r["tiled_us"] if i < k else (r["band4_us"] if i < j else r["band8_us"]))
        return total

    k, j = min(((k, j) for k in range(n + 1) for j in range(k, n + 1)), key=lambda kj: (cost(*kj), -kj[0], kj[1]))

    def place(i: int) -> int | None:
        if i >= n:
            return None
        return 0 if i == 0 else round((counts[i - 1] * counts[i]) ** 0.5)

    return place(k), (place(j) if k < n else None)


# Fitted to profiles/dispatch_sweep.md (tests/test_host_cpu.py re-derives it from that table).
_GFX950_POLICY = HipDispatchPolicy(arch="gfx950", boundaries=((64, 64), (128, 32)))
_HIP_POLICY_BY_ARCH = {"gfx950": _GFX950_POLICY}


def current_gcn_arch(device: int | torch.device | None = None) -> str | None:
    """The device's gfx target without feature suffixes (``gfx950:sramecc+:xnack-`` -> ``gfx950``)."""
    try:
        if not torch.cuda.is_available():
            return None
        props = torch.cuda.get_device_properties(device if device is not None else torch.cuda.current_device())
        return str(getattr(props, "gcnArchName", "")).split(":")[0] or None
    except Exception:  # pragma: no cover - defensive
        return None


def get_hip_dispatch_policy(arch: str | None = None) -> HipDispatchPolicy | None:
    """The calibrated routing policy for ``arch`` (default: the current device), else None."""
    arch = current_gcn_arch() if arch is None else arch.split(":")[0]
    return _HIP_POLICY_BY_ARCH.get(arch) if arch else None


def hip_short_max(head_dim: int, arch: str | None = None, max_seqlen: int | None = None) -> int:
    """The routing boundary the HIP op uses: the calibrated policy's, else gfx950's."""
    policy = get_hip_dispatch_policy(arch) or _GFX950_POLICY
    return policy.short_max(head_dim, max_seqlen)


def _arch_of(compute_capability: tuple[int, int] | None, device_name: str | None) -> str | None:
    """gfx950 from what torch reports for it: compute capability (9, 5), or an MI350-series name."""
    name = (device_name or "").casefold()
    if compute_capability is not None and tuple(compute_capability) == (9, 5):
        return "gfx950"
    if "mi355" in name or "mi350" in name or "gfx950" in name:
        return "gfx950"
    return None


def get_packed_inference_policy(compute_capability: tuple[int, int] | None = None,
                                device_name: str | None = None, *,
                                for_cuda_graph: bool = False) -> HipDispatchPolicy | None:
    """The calibrated policy of a device (default: the current one), or None (the reference's
    entry point, attention_dispatch.py:164-205). Graph replay does not change which kernel is
    faster for a segment (the sweep itself is graph-replayed), so ``for_cuda_graph`` selects the
    same policy."""
    del for_cuda_graph
    if compute_capability is None and device_name is None:
        arch = current_gcn_arch()
    else:
        arch = _arch_of(compute_capability, device_name)
    return _HIP_POLICY_BY_ARCH.get(arch) if arch else None
