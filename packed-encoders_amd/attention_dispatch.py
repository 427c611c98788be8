"""Packed attention dispatch policies: the reference's exact-card score policies and the gfx950
routing policy between the LDS-resident short kernel and the tiled MFMA kernel.

Restates packed_encoders/attention_dispatch.py:17-205. ``AttentionWorkload``,
``FlashScorePolicy`` and ``get_packed_inference_policy`` keep their names, fields, integer
score and exact-card tables (the reference's measured Triton/Flash crossovers on NVIDIA cards,
kept as data so callers and tests that consult them behave identically). Those tables never
match an MI355X: on gfx950 the choice is not Triton versus Flash but, per segment on the
device, short kernel versus tiled kernel, and ``get_hip_dispatch_policy`` returns that policy.

Every input is a host-visible shape statistic; no policy reads ``cu_seqlens`` values, so the
same decision is safe before eager execution and while capturing a graph.
"""

from __future__ import annotations

from dataclasses import dataclass, replace
from typing import Sequence

import torch


@dataclass(frozen=True)
class AttentionWorkload:
    """Capture-safe summary of an already-packed attention workload."""

    n_sequences: int
    live_tokens: int
    max_seqlen: int
    rectangle_tokens: int
    fragmentation_tokens: int

    @classmethod
    def from_lengths(cls, lengths: Sequence[int]) -> "AttentionWorkload":
        values = tuple(int(length) for length in lengths)
        if not values or any(length < 0 for length in values):
            raise ValueError("sequence lengths must be a non-empty sequence of non-negative integers")
        return cls.from_summary(n_sequences=len(values), live_tokens=sum(values), max_seqlen=max(values))

    @classmethod
    def from_summary(cls, *, n_sequences: int, live_tokens: int, max_seqlen: int) -> "AttentionWorkload":
        n, m, s = int(n_sequences), int(live_tokens), int(max_seqlen)
        if n <= 0 or m < 0 or s <= 0 or m > n * s:
            raise ValueError(f"invalid packed workload N={n}, M={m}, Smax={s}")
        rectangle = n * s
        return cls(n_sequences=n, live_tokens=m, max_seqlen=s, rectangle_tokens=rectangle,
                   fragmentation_tokens=rectangle - m)


@dataclass(frozen=True)
class FlashScorePolicy:
    """Integer scalar score; Flash is selected at ``score >= threshold``
    (attention_dispatch.py:58-88)."""

    threshold: int
    live_token_weight: int = 0
    sequence_weight: int = 0
    max_seqlen_weight: int = 0
    rectangle_pair_weight: int = 0
    mean_square_work_weight: int = 0
    live_max_weight: int = 0
    query_cta_weight: int = 0

    def score(self, workload: AttentionWorkload) -> int:
        n, m, s = workload.n_sequences, workload.live_tokens, workload.max_seqlen
        block_m = 16 if s <= 64 else 64
        query_ctas = n * ((s + block_m - 1) // block_m)
        return (
            self.live_token_weight * m
            + self.sequence_weight * n
            + self.max_seqlen_weight * s
            + self.rectangle_pair_weight * n * s * s
            + self.mean_square_work_weight * (m * m // n)
            + self.live_max_weight * m * s
            + self.query_cta_weight * query_ctas
        )

    def use_flash(self, workload: AttentionWorkload) -> bool:
        return self.score(workload) >= self.threshold


# The reference's exact-card tables (attention_dispatch.py:91-143), kept as data.
_RTX_5090_PACKED_POLICY = FlashScorePolicy(live_token_weight=1, threshold=20_736)
_A100_PACKED_POLICY = FlashScorePolicy(sequence_weight=-203_715, mean_square_work_weight=24,
                                       query_cta_weight=41_801, threshold=9_422_745)
_L40S_PACKED_POLICY = FlashScorePolicy(live_token_weight=4_260, rectangle_pair_weight=-7,
                                       query_cta_weight=-11_752, threshold=77_166_921)
_L40S_PACKED_GRAPH_POLICY = replace(_L40S_PACKED_POLICY, threshold=74_000_000)
_H200_PACKED_POLICY = FlashScorePolicy(live_token_weight=1, threshold=131_073)
_B200_PACKED_POLICY = FlashScorePolicy(live_token_weight=1, threshold=131_073)

_PACKED_INFERENCE_POLICY_BY_DEVICE = {
    ((12, 0), "RTX 5090"): _RTX_5090_PACKED_POLICY,
    ((8, 0), "A100-SXM4-40GB"): _A100_PACKED_POLICY,
    ((8, 9), "L40S"): _L40S_PACKED_POLICY,
    ((9, 0), "H200"): _H200_PACKED_POLICY,
    ((10, 0), "B200"): _B200_PACKED_POLICY,
}
_PACKED_GRAPH_POLICY_BY_DEVICE = {((8, 9), "L40S"): _L40S_PACKED_GRAPH_POLICY}


def current_compute_capability() -> tuple[int, int] | None:
    try:
        if not torch.cuda.is_available():
            return None
        return torch.cuda.get_device_capability()
    except Exception:  # pragma: no cover - defensive
        return None


def current_device_name() -> str | None:
    try:
        if not torch.cuda.is_available():
            return None
        return torch.cuda.get_device_name()
    except Exception:  # pragma: no cover - defensive
        return None


def get_packed_inference_policy(compute_capability: tuple[int, int] | None = None,
                                device_name: str | None = None, *,
                                for_cuda_graph: bool = False) -> FlashScorePolicy | None:
    """Exact-card Triton/Flash policy, if calibrated (attention_dispatch.py:164-205).

    ``None`` for every card without a measured table, MI355X included: crossovers are never
    borrowed from another GPU."""
    infer_device = compute_capability is None
    cc = current_compute_capability() if infer_device else compute_capability
    if cc is None:
        return None
    if device_name is None and infer_device:
        device_name = current_device_name()
    if device_name is None:
        return None
    normalized = device_name.casefold()
    if for_cuda_graph:
        for (candidate_cc, fragment), policy in _PACKED_GRAPH_POLICY_BY_DEVICE.items():
            if candidate_cc == cc and fragment.casefold() in normalized:
                return policy
    for (candidate_cc, fragment), policy in _PACKED_INFERENCE_POLICY_BY_DEVICE.items():
        if candidate_cc == cc and fragment.casefold() in normalized:
            return policy
    return None


# ------------------------------------------------------------------------------ gfx950 (HIP)


@dataclass(frozen=True)
class HipDispatchPolicy:
    """Per-segment routing for the HIP kernels on one GPU architecture.

    A segment of length ``L`` runs the LDS-resident short kernel when ``L <= short_max`` for its
    head dim, else the tiled MFMA kernel; both launch in one call and each segment is claimed by
    exactly one of them on the device, so a batch mixing queries and documents is split with no
    host read. ``short_max = 0`` sends every segment to the tiled kernel."""

    arch: str
    short_max_by_head_dim: tuple[tuple[int, int], ...]

    def short_max(self, head_dim: int) -> int:
        return dict(self.short_max_by_head_dim).get(int(head_dim), 0)

    def route(self, lengths: Sequence[int], head_dim: int) -> tuple[list[int], list[int]]:
        """Indices of the segments each kernel serves: (short, tiled); empty segments in neither."""
        sm = self.short_max(head_dim)
        short = [i for i, n in enumerate(lengths) if 0 < n <= sm]
        tiled = [i for i, n in enumerate(lengths) if n > sm]
        return short, tiled


# gfx950 (MI355X / MI350X): boundary measured with bench.py's per-kernel sweep; the short kernel
# covers head_dim <= 128 and holds at most 128 keys in LDS.
_GFX950_POLICY = HipDispatchPolicy(arch="gfx950", short_max_by_head_dim=((64, 64), (128, 64), (256, 0)))
_HIP_POLICY_BY_ARCH = {"gfx950": _GFX950_POLICY}


def current_gcn_arch(device: int | torch.device | None = None) -> str | None:
    """The device's gfx target without feature suffixes (``gfx950:sramecc+:xnack-`` → ``gfx950``)."""
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


def hip_short_max(head_dim: int, arch: str | None = None) -> int:
    """The routing boundary the HIP op uses: the calibrated policy's, else gfx950's."""
    policy = get_hip_dispatch_policy(arch) or _GFX950_POLICY
    return policy.short_max(head_dim)
