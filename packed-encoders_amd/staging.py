"""Batch metadata built on the host and moved to the GPU in one pinned copy.

The packed path needs small index tensors: ``cu_seqlens``, per-token positions and the gather
indices that strip padding. Built on the GPU from a device attention mask they cost two
device-to-host synchronisations (the packed length sizes the gather, ``max_seqlen`` is a host
int; packed_encoders/forward.py:395-415). When the mask or the lengths are on the host, as a
collator produces them, they are computed there and staged with one non-blocking copy
(``PinnedStager.put`` and ``packed_layout_host`` keep the names of the reference's
runtime/staging.py:21-55).

The stager copies through a ring of pinned slots rather than one buffer. A non-blocking copy is
queued behind the work already on the stream, so with a single buffer the host could not stage
batch i+1 before the GPU had reached batch i's copy, which keeps the host from running ahead
of a busy GPU. With two slots a ``put`` waits only for the copy issued two calls earlier.
"""

from __future__ import annotations

from collections.abc import Sequence

import numpy as np
import torch
from torch import Tensor


class PinnedStager:
    """Copies 1-D integer host tensors to ``device`` in one non-blocking transfer per ``put`` and
    returns device int64 views in input order. ``slots`` pinned int64 buffers are used in turn;
    a slot is refilled only after the event recorded behind its previous copy has completed."""

    def __init__(self, device: torch.device, capacity: int = 1 << 16, slots: int = 2):
        if slots < 1:
            raise ValueError("a stager needs at least one slot")
        self.device = torch.device(device)
        self._min_capacity = int(capacity)
        self._buffers: list[Tensor | None] = [None] * slots
        self._copied: list[torch.cuda.Event | None] = [None] * slots
        self._turn = 0

    def _slot(self, words: int) -> tuple[int, Tensor]:
        i = self._turn
        self._turn = (i + 1) % len(self._buffers)
        if self._copied[i] is not None:
            self._copied[i].synchronize()  # that slot's previous copy may still be reading it
        buf = self._buffers[i]
        if buf is None or buf.numel() < words:
            size = max(self._min_capacity, 1 << max(words - 1, 0).bit_length())
            buf = self._buffers[i] = torch.empty(size, dtype=torch.int64, pin_memory=True)
        return i, buf

    def put(self, parts: Sequence[Tensor]) -> list[Tensor]:
        sizes = [int(p.numel()) for p in parts]
        words = sum(sizes)
        i, buf = self._slot(words)
        if words:
            torch.cat([p.reshape(-1).to(torch.int64) for p in parts], out=buf[:words])
        with torch.cuda.device(self.device):  # the event follows the copy on that device's stream
            dev = buf[:words].to(self.device, non_blocking=True)
            done = torch.cuda.Event()
            done.record()
        self._copied[i] = done
        return list(dev.split(sizes))


_STAGERS: dict[torch.device, PinnedStager] = {}


def stager_for(device: torch.device) -> PinnedStager:
    """The process-wide stager of ``device``."""
    device = torch.device(device)
    if device.index is None:
        device = torch.device(device.type, torch.cuda.current_device())
    if device not in _STAGERS:
        _STAGERS[device] = PinnedStager(device)
    return _STAGERS[device]


def packed_layout_host(lengths: Sequence[int]) -> tuple[Tensor, Tensor]:
    """``(cu_seqlens [N+1], positions [T])``, int64 on the host, for sequences of ``lengths``
    packed back to back; positions restart at 0 in every sequence.

    Positions are a running count with a reset at each non-empty sequence's first token: the
    per-token increment is 1, except there, where it is ``1 - (length of the previous
    non-empty sequence)``; one cumulative sum then gives every position."""
    lens = np.fromiter((int(n) for n in lengths), dtype=np.int64)
    if lens.size and lens.min() < 0:
        raise ValueError("sequence lengths must be non-negative")
    cu = np.zeros(lens.size + 1, dtype=np.int64)
    np.cumsum(lens, out=cu[1:])
    step = np.ones(int(cu[-1]), dtype=np.int64)
    starts = cu[:-1][lens > 0]
    step[starts[1:]] = 1 - np.diff(starts)
    positions = np.cumsum(step) - 1
    return torch.from_numpy(cu), torch.from_numpy(positions)


def padded_layout_host(attention_mask: Tensor) -> tuple[Tensor, Tensor, Tensor, int]:
    """For a host ``attention_mask [B, S]`` (1 = real token): the flat indices of the real tokens
    in ``[B * S]`` order, ``cu_seqlens [B+1]``, positions (each token's column, the RoPE
    position Hugging Face ModernBERT gives it) and ``max_seqlen``, all int64 on the host."""
    if attention_mask.device.type != "cpu" or attention_mask.ndim != 2:
        raise ValueError("padded_layout_host takes a [B, S] host attention mask")
    b, s = attention_mask.shape
    real = attention_mask.reshape(-1) != 0
    indices = torch.nonzero(real, as_tuple=False).flatten()
    seqlens = real.view(b, s).sum(dim=1, dtype=torch.int64)
    cu = torch.zeros(b + 1, dtype=torch.int64)
    torch.cumsum(seqlens, 0, out=cu[1:])
    max_seqlen = int(seqlens.max()) if b else 0
    return indices, cu, indices % s, max_seqlen
