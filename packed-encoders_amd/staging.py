"""Batch metadata built on the host and moved to the GPU in one pinned copy.

The packed path needs small index tensors — ``cu_seqlens``, per-token positions, the gather
indices that strip padding. Built on the GPU from a device attention mask they cost two
device-to-host synchronisations (the packed length sizes the gather, ``max_seqlen`` is a host
int; packed_encoders/forward.py:395-415). When the mask (or the lengths) is on the host, as a
collator produces it, everything can be computed there and staged with one non-blocking copy
from a reused pinned buffer, leaving the launch stream free of syncs (the reference's
runtime/staging.py and benchmarks/helpers/packed_collator.py:68-196 follow the same plan).

The pinned buffer is reused; an event recorded after each copy makes the next ``put`` wait
until the previous copy has left the buffer before overwriting it.
"""

from __future__ import annotations

from collections.abc import Sequence

import torch
from torch import Tensor


class PinnedStager:
    """Copies several 1-D integer host tensors to ``device`` in one non-blocking transfer through
    a reused pinned int64 buffer; returns device int64 views in input order."""

    def __init__(self, device: torch.device, capacity: int = 1 << 16):
        self.device = torch.device(device)
        self._capacity = int(capacity)
        self._buf: Tensor | None = None
        self._done: torch.cuda.Event | None = None

    def _buffer(self, n: int) -> Tensor:
        if self._buf is None or self._buf.numel() < n:
            self._capacity = max(self._capacity, n, 2 * (self._buf.numel() if self._buf is not None else 0))
            self._buf = torch.empty(self._capacity, dtype=torch.int64, pin_memory=True)
        return self._buf

    def put(self, parts: Sequence[Tensor]) -> list[Tensor]:
        sizes = [int(p.numel()) for p in parts]
        total = sum(sizes)
        if self._done is not None and not self._done.query():
            self._done.synchronize()  # the previous copy is still reading the buffer
        buf = self._buffer(max(total, 1))
        off = 0
        for part, n in zip(parts, sizes):
            buf[off:off + n].copy_(part.reshape(-1))
            off += n
        with torch.cuda.device(self.device):
            dev = buf[:total].to(self.device, non_blocking=True)
            self._done = torch.cuda.Event()
            self._done.record()
        return list(dev.split(sizes))


_STAGERS: dict[torch.device, PinnedStager] = {}


def stager_for(device: torch.device) -> PinnedStager:
    """The process-wide stager of ``device`` (one pinned buffer per device)."""
    device = torch.device(device)
    if device.index is None:
        device = torch.device(device.type, torch.cuda.current_device())
    st = _STAGERS.get(device)
    if st is None:
        st = _STAGERS[device] = PinnedStager(device)
    return st


def packed_layout_host(lengths: Sequence[int]) -> tuple[Tensor, Tensor]:
    """``(cu_seqlens [N+1], positions [T])`` (int64, host) for sequences of ``lengths`` packed
    back to back, positions restarting at 0 in every sequence."""
    lens = torch.as_tensor(list(lengths), dtype=torch.int64)
    cu = torch.zeros(lens.numel() + 1, dtype=torch.int64)
    if lens.numel():
        torch.cumsum(lens, 0, out=cu[1:])
    starts = torch.repeat_interleave(cu[:-1], lens)
    positions = torch.arange(int(cu[-1]), dtype=torch.int64) - starts
    return cu, positions


def padded_layout_host(attention_mask: Tensor) -> tuple[Tensor, Tensor, Tensor, int]:
    """For a host ``attention_mask [B, S]`` (1 = real token): the flat indices of the real tokens
    in ``[B * S]`` order, ``cu_seqlens [B+1]``, positions (each token's column, the RoPE
    position Hugging Face ModernBERT gives it) and ``max_seqlen`` — all int64 on the host."""
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
