"""Packed input metadata (packed_encoders/batch.py:11-30).

Construction never reads, derives or validates tensor values: the caller (a collator) owns
their consistency, and the packed engine checks only shapes, dtypes and devices, which needs no
device-to-host transfer.
"""

from __future__ import annotations

from dataclasses import dataclass

from torch import Tensor


@dataclass(frozen=True)
class PackedBatch:
    """Real token ids of every sequence back to back; the output keeps that order, ``[T, hidden]``.

    The HIP ModernBERT engine needs device ``cu_seqlens`` (int32 ``[N+1]``), a host ``max_seqlen``
    bounding every length, and device ``position_ids`` (int64, each token's index within its
    sequence). ``host_lengths`` is optional.
    """

    input_ids: Tensor
    cu_seqlens: Tensor | None = None
    max_seqlen: int | None = None
    position_ids: Tensor | None = None
    host_lengths: tuple[int, ...] | None = None
