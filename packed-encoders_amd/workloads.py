"""Seeded synthetic packed batches for the benchmark configurations (host-side generators).

Segment lengths come from a counter-free splitmix64 stream with Box–Muller normals, so every
configuration is reproducible bit-for-bit on any host without numpy's or torch's generators.
Tensor data (Q/K/V, gates, token ids) is drawn separately with a seeded ``torch.Generator``.

Configurations (the workloads the benchmark baseline names):
  C1  32 segments, L ~ U{16..64}, 12 heads x 64, global                       (CPU-runnable)
  C2  ModernBERT-base: 64 docs, L = clip(round(LogNormal(ln 400, 0.8)), 32, 2048), 12 x 64,
      22 layers: every 3rd global, the rest a +-64 band
  C3  512 queries L ~ U{8..48} then 64 docs L = clip(round(LogNormal(ln 700, 0.8)), 256, 8192),
      12 x 64, global (sigma 0.8 is an assumption: the configuration names none); C3-shuffled is
      the same 576 segments in a seeded Fisher–Yates order (queries and documents interleaved)
  C4  16 x 8192, 16 heads x 64, global and +-64 band
  C5  256 segments, L ~ U{16..512}, 8 query / 2 kv heads x 256, causal, sigmoid gate
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

_MASK = (1 << 64) - 1


class SplitMix64:
    """splitmix64 (Steele, Lea & Flood 2014): state += golden gamma, then two xor-shift-multiply
    finalisation rounds."""

    def __init__(self, seed: int):
        self.state = seed & _MASK

    def next_u64(self) -> int:
        self.state = (self.state + 0x9E3779B97F4A7C15) & _MASK
        z = self.state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _MASK
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _MASK
        return z ^ (z >> 31)

    def uniform(self) -> float:
        """Uniform in [0, 1) with 53 random bits."""
        return (self.next_u64() >> 11) * (1.0 / (1 << 53))

    def randint(self, lo: int, hi: int) -> int:
        """Uniform integer in [lo, hi] (inclusive)."""
        return lo + min(hi - lo, int(self.uniform() * (hi - lo + 1)))

    def normal(self) -> float:
        """Standard normal by Box–Muller (one of the pair; the other is discarded)."""
        u1 = self.uniform()
        u2 = self.uniform()
        return math.sqrt(-2.0 * math.log(1.0 - u1)) * math.cos(2.0 * math.pi * u2)

    def lognormal_length(self, median: float, sigma: float, lo: int, hi: int) -> int:
        return int(min(hi, max(lo, round(math.exp(math.log(median) + sigma * self.normal())))))


@dataclass(frozen=True)
class AttentionLayer:
    """One attention call of a workload: window (-1 unbounded), causal, gate."""

    window: tuple[int, int] = (-1, -1)
    causal: bool = False
    gate: bool = False


@dataclass(frozen=True)
class Workload:
    name: str
    lengths: tuple[int, ...]
    n_heads_q: int
    n_heads_kv: int
    head_dim: int
    layers: tuple[AttentionLayer, ...]
    description: str = ""
    extra: dict = field(default_factory=dict)

    @property
    def total_tokens(self) -> int:
        return sum(self.lengths)

    @property
    def max_seqlen(self) -> int:
        return max(self.lengths)

    @property
    def scale(self) -> float:
        return self.head_dim ** -0.5

    def cu_seqlens(self) -> list[int]:
        out = [0]
        for n in self.lengths:
            out.append(out[-1] + n)
        return out


GLOBAL = AttentionLayer()
BAND64 = AttentionLayer(window=(64, 64))


def modernbert_layers(n_layers: int = 22, every: int = 3, half_window: int = 64) -> tuple[AttentionLayer, ...]:
    """Layer i is global when i % every == 0, else the +-half_window band (config.py:39-47)."""
    band = AttentionLayer(window=(half_window, half_window))
    return tuple(GLOBAL if i % every == 0 else band for i in range(n_layers))


def c1(seed: int = 1) -> Workload:
    rng = SplitMix64(seed)
    lengths = tuple(rng.randint(16, 64) for _ in range(32))
    return Workload("C1", lengths, 12, 12, 64, (GLOBAL,), "32 x U{16..64}, 12x64, global")


def c2(seed: int = 2) -> Workload:
    rng = SplitMix64(seed)
    lengths = tuple(rng.lognormal_length(400, 0.8, 32, 2048) for _ in range(64))
    return Workload("C2", lengths, 12, 12, 64, modernbert_layers(),
                    "ModernBERT-base 22 layers (8 global + 14 +-64), 64 docs LogNormal(400, 0.8) in [32, 2048]")


def c3(seed: int = 3, shuffled: bool = False) -> Workload:
    rng = SplitMix64(seed)
    queries = [rng.randint(8, 48) for _ in range(512)]
    docs = [rng.lognormal_length(700, 0.8, 256, 8192) for _ in range(64)]
    lengths = queries + docs
    if shuffled:  # Fisher–Yates with the same stream
        for i in range(len(lengths) - 1, 0, -1):
            j = rng.randint(0, i)
            lengths[i], lengths[j] = lengths[j], lengths[i]
    order = ", shuffled" if shuffled else ""
    return Workload("C3-shuffled" if shuffled else "C3", tuple(lengths), 12, 12, 64, (GLOBAL,),
                    f"512 queries U{{8..48}} + 64 docs LogNormal(700, 0.8) in [256, 8192]{order}, 12x64, global",
                    {"n_queries": 512})


def c4(band: bool = False) -> Workload:
    layer = BAND64 if band else GLOBAL
    return Workload("C4-band" if band else "C4", (8192,) * 16, 16, 16, 64, (layer,),
                    "16 x 8192, 16x64, " + ("+-64 band" if band else "global"))


def c5(seed: int = 5) -> Workload:
    rng = SplitMix64(seed)
    lengths = tuple(rng.randint(16, 512) for _ in range(256))
    return Workload("C5", lengths, 8, 2, 256, (AttentionLayer(causal=True, gate=True),),
                    "256 x U{16..512}, GQA 8:2 x 256, causal, sigmoid gate")


def query_sweep(n: int = 4096, seed: int = 6) -> Workload:
    """Scaled query batch (n x U{16..64}) where the HBM fraction of the short kernel is measurable."""
    rng = SplitMix64(seed)
    lengths = tuple(rng.randint(16, 64) for _ in range(n))
    return Workload(f"Q{n}", lengths, 12, 12, 64, (GLOBAL,), f"{n} x U{{16..64}}, 12x64, global")


CONFIGS = {"C1": c1, "C2": c2, "C3": c3, "C4": c4, "C5": c5}
