"""Writes tests/golden/ref_cpu_attention.npz from the reference's own compiled CPU kernel.

The reference ships no golden vectors for packed attention (its tests draw seeded inputs on the
fly). This script makes some from its native CPU packed attention, ``pe_local_attention``
(packed_encoders/cpu/local_attention_x86.c:192-234), compiled from the reference source by
oracle/Makefile into oracle/_ref/ (only where /root/reference is present). The fixture then
travels with the tests, so the GPU parity tests compare the HIP kernels with the reference's
outputs on a box that has no reference checkout.

Inputs: head-major ``[2, T, 64]`` Q/K/V drawn N(0, 1) from numpy's PCG64 (seed 20261201) and
rounded to bf16, stored as their raw bf16 bit patterns (uint16), so the bf16 GPU path reads
exactly the numbers the reference read as fp32. Row 0 of Q is zero (uniform softmax) and row 1
is scaled by 8 (a sharp row). Segment lengths cover every short-segment path of the reference
kernel (full-window 16 and 32, tails, 1) and segments long enough for its tiled path and for
this library's tiled kernel. Outputs: the reference kernel's fp32 result for each half width in
``HALVES`` (``half >= longest`` is global attention), scale 0.125 (fixed by the reference
kernel).

Run: python tests/golden/make_golden.py   (needs oracle/_ref built: make -C oracle)
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import attention as oa  # noqa: E402
from oracle import cpu  # noqa: E402

SEED = 20261201
HEADS, DIM = 2, 64
LENGTHS = (16, 32, 1, 15, 17, 31, 33, 65, 129, 7)
HALVES = (0, 16, 64, 129)
OUT = Path(__file__).resolve().parent / "ref_cpu_attention.npz"


def main() -> None:
    cpu.build()
    if not cpu.available("reference"):
        raise SystemExit("oracle/_ref is not built: the reference checkout is needed to write this fixture")
    rng = np.random.default_rng(SEED)
    T = sum(LENGTHS)
    q, k, v = (oa.to_bf16(rng.standard_normal((HEADS, T, DIM)).astype(np.float32)) for _ in range(3))
    q[:, 0] = 0.0
    q[:, 1] *= 8.0  # exact in bf16 (a power of two)
    outs = {}
    for half in HALVES:
        outs[f"out_half{half}"] = cpu.local_attention(q, k, v, LENGTHS, half, kind="reference", threads=1, tile=64)
    bits = {name: (np.ascontiguousarray(x).view(np.uint32) >> 16).astype(np.uint16)
            for name, x in (("q_bf16", q), ("k_bf16", k), ("v_bf16", v))}
    np.savez_compressed(OUT, **bits, lengths=np.asarray(LENGTHS, dtype=np.int32),
                        halves=np.asarray(HALVES, dtype=np.int32), scale=np.float32(0.125), **outs)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
