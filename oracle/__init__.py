"""Oracle for the packed varlen attention path — TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import, call, link or run anything in this directory, and only as the checker (or the timed CPU
baseline), never as the thing measured or shipped. The product path (``packed-encoders_amd/``)
never imports it and fails loudly when its HIP library is missing.

Contents:
- ``attention.py``: CPU restatement of the reference's packed attention semantics in numpy
  (float64), its brute-force loop form for tiny inputs, bf16 rounding, the sigmoid gate.
- ``cpu_attention.c`` + ``cpu.py``: C/OpenMP restatement of the reference's native CPU packed
  attention (``packed_encoders/cpu/local_attention_x86.c:132-234``), the CPU baseline.
- ``Makefile``: builds ``build/`` (this restatement) and ``_ref/`` (the reference's own C file,
  compiled from ``/root/reference`` when present) for the parity checks.
"""
