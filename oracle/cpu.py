"""ctypes access to the CPU attention libraries — TEST INFRASTRUCTURE / CPU BASELINE ONLY.

``port``: this repo's C restatement (oracle/cpu_attention.c).
``reference``: the reference's own ``pe_local_attention``
(packed_encoders/cpu/local_attention_x86.c:192-234), built from its source by oracle/Makefile
into ``oracle/_ref/``. Its ABI: ``int pe_local_attention(const float *q, const float *k,
const float *v, float *out, const int *lengths, int tokens, int heads, int sequences, int tile,
int half, int token_major, int workers, void *pool, float *scratch, size_t scratch_floats)``,
head_dim 64 and scale 0.125 fixed, scratch ``workers * (64 + tile) * ld`` floats with
``ld = round_up(min(tile + 2 * half, longest), 16)`` (cpu/attention.py:409-440).
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from functools import lru_cache
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def cpu_level() -> str:
    """x86-64 microarchitecture level the host supports: "v4" (AVX-512) or "v3" (AVX2)."""
    try:
        flags = set()
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    flags = set(line.split(":", 1)[1].split())
                    break
    except OSError:
        return "v3"
    return "v4" if {"avx512f", "avx512bw", "avx512vl", "avx512dq", "avx512cd"} <= flags else "v3"


def build(quiet: bool = True) -> None:
    """Run oracle/Makefile (the restatement always; the reference build when its source exists)."""
    out = subprocess.run(["make", "-C", str(HERE), "-j4"], capture_output=True, text=True)
    if out.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{out.stdout}\n{out.stderr}")
    if not quiet:
        print(out.stdout)


@lru_cache(maxsize=None)
def _load(kind: str) -> ctypes.CDLL | None:
    level = cpu_level()
    if kind == "port":
        path = HERE / "build" / f"libpe_oracle_cpu_{level}.so"
    else:
        path = HERE / "_ref" / f"libref_local_attention_{level}.so"
    if not path.exists():
        return None
    lib = ctypes.CDLL(str(path))
    if kind == "port":
        fn = lib.pe_oracle_local_attention
        fn.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 8 + [ctypes.c_float]
    else:
        fn = lib.pe_local_attention
        fn.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 7 + [ctypes.c_void_p] * 2 + [ctypes.c_size_t]
    fn.restype = ctypes.c_int
    return lib


def available(kind: str) -> bool:
    return _load(kind) is not None


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def local_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, lengths, half: int, *, kind: str = "port",
                    threads: int = 1, tile: int = 64, token_major: bool = False, scale: float = 0.125,
                    out: np.ndarray | None = None) -> np.ndarray:
    """FP32 packed attention over head-major ``[H, T, D]`` arrays with ``|i - j| <= half``.

    ``kind="reference"`` runs the reference's compiled kernel (head_dim 64, scale 0.125 only)."""
    lib = _load(kind)
    if lib is None:
        raise FileNotFoundError(f"oracle CPU library '{kind}' is not built (make -C oracle)")
    q, k, v = (np.ascontiguousarray(t, dtype=np.float32) for t in (q, k, v))
    heads, tokens, dim = q.shape
    lens = np.ascontiguousarray(np.asarray(lengths, dtype=np.int32))
    shape = (tokens, heads * dim) if token_major else (heads, tokens, dim)
    if out is None or out.shape != shape:
        out = np.empty(shape, dtype=np.float32)
    if kind == "port":
        rc = lib.pe_oracle_local_attention(_ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(lens), tokens, heads, len(lens),
                                           dim, tile, half, int(token_major), threads, scale)
    else:
        if dim != 64 or abs(scale - 0.125) > 0:
            raise ValueError("the reference CPU kernel is fixed to head_dim 64 and scale 0.125")
        longest = int(lens.max())
        eff_half = min(half, longest)
        columns = min(tile + 2 * eff_half, longest)
        ld = (columns + 15) // 16 * 16
        workers = max(1, min(threads, heads * len(lens)))
        scratch = np.empty(workers * (64 + tile) * ld, dtype=np.float32)
        rc = lib.pe_local_attention(_ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(lens), tokens, heads, len(lens), tile,
                                    half, int(token_major), workers, None, _ptr(scratch), scratch.size)
    if rc != 0:
        raise RuntimeError(f"{kind} CPU attention returned {rc}")
    return out


def physical_cores() -> int:
    """Physical cores in this process's affinity mask (the rule of cpu/topology.py:9-27)."""
    try:
        cpus = os.sched_getaffinity(0)
    except (AttributeError, OSError):
        return os.cpu_count() or 1
    cores = set()
    for cpu in cpus:
        base = Path(f"/sys/devices/system/cpu/cpu{cpu}/topology")
        try:
            cores.add((int((base / "physical_package_id").read_text()), int((base / "core_id").read_text())))
        except (OSError, ValueError):
            return len(cpus)
    return len(cores) or len(cpus)
