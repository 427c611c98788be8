"""Build libpe_attn.so (the HIP kernels and their C ABI) in-tree for gfx950.

The library is compiled ahead of time with hipcc, next to this file, so it travels with the
source tree; nothing is JIT-compiled at import time. ``build_library()`` always recompiles.
"""

from __future__ import annotations

import hashlib
import os
import re
import shutil
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
INCLUDE = HERE.parent / "include"
LIBRARY = HERE / "libpe_attn.so"
PEAKS_LIBRARY = HERE / "libpe_peaks.so"  # achieved-peak microbenchmarks (include/pe_peaks.h)
ARCH = "gfx950"

# hipcc flags. Packed FP32 instructions are disabled for device code; hipcc's host pass warns
# that it does not know the feature, which is harmless.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # keep MFMA accumulators in ordinary VGPRs: the softmax reads every score element, and
    # AGPR-resident accumulators would cost a v_accvgpr_read per element and per rescale
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]
SOURCES = ["pe_attn_capi.hip"]
PEAKS_SOURCES = ["pe_peaks.hip"]


def _code_only(text: str) -> str:
    """C/C++ source with comments removed and whitespace collapsed (no string literal in these
    sources holds a comment marker)."""
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    text = re.sub(r"//[^\n]*", " ", text)
    return " ".join(text.split())


def source_digest() -> str:
    """A short sha256 over the code of the attention library's HIP sources and public header
    (comments and layout excluded; the peaks microbenchmarks are not part of it) and the
    compile flags: what ties a committed profile of the kernels to the code it measured."""
    h = hashlib.sha256(" ".join(HIPCC_FLAGS).encode())
    files = [p for p in [*CSRC.iterdir(), *INCLUDE.iterdir()] if p.is_file() and "peaks" not in p.name]
    for path in sorted(files):
        h.update(path.name.encode())
        h.update(_code_only(path.read_text()).encode())
    return h.hexdigest()[:16]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the HIP attention library cannot be built")
    return path


def build_library(verbose: bool = False) -> Path:
    """Compile the attention library ``libpe_attn.so`` and the peaks microbenchmarks
    ``libpe_peaks.so`` (each an atomic replace); returns the attention library's path."""
    _compile(SOURCES, LIBRARY, verbose)
    _compile(PEAKS_SOURCES, PEAKS_LIBRARY, verbose)
    return LIBRARY


def _compile(sources: list[str], target: Path, verbose: bool) -> None:
    tmp = target.with_name(f"{target.name}.tmp{os.getpid()}")
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", *(str(CSRC / s) for s in sources), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "packed-fp32-ops' is not a recognized feature"
    stderr = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        tmp.unlink(missing_ok=True)
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{' '.join(cmd)}\n{stderr}")
    if verbose and stderr.strip():
        print(stderr)
    os.replace(tmp, target)


if __name__ == "__main__":
    print(build_library(verbose=True))
