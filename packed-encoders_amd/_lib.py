"""ctypes binding of libpe_attn.so, the C ABI declared in include/pe_attn.h.

Loading fails loudly: a missing or stale library raises ``ImportError`` (the reference's
"backend unavailable" signal, packed_encoders/ops.py:345-352), never a silent fallback.
"""

from __future__ import annotations

import ctypes
from functools import lru_cache
from pathlib import Path

from ._build import LIBRARY

ABI_VERSION = 9
DTYPE_BF16 = 1

OK, EINVAL, EUNSUPPORTED, EWORKSPACE, ELAUNCH, ESCRATCH = 0, -1, -2, -3, -4, -5
STATIC_SCRATCH_BYTES = 1 << 20  # PE_ATTN_STATIC_SCRATCH_BYTES
# PE_ATTN_KERNEL_*: the long-segment kernel pe_attn_kernels reports
KERNEL_NONE, KERNEL_TILED, KERNEL_GLOBAL64, KERNEL_BAND64, KERNEL_WIDE, KERNEL_WIDE16 = range(6)

EXPORTED = (
    "pe_attn_abi_version",
    "pe_attn_strerror",
    "pe_attn_workspace_size",
    "pe_varlen_attn_fwd",
    "pe_varlen_attn_fwd_noalloc",
    "pe_attn_plan",
    "pe_attn_short_fwd",
    "pe_attn_tiled_fwd",
    "pe_packed_short_attn_fwd",
    "pe_attn_short_config",
    "pe_attn_kernels",
    "pe_rope_qkv_fwd",
)


class AttnArgs(ctypes.Structure):
    """Mirror of ``pe_attn_args``."""

    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("dtype", ctypes.c_int32),
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("gate", ctypes.c_void_p),
        ("cu_seqlens", ctypes.c_void_p),
        ("q_stride_token", ctypes.c_int64),
        ("q_stride_head", ctypes.c_int64),
        ("k_stride_token", ctypes.c_int64),
        ("k_stride_head", ctypes.c_int64),
        ("v_stride_token", ctypes.c_int64),
        ("v_stride_head", ctypes.c_int64),
        ("o_stride_token", ctypes.c_int64),
        ("o_stride_head", ctypes.c_int64),
        ("gate_stride_token", ctypes.c_int64),
        ("gate_stride_head", ctypes.c_int64),
        ("n_seq", ctypes.c_int32),
        ("total_tokens", ctypes.c_int32),
        ("max_seqlen", ctypes.c_int32),
        ("n_heads_q", ctypes.c_int32),
        ("n_heads_kv", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float),
        ("window_left", ctypes.c_int32),
        ("window_right", ctypes.c_int32),
        ("causal", ctypes.c_int32),
        ("short_max", ctypes.c_int32),
        ("strip", ctypes.c_int32),
        ("cu_seqlens_k", ctypes.c_void_p),
        ("total_tokens_k", ctypes.c_int32),
        ("max_seqlen_k", ctypes.c_int32),
        ("band_kernel", ctypes.c_int32),
        ("min_seqlen", ctypes.c_int32),
        ("rope_cos", ctypes.c_void_p),
        ("rope_sin", ctypes.c_void_p),
        ("rope_table_stride", ctypes.c_int64),
        ("rope_table_rows", ctypes.c_int32),
    ]


class RopeArgs(ctypes.Structure):
    """Mirror of ``pe_rope_args``."""

    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("dtype", ctypes.c_int32),
        ("qkv", ctypes.c_void_p),
        ("cos", ctypes.c_void_p),
        ("sin", ctypes.c_void_p),
        ("q_out", ctypes.c_void_p),
        ("k_out", ctypes.c_void_p),
        ("qkv_stride_row", ctypes.c_int64),
        ("table_stride_row", ctypes.c_int64),
        ("table_rows", ctypes.c_int32),
        ("n_rows", ctypes.c_int32),
        ("n_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
    ]


@lru_cache(maxsize=1)
def library(path: str | None = None) -> ctypes.CDLL:
    """Load the in-tree library once; ``ImportError`` if it is missing or mismatched."""
    lib_path = Path(path) if path else LIBRARY
    if not lib_path.exists():
        raise ImportError(
            f"{lib_path} is not built: run __graft_entry__.build() (hipcc --offload-arch=gfx950)"
        )
    try:
        lib = ctypes.CDLL(str(lib_path))
    except OSError as exc:  # pragma: no cover - depends on the HIP runtime being present
        raise ImportError(f"cannot load {lib_path}: {exc}") from exc
    lib.pe_attn_abi_version.restype = ctypes.c_int
    lib.pe_attn_abi_version.argtypes = []
    lib.pe_attn_strerror.restype = ctypes.c_char_p
    lib.pe_attn_strerror.argtypes = [ctypes.c_int]
    lib.pe_attn_workspace_size.restype = ctypes.c_int
    lib.pe_attn_workspace_size.argtypes = [ctypes.POINTER(AttnArgs), ctypes.POINTER(ctypes.c_size_t)]
    lib.pe_varlen_attn_fwd.restype = ctypes.c_int
    lib.pe_varlen_attn_fwd.argtypes = [ctypes.POINTER(AttnArgs), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    lib.pe_varlen_attn_fwd_noalloc.restype = ctypes.c_int
    lib.pe_varlen_attn_fwd_noalloc.argtypes = [ctypes.POINTER(AttnArgs), ctypes.c_void_p]
    lib.pe_attn_plan.restype = ctypes.c_int
    lib.pe_attn_plan.argtypes = [ctypes.POINTER(AttnArgs), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    lib.pe_attn_short_fwd.restype = ctypes.c_int
    lib.pe_attn_short_fwd.argtypes = [ctypes.POINTER(AttnArgs), ctypes.c_void_p]
    lib.pe_attn_tiled_fwd.restype = ctypes.c_int
    lib.pe_attn_tiled_fwd.argtypes = [ctypes.POINTER(AttnArgs), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    lib.pe_packed_short_attn_fwd.restype = ctypes.c_int
    lib.pe_packed_short_attn_fwd.argtypes = [ctypes.POINTER(AttnArgs), ctypes.c_void_p]
    lib.pe_attn_short_config.restype = ctypes.c_int
    lib.pe_attn_short_config.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.POINTER(ctypes.c_int32)]
    lib.pe_attn_kernels.restype = ctypes.c_int
    lib.pe_attn_kernels.argtypes = [ctypes.POINTER(AttnArgs), ctypes.POINTER(ctypes.c_int32)]
    lib.pe_rope_qkv_fwd.restype = ctypes.c_int
    lib.pe_rope_qkv_fwd.argtypes = [ctypes.POINTER(RopeArgs), ctypes.c_void_p]
    version = lib.pe_attn_abi_version()
    if version != ABI_VERSION:
        raise ImportError(f"{lib_path} has ABI {version}, expected {ABI_VERSION}: rebuild it")
    return lib


def strerror(status: int) -> str:
    return library().pe_attn_strerror(status).decode()


def check(status: int, what: str) -> None:
    """Map a C status to the reference's exception types (ValueError / RuntimeError)."""
    if status == OK:
        return
    message = f"{what}: {strerror(status)} ({status})"
    if status in (EINVAL, EUNSUPPORTED, EWORKSPACE, ESCRATCH):
        raise ValueError(message)
    raise RuntimeError(message)
