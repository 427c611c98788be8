"""libpe_attn.so loads on the CPU host and exports every entry point include/pe_attn.h declares.

Only host-side entry points are called here (ABI version, status text, workspace sizing, the
static short-kernel table and argument rejection); nothing launches a kernel.
"""

from __future__ import annotations

import ctypes
import re
import subprocess

import pytest

from conftest import ROOT

HEADER = ROOT / "include" / "pe_attn.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s+\**\s*(pe_\w+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def lib(pe):
    from packed_encoders_amd import _lib

    return _lib.library()


def test_header_declares_the_expected_entry_points():
    from packed_encoders_amd import _lib

    assert _declared() == sorted(_lib.EXPORTED)


@pytest.mark.parametrize("struct,cname", [("AttnArgs", "pe_attn_args"), ("RopeArgs", "pe_rope_args")])
def test_ctypes_structs_match_the_header_layout(pe, tmp_path, struct, cname):
    """Every field of the ctypes mirror sits at the offset, and has the size, that the C compiler
    gives the header's struct (compiled on the host with gcc against include/pe_attn.h), and the
    two structs have the same size: a field reordered or retyped on either side fails here, not
    as a wrong argument on the GPU."""
    import shutil

    from packed_encoders_amd import _lib

    gcc, hip_include = shutil.which("gcc"), "/opt/rocm/include"
    if gcc is None or not (ROOT / "include").is_dir() or not __import__("os").path.isdir(hip_include):
        pytest.skip("gcc or the HIP headers are not available")
    cls = getattr(_lib, struct)
    names = [f[0] for f in cls._fields_]
    body = "".join(f'    printf("%s %zu %zu\\n", "{n}", offsetof({cname}, {n}), sizeof((({cname} *)0)->{n}));\n'
                   for n in names)
    src = tmp_path / "layout.c"
    src.write_text('#include <stdio.h>\n#include "pe_attn.h"\nint main(void) {\n'
                   f'    printf("sizeof %zu 0\\n", sizeof({cname}));\n{body}    return 0;\n}}\n')
    exe = tmp_path / "layout"
    subprocess.run([gcc, "-D__HIP_PLATFORM_AMD__", "-I", str(ROOT / "include"), "-I", hip_include, str(src), "-o",
                    str(exe)], check=True, capture_output=True)
    got = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines():
        name, off, size = line.split()
        got[name] = (int(off), int(size))
    assert got.pop("sizeof")[0] == ctypes.sizeof(cls)
    want = {n: (getattr(cls, n).offset, getattr(cls, n).size) for n in names}
    assert got == want


def test_python_constants_match_the_header_macros(pe, tmp_path):
    """The ABI version, dtype code, status codes, static scratch size and kernel codes that
    _lib.py mirrors equal the header's macros, as the C compiler evaluates them."""
    import os
    import shutil

    from packed_encoders_amd import _lib

    gcc, hip_include = shutil.which("gcc"), "/opt/rocm/include"
    if gcc is None or not os.path.isdir(hip_include):
        pytest.skip("gcc or the HIP headers are not available")
    mirror = {"ABI_VERSION": _lib.ABI_VERSION, "DTYPE_BF16": _lib.DTYPE_BF16, "OK": _lib.OK, "EINVAL": _lib.EINVAL,
              "EUNSUPPORTED": _lib.EUNSUPPORTED, "EWORKSPACE": _lib.EWORKSPACE, "ELAUNCH": _lib.ELAUNCH,
              "ESCRATCH": _lib.ESCRATCH, "STATIC_SCRATCH_BYTES": _lib.STATIC_SCRATCH_BYTES,
              "KERNEL_NONE": _lib.KERNEL_NONE, "KERNEL_TILED": _lib.KERNEL_TILED,
              "KERNEL_GLOBAL64": _lib.KERNEL_GLOBAL64, "KERNEL_BAND64": _lib.KERNEL_BAND64,
              "KERNEL_WIDE": _lib.KERNEL_WIDE, "KERNEL_WIDE16": _lib.KERNEL_WIDE16}
    declared = set(re.findall(r"^#define PE_ATTN_(\w+) ", HEADER.read_text(), flags=re.M))
    assert set(mirror) <= declared, set(mirror) - declared
    body = "".join(f'    printf("{n} %lld\\n", (long long)(PE_ATTN_{n}));\n' for n in mirror)
    src = tmp_path / "macros.c"
    src.write_text('#include <stdio.h>\n#include "pe_attn.h"\nint main(void) {\n' + body + "    return 0;\n}\n")
    exe = tmp_path / "macros"
    subprocess.run([gcc, "-D__HIP_PLATFORM_AMD__", "-I", str(ROOT / "include"), "-I", hip_include, str(src), "-o",
                    str(exe)], check=True, capture_output=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    got = {n: int(v) for n, v in (line.split() for line in out.splitlines())}
    assert got == mirror


def test_library_exports_every_declared_symbol(lib):
    from packed_encoders_amd import _build

    out = subprocess.run(["nm", "-D", "--defined-only", str(_build.LIBRARY)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    for name in _declared():
        assert name in exported, name
        assert hasattr(lib, name)


def test_peaks_library_exports_its_header():
    """libpe_peaks.so (achieved-peak microbenchmarks) exports every entry point
    include/pe_peaks.h declares."""
    from packed_encoders_amd import _build

    text = (ROOT / "include" / "pe_peaks.h").read_text()
    declared = set(re.findall(r"^\s*int\s+(pe_peak_\w+)\s*\(", text, flags=re.M))
    assert declared == {"pe_peak_mfma_bf16", "pe_peak_read", "pe_peak_copy", "pe_peak_read_lds"}
    out = subprocess.run(["nm", "-D", "--defined-only", str(_build.PEAKS_LIBRARY)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    assert declared <= exported
    assert b"gfx950" in _build.PEAKS_LIBRARY.read_bytes()


def test_library_holds_gfx950_code():
    from packed_encoders_amd import _build

    data = _build.LIBRARY.read_bytes()
    assert b"gfx950" in data


def test_abi_version_and_status_text(lib):
    assert lib.pe_attn_abi_version() == 9
    assert lib.pe_attn_strerror(0) == b"ok"
    assert lib.pe_attn_strerror(-3) == b"workspace missing or too small"
    assert lib.pe_attn_strerror(-99) == b"unknown status"


def _args(**kw):
    from packed_encoders_amd import _lib

    a = _lib.AttnArgs()
    a.struct_size = ctypes.sizeof(_lib.AttnArgs)
    a.dtype = 1
    a.n_seq, a.total_tokens, a.max_seqlen = 64, 32438, 2048
    a.n_heads_q, a.n_heads_kv, a.head_dim = 12, 12, 64
    a.softmax_scale = 0.125
    a.window_left = a.window_right = -1
    a.short_max = -1
    for name, value in kw.items():
        setattr(a, name, value)
    return a


def _ws(lib, a):
    size = ctypes.c_size_t(12345)
    rc = lib.pe_attn_workspace_size(ctypes.byref(a), ctypes.byref(size))
    return rc, size.value


def test_workspace_size_is_host_arithmetic(lib):
    # 64 segments, max 2048, global head_dim 64: tiles of 256 rows (four waves of 64);
    # bound min(N*ceil(S/256), (T + N_long*255)/256)
    rc, size = _ws(lib, _args())
    assert rc == 0
    n_long = min(64, 32438 // 65)
    cap = min(64 * 8, (32438 + n_long * 255) // 256)
    assert size == 256 + 16 * cap
    # windowed head_dim 64: tiles of 128 rows (four waves of 32)
    rc, size = _ws(lib, _args(window_left=64, window_right=64))
    assert rc == 0 and size == 256 + 16 * min(64 * 16, (32438 + n_long * 127) // 128)
    # every segment fits the short kernel: no workspace
    rc, size = _ws(lib, _args(max_seqlen=64))
    assert rc == 0 and size == 0
    # GQA 4:1 packs 4 heads per tile; head_dim 256 tiles are four 16-row waves: 16-row tiles
    rc, size = _ws(lib, _args(n_heads_q=8, n_heads_kv=2, head_dim=256, max_seqlen=512, n_seq=256, total_tokens=71104))
    assert rc == 0
    assert size == 256 + 16 * min(256 * 32, (71104 + 256 * 15) // 16)
    # head_dim 128 keeps 32-row waves: 4 heads of 32 rows
    rc, size = _ws(lib, _args(n_heads_q=8, n_heads_kv=2, head_dim=128, max_seqlen=512, n_seq=256, total_tokens=71104))
    assert rc == 0
    assert size == 256 + 16 * min(256 * 16, (71104 + 256 * 31) // 32)
    # strips of 4 query tiles: min(N * ceil(ceil(S/256)/4), (tiles_by_tokens + N_long*3) // 4)
    rc, size = _ws(lib, _args(strip=4))
    tiles = (32438 + n_long * 255) // 256
    assert rc == 0 and size == 256 + 16 * min(64 * 2, (tiles + n_long * 3) // 4)


@pytest.mark.parametrize("field,value,status", [
    ("struct_size", 8, -1), ("dtype", 7, -2), ("head_dim", 96, -2), ("n_heads_kv", 5, -1),
    ("softmax_scale", 0.0, -1), ("window_left", -2, -1), ("causal", 2, -1), ("short_max", 129, -1),
    ("strip", 65, -1), ("strip", -1, -1), ("band_kernel", 3, -1), ("band_kernel", -1, -1),
    ("min_seqlen", -1, -1), ("min_seqlen", 2049, -1),
])
def test_bad_arguments_are_rejected_before_any_launch(lib, field, value, status):
    rc, _ = _ws(lib, _args(**{field: value}))
    assert rc == status
    a = _args(**{field: value})
    assert lib.pe_varlen_attn_fwd(ctypes.byref(a), None, 0, None) == status


def test_key_segment_sizes_are_checked_and_size_the_workspace(lib):
    """With cu_seqlens_k given, negative key sizes are rejected; a batch whose query segments
    are all short still needs the tiled workspace when its key segments are long, and that
    workspace counts every segment as possibly long."""
    a = _args(max_seqlen=64)
    a.cu_seqlens_k = 8  # any non-NULL value: only sizes are read here
    a.total_tokens_k, a.max_seqlen_k = -1, 100
    rc, _ = _ws(lib, a)
    assert rc == -1
    a.total_tokens_k, a.max_seqlen_k = 5000, 300
    rc, size = _ws(lib, a)
    n = a.n_seq
    assert rc == 0 and size == 256 + 16 * min(n * 1, (a.total_tokens + n * 127) // 128)
    rc, size = _ws(lib, _args(max_seqlen=64))  # same queries, keys shared: no tiled work
    assert rc == 0 and size == 0


def test_missing_device_pointers_are_rejected(lib):
    a = _args()  # q/k/v/o/cu are NULL with work to do
    assert lib.pe_varlen_attn_fwd(ctypes.byref(a), None, 0, None) == -1
    assert lib.pe_packed_short_attn_fwd(ctypes.byref(_args(max_seqlen=64)), None) == -1
    assert lib.pe_packed_short_attn_fwd(ctypes.byref(_args(max_seqlen=129)), None) == -2


def test_empty_batch_is_a_no_op(lib):
    a = _args(n_seq=0, total_tokens=0)
    assert lib.pe_varlen_attn_fwd(ctypes.byref(a), None, 0, None) == 0


def test_short_config_table(lib):
    out = (ctypes.c_int32 * 4)()
    expected = {1: (32, 32, 4, 4), 32: (32, 32, 4, 4), 33: (32, 64, 4, 4), 64: (32, 64, 4, 4),
                65: (32, 128, 2, 4), 128: (32, 128, 2, 4)}
    for max_seqlen, want in expected.items():
        assert lib.pe_attn_short_config(max_seqlen, 64, out) == 0
        assert tuple(out) == want
    assert lib.pe_attn_short_config(129, 64, out) == -1
    assert lib.pe_attn_short_config(64, 256, out) == -1


def test_python_config_mirror(pe):
    """The reference's keys (its dispatch bench reads config['block_n']) plus this kernel's own;
    any length gets an answer, past 128 the largest shape."""
    cfg = pe.select_packed_short_attention_config(100)
    assert cfg == {"block_m": 32, "block_n": 128, "num_warps": 4, "num_stages": 1, "key_capacity": 128,
                   "heads_per_workgroup": 2, "num_waves": 4}
    assert {"block_m", "block_n", "num_warps", "num_stages"} <= set(pe.select_packed_short_attention_config(20))
    assert pe.select_packed_short_attention_config(20)["block_n"] == 32
    assert pe.select_packed_short_attention_config(4096) == pe.select_packed_short_attention_config(128)
    assert pe.select_packed_short_attention_config(0)["block_n"] == 32


def _rope_args(**kw):
    from packed_encoders_amd import _lib

    a = _lib.RopeArgs()
    a.struct_size = ctypes.sizeof(_lib.RopeArgs)
    a.dtype = 1
    a.qkv_stride_row, a.table_stride_row = 3 * 12 * 64, 64
    a.table_rows, a.n_rows, a.n_heads, a.head_dim = 128, 128, 12, 64
    for name, value in kw.items():
        setattr(a, name, value)
    return a


@pytest.mark.parametrize("field,value,status", [
    ("struct_size", 8, -1), ("dtype", 2, -2), ("head_dim", 96, -2), ("n_heads", 0, -1), ("table_rows", 0, -1),
    ("n_rows", -1, -1),
])
def test_rope_bad_arguments_are_rejected_before_any_launch(lib, field, value, status):
    assert lib.pe_rope_qkv_fwd(ctypes.byref(_rope_args(**{field: value})), None) == status


def test_rope_missing_pointers_misaligned_strides_and_empty_input(lib):
    assert lib.pe_rope_qkv_fwd(ctypes.byref(_rope_args()), None) == -1  # NULL pointers, rows to do
    assert lib.pe_rope_qkv_fwd(ctypes.byref(_rope_args(n_rows=0)), None) == 0  # nothing to do
    buf = ctypes.create_string_buffer(64)
    p = (ctypes.addressof(buf) + 15) & ~15
    a = _rope_args(qkv=p, cos=p, sin=p, q_out=p, k_out=p, qkv_stride_row=3 * 12 * 64 + 4)
    assert lib.pe_rope_qkv_fwd(ctypes.byref(a), None) == -1  # row stride not a multiple of 8
    a = _rope_args(qkv=p, cos=p, sin=p, q_out=p, k_out=p, qkv_stride_row=3 * 12 * 64 - 8)
    assert lib.pe_rope_qkv_fwd(ctypes.byref(a), None) == -1  # rows narrower than 3HD
    a = _rope_args(qkv=p + 2, cos=p, sin=p, q_out=p, k_out=p)
    assert lib.pe_rope_qkv_fwd(ctypes.byref(a), None) == -1  # misaligned base


def test_noalloc_entry_point_rejects_calls_past_its_static_scratch(lib):
    """pe_varlen_attn_fwd_noalloc holds the plan list in a fixed device array: a call whose
    workspace would exceed it is refused with PE_ATTN_ESCRATCH before anything is launched or
    any device pointer is read (here there are none)."""
    from packed_encoders_amd import _lib

    big = _args(n_seq=200000, total_tokens=1 << 27, max_seqlen=4096, short_max=0)
    rc, size = _ws(lib, big)
    assert rc == 0 and size > _lib.STATIC_SCRATCH_BYTES
    assert lib.pe_varlen_attn_fwd_noalloc(ctypes.byref(big), None) == _lib.ESCRATCH
    assert lib.pe_attn_strerror(_lib.ESCRATCH).startswith(b"needs more than the static scratch")
    # malformed arguments are still reported as such
    assert lib.pe_varlen_attn_fwd_noalloc(ctypes.byref(_args(head_dim=96)), None) == -2
    assert lib.pe_varlen_attn_fwd_noalloc(ctypes.byref(_args(n_seq=0, total_tokens=0)), None) == 0


def _kernels(lib, short=False, **kw):
    out = (ctypes.c_int32 * 6)()
    a = _args(**kw)
    rc = lib.pe_attn_kernels(ctypes.byref(a), out)
    assert rc == 0, rc
    return tuple(out)[4:] if short else tuple(out)[:4]


def test_short_kernel_heads_per_workgroup(lib):
    """pe_attn_kernels reports the short kernel's heads per workgroup and its workgroups: the
    shape's default (pe_attn_short_config) halved while the batch would give fewer than eight
    workgroups per CU (2,048 on 256 CUs), so a small batch spreads over more, smaller workgroups."""
    q = dict(max_seqlen=64, total_tokens=1307)
    assert _kernels(lib, short=True, n_seq=32, **q) == (1, 32 * 12)  # C1
    assert _kernels(lib, short=True, n_seq=100, **q) == (1, 100 * 12)
    assert _kernels(lib, short=True, n_seq=342, **q) == (2, 342 * 6)
    assert _kernels(lib, short=True, n_seq=683, **q) == (4, 683 * 3)
    assert _kernels(lib, short=True, n_seq=576, max_seqlen=2000, total_tokens=60000) == (2, 576 * 6)  # C3
    assert _kernels(lib, short=True, n_seq=4096, max_seqlen=64, total_tokens=164139) == (4, 4096 * 3)  # Q4096
    assert _kernels(lib, short=True, n_seq=300, max_seqlen=128, total_tokens=20000) == (1, 300 * 12)
    assert _kernels(lib, short=True, head_dim=128, n_seq=4096, max_seqlen=128, total_tokens=300000) == (1, 4096 * 12)
    assert _kernels(lib, short=True, head_dim=128, n_seq=40, max_seqlen=32, total_tokens=800) == (1, 40 * 12)
    assert _kernels(lib, short=True, head_dim=256, n_heads_q=8, n_heads_kv=2) == (0, 0)


def test_kernel_choice_per_call(lib):
    """pe_attn_kernels reports (short capacity, long-segment kernel, strip, tile rows): the
    global head_dim 64 kernel, the tiled kernel for band calls below 17667 query tiles and the
    streaming band kernel from there (strip 8; strip 4 when forced on a smaller call),
    band_kernel overriding the size rule only where the window shape, an odd GQA ratio and
    shared key segments allow it."""
    from packed_encoders_amd import _lib

    band = dict(window_left=64, window_right=64)
    assert _kernels(lib) == (64, _lib.KERNEL_GLOBAL64, 1, 256)
    assert _kernels(lib, **band) == (64, _lib.KERNEL_TILED, 1, 128)  # C2: 3041 tiles
    assert _kernels(lib, band_kernel=1, **band) == (64, _lib.KERNEL_BAND64, 4, 128)
    c4 = dict(n_seq=16, total_tokens=131072, max_seqlen=8192, n_heads_q=16, n_heads_kv=16)
    assert _kernels(lib, **c4, **band) == (64, _lib.KERNEL_TILED, 1, 128)  # 16384 tiles
    assert _kernels(lib, **c4, band_kernel=1, **band) == (64, _lib.KERNEL_BAND64, 4, 128)
    big = dict(n_seq=512, total_tokens=253948, max_seqlen=2048)  # 23796 tiles
    assert _kernels(lib, **big, **band) == (64, _lib.KERNEL_BAND64, 8, 128)
    assert _kernels(lib, **big, band_kernel=2, **band) == (64, _lib.KERNEL_TILED, 1, 128)
    assert _kernels(lib, band_kernel=1, n_heads_q=12, n_heads_kv=4, **band)[1] == _lib.KERNEL_BAND64  # GQA 3:1
    assert _kernels(lib, band_kernel=1, n_heads_q=12, n_heads_kv=6, **band)[1] == _lib.KERNEL_TILED  # GQA 2:1
    assert _kernels(lib, band_kernel=1, window_left=5, window_right=7)[1] == _lib.KERNEL_TILED
    assert _kernels(lib, band_kernel=1, window_left=33, window_right=64)[1] == _lib.KERNEL_BAND64
    assert _kernels(lib, band_kernel=1, window_left=64, window_right=-1, causal=1)[1] == _lib.KERNEL_TILED
    assert _kernels(lib, head_dim=128) == (32, _lib.KERNEL_WIDE, 1, 128)
    assert _kernels(lib, head_dim=256, n_heads_q=8, n_heads_kv=2) == (0, _lib.KERNEL_WIDE16, 1, 16)
    assert _kernels(lib, max_seqlen=64, **band) == (64, _lib.KERNEL_NONE, 0, 0)
    a = _args(band_kernel=1, **band)
    a.cu_seqlens_k = 8  # sizes only
    a.total_tokens_k, a.max_seqlen_k = 32438, 2048
    out = (ctypes.c_int32 * 6)()
    assert lib.pe_attn_kernels(ctypes.byref(a), out) == 0 and out[1] == _lib.KERNEL_TILED
    # the band kernel's strips size the workspace: 4 tiles of 128 rows per entry
    rc, size = _ws(lib, _args(band_kernel=1, **band))
    n_long = min(64, 32438 // 65)
    tiles = (32438 + n_long * 127) // 128
    assert rc == 0 and size == 256 + 16 * min(64 * 4, (tiles + n_long * 3) // 4)


def test_band_kernel_envelope_is_the_tested_one(lib):
    """Every (left, right, causal) the streaming band kernel accepts (band_kernel=1, host-only
    kernel choice) lies in a block-count class whose extreme shapes the GPU tests force onto it
    (tests/test_band_kernel_gpu.py: BAND_WINDOWS and CLASS_EXTREMES), inside those extremes."""
    import math

    from packed_encoders_amd import _lib

    # block-count class (ceil(left / 32), ceil(right / 32)) -> tested (min, max) of left and right
    tested = {(0, 4): ((0, 0), (97, 128)), (4, 0): ((97, 128), (0, 0)), (1, 3): ((1, 32), (65, 96)),
              (3, 1): ((65, 96), (1, 32)), (2, 2): ((33, 64), (33, 64))}
    admitted = 0
    for causal in (0, 1):
        for wl in range(-1, 200):
            for wr in ([-1] if causal else range(-1, 200)):
                out = (ctypes.c_int32 * 6)()
                a = _args(band_kernel=1, window_left=wl, window_right=wr, causal=causal)
                assert lib.pe_attn_kernels(ctypes.byref(a), out) == 0
                if out[1] != _lib.KERNEL_BAND64:
                    continue
                admitted += 1
                right = 0 if causal else wr
                cls = (math.ceil(wl / 32), math.ceil(right / 32))
                assert cls in tested, (wl, wr, causal)
                (l0, l1), (r0, r1) = tested[cls]
                assert l0 <= wl <= l1 and r0 <= right <= r1, (wl, wr, causal)
    assert admitted == 32 + 32 + 32 * 32 * 2 + 32 * 32 + 32, admitted


def test_min_seqlen_above_the_boundary_skips_the_short_pass(lib):
    """A host lower bound on the lengths above the routing boundary leaves no segment short:
    no short kernel, every segment planned for the tiled kernel (the workspace bound counts
    all N segments as long); at or below the boundary, or 0 (unknown), routing is unchanged."""
    from packed_encoders_amd import _lib

    assert _kernels(lib, min_seqlen=98) == (0, _lib.KERNEL_GLOBAL64, 1, 256)
    assert _kernels(lib, min_seqlen=64) == (64, _lib.KERNEL_GLOBAL64, 1, 256)
    assert _kernels(lib, min_seqlen=0) == (64, _lib.KERNEL_GLOBAL64, 1, 256)
    assert _kernels(lib, head_dim=128, min_seqlen=33) == (0, _lib.KERNEL_WIDE, 1, 128)
    assert _kernels(lib, short_max=100, min_seqlen=98) == (128, _lib.KERNEL_GLOBAL64, 1, 256)  # capacity 128
    # every segment short by max_seqlen: the bound cannot exceed it, routing stays all-short
    assert _kernels(lib, max_seqlen=64, min_seqlen=64) == (64, _lib.KERNEL_NONE, 0, 0)
    rc, size = _ws(lib, _args(min_seqlen=98))
    assert rc == 0 and size == 256 + 16 * min(64 * 8, (32438 + 64 * 255) // 256)
