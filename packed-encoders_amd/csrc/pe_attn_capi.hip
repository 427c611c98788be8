// C ABI of libpe_attn.so (declared in include/pe_attn.h): argument checks, host-side sizing
// and the launches of the plan, short, tiled and RoPE kernels on the caller's stream.
//
// Nothing here reads device memory, synchronises or allocates, so every entry point can be
// captured into a HIP graph. No exception crosses the ABI; failures are status codes.
#include "../../include/pe_attn.h"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <mutex>

#include "pe_attn_band64.h"
#include "pe_attn_device.h"
#include "pe_attn_global64.h"
#include "pe_attn_plan.h"
#include "pe_attn_short.h"
#include "pe_attn_tiled.h"
#include "pe_attn_tiled_wide16.h"
#include "pe_rope.h"

namespace pe {
// Workspace of pe_varlen_attn_fwd_noalloc: one copy per GPU, in device memory for the life of
// the process. In host code `scratch` names a host-side stand-in, never the device array: the
// array is reached only through the address hipGetSymbolAddress returns for the current
// device, kept per device (static_scratch below).
__device__ __align__(256) unsigned char scratch[PE_ATTN_STATIC_SCRATCH_BYTES];
}  // namespace pe

namespace {

using pe::AttnParams;

constexpr int kMaxDevices = 64;
std::mutex scratch_lock;
void *scratch_ptr[kMaxDevices];

// The current device's address of pe::scratch, looked up once per device.
int static_scratch(void **ptr) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return PE_ATTN_ELAUNCH;
    std::lock_guard<std::mutex> guard(scratch_lock);
    if (!scratch_ptr[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(pe::scratch)) != hipSuccess || !p) return PE_ATTN_ELAUNCH;
        scratch_ptr[dev] = p;
    }
    *ptr = scratch_ptr[dev];
    return PE_ATTN_OK;
}

// gfx950 routing boundary for batches longer than the short kernel's largest key capacity,
// per head dim, fitted to the short-vs-tiled sweep (bench.py --dispatch-sweep): 64 for head_dim
// 64, 32 for head_dim 128. Batches whose longest segment fits that capacity run every segment
// in the short kernel.
constexpr int kShortCapacity = 128;
constexpr int default_boundary(int head_dim) { return head_dim == 64 ? 64 : 32; }
constexpr int kMaxStrip = 64;         // query tiles per tiled-kernel workgroup, at most

int gcd_int(int a, int b) {
    while (b) {
        const int t = a % b;
        a = b;
        b = t;
    }
    return a;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Structural checks shared by every entry point; pointers and strides only when a launch
// will read them (workspace sizing needs sizes alone).
int check_args(const pe_attn_args *a, bool need_pointers = true) {
    if (!a || a->struct_size != sizeof(pe_attn_args)) return PE_ATTN_EINVAL;
    if (a->dtype != PE_ATTN_DTYPE_BF16) return PE_ATTN_EUNSUPPORTED;
    if (a->n_seq < 0 || a->total_tokens < 0 || a->max_seqlen < 0) return PE_ATTN_EINVAL;
    if (a->n_heads_q < 1 || a->n_heads_kv < 1 || a->n_heads_q % a->n_heads_kv) return PE_ATTN_EINVAL;
    if (a->head_dim != 64 && a->head_dim != 128 && a->head_dim != 256) return PE_ATTN_EUNSUPPORTED;
    if (!(a->softmax_scale > 0.0f) || a->softmax_scale != a->softmax_scale) return PE_ATTN_EINVAL;
    if (a->window_left < -1 || a->window_right < -1) return PE_ATTN_EINVAL;
    if (a->causal != 0 && a->causal != 1) return PE_ATTN_EINVAL;
    if (a->short_max < -1 || a->short_max > 128) return PE_ATTN_EINVAL;
    if (a->strip < 0 || a->strip > kMaxStrip) return PE_ATTN_EINVAL;
    if (a->band_kernel < 0 || a->band_kernel > 2) return PE_ATTN_EINVAL;
    if (a->min_seqlen < 0 || a->min_seqlen > a->max_seqlen) return PE_ATTN_EINVAL;
    if (a->cu_seqlens_k && (a->total_tokens_k < 0 || a->max_seqlen_k < 0)) return PE_ATTN_EINVAL;
    if (a->rope_cos || a->rope_sin) {
        if (!a->rope_cos || !a->rope_sin || a->rope_table_rows < 1 || a->rope_table_stride < a->head_dim ||
            (a->rope_table_stride & 7) || !aligned16(a->rope_cos) || !aligned16(a->rope_sin))
            return PE_ATTN_EINVAL;
        // The fused prologue lives in the short kernel (prepare() also needs every segment short),
        // which reads the tables through a buffer resource with 32-bit offsets.
        if (a->head_dim > 128 || a->cu_seqlens_k) return PE_ATTN_EUNSUPPORTED;
        if ((int64_t)a->rope_table_rows * a->rope_table_stride * 2 >= (int64_t)1 << 31) return PE_ATTN_EUNSUPPORTED;
    }
    if (!need_pointers || a->n_seq == 0 || a->total_tokens == 0) return PE_ATTN_OK;
    if (!a->q || !a->k || !a->v || !a->o || !a->cu_seqlens) return PE_ATTN_EINVAL;
    const void *ptrs[4] = {a->q, a->k, a->v, a->o};
    for (const void *p : ptrs)
        if (!aligned16(p)) return PE_ATTN_EINVAL;
    const int64_t strides[8] = {a->q_stride_token, a->q_stride_head, a->k_stride_token, a->k_stride_head,
                                a->v_stride_token, a->v_stride_head, a->o_stride_token, a->o_stride_head};
    for (int64_t s : strides)
        if (s < 0 || (s & 7)) return PE_ATTN_EINVAL;
    if (a->gate) {
        if (!aligned16(a->gate) || a->gate_stride_token < 0 || a->gate_stride_head < 0 ||
            (a->gate_stride_token & 7) || (a->gate_stride_head & 7))
            return PE_ATTN_EINVAL;
    }
    // Kernels address a segment through 32-bit buffer offsets bounded by its last row: rows
    // must not overlap (token stride >= head_dim) and a segment must span < 2 GiB per tensor.
    const int64_t kv_rows = a->cu_seqlens_k ? a->total_tokens_k : a->total_tokens;
    const int64_t kv_max = a->cu_seqlens_k ? a->max_seqlen_k : a->max_seqlen;
    const int64_t token_strides[5] = {a->q_stride_token, a->k_stride_token, a->v_stride_token, a->o_stride_token,
                                      a->gate ? a->gate_stride_token : a->head_dim};
    for (int i = 0; i < 5; ++i) {
        const int64_t s = token_strides[i];
        const bool kv = i == 1 || i == 2;
        if ((kv ? kv_rows : a->total_tokens) > 1 && s < a->head_dim) return PE_ATTN_EINVAL;
        if ((kv ? kv_max : (int64_t)a->max_seqlen) * s * 2 + 2 * a->head_dim >= (int64_t)1 << 31)
            return PE_ATTN_EUNSUPPORTED;
    }
    return PE_ATTN_OK;
}

int routing_boundary(const pe_attn_args *a) {
    if (a->head_dim > 128) return 0;  // the short kernel covers head_dim <= 128
    if (a->short_max >= 0) return a->short_max;
    const int32_t longest = a->cu_seqlens_k && a->max_seqlen_k > a->max_seqlen ? a->max_seqlen_k : a->max_seqlen;
    return longest > 0 && longest <= kShortCapacity ? longest : default_boundary(a->head_dim);
}

// The boundary a call routes by: 0 (every segment to the tiled kernels) when the caller's
// lower bound on the lengths leaves no segment short, which spares the short pass's launch.
int effective_short_max(const pe_attn_args *a) {
    const int sm = routing_boundary(a);
    return a->min_seqlen > sm ? 0 : sm;
}

int heads_per_tile(const pe_attn_args *a) { return gcd_int(a->n_heads_q / a->n_heads_kv, 4); }

// Upper bound on (segment, strip) entries the plan can emit, from host-known sizes only:
// a segment of L > short_max tokens has ceil(L / bm) query tiles in ceil(tiles / strip) strips.
int64_t tile_capacity(const pe_attn_args *a, int short_max, int bm, int strip) {
    const int32_t max_k = a->cu_seqlens_k ? a->max_seqlen_k : a->max_seqlen;
    if (a->n_seq == 0 || a->total_tokens == 0 || (a->max_seqlen <= short_max && max_k <= short_max)) return 0;
    const int64_t n = a->n_seq, t = a->total_tokens;
    // With separate key segments a segment of few queries can still be long (its keys): every
    // segment may then reach the tiled kernel.
    const int64_t n_long = short_max > 0 && !a->cu_seqlens_k ? (t / (short_max + 1) < n ? t / (short_max + 1) : n) : n;
    const int64_t tiles_per_seg = (a->max_seqlen + bm - 1) / bm;
    const int64_t by_shape = n * ((tiles_per_seg + strip - 1) / strip);
    const int64_t tiles_by_tokens = (t + n_long * (bm - 1)) / bm;
    const int64_t by_tokens = (tiles_by_tokens + n_long * (strip - 1)) / strip;
    return by_shape < by_tokens ? by_shape : by_tokens;
}

// Query tiles (128 rows x heads) of a call, from host-known sizes.
int64_t query_tiles(const pe_attn_args *a) { return (int64_t)a->total_tokens / 128 * a->n_heads_q; }

// Whether a call's long segments run the streaming band kernel (band64_attn_kernel) rather than
// the tiled kernel: its window shape, one query head per kv head group, shared key segments,
// and the caller's band_kernel choice; by default a call of at least kBandMinTiles query tiles.
// Both thresholds are fitted to a sweep of C2-like document mixes and equal-length batches
// (12 heads, +-64; attention_dispatch.fit_band_rule): the tiled kernel's short-lived
// workgroups (three per CU) win every call below about 13K tiles, the band kernel's strips
// (two workgroups per CU, each key block staged once) win large document mixes by 1-6% from
// about 24K tiles, at strip 8; the thresholds sit halfway (geometric) between those points.
constexpr int64_t kBandMinTiles = 17667;
constexpr int64_t kBandStrip8Tiles = 17667;
bool uses_band64(const pe_attn_args *a) {
    const int wr = a->causal ? 0 : a->window_right;
    const bool shape = a->head_dim == 64 && !a->cu_seqlens_k && heads_per_tile(a) == 1 &&
                       pe::band64_window(a->window_left, wr);
    if (!shape || a->band_kernel == 2) return false;
    return a->band_kernel == 1 || query_tiles(a) >= kBandMinTiles;
}

// Query tiles per tiled-kernel workgroup: the caller's choice, else the gfx950 default. The
// band kernel streams its key blocks along a strip: 8 tiles from kBandStrip8Tiles on, 4 on the
// smaller calls that force it (band_kernel = 1).
int effective_strip(const pe_attn_args *a) {
    if (a->strip > 0) return a->strip;
    if (!uses_band64(a)) return 1;
    return query_tiles(a) >= kBandStrip8Tiles ? 8 : 4;
}

AttnParams make_params(const pe_attn_args *a, int short_max) {
    AttnParams p;
    std::memset(&p, 0, sizeof(p));
    p.q = static_cast<const __bf16 *>(a->q);
    p.k = static_cast<const __bf16 *>(a->k);
    p.v = static_cast<const __bf16 *>(a->v);
    p.g = static_cast<const __bf16 *>(a->gate);
    p.o = static_cast<__bf16 *>(a->o);
    p.cu = a->cu_seqlens;
    p.cuk = a->cu_seqlens_k ? a->cu_seqlens_k : a->cu_seqlens;
    p.q_st = a->q_stride_token;
    p.q_sh = a->q_stride_head;
    p.k_st = a->k_stride_token;
    p.k_sh = a->k_stride_head;
    p.v_st = a->v_stride_token;
    p.v_sh = a->v_stride_head;
    p.o_st = a->o_stride_token;
    p.o_sh = a->o_stride_head;
    p.g_st = a->gate_stride_token;
    p.g_sh = a->gate_stride_head;
    p.n_seq = a->n_seq;
    p.hq = a->n_heads_q;
    p.group = a->n_heads_q / a->n_heads_kv;
    p.wl = a->window_left;
    p.wr = a->window_right;
    if (a->causal) p.wr = 0;  // causal = no key to the right of the query
    p.short_max = short_max;
    p.max_seqlen = a->max_seqlen;
    p.max_seqlen_k = a->cu_seqlens_k ? a->max_seqlen_k : a->max_seqlen;
    p.strip = effective_strip(a);
    p.band = uses_band64(a) ? 1 : 0;
    p.c = a->softmax_scale * pe::kLog2e;
    p.rcos = static_cast<const __bf16 *>(a->rope_cos);
    p.rsin = static_cast<const __bf16 *>(a->rope_sin);
    p.rst = a->rope_table_stride;
    p.rrows = a->rope_table_rows;
    return p;
}

template <int D, int SK, int HPW, bool GATE>
int launch_short_t(const AttnParams &p, hipStream_t stream) {
    dim3 grid(p.n_seq, (p.hq + HPW - 1) / HPW);
    if (p.rcos)
        hipLaunchKernelGGL((pe::short_attn_kernel<D, SK, HPW, GATE, true>), grid, dim3(256), 0, stream, p);
    else
        hipLaunchKernelGGL((pe::short_attn_kernel<D, SK, HPW, GATE, false>), grid, dim3(256), 0, stream, p);
    return hipGetLastError() == hipSuccess ? PE_ATTN_OK : PE_ATTN_ELAUNCH;
}

// Compute units of an MI355X.
constexpr int64_t kCUs = 256;

// Static short-kernel choice: key capacity SK (32/64/128) and heads per workgroup, sized so
// the workgroup's K and V^T stay within ~75 KB of LDS (two workgroups per CU).
void short_shape(int max_len, int d, int *sk, int *hpw) {
    *sk = max_len <= 32 ? 32 : (max_len <= 64 ? 64 : 128);
    if (d == 64)
        *hpw = *sk == 128 ? 2 : 4;
    else
        *hpw = *sk == 32 ? 4 : (*sk == 64 ? 2 : 1);
}

// hpw never exceeds the shape's default (short_shape), the most heads whose K and V fit LDS.
template <int D, int SK, bool GATE>
int launch_short_h(const AttnParams &p, int hpw, hipStream_t stream) {
    constexpr int kMax = (D == 64 ? 4 : 2) * 64 / SK;  // short_shape's hpw (4, 4, 2 / 4, 2, 1)
    if constexpr (kMax >= 4)
        if (hpw == 4) return launch_short_t<D, SK, 4, GATE>(p, stream);
    if constexpr (kMax >= 2)
        if (hpw == 2) return launch_short_t<D, SK, 2, GATE>(p, stream);
    return launch_short_t<D, SK, 1, GATE>(p, stream);
}

template <int D, bool GATE>
int launch_short_d(const AttnParams &p, int sk, int hpw, hipStream_t stream) {
    if (sk == 32) return launch_short_h<D, 32, GATE>(p, hpw, stream);
    if (sk == 64) return launch_short_h<D, 64, GATE>(p, hpw, stream);
    return launch_short_h<D, 128, GATE>(p, hpw, stream);
}

// Heads per short-kernel workgroup for a call: the shape's default, halved while the call
// would give fewer than eight workgroups per CU (a small batch: more, smaller workgroups, which
// fit more per CU and hide each other's load latency). Measured on gfx950: C3's 512 query
// segments (1,536 four-head workgroups, three rounds of two per CU) run their short pass 12 %
// faster with two heads per workgroup and 1 % slower with one; a 4,096-segment query batch
// keeps four heads (two: 1 % slower, one: 10 % slower); C1's 32 segments run one head each.
int short_heads(int hpw, int64_t n_seq, int hq) {
    while (hpw > 1 && n_seq * ((hq + hpw - 1) / hpw) < 8 * kCUs) hpw /= 2;
    return hpw;
}

int launch_short(const AttnParams &p, int d, bool gate, int short_max, hipStream_t stream) {
    int sk, hpw;
    short_shape(short_max, d, &sk, &hpw);
    hpw = short_heads(hpw, p.n_seq, p.hq);
    if (d == 64) return gate ? launch_short_d<64, true>(p, sk, hpw, stream) : launch_short_d<64, false>(p, sk, hpw, stream);
    if (d == 128) return gate ? launch_short_d<128, true>(p, sk, hpw, stream) : launch_short_d<128, false>(p, sk, hpw, stream);
    return PE_ATTN_EUNSUPPORTED;
}

// head_dim 256 runs wide16_attn_kernel with kWide16Waves waves of 16 query rows per workgroup:
// four waves (one per SIMD) and a 64 KB ring, so two workgroups share a CU and run out of
// step (one's softmax and epilogue under the other's MFMAs); eight waves with a 128 KB ring,
// one workgroup per CU, measured 6% slower on C5.
constexpr int kWide16Waves = 4;

// Key tile and LDS ring depth per head dim: 48 KB (head_dim 64: three workgroups per CU, two
// tiles in flight each), 64 KB (head_dim 128 and 256: two workgroups per CU).
template <int D>
struct TiledShape {
    static constexpr int BN = D >= 256 ? 32 : 64;
    static constexpr int NS = D == 64 ? 3 : (D == 256 ? (kWide16Waves == 8 ? 4 : 2) : 2);
};

// Query rows per tiled-kernel tile for g query heads per workgroup (the plan's tile height).
// Global head_dim 64 calls run global64_attn_kernel, whose waves hold 64 query rows.
bool global64(const pe_attn_args *a) {
    return a->head_dim == 64 && a->window_left < 0 && a->window_right < 0 && !a->causal;
}

int tile_rows(const pe_attn_args *a, int g) {
    if (a->head_dim == 256) return 16 * kWide16Waves / g;
    return (global64(a) ? 64 : 32) * (4 / g);
}

template <int D, int G, bool GATE, bool WIN>
int launch_tiled_t(AttnParams p, int64_t cap, hipStream_t stream) {
    constexpr int BN = TiledShape<D>::BN, NS = TiledShape<D>::NS;
    p.hgroups = p.hq / G;
    // Banded head_dim 64 launches deal work to the 8 XCDs in runs (tiled_attn_kernel): whole
    // rounds of runs, the surplus workgroups exiting at once.
    // head_dim 128 / 256 launches deal every call that way, in runs of the workgroups an XCD
    // holds at once.
    const int64_t run = D == 64    ? 8LL * pe::kXcdRun * p.hgroups
                        : D == 256 ? 8LL * pe::wide16_run<kWide16Waves, NS>(p.hgroups)
                                   : 8LL * pe::wide_run(p.hgroups);
    const int64_t blocks = (D > 64 || WIN) ? (cap * p.hgroups + run - 1) / run * run : cap * p.hgroups;
    if (blocks <= 0) return PE_ATTN_OK;
    if (blocks > 0x7fffffffLL) return PE_ATTN_EUNSUPPORTED;
    if constexpr (D == 64 && !WIN)
        hipLaunchKernelGGL((pe::global64_attn_kernel<G, GATE>), dim3((unsigned)blocks), dim3(256), 0, stream, p);
    else if constexpr (D == 64 && G == 1)
        if (p.band)
            hipLaunchKernelGGL((pe::band64_attn_kernel<GATE>), dim3((unsigned)blocks), dim3(256), 0, stream, p);
        else
            hipLaunchKernelGGL((pe::tiled_attn_kernel<D, G, BN, NS, GATE, WIN>), dim3((unsigned)blocks), dim3(256), 0,
                               stream, p);
    else if constexpr (D == 64)
        hipLaunchKernelGGL((pe::tiled_attn_kernel<D, G, BN, NS, GATE, WIN>), dim3((unsigned)blocks), dim3(256), 0,
                           stream, p);
    else if constexpr (D == 256)
        hipLaunchKernelGGL((pe::wide16_attn_kernel<D, kWide16Waves, G, NS, GATE, WIN>), dim3((unsigned)blocks),
                           dim3(64 * kWide16Waves), 0, stream, p);
    else
        hipLaunchKernelGGL((pe::wide_attn_kernel<D, G, BN, NS, GATE, WIN>), dim3((unsigned)blocks), dim3(256), 0,
                           stream, p);
    return hipGetLastError() == hipSuccess ? PE_ATTN_OK : PE_ATTN_ELAUNCH;
}

template <int D, bool GATE, bool WIN>
int launch_tiled_g(const AttnParams &p, int g, int64_t cap, hipStream_t stream) {
    if (g == 4) return launch_tiled_t<D, 4, GATE, WIN>(p, cap, stream);
    if (g == 2) return launch_tiled_t<D, 2, GATE, WIN>(p, cap, stream);
    return launch_tiled_t<D, 1, GATE, WIN>(p, cap, stream);
}

template <int D>
int launch_tiled_d(const AttnParams &p, int g, bool gate, int64_t cap, hipStream_t stream) {
    const bool win = p.wl >= 0 || p.wr >= 0;
    if (gate) return win ? launch_tiled_g<D, true, true>(p, g, cap, stream) : launch_tiled_g<D, true, false>(p, g, cap, stream);
    return win ? launch_tiled_g<D, false, true>(p, g, cap, stream) : launch_tiled_g<D, false, false>(p, g, cap, stream);
}

int launch_tiled(const AttnParams &p, int d, int g, bool gate, int64_t cap, hipStream_t stream) {
    if (d == 64) return launch_tiled_d<64>(p, g, gate, cap, stream);
    if (d == 128) return launch_tiled_d<128>(p, g, gate, cap, stream);
    if (d == 256) return launch_tiled_d<256>(p, g, gate, cap, stream);
    return PE_ATTN_EUNSUPPORTED;
}

constexpr size_t kWorkspaceHeader = 256;  // the entry counts live here, list follows aligned

// Workspace layout: [0, 256) header (int32 entries written, int32 entries needed), then the
// list of (segment, first query tile, query start, query rows) int4 entries.
struct Plan {
    int sm, g, bm, strip;
    int64_t cap;
};

int prepare(const pe_attn_args *a, Plan *plan) {
    int rc = check_args(a);
    if (rc) return rc;
    plan->sm = effective_short_max(a);
    // RoPE tables: the fused prologue is the short kernel's, so no segment may reach a tiled one.
    if (a->rope_cos && (plan->sm == 0 || a->max_seqlen > plan->sm)) return PE_ATTN_EUNSUPPORTED;
    plan->g = heads_per_tile(a);
    plan->bm = tile_rows(a, plan->g);
    plan->strip = effective_strip(a);
    plan->cap = tile_capacity(a, plan->sm, plan->bm, plan->strip);
    if (plan->cap > 0x7fffffffLL) return PE_ATTN_EUNSUPPORTED;
    return PE_ATTN_OK;
}

int check_workspace(const Plan &plan, const void *workspace, size_t bytes) {
    if (plan.cap > 0 && (!workspace || !aligned16(workspace) ||
                         bytes < kWorkspaceHeader + (size_t)plan.cap * sizeof(int4)))
        return PE_ATTN_EWORKSPACE;
    return PE_ATTN_OK;
}

template <int D>
int launch_rope(const pe::RopeParams &p, hipStream_t stream) {
    const int64_t threads = (int64_t)p.n_rows * 2 * p.heads * (D / 16);
    const int64_t blocks = (threads + 255) / 256;
    if (blocks > 0x7fffffffLL) return PE_ATTN_EUNSUPPORTED;
    hipLaunchKernelGGL(pe::rope_qkv_kernel<D>, dim3((unsigned)blocks), dim3(256), 0, stream, p);
    return hipGetLastError() == hipSuccess ? PE_ATTN_OK : PE_ATTN_ELAUNCH;
}

}  // namespace

extern "C" {

int pe_attn_abi_version(void) { return PE_ATTN_ABI_VERSION; }

const char *pe_attn_strerror(int status) {
    switch (status) {
        case PE_ATTN_OK: return "ok";
        case PE_ATTN_EINVAL: return "invalid argument";
        case PE_ATTN_EUNSUPPORTED: return "unsupported configuration";
        case PE_ATTN_EWORKSPACE: return "workspace missing or too small";
        case PE_ATTN_ELAUNCH: return "kernel launch failed";
        case PE_ATTN_ESCRATCH: return "needs more than the static scratch (PE_ATTN_STATIC_SCRATCH_BYTES)";
        default: return "unknown status";
    }
}

int pe_attn_workspace_size(const pe_attn_args *a, size_t *bytes) {
    if (!bytes) return PE_ATTN_EINVAL;
    const int rc = check_args(a, false);
    if (rc) return rc;
    const int sm = effective_short_max(a);
    const int g = heads_per_tile(a);
    const int64_t cap = tile_capacity(a, sm, tile_rows(a, g), effective_strip(a));
    *bytes = cap > 0 ? kWorkspaceHeader + (size_t)cap * sizeof(int4) : 0;
    return PE_ATTN_OK;
}

int pe_attn_plan(const pe_attn_args *a, void *workspace, size_t workspace_bytes, hipStream_t stream) {
    Plan plan;
    int rc = prepare(a, &plan);
    if (rc) return rc;
    if (plan.cap == 0) return PE_ATTN_OK;
    rc = check_workspace(plan, workspace, workspace_bytes);
    if (rc) return rc;
    int32_t *count = static_cast<int32_t *>(workspace);
    int4 *work = reinterpret_cast<int4 *>(static_cast<char *>(workspace) + kWorkspaceHeader);
    const int wr = a->causal ? 0 : a->window_right;
    hipLaunchKernelGGL(pe::plan_kernel, dim3(1), dim3(1024), 0, stream, a->cu_seqlens,
                       a->cu_seqlens_k ? a->cu_seqlens_k : a->cu_seqlens, a->n_seq, plan.sm, a->max_seqlen,
                       a->cu_seqlens_k ? a->max_seqlen_k : a->max_seqlen, plan.bm, plan.strip, a->window_left, wr,
                       a->head_dim > 64 ? 1 : 0, work, count, (int)plan.cap);
    return hipGetLastError() == hipSuccess ? PE_ATTN_OK : PE_ATTN_ELAUNCH;
}

int pe_attn_short_fwd(const pe_attn_args *a, hipStream_t stream) {
    Plan plan;
    const int rc = prepare(a, &plan);
    if (rc) return rc;
    if (plan.sm == 0 || a->n_seq == 0 || a->total_tokens == 0) return PE_ATTN_OK;
    const AttnParams p = make_params(a, plan.sm);
    return launch_short(p, a->head_dim, a->gate != nullptr, plan.sm, stream);
}

int pe_attn_tiled_fwd(const pe_attn_args *a, const void *workspace, size_t workspace_bytes, hipStream_t stream) {
    Plan plan;
    int rc = prepare(a, &plan);
    if (rc) return rc;
    if (plan.cap == 0) return PE_ATTN_OK;
    rc = check_workspace(plan, workspace, workspace_bytes);
    if (rc) return rc;
    AttnParams p = make_params(a, plan.sm);
    p.work_count = static_cast<const int32_t *>(workspace);
    p.work = reinterpret_cast<const int4 *>(static_cast<const char *>(workspace) + kWorkspaceHeader);
    p.work_cap = (int)plan.cap;
    return launch_tiled(p, a->head_dim, plan.g, a->gate != nullptr, plan.cap, stream);
}

int pe_varlen_attn_fwd(const pe_attn_args *a, void *workspace, size_t workspace_bytes, hipStream_t stream) {
    Plan plan;
    int rc = prepare(a, &plan);
    if (rc) return rc;
    rc = check_workspace(plan, workspace, workspace_bytes);
    if (rc) return rc;
    if ((rc = pe_attn_short_fwd(a, stream))) return rc;
    if ((rc = pe_attn_plan(a, workspace, workspace_bytes, stream))) return rc;
    return pe_attn_tiled_fwd(a, workspace, workspace_bytes, stream);
}

int pe_varlen_attn_fwd_noalloc(const pe_attn_args *a, hipStream_t stream) {
    size_t need = 0;
    int rc = pe_attn_workspace_size(a, &need);
    if (rc) return rc;
    if (need > PE_ATTN_STATIC_SCRATCH_BYTES) return PE_ATTN_ESCRATCH;
    void *ws = nullptr;
    if (need > 0 && (rc = static_scratch(&ws))) return rc;
    // Nothing in the workspace needs clearing: the plan writes the entry counts before the
    // tiled kernel reads them, and entries only up to that count.
    return pe_varlen_attn_fwd(a, ws, need, stream);
}

int pe_packed_short_attn_fwd(const pe_attn_args *a, hipStream_t stream) {
    int rc = check_args(a, false);
    if (rc) return rc;
    const int32_t smax = a->cu_seqlens_k && a->max_seqlen_k > a->max_seqlen ? a->max_seqlen_k : a->max_seqlen;
    if (smax <= 0 || smax > 128) return PE_ATTN_EUNSUPPORTED;
    if (a->head_dim > 128) return PE_ATTN_EUNSUPPORTED;
    rc = check_args(a);
    if (rc) return rc;
    if (a->n_seq == 0 || a->total_tokens == 0) return PE_ATTN_OK;
    AttnParams p = make_params(a, smax);
    return launch_short(p, a->head_dim, a->gate != nullptr, smax, stream);
}

int pe_attn_short_config(int32_t max_seqlen, int32_t head_dim, int32_t out[4]) {
    if (!out || max_seqlen <= 0 || max_seqlen > 128 || (head_dim != 64 && head_dim != 128)) return PE_ATTN_EINVAL;
    int sk, hpw;
    short_shape(max_seqlen, head_dim, &sk, &hpw);
    out[0] = 32;
    out[1] = sk;
    out[2] = hpw;
    out[3] = 4;
    return PE_ATTN_OK;
}

int pe_attn_kernels(const pe_attn_args *a, int32_t out[6]) {
    int rc = check_args(a, false);
    if (rc) return rc;
    if (!out) return PE_ATTN_EINVAL;
    const int sm = effective_short_max(a);
    int sk = 0, hpw = 0;
    if (sm > 0) short_shape(sm, a->head_dim, &sk, &hpw);
    const int g = heads_per_tile(a);
    const int32_t max_k = a->cu_seqlens_k ? a->max_seqlen_k : a->max_seqlen;
    const bool tiled = a->n_seq > 0 && a->total_tokens > 0 && (a->max_seqlen > sm || max_k > sm);
    int kernel = PE_ATTN_KERNEL_NONE;
    if (tiled) {
        if (a->head_dim == 256) kernel = PE_ATTN_KERNEL_WIDE16;
        else if (a->head_dim == 128) kernel = PE_ATTN_KERNEL_WIDE;
        else if (global64(a)) kernel = PE_ATTN_KERNEL_GLOBAL64;
        else kernel = uses_band64(a) ? PE_ATTN_KERNEL_BAND64 : PE_ATTN_KERNEL_TILED;
    }
    out[0] = sk;
    out[1] = kernel;
    out[2] = tiled ? effective_strip(a) : 0;
    out[3] = tiled ? tile_rows(a, g) : 0;
    const int heads = sk ? short_heads(hpw, a->n_seq, a->n_heads_q) : 0;
    const int64_t groups = heads ? (int64_t)a->n_seq * ((a->n_heads_q + heads - 1) / heads) : 0;
    out[4] = heads;
    out[5] = (int32_t)(groups < 0x7fffffff ? groups : 0x7fffffff);
    return PE_ATTN_OK;
}

int pe_rope_qkv_fwd(const pe_rope_args *a, hipStream_t stream) {
    if (!a || a->struct_size != sizeof(pe_rope_args)) return PE_ATTN_EINVAL;
    if (a->dtype != PE_ATTN_DTYPE_BF16) return PE_ATTN_EUNSUPPORTED;
    if (a->head_dim != 64 && a->head_dim != 128 && a->head_dim != 256) return PE_ATTN_EUNSUPPORTED;
    if (a->n_rows < 0 || a->n_heads < 1 || a->table_rows < 1) return PE_ATTN_EINVAL;
    if (a->n_rows == 0) return PE_ATTN_OK;
    if (!a->qkv || !a->cos || !a->sin || !a->q_out || !a->k_out) return PE_ATTN_EINVAL;
    const void *ptrs[5] = {a->qkv, a->cos, a->sin, a->q_out, a->k_out};
    for (const void *p : ptrs)
        if (!aligned16(p)) return PE_ATTN_EINVAL;
    const int64_t width = 3LL * a->n_heads * a->head_dim;
    if (a->qkv_stride_row < width || (a->qkv_stride_row & 7)) return PE_ATTN_EINVAL;
    if (a->table_stride_row < a->head_dim || (a->table_stride_row & 7)) return PE_ATTN_EINVAL;
    pe::RopeParams p;
    p.qkv = static_cast<const __bf16 *>(a->qkv);
    p.cos = static_cast<const __bf16 *>(a->cos);
    p.sin = static_cast<const __bf16 *>(a->sin);
    p.q_out = static_cast<__bf16 *>(a->q_out);
    p.k_out = static_cast<__bf16 *>(a->k_out);
    p.qkv_st = a->qkv_stride_row;
    p.table_st = a->table_stride_row;
    p.table_rows = a->table_rows;
    p.n_rows = a->n_rows;
    p.heads = a->n_heads;
    if (a->head_dim == 64) return launch_rope<64>(p, stream);
    if (a->head_dim == 128) return launch_rope<128>(p, stream);
    return launch_rope<256>(p, stream);
}

}  // extern "C"
