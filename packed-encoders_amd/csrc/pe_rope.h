// Split-half rotary embedding read straight from the packed QKV projection (gfx950).
//
// qkv is [n_rows, 3 * H * D] (q at column 0, k at H * D, v at 2 * H * D, left untouched): the
// attention kernels read v as a strided view of it, and q, k come out of this kernel RoPE'd and
// contiguous [n_rows, H, D]. Row r uses row r % table_rows of the cos / sin tables [*, D]: the
// per-token gathered tables of a packed batch (table_rows = n_rows), or the [S, D] tables of a
// dense [B, S] batch (row = b * S + s).
//
// out[i]         = bf16(x[i] * cos[i]         - x[i + D/2] * sin[i])
// out[i + D/2]   = bf16(x[i + D/2] * cos[i + D/2] + x[i] * sin[i + D/2])        (i < D/2)
// in fp32, each product rounded to fp32 and then summed (no fused multiply-add): the rounding
// of the fp32 formula x * cos + rotate_half(x) * sin.
//
// One thread = one 8-element chunk of the low half of one head of q or k and the matching
// chunk of the high half: 16-byte loads and stores, no exchange between lanes. Consecutive
// threads cover a row's 2 * H * D q and k elements in order, so reads and writes are
// coalesced. HBM-bound: per row, q and k are read once and written once (4 * H * D * 2 bytes)
// plus the two table rows (cache-resident for a dense batch).
#pragma once

#include "pe_attn_device.h"

namespace pe {

struct RopeParams {
    const __bf16 *qkv;
    const __bf16 *cos;
    const __bf16 *sin;
    __bf16 *q_out;
    __bf16 *k_out;
    int64_t qkv_st;    // qkv row stride, elements
    int64_t table_st;  // cos / sin row stride, elements
    int32_t table_rows;
    int32_t n_rows;
    int32_t heads;
};

// Split-half RoPE of 8 elements of a head's low half (lo) and their high-half partners (hi),
// in place, with the table elements of the same dims: each product rounded to fp32, then
// summed (no fused multiply-add), then rounded to bf16. The attention kernels' fused prologue
// uses the same function, so fused and separate RoPE agree bit for bit.
__device__ __forceinline__ void rope8(bf16x8 &lo, bf16x8 &hi, const bf16x8 &cl, const bf16x8 &ch, const bf16x8 &sl,
                                      const bf16x8 &sh) {
#pragma clang fp contract(off)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float a = (float)lo[j], b = (float)hi[j];
        const float l1 = a * (float)cl[j], l2 = b * (float)sl[j];
        const float h1 = b * (float)ch[j], h2 = a * (float)sh[j];
        lo[j] = (__bf16)(l1 - l2);
        hi[j] = (__bf16)(h1 + h2);
    }
}

template <int D>
__global__ __launch_bounds__(256) void rope_qkv_kernel(RopeParams p) {
    constexpr int CH = D / 16;  // chunk pairs per head
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t per_row = 2LL * p.heads * CH;
    const int64_t row = g / per_row;
    if (row >= p.n_rows) return;
    const int rem = (int)(g - row * per_row);
    const int which = rem / (p.heads * CH);  // 0: q, 1: k
    const int hc = rem - which * p.heads * CH;
    const int h = hc / CH, c = hc - h * CH;
    const int lo = 8 * c, hi = D / 2 + 8 * c;

    const __bf16 *x = p.qkv + row * p.qkv_st + (int64_t)which * p.heads * D + (int64_t)h * D;
    const int64_t trow = row % p.table_rows;
    const __bf16 *cs = p.cos + trow * p.table_st;
    const __bf16 *sn = p.sin + trow * p.table_st;
    bf16x8 ol = ld_g16(x + lo), oh = ld_g16(x + hi);
    const bf16x8 cl = ld_g16(cs + lo), ch = ld_g16(cs + hi);
    const bf16x8 sl = ld_g16(sn + lo), sh = ld_g16(sn + hi);
    rope8(ol, oh, cl, ch, sl, sh);
    __bf16 *out = (which == 0 ? p.q_out : p.k_out) + (row * p.heads + h) * D;
    *reinterpret_cast<bf16x8 *>(out + lo) = ol;
    *reinterpret_cast<bf16x8 *>(out + hi) = oh;
}

}  // namespace pe
