// Device-side building blocks shared by the packed attention kernels (gfx950 / CDNA4).
//
// Conventions used by every kernel in this library:
//  * A wave is 64 lanes. Lane l is split as col = l % 32, kg = l / 32.
//  * Scores are computed transposed, S^T = K . Q^T, with v_mfma_f32_32x32x16_bf16:
//    A = 32 keys x 16 dims (row = key col, 8 dims per lane group kg),
//    B = 16 dims x 32 queries (query col, the same 8 dims per lane group),
//    so after the product lane l holds, for ONE query (col) and 16 keys, the accumulator
//    element j at key 8*(j/4) + 4*kg + (j%4) of the 32-key block. Every softmax statistic is
//    therefore a per-lane scalar, combined with the partner lane l ^ 32 only.
//  * The output is accumulated transposed too, O^T = V^T . P^T: A = 32 dims x 16 keys read
//    from the row-major V tile in LDS with ds_read_b64_tr_b16 (its 16-lane transpose hands a
//    lane four keys of one dim per read), B = the lane's own probabilities (8 of them), so no
//    probability ever leaves its register. The MFMA reduces over its K dimension, so any key
//    order shared by A and B is exact.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pe {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kLog2e = 1.4426950408889634f;

// Kernel parameters (one struct for every kernel; passed by value).
struct AttnParams {
    const __bf16 *q, *k, *v, *g;
    __bf16 *o;
    const int32_t *cu;
    const int32_t *cuk;  // key/value segment boundaries (cu when keys and queries share them)
    int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, o_st, o_sh, g_st, g_sh;
    int32_t n_seq;
    int32_t hq;      // query heads
    int32_t group;   // query heads per kv head
    int32_t wl, wr;  // window (-1: unbounded); causal already folded into wr = 0
    int32_t short_max;
    int32_t max_seqlen;    // the caller's bound on query segment lengths (32-bit offsets were sized for it)
    int32_t max_seqlen_k;  // and on key segment lengths
    int32_t hgroups; // head groups per work entry (tiled kernel)
    int32_t strip;   // query tiles per work entry (tiled kernel)
    int32_t band;    // 1: windowed head_dim 64 calls run the streaming band kernel
    float c;         // softmax_scale * log2(e)
    const int4 *work;          // tiled kernels: (segment, first q-tile, query start, query rows)
    const int32_t *work_count; // tiled kernels: number of valid entries
    int32_t work_cap;          // entries the workspace holds
    const __bf16 *rcos, *rsin; // short kernel's fused RoPE tables [rows, D] (NULL: none)
    int64_t rst;               // table row stride, elements
    int32_t rrows;             // table rows: packed row r takes row r % rrows
};

// A tiled kernel's work item: the plan's (segment, first query tile, query start, query rows)
// and the segment's keys. The entry is loaded together with the entry count, its index clamped
// to the list's capacity so the read stays inside the workspace: the two loads overlap, and the
// segment's bounds come with the entry instead of a further dependent read of cu_seqlens (keys
// are read from cu_seqlens_k only when it differs from cu_seqlens). `valid` is false for an
// index past the count or an entry planned for other arguments.
struct WorkItem {
    int seg, qt_first, start, L, kstart, Lk;
    bool valid;
};

__device__ __forceinline__ WorkItem load_work(const AttnParams &p, int entry) {
    const int count = p.work_count[0];
    const int4 w = p.work[min(max(entry, 0), p.work_cap - 1)];
    WorkItem it;
    it.seg = w.x;
    it.qt_first = w.y;
    it.start = w.z;
    it.L = w.w;
    it.valid = entry >= 0 && entry < count && w.x >= 0 && w.x < p.n_seq && w.y >= 0 && p.strip >= 1;
    it.kstart = w.z;
    it.Lk = w.w;
    if (p.cuk != p.cu && it.valid) {
        it.kstart = p.cuk[w.x];
        it.Lk = p.cuk[w.x + 1] - it.kstart;
    }
    return it;
}

typedef int i32x4 __attribute__((ext_vector_type(4)));

// Buffer resources. A raw buffer (stride 0) whose range ends at the last byte of a segment's
// last row makes the hardware return 0 for any load beyond it and drop any store beyond it,
// so segment tails need no branches; offsets are 32-bit (voffset VGPR + soffset SGPR).
// Word 3 is the gfx9 raw-buffer configuration (32-bit data format, no swizzle).
constexpr int kBufferWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, kBufferWord3);
}

// Range of `rows` rows of `d` bf16 elements `stride` elements apart (0 rows: empty range).
__device__ __forceinline__ uint32_t rows_bytes(int rows, int64_t stride, int d) {
    return rows > 0 ? (uint32_t)((int64_t)(rows - 1) * stride * 2 + d * 2) : 0u;
}

__device__ __forceinline__ bf16x8 buf_ld16(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
__device__ __forceinline__ void buf_st16(__amdgpu_buffer_rsrc_t r, int voff, bf16x8 x) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, x), r, voff, 0, 0);
}

// Wave-uniform value as a scalar (lets the compiler branch on SCC instead of EXEC masks).
__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// True when `pred` holds on any lane of the wave (a scalar result).
__device__ __forceinline__ bool wave_any(bool pred) { return __builtin_amdgcn_ballot_w64(pred) != 0; }

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 ld_g16(const __bf16 *p) {
    return *reinterpret_cast<const bf16x8 *>(p);
}
__device__ __forceinline__ bf16x8 ld_s16(const __bf16 *p) {
    return *reinterpret_cast<const bf16x8 *>(p);
}
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Key index (within its 32-key block) of accumulator element j held by lane group kg.
__device__ __forceinline__ int acc_key(int j, int kg) { return 8 * (j >> 2) + 4 * kg + (j & 3); }

// Round 8 fp32 probabilities to bf16 (round to nearest even) as one MFMA operand.
__device__ __forceinline__ bf16x8 to_bf16x8(const f32x16 &s, int base) {
    bf16x8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = (__bf16)s[base + i];
    return r;
}

// acc + p[2i] + p[2i + 1] for one bf16 pair of an MFMA operand, summed in fp32 (v_dot2 with
// ones): the probabilities the P.V product uses, added without a separate conversion.
__device__ __forceinline__ float sum2(const bf16x8 &p, int i, float acc) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const bf16x2 pair = {p[2 * i], p[2 * i + 1]};
    const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};
    return __builtin_amdgcn_fdot2_f32_bf16(pair, ones, acc, false);
}

// p[2i] + p[2i + 1] in fp32, starting a sum: the VOP3P form of v_dot2 with an inline zero
// accumulator, which needs no register cleared beforehand (the compiler selects the
// accumulating VOP2 form, v_dot2c, and clears its destination with a separate move).
__device__ __forceinline__ float sum2_first(const bf16x8 &p, int i) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const bf16x2 pair = {p[2 * i], p[2 * i + 1]};
    float r;
    asm("v_dot2_f32_bf16 %0, %1, %2, 0" : "=v"(r) : "v"(pair), "s"(0x3f803f80u));
    return r;
}

// acc + p[2i] + p[2i + 1] in fp32 into a new register, acc kept: the VOP3P form of v_dot2 (the
// accumulating VOP2 form would first copy acc with a separate move).
__device__ __forceinline__ float sum2_from(const bf16x8 &p, int i, float acc) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const bf16x2 pair = {p[2 * i], p[2 * i + 1]};
    float r;
    asm("v_dot2_f32_bf16 %0, %1, %2, %3" : "=v"(r) : "v"(pair), "s"(0x3f803f80u), "v"(acc));
    return r;
}

// Bits lo..hi (clamped to 0..31) of a 32-bit mask; 0 when the range is empty. lo >= 0.
__device__ __forceinline__ uint32_t bit_range(int lo, int hi) {
    hi = min(hi, 31);
    const uint32_t upto = hi >= 31 ? 0xffffffffu : (1u << (max(hi, -1) + 1)) - 1u;
    const uint32_t below = lo >= 32 ? 0xffffffffu : (1u << lo) - 1u;
    return hi < lo ? 0u : upto & ~below;
}

// Per-lane mask of the keys of 32-key block kb0 that row `row` may read, bit x standing for key
// kb0 + 4 kg + x (the keys of accumulator elements x = acc_key(j, 0) of lane group kg): keys
// below L and inside the window [row - wl, row + wr] (a negative bound is unbounded).
__device__ __forceinline__ uint32_t key_mask(int kb0, int kg, int row, int L, int wl, int wr) {
    const int base = kb0 + 4 * kg;
    int lo = 0, hi = L - 1 - base;
    if (wl >= 0) lo = max(lo, row - wl - base);
    if (wr >= 0) hi = min(hi, row + wr - base);
    return bit_range(lo, hi);
}

// Score a, or -inf where bit x of mask m is clear (two VALU: a signed bitfield extract and a
// bitwise select).
__device__ __forceinline__ float mask_score(float a, uint32_t m, int x) {
    const int keep = (int)(m << (31 - x)) >> 31;
    return __builtin_bit_cast(float, (__builtin_bit_cast(int, a) & keep) | (~keep & (int)0xff800000));
}

// Rows passed to the mask helpers below are key positions: query row r of a segment whose key
// segment is Lk long and query segment Lq long sits at key position r + (Lk - Lq) (queries are
// the tail of their keys; 0 when both are the same segment).

// Whether key block [kb0, kb0 + 32) intersects the keys any row in [r0, r1) may read.
__device__ __forceinline__ bool block_live(int kb0, int L, int r0, int r1, int wl, int wr) {
    if (kb0 >= L) return false;
    if (wl >= 0 && kb0 + 31 < r0 - wl) return false;
    if (wr >= 0 && kb0 > r1 - 1 + wr) return false;
    return true;
}

// Whether every (row, key) of rows [r0, r1) x keys [kb0, kb0 + 32) is allowed (no masking).
__device__ __forceinline__ bool block_full(int kb0, int L, int r0, int r1, int wl, int wr) {
    if (kb0 + 32 > L) return false;
    if (wl >= 0 && (r1 - 1) - kb0 > wl) return false;
    if (wr >= 0 && (kb0 + 31) - r0 > wr) return false;
    return true;
}

// Output rounding and the optional fused sigmoid gate: y = bf16(bf16(o) * bf16(sigmoid(g))),
// the rounding order of the reference's gate kernel (packed_encoders/_kernels/hybrid.py:197-206).
// Roundings go two at a time (v_cvt_pk_bf16_f32). The sigmoid's reciprocal is v_rcp_f32
// (1 ulp) rather than an IEEE division (about ten instructions): its result is rounded to bf16
// next, which a 1-ulp fp32 difference can move by one bf16 step only when the quotient lies
// within that ulp of a rounding boundary.

// bf16(sigmoid(g)) of 4 gate values.
__device__ __forceinline__ bf16x4 sigmoid4(bf16x4 g) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    float sg[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) sg[i] = __builtin_amdgcn_rcpf(1.0f + __expf(-(float)g[i]));
    const bf16x2 s01 = __builtin_convertvector(f32x2{sg[0], sg[1]}, bf16x2);
    const bf16x2 s23 = __builtin_convertvector(f32x2{sg[2], sg[3]}, bf16x2);
    return bf16x4{s01[0], s01[1], s23[0], s23[1]};
}

// bf16(bf16(a) * s) for 4 outputs a and 4 bf16 gate factors s (SCALED), or bf16(a).
template <bool SCALED>
__device__ __forceinline__ bf16x4 round4(float a0, float a1, float a2, float a3, bf16x4 s) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    const bf16x2 r01 = __builtin_convertvector(f32x2{a0, a1}, bf16x2);
    const bf16x2 r23 = __builtin_convertvector(f32x2{a2, a3}, bf16x2);
    if constexpr (!SCALED) {
        return bf16x4{r01[0], r01[1], r23[0], r23[1]};
    } else {
        const bf16x2 s01 = {s[0], s[1]}, s23 = {s[2], s[3]};
        const bf16x2 y01 = __builtin_convertvector(
            __builtin_convertvector(r01, f32x2) * __builtin_convertvector(s01, f32x2), bf16x2);
        const bf16x2 y23 = __builtin_convertvector(
            __builtin_convertvector(r23, f32x2) * __builtin_convertvector(s23, f32x2), bf16x2);
        return bf16x4{y01[0], y01[1], y23[0], y23[1]};
    }
}


// Two rounded 4-dim chunks of one query row, x held by lanes (col, kg) for dims d + 4 kg and y
// for dims d + 8 + 4 kg, regrouped by one v_permlane32_swap per dword (x's lanes 32-63 with
// y's lanes 0-31) into 8 contiguous dims per lane: d + 8 kg .. + 7.
__device__ __forceinline__ bf16x8 swap32_pair(bf16x4 x, bf16x4 y) {
    typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
    u32x2 a = __builtin_bit_cast(u32x2, x), b = __builtin_bit_cast(u32x2, y);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const auto s = __builtin_amdgcn_permlane32_swap(a[k], b[k], false, false);
        a[k] = s[0];
        b[k] = s[1];
    }
    const bf16x4 lo = __builtin_bit_cast(bf16x4, a), hi = __builtin_bit_cast(bf16x4, b);
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// bf16(x * bf16(sigmoid(g))) of 8 outputs x already rounded to bf16 and their 8 raw gate values:
// with x exact in bf16 this is round4<true>'s bf16(bf16(o) * bf16(sigmoid(g))).
__device__ __forceinline__ bf16x8 gate8(bf16x8 x, bf16x8 g) {
    const bf16x4 lo = round4<true>((float)x[0], (float)x[1], (float)x[2], (float)x[3],
                                   sigmoid4(bf16x4{g[0], g[1], g[2], g[3]}));
    const bf16x4 hi = round4<true>((float)x[4], (float)x[5], (float)x[6], (float)x[7],
                                   sigmoid4(bf16x4{g[4], g[5], g[6], g[7]}));
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Epilogue of a wave's 32-row query block in the 32x32 accumulator layout: lane (col, kg) holds
// row `col` of O^T in o[db][4 jj + i] = dims 32 db + 8 jj + 4 kg + i. Scales by inv, rounds to
// bf16, and for each pair of chunks (jj = 2m, 2m + 1) swaps halves with the partner lane l ^ 32
// (swap32_pair), so that every lane stores 16 contiguous bytes, dims 32 db + 16 m + 8 kg .. + 7
// (2 DB stores instead of 4 DB). With a gate, its 16-byte pieces for those dims are all loaded
// first (each wait then covers only the pieces before it) and applied after the swap. The
// caller keeps the whole wave in the call (the swaps read the partner lanes).
template <int DB, bool GATE>
__device__ __forceinline__ void store_block(const f32x16 (&o)[DB], float inv, int kg, __amdgpu_buffer_rsrc_t o_rs,
                                            int ooff, __amdgpu_buffer_rsrc_t g_rs, int goff) {
    constexpr int NP = 2 * DB;
    auto dim0 = [&](int q) { return (q >> 1) * 32 + 16 * (q & 1) + 8 * kg; };
    bf16x8 g[GATE ? NP : 1];
    if constexpr (GATE) {
#pragma unroll
        for (int q = 0; q < NP; ++q) g[q] = buf_ld16(g_rs, goff + dim0(q) * 2, 0);
    }
#pragma unroll
    for (int q = 0; q < NP; ++q) {
        const int db = q >> 1, b = 8 * (q & 1);
        const bf16x4 x = round4<false>(o[db][b] * inv, o[db][b + 1] * inv, o[db][b + 2] * inv, o[db][b + 3] * inv,
                                       bf16x4{});
        const bf16x4 y = round4<false>(o[db][b + 4] * inv, o[db][b + 5] * inv, o[db][b + 6] * inv,
                                       o[db][b + 7] * inv, bf16x4{});
        bf16x8 z = swap32_pair(x, y);
        if constexpr (GATE) z = gate8(z, g[q]);
        buf_st16(o_rs, ooff + dim0(q) * 2, z);
    }
}

}  // namespace pe
