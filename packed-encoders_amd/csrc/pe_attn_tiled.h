// Tiled flash-style packed attention for long segments (gfx950 MFMA).
//
// One workgroup = 4 waves = one strip of consecutive query tiles of one segment, for one group
// of G query heads. A query tile has 32*4/G rows: the G heads share one kv head (G divides the
// GQA ratio), so every K/V tile staged in LDS serves 128 query rows, 4 waves x 32 rows split
// over the G heads. Each wave keeps its 32 query rows in registers as MFMA B operands.
//
// K/V staging: an LDS ring of NS stages, each holding one BN-key K tile and one V tile,
// row-major and unpadded. They are filled by direct global-to-LDS loads (buffer_load_dwordx4
// ... lds: 64 lanes x 16 bytes, contiguous in lane order), so no data in flight occupies a
// VGPR and NS - 1 tiles can be in flight per workgroup. The loads are issued through inline
// asm, out of the compiler's sight, and completion is waited for explicitly (s_waitcnt vmcnt)
// before the one barrier per step; the compiler therefore never serialises the ring with its
// own conservative LDS-DMA waits. Bank conflicts are avoided by an XOR swizzle of the 16-byte
// units of a row (swz below), applied when choosing which global 16 bytes a lane loads. K is
// read as the MFMA A operand with ds_read_b128; V^T is read with ds_read_b64_tr_b16, whose
// 16-lane transpose turns four keys x sixteen dims of the row-major V tile into four keys per
// lane for one dim each — two of them make one A operand of O^T = V^T . P^T.
//
// The workgroup walks its strip as one flat sequence of steps, (query tile, key tile) pairs,
// through the same ring; the next query tile's Q fragments are prefetched during the last
// step of the current one (head_dim <= 128). Every global access goes through a buffer
// resource bounded by the segment, so rows past the segment read as zero with no branch.
// Block decisions are scalar: each wave skips 32-key blocks outside its rows' band (window /
// causal), and only blocks crossing a segment or band edge are masked.
//
// Softmax: online, fp32, log2 domain. The running maximum is raised lazily — only when a new
// tile's maximum exceeds it by more than 2^8 on some lane of the wave — so the accumulator
// rescale (and the exchange of maxima between the two lanes of a query row) is skipped on
// almost every tile; numerator and denominator always share the stale maximum, so the result
// is the same up to rounding. Probabilities are rounded to bf16 for the P.V MFMA and summed
// unrounded in fp32 (the reference's precision strategy,
// packed_encoders/_kernels/triton_packed_attention.py:122-136).
//
// Work entries (segment, first query tile of the strip) come from the device-built,
// cost-ordered list of plan_kernel; the 1-D grid walks entries with the head group fastest,
// so the most expensive strips of every head are dispatched first
// (longest-processing-time order).
#pragma once

#include "pe_attn_device.h"

namespace pe {

constexpr float kLazyRescale = 8.0f;  // log2 of the largest unnormalised probability allowed

#define PE_LDS __attribute__((address_space(3)))

// 16-byte unit of a row after the XOR swizzle: rows of CPR units; ds_read_b128 serves 16 lanes
// (16 keys, one unit column) per pass over 64 banks, which this makes conflict-free.
template <int CPR>
__device__ __forceinline__ int swz(int key) {
    return CPR == 8 ? (key >> 1) & 7 : key & 15;
}

// Global -> LDS, 16 bytes per lane: lane l's data lands at lds_base + 16 * l.
__device__ __forceinline__ void dma16(uint32_t lds_base, int voffset, __amdgpu_buffer_rsrc_t rsrc) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(lds_base), "v"(voffset), "s"(rsrc)
                 : "memory", "m0");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const PE_LDS void *)p;
}

// ds_read_b64_tr_b16 at an LDS element address: in each 16-lane group, lane j receives element
// j % 4 of the 4-element rows addressed by lanes j / 4, j / 4 + 4, j / 4 + 8 and j / 4 + 12.
__device__ __forceinline__ bf16x4 tr16(const __bf16 *p) {
    typedef __bf16 lds_bf16x4 __attribute__((ext_vector_type(4)));
    return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((PE_LDS lds_bf16x4 *)(PE_LDS void *)p);
}

// WIN: the call has a window or causal bound. Without one (global attention) every window
// test folds away at compile time, which also gives global and windowed launches distinct
// kernel names in traces.
template <int D, int G, int BN, int NS, bool GATE, bool WIN>
__global__ __launch_bounds__(256) void tiled_attn_kernel(AttnParams p) {
    static_assert(D % 32 == 0 && BN % 32 == 0 && (4 % G) == 0 && NS >= 2, "tile shape");
    constexpr int WPH = 4 / G;       // waves per query head
    constexpr int BM = 32 * WPH;     // query rows per query tile
    constexpr int NB = BN / 32;      // 32-key blocks per tile
    constexpr int DC = D / 16;       // 16-dim chunks for S^T
    constexpr int DB = D / 32;       // 32-dim blocks for O^T
    constexpr int CPR = D / 8;       // 16-byte units per K/V row
    constexpr int TILE = BN * D;     // elements of one K (or V) tile
    constexpr int UPW = TILE / 8 / 64 / 4;  // 1 KB wave-loads per tensor per wave and tile
    constexpr int LPS = 2 * UPW;     // loads per thread per step (K and V)
    constexpr bool PREFETCH_Q = false;  // next tile's Q fragments loaded one step early (costs a VGPR occupancy step)
    static_assert(UPW >= 1 && TILE % (8 * 64 * 4) == 0, "tile must split into 1 KB wave loads");

    __shared__ __attribute__((aligned(16))) __bf16 ring[NS][2][TILE];

    const int entry = blockIdx.x / p.hgroups;
    const int hg = blockIdx.x - entry * p.hgroups;
    if (entry >= *p.work_count) return;
    const int2 w = p.work[entry];
    const int seg = w.x, qt_first = w.y;
    if (seg < 0 || seg >= p.n_seq || qt_first < 0 || p.strip < 1) return;  // a plan made for other arguments
    const int start = p.cu[seg];
    const int L = p.cu[seg + 1] - start;
    const int nq = (L + BM - 1) / BM;
    if (qt_first >= nq) return;
    const int qt_end = min(nq, qt_first + p.strip);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = uniform(tid >> 6);
    const int col = lane & 31, kg = lane >> 5;
    const int slot = wave / WPH, rb = wave - slot * WPH;
    const int qh = hg * G + slot;
    const int kvh = (hg * G) / p.group;
    const int wl = WIN ? p.wl : -1, wr = WIN ? p.wr : -1;

    const __amdgpu_buffer_rsrc_t q_rs = make_rsrc(p.q + (int64_t)start * p.q_st + (int64_t)qh * p.q_sh, rows_bytes(L, p.q_st, D));
    const __amdgpu_buffer_rsrc_t k_rs = make_rsrc(p.k + (int64_t)start * p.k_st + (int64_t)kvh * p.k_sh, rows_bytes(L, p.k_st, D));
    const __amdgpu_buffer_rsrc_t v_rs = make_rsrc(p.v + (int64_t)start * p.v_st + (int64_t)kvh * p.v_sh, rows_bytes(L, p.v_st, D));
    const __amdgpu_buffer_rsrc_t o_rs = make_rsrc(p.o + (int64_t)start * p.o_st + (int64_t)qh * p.o_sh, rows_bytes(L, p.o_st, D));
    __amdgpu_buffer_rsrc_t g_rs = o_rs;
    if constexpr (GATE) g_rs = make_rsrc(p.g + (int64_t)start * p.g_st + (int64_t)qh * p.g_sh, rows_bytes(L, p.g_st, D));
    const int k_row = (int)p.k_st * 2, v_row = (int)p.v_st * 2;

    // Key range [klo, klo + ntiles * BN) of query tile qt: the union of its rows' windows.
    auto key_range = [&](int qt, int &klo, int &ntiles) {
        const int q0 = qt * BM, rows_end = min(L, q0 + BM);
        klo = wl >= 0 ? max(0, q0 - wl) : 0;
        const int khi = wr >= 0 ? min(L, rows_end + wr) : L;
        ntiles = khi > klo ? (khi - klo + BN - 1) / BN : 0;
    };
    // This wave's 32 query rows of query tile qt as B operands (zero beyond the segment).
    auto load_q = [&](int qt, bf16x8 (&dst)[DC]) {
        const int qoff = (qt * BM + rb * 32 + col) * (int)p.q_st * 2 + kg * 16;
#pragma unroll
        for (int c = 0; c < DC; ++c) dst[c] = buf_ld16(q_rs, qoff + c * 32, 0);
    };

    // DMA geometry: wave-load j of this wave fills units [(wave * UPW + j) * 64, +64) of a tile;
    // unit u holds key u / CPR, global 16-byte column (u % CPR) ^ swz(key).
    int koff[UPW], voff[UPW];
#pragma unroll
    for (int j = 0; j < UPW; ++j) {
        const int u = (wave * UPW + j) * 64 + lane;
        const int key = u / CPR, ch = (u % CPR) ^ swz<CPR>(key);
        koff[j] = key * k_row + ch * 16;
        voff[j] = key * v_row + ch * 16;
    }
    const uint32_t ring_base = uniform((int)lds_addr(&ring[0][0][0]));
    constexpr uint32_t kStageBytes = 2 * TILE * 2, kTileBytes = TILE * 2;
    auto issue = [&](int stage, int kt0) {
        const uint32_t kb = ring_base + stage * kStageBytes + wave * UPW * 1024;
        const int kbase = kt0 * k_row, vbase = kt0 * v_row;
#pragma unroll
        for (int j = 0; j < UPW; ++j) dma16(kb + j * 1024, koff[j] + kbase, k_rs);
#pragma unroll
        for (int j = 0; j < UPW; ++j) dma16(kb + kTileBytes + j * 1024, voff[j] + vbase, v_rs);
    };

    // Per-lane LDS read offsets (elements within a tile). K: key 32b + col, unit 2c + kg.
    // V^T (tr16): in 16-lane group g = lane / 16, source lane i = lane % 16 points at key
    // 16h + 4 * (g / 2) + i / 4 (+ 8 for the second half of the operand) and dims
    // 32 db + 16 (g % 2) + 4 (i % 4); the transpose hands lane (m = dim, kg) four keys of its dim.
    // Both swizzles depend only on bits of the key below 32 that the block / 16-key-half loops
    // leave fixed, so every address is a per-lane base plus a compile-time offset.
    int kbase_c[DC];
#pragma unroll
    for (int c = 0; c < DC; ++c) kbase_c[c] = col * D + ((2 * c + kg) ^ swz<CPR>(col)) * 8;
    const int vi = lane & 15, vg = lane >> 4;
    const int vkey0 = 4 * (vg >> 1) + (vi >> 2);
    const int vdim0 = 16 * (vg & 1) + 4 * (vi & 3);
    int vbase[2][DB];  // [second 4-key half of the operand][32-dim block]
#pragma unroll
    for (int half = 0; half < 2; ++half)
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const int key = 8 * half + vkey0, dim = 32 * db + vdim0;
            vbase[half][db] = key * D + (((dim >> 3) ^ swz<CPR>(key)) * 8) + (dim & 4);
        }

    f32x16 o[DB];
    float m;
    float ls[4];
    auto reset = [&]() {
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int j = 0; j < 16; ++j) o[db][j] = 0.0f;
        m = kNegInf;
#pragma unroll
        for (int i = 0; i < 4; ++i) ls[i] = 0.0f;
    };
    const float c2 = p.c;

    // Current query tile.
    int qt = qt_first, klo, ntiles;
    key_range(qt, klo, ntiles);
    int r0 = qt * BM + rb * 32;
    int myrow = r0 + col;
    bool wave_active = r0 < L;
    int wr1 = min(L, r0 + 32);
    bf16x8 qf[DC], qn[DC];
    load_q(qt, qf);
    reset();

    // Step bookkeeping: a step is (query tile, key tile). `adv` moves a cursor one step ahead.
    struct Cursor {
        int qt, t, klo, ntiles;
    };
    auto adv = [&](Cursor &c) {
        if (++c.t >= c.ntiles) {
            ++c.qt;
            c.t = 0;
            if (c.qt < qt_end) key_range(c.qt, c.klo, c.ntiles);
        }
    };
    auto valid = [&](const Cursor &c) { return c.qt < qt_end && c.t < c.ntiles; };

    // Prologue: issue the first NS - 1 steps.
    Cursor ld{qt, 0, klo, ntiles};  // next step to issue
    int issued = 0;
#pragma unroll
    for (int s = 0; s < NS - 1; ++s) {
        if (valid(ld)) {
            issue(issued % NS, ld.klo + ld.t * BN);
            ++issued;
            adv(ld);
        }
    }

    int t = 0, step = 0;
    bool first = true;
    while (true) {
        // This step's loads are complete once at most the later steps' loads are in flight
        // (loads complete in issue order).
        const int later = issued - step - 1;
        if (NS >= 3 && later >= 2) wait_vmcnt<2 * LPS>();
        else if (later >= 1) wait_vmcnt<LPS>();
        else wait_vmcnt<0>();
        __syncthreads();
        if (first) {
            // The query fragments were loaded before this step's K/V (or with the previous
            // step); ending their load scope here keeps the compiler from waiting on the
            // vector memory counter inside the loop, which would also drain the ring.
#pragma unroll
            for (int c = 0; c < DC; ++c) asm volatile("" : "+v"(qf[c]));
            first = false;
        }
        // The next query tile's Q fragments, during this tile's last step and before the
        // refill below, so the next step's wait covers them.
        const bool last_of_tile = t + 1 >= ntiles;
        const bool more = qt + 1 < qt_end;
        if constexpr (PREFETCH_Q) {
            if (last_of_tile && more) load_q(qt + 1, qn);
        }
        // Refill the stage freed by the previous step (all waves passed the barrier after it).
        if (valid(ld)) {
            issue(issued % NS, ld.klo + ld.t * BN);
            ++issued;
            adv(ld);
        }

        const __bf16 *kt = &ring[step % NS][0][0];
        const __bf16 *vt = &ring[step % NS][1][0];
        if (wave_active && t < ntiles) {
            const int kt0 = klo + t * BN;
            f32x16 s[NB];
            bool live[NB];
            float mp[4] = {kNegInf, kNegInf, kNegInf, kNegInf};  // partial maxima (4 chains)
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int kb0 = kt0 + 32 * b;
                live[b] = block_live(kb0, L, r0, wr1, wl, wr);
                if (live[b]) {
                    f32x16 acc;
#pragma unroll
                    for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
#pragma unroll
                    for (int c = 0; c < DC; ++c) acc = mfma32(ld_s16(kt + 32 * b * D + kbase_c[c]), qf[c], acc);
                    if (!block_full(kb0, L, r0, wr1, wl, wr)) {
#pragma unroll
                        for (int j = 0; j < 16; ++j) {
                            const int kk = kb0 + acc_key(j, kg);
                            const bool ok = (kk < L) & ((wl < 0) | (myrow - kk <= wl)) & ((wr < 0) | (kk - myrow <= wr));
                            acc[j] = ok ? acc[j] : kNegInf;
                        }
                    }
                    s[b] = acc;
#pragma unroll
                    for (int j = 0; j < 16; ++j) mp[j & 3] = fmaxf(mp[j & 3], acc[j]);
                }
            }
            // Each lane tests its own maximum: the two lanes of a query row share m, so "some
            // lane exceeds m" is "some row exceeds m"; only a rescale combines the pair.
            const float mx = fmaxf(fmaxf(mp[0], mp[1]), fmaxf(mp[2], mp[3]));
            if (wave_any(mx * c2 > m + kLazyRescale)) {
                const float mnew = fmaxf(m, fmaxf(mx, __shfl_xor(mx, 32)) * c2);
                const float alpha = mnew == kNegInf ? 1.0f : exp2_fast(m - mnew);
                m = mnew;
#pragma unroll
                for (int i = 0; i < 4; ++i) ls[i] *= alpha;
#pragma unroll
                for (int db = 0; db < DB; ++db)
#pragma unroll
                    for (int j = 0; j < 16; ++j) o[db][j] *= alpha;
            }
            const float muse = m == kNegInf ? 0.0f : m;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if (live[b]) {
#pragma unroll
                    for (int j = 0; j < 16; ++j) {
                        const float e = exp2_fast(fmaf(s[b][j], c2, -muse));
                        s[b][j] = e;
                        ls[j & 3] += e;
                    }
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const bf16x8 pb = to_bf16x8(s[b], 8 * h);
#pragma unroll
                        for (int db = 0; db < DB; ++db) {
                            // keys 32b + 16h + 8 half + vkey0: the swizzle sees only the bits of
                            // 8 half + vkey0 (32b + 16h changes neither)
                            const bf16x4 lo = tr16(vt + (32 * b + 16 * h) * D + vbase[0][db]);
                            const bf16x4 hi = tr16(vt + (32 * b + 16 * h) * D + vbase[1][db]);
                            const bf16x8 va = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                            o[db] = mfma32(va, pb, o[db]);
                        }
                    }
                }
            }
        }

        if (last_of_tile) {
            // Last key tile of this query tile: normalise, apply the gate, store, reset.
            const float lsum = (ls[0] + ls[1]) + (ls[2] + ls[3]);
            const float lt = lsum + __shfl_xor(lsum, 32);
            if (wave_active) {
                const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
                const int ooff = myrow * (int)p.o_st * 2;
                const int goff = GATE ? myrow * (int)p.g_st * 2 : 0;
#pragma unroll
                for (int db = 0; db < DB; ++db)
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) {
                        const int d0 = db * 32 + 8 * jj + 4 * kg;
                        bf16x4 g4 = {};
                        if constexpr (GATE) g4 = buf_ld8(g_rs, goff + d0 * 2, 0);
                        buf_st8(o_rs, ooff + d0 * 2,
                                out4<GATE>(o[db][4 * jj] * inv, o[db][4 * jj + 1] * inv, o[db][4 * jj + 2] * inv,
                                           o[db][4 * jj + 3] * inv, g4));
                    }
            }
            reset();
            if (!more) break;
            ++qt;
            key_range(qt, klo, ntiles);
            r0 = qt * BM + rb * 32;
            myrow = r0 + col;
            wave_active = r0 < L;
            wr1 = min(L, r0 + 32);
            if constexpr (PREFETCH_Q) {
#pragma unroll
                for (int c = 0; c < DC; ++c) qf[c] = qn[c];
            } else {
                load_q(qt, qf);
            }
            first = true;  // end the new fragments' load scope after the next barrier
            t = 0;
        } else {
            ++t;
        }
        ++step;
    }
}

}  // namespace pe
