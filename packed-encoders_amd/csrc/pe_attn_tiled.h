// Tiled flash-style packed attention for long segments (gfx950 MFMA).
//
// One workgroup = 4 waves = one (segment, 32*4/G-row query tile, group of G query heads).
// The G heads share one kv head (G divides the GQA ratio), so every K/V tile staged in LDS
// serves 128 query rows: 4 waves x 32 rows, split over the G heads. Each wave keeps its 32
// query rows in registers as MFMA B operands for the whole key loop.
//
// Key loop: BN-key tiles of K (row-major) and V (transposed, see pe_attn_device.h) are
// double-buffered in LDS: tile t+1 is fetched into registers while tile t is consumed and
// written to the other buffer afterwards, one barrier per tile. Every global access goes
// through a buffer resource bounded by the segment, so rows past the segment read as zero
// with no branch. Block decisions are scalar: each wave skips 32-key blocks outside its rows'
// band (window / causal), and only blocks crossing a segment or band edge are masked.
//
// Softmax: online, fp32, log2 domain. The running maximum is raised lazily — only when a new
// tile's maximum exceeds it by more than 2^8 on some lane of the wave — so the accumulator
// rescale (and the exchange of maxima between the two lanes of a query row) is skipped on
// almost every tile; numerator and denominator always share the stale maximum, so the result
// is the same up to rounding. Probabilities are rounded to bf16 for the
// P.V MFMA (the reference's precision strategy,
// packed_encoders/_kernels/triton_packed_attention.py:122-136).
//
// Work entries (segment, q-tile) come from the device-built, cost-ordered list of plan_kernel;
// the 1-D grid walks entries with the head group fastest, so the most expensive tiles of every
// head are dispatched first (longest-processing-time order).
#pragma once

#include "pe_attn_device.h"

namespace pe {

constexpr float kLazyRescale = 8.0f;  // log2 of the largest unnormalised probability allowed

// WIN: the call has a window or causal bound. Without one (global attention) every window
// test folds away at compile time, which also gives global and windowed launches distinct
// kernel names in traces.
template <int D, int G, int BN, bool GATE, bool WIN>
__global__ __launch_bounds__(256) void tiled_attn_kernel(AttnParams p) {
    static_assert(D % 32 == 0 && BN % 32 == 0 && (4 % G) == 0, "tile shape");
    constexpr int WPH = 4 / G;       // waves per query head
    constexpr int BM = 32 * WPH;     // query rows per workgroup
    constexpr int KP = D + 8;        // K tile row pitch (elements): 16-byte pad
    constexpr int VP = BN + 8;       // V^T tile row pitch
    constexpr int NB = BN / 32;      // 32-key blocks per tile
    constexpr int DC = D / 16;       // 16-dim chunks for S^T
    constexpr int DB = D / 32;       // 32-dim blocks for O^T
    constexpr int KQ = BN * D / 2048;  // 16-byte K chunks per thread = keys per V chunk
    constexpr int NKQ = BN / KQ;       // V chunks along the keys
    static_assert(KQ == 2 || KQ == 4, "every thread loads KQ K chunks and one KQ-key V chunk");

    __shared__ __attribute__((aligned(16))) __bf16 Ks[2][BN * KP];
    __shared__ __attribute__((aligned(16))) __bf16 Vt[2][D * VP];

    const int entry = blockIdx.x / p.hgroups;
    const int hg = blockIdx.x - entry * p.hgroups;
    if (entry >= *p.work_count) return;
    const int2 w = p.work[entry];
    const int seg = w.x, tile = w.y;
    if (seg < 0 || seg >= p.n_seq || tile < 0) return;  // a plan made for other arguments
    const int start = p.cu[seg];
    const int L = p.cu[seg + 1] - start;
    const int q0 = tile * BM;
    if (q0 >= L) return;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = uniform(tid >> 6);
    const int col = lane & 31, kg = lane >> 5;
    const int slot = wave / WPH, rb = wave - slot * WPH;
    const int qh = hg * G + slot;
    const int kvh = (hg * G) / p.group;
    const int r0 = q0 + rb * 32;
    const int myrow = r0 + col;
    const int wl = WIN ? p.wl : -1, wr = WIN ? p.wr : -1;

    const int rows_end = min(L, q0 + BM);
    const int klo = wl >= 0 ? max(0, q0 - wl) : 0;
    const int khi = wr >= 0 ? min(L, rows_end + wr) : L;
    const bool wave_active = r0 < L;
    const int wr1 = min(L, r0 + 32);

    const __amdgpu_buffer_rsrc_t q_rs = make_rsrc(p.q + (int64_t)start * p.q_st + (int64_t)qh * p.q_sh, rows_bytes(L, p.q_st, D));
    const __amdgpu_buffer_rsrc_t k_rs = make_rsrc(p.k + (int64_t)start * p.k_st + (int64_t)kvh * p.k_sh, rows_bytes(L, p.k_st, D));
    const __amdgpu_buffer_rsrc_t v_rs = make_rsrc(p.v + (int64_t)start * p.v_st + (int64_t)kvh * p.v_sh, rows_bytes(L, p.v_st, D));
    const int k_row = (int)p.k_st * 2, v_row = (int)p.v_st * 2;

    // This wave's 32 query rows as B operands (zero beyond the segment).
    bf16x8 qf[DC];
    {
        const int qoff = myrow * (int)p.q_st * 2 + kg * 16;
#pragma unroll
        for (int c = 0; c < DC; ++c) qf[c] = buf_ld16(q_rs, qoff + c * 32, 0);
    }

    // Per-thread tile chunks: KQ 16-byte K chunks (row-major) and one KQ-key x 8-dim V chunk.
    int koff[KQ], klds[KQ];
#pragma unroll
    for (int i = 0; i < KQ; ++i) {
        const int c = tid + i * 256;
        const int key = c / (D / 8), dc = c - key * (D / 8);
        koff[i] = key * k_row + dc * 16;
        klds[i] = key * KP + dc * 8;
    }
    const int vkq = tid % NKQ, vdc = tid / NKQ;  // key group fastest: LDS writes spread over banks
    const int voff = vkq * KQ * v_row + vdc * 16;
    const int vlds = (vdc * 8) * VP + vperm(vkq * KQ);

    // The tile offset goes into the VGPR offset, never the SGPR one: only the former is
    // guaranteed to take part in the buffer range check that zeroes rows past the segment.
    bf16x8 kreg[KQ], vreg[KQ];
    auto gload = [&](int kt0) {
        const int kbase = kt0 * k_row, vbase = kt0 * v_row;
#pragma unroll
        for (int i = 0; i < KQ; ++i) kreg[i] = buf_ld16(k_rs, koff[i] + kbase, 0);
#pragma unroll
        for (int r = 0; r < KQ; ++r) vreg[r] = buf_ld16(v_rs, voff + vbase + r * v_row, 0);
    };
    auto swrite = [&](int buf) {
#pragma unroll
        for (int i = 0; i < KQ; ++i) st_s16(&Ks[buf][klds[i]], kreg[i]);
#pragma unroll
        for (int dd = 0; dd < 8; ++dd) {
            if constexpr (KQ == 4) {
                bf16x4 t;
                t[0] = vreg[0][dd];
                t[1] = vreg[1][dd];
                t[2] = vreg[2][dd];
                t[3] = vreg[3][dd];
                st_s8(&Vt[buf][vlds + dd * VP], t);
            } else {
                typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
                bf16x2 t;
                t[0] = vreg[0][dd];
                t[1] = vreg[1][dd];
                *reinterpret_cast<bf16x2 *>(&Vt[buf][vlds + dd * VP]) = t;
            }
        }
    };

    f32x16 o[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int j = 0; j < 16; ++j) o[db][j] = 0.0f;
    // Running maximum (log2 domain) and row sum; the sum is kept as 4 partial sums so the
    // 16 additions of a block form 4 independent chains instead of one serial chain.
    float m = kNegInf;
    float ls[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const float c2 = p.c;

    const int ntiles = khi > klo ? (khi - klo + BN - 1) / BN : 0;
    if (ntiles > 0) {
        gload(klo);
        swrite(0);
    }
    __syncthreads();
    // The query fragments arrived before tile 0 (issued earlier, and loads complete in
    // order). Re-defining them through an empty asm ends their load's scope here: otherwise
    // the compiler, seeing them possibly in flight at the loop header, waits on the vector
    // memory counter before the first MFMA of every tile, which also drains the next
    // tile's prefetch and serialises the double buffer.
#pragma unroll
    for (int c = 0; c < DC; ++c) asm volatile("" : "+v"(qf[c]));

    for (int t = 0; t < ntiles; ++t) {
        const int buf = t & 1;
        const int kt0 = klo + t * BN;
        if (t + 1 < ntiles) gload(kt0 + BN);

        if (wave_active) {
            f32x16 s[NB];
            bool live[NB];
            float mp[4] = {kNegInf, kNegInf, kNegInf, kNegInf};  // partial maxima (4 chains)
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int kb0 = kt0 + 32 * b;
                live[b] = block_live(kb0, L, r0, wr1, wl, wr);
                if (live[b]) {
                    const __bf16 *ka = &Ks[buf][(32 * b + col) * KP + kg * 8];
                    f32x16 acc;
#pragma unroll
                    for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
#pragma unroll
                    for (int c = 0; c < DC; ++c) acc = mfma32(ld_s16(ka + c * 16), qf[c], acc);
                    if (!block_full(kb0, L, r0, wr1, wl, wr)) {
#pragma unroll
                        for (int j = 0; j < 16; ++j) {
                            const int key = kb0 + acc_key(j, kg);
                            const bool ok = (key < L) & ((wl < 0) | (myrow - key <= wl)) & ((wr < 0) | (key - myrow <= wr));
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
                        const __bf16 *va = &Vt[buf][col * VP + 32 * b + 16 * h + 8 * kg];
#pragma unroll
                        for (int db = 0; db < DB; ++db) o[db] = mfma32(ld_s16(va + db * 32 * VP), pb, o[db]);
                    }
                }
            }
        }
        if (t + 1 < ntiles) swrite(buf ^ 1);
        __syncthreads();
    }

    const float lsum = (ls[0] + ls[1]) + (ls[2] + ls[3]);
    const float lt = lsum + __shfl_xor(lsum, 32);
    if (!wave_active) return;
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    const __amdgpu_buffer_rsrc_t o_rs = make_rsrc(p.o + (int64_t)start * p.o_st + (int64_t)qh * p.o_sh, rows_bytes(L, p.o_st, D));
    const int ooff = myrow * (int)p.o_st * 2;
    __amdgpu_buffer_rsrc_t g_rs = o_rs;
    int goff = 0;
    if constexpr (GATE) {
        g_rs = make_rsrc(p.g + (int64_t)start * p.g_st + (int64_t)qh * p.g_sh, rows_bytes(L, p.g_st, D));
        goff = myrow * (int)p.g_st * 2;
    }
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

}  // namespace pe
