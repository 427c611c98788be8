// Tiled flash-style packed attention for long segments (gfx950 MFMA).
//
// One workgroup = 4 waves = one (segment, 32*4/G-row query tile, group of G query heads).
// The G heads share one kv head (G divides the GQA ratio), so every K/V tile staged in LDS
// serves 128 query rows: 4 waves x 32 rows, split over the G heads. Each wave keeps its 32
// query rows in registers as MFMA B operands for the whole key loop.
//
// Key loop: BN-key tiles of K (row-major) and V (transposed, see pe_attn_device.h) are
// double-buffered in LDS: tile t+1 is fetched into registers while tile t is consumed and
// written to the other buffer afterwards, one barrier per tile. Inside a tile each wave skips
// 32-key blocks outside its rows' band (window / causal), and only blocks crossing a segment
// or band edge are masked. Online softmax in fp32 in the log2 domain; probabilities are
// rounded to bf16 for the P.V MFMA (the reference's precision strategy,
// packed_encoders/_kernels/triton_packed_attention.py:122-136).
//
// Work entries (segment, q-tile) come from the device-built, cost-ordered list of
// pe_attn_plan_kernel; the 1-D grid walks entries with the head group fastest, so the most
// expensive tiles of every head are dispatched first (longest-processing-time order).
#pragma once

#include "pe_attn_device.h"

namespace pe {

template <int D, int G, int BN, bool GATE>
__global__ __launch_bounds__(256) void tiled_attn_kernel(AttnParams p) {
    static_assert(D % 32 == 0 && BN % 32 == 0 && (4 % G) == 0, "tile shape");
    constexpr int WPH = 4 / G;       // waves per query head
    constexpr int BM = 32 * WPH;     // query rows per workgroup
    constexpr int KP = D + 8;        // K tile row pitch (elements): 16-byte pad
    constexpr int VP = BN + 8;       // V^T tile row pitch
    constexpr int NB = BN / 32;      // 32-key blocks per tile
    constexpr int DC = D / 16;       // 16-dim chunks for S^T
    constexpr int DB = D / 32;       // 32-dim blocks for O^T
    constexpr int KCH = BN * D / 8;  // 16-byte chunks in a K tile
    constexpr int KPT = (KCH + 255) / 256;
    constexpr int VCH = (BN / 4) * (D / 8);  // 4-key x 8-dim chunks in a V tile
    constexpr int VPT = (VCH + 255) / 256;

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

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 31, kg = lane >> 5;
    const int slot = wave / WPH, rb = wave - slot * WPH;
    const int qh = hg * G + slot;
    const int kvh = (hg * G) / p.group;
    const int r0 = q0 + rb * 32;
    const int myrow = r0 + col;

    const int rows_end = min(L, q0 + BM);
    int klo = 0, khi = L;
    if (p.wl >= 0) klo = max(0, q0 - p.wl);
    if (p.wr >= 0) khi = min(L, rows_end + p.wr);
    const bool wave_active = r0 < L;
    const int wr1 = min(L, r0 + 32);

    // This wave's 32 query rows as B operands (zero beyond the segment).
    bf16x8 qf[DC];
    {
        const __bf16 *qrow = p.q + (int64_t)(start + myrow) * p.q_st + (int64_t)qh * p.q_sh + kg * 8;
        const bool ok = myrow < L;
#pragma unroll
        for (int c = 0; c < DC; ++c) qf[c] = ok ? ld_g16(qrow + c * 16) : zero8();
    }

    f32x16 o[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int j = 0; j < 16; ++j) o[db][j] = 0.0f;
    float m = kNegInf, lsum = 0.0f;

    const __bf16 *kbase = p.k + (int64_t)start * p.k_st + (int64_t)kvh * p.k_sh;
    const __bf16 *vbase = p.v + (int64_t)start * p.v_st + (int64_t)kvh * p.v_sh;
    bf16x8 kreg[KPT];
    bf16x8 vreg[VPT][4];

    auto gload = [&](int kt0) {
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int c = tid + i * 256;
            if (c < KCH) {
                const int key = c / (D / 8), dc = c - key * (D / 8);
                const int kk = kt0 + key;
                kreg[i] = kk < khi ? ld_g16(kbase + (int64_t)kk * p.k_st + dc * 8) : zero8();
            }
        }
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int c = tid + i * 256;
            if (c < VCH) {
                const int kq = c / (D / 8), dc = c - kq * (D / 8);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int kk = kt0 + 4 * kq + r;
                    vreg[i][r] = kk < khi ? ld_g16(vbase + (int64_t)kk * p.v_st + dc * 8) : zero8();
                }
            }
        }
    };
    auto swrite = [&](int buf) {
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int c = tid + i * 256;
            if (c < KCH) {
                const int key = c / (D / 8), dc = c - key * (D / 8);
                st_s16(&Ks[buf][key * KP + dc * 8], kreg[i]);
            }
        }
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int c = tid + i * 256;
            if (c < VCH) {
                const int kq = c / (D / 8), dc = c - kq * (D / 8);
                store_vt_chunk(&Vt[buf][(dc * 8) * VP + vperm(4 * kq)], VP, vreg[i]);
            }
        }
    };

    const int ntiles = khi > klo ? (khi - klo + BN - 1) / BN : 0;
    if (ntiles > 0) {
        gload(klo);
        swrite(0);
    }
    __syncthreads();

    for (int t = 0; t < ntiles; ++t) {
        const int buf = t & 1;
        const int kt0 = klo + t * BN;
        if (t + 1 < ntiles) gload(kt0 + BN);

        if (wave_active) {
            f32x16 s[NB];
            bool live[NB];
            float mx = kNegInf;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int kb0 = kt0 + 32 * b;
                live[b] = block_live(kb0, L, r0, wr1, p.wl, p.wr);
                if (live[b]) {
#pragma unroll
                    for (int j = 0; j < 16; ++j) s[b][j] = 0.0f;
                    const __bf16 *ka = &Ks[buf][(32 * b + col) * KP + kg * 8];
#pragma unroll
                    for (int c = 0; c < DC; ++c) s[b] = mfma32(ld_s16(ka + c * 16), qf[c], s[b]);
                    if (!block_full(kb0, L, r0, wr1, p.wl, p.wr)) {
#pragma unroll
                        for (int j = 0; j < 16; ++j) {
                            const int key = kb0 + acc_key(j, kg);
                            const bool ok = key < L && (p.wl < 0 || myrow - key <= p.wl) &&
                                            (p.wr < 0 || key - myrow <= p.wr);
                            s[b][j] = ok ? s[b][j] : kNegInf;
                        }
                    }
#pragma unroll
                    for (int j = 0; j < 16; ++j) mx = fmaxf(mx, s[b][j]);
                }
            }
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const float mnew = fmaxf(m, mx * p.c);
            const float muse = mnew == kNegInf ? 0.0f : mnew;
            const float alpha = exp2_fast(m - muse);
            m = mnew;
            float ts = 0.0f;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if (live[b]) {
#pragma unroll
                    for (int j = 0; j < 16; ++j) {
                        const float e = exp2_fast(fmaf(s[b][j], p.c, -muse));
                        s[b][j] = e;
                        ts += e;
                    }
                }
            }
            lsum = lsum * alpha + ts;
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int j = 0; j < 16; ++j) o[db][j] *= alpha;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if (live[b]) {
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const bf16x8 pb = to_bf16x8(s[b], 8 * h);
                        const __bf16 *va = &Vt[buf][col * VP + 32 * b + 16 * h + 8 * kg];
#pragma unroll
                        for (int db = 0; db < DB; ++db)
                            o[db] = mfma32(ld_s16(va + db * 32 * VP), pb, o[db]);
                    }
                }
            }
        }
        if (t + 1 < ntiles) swrite(buf ^ 1);
        __syncthreads();
    }

    const float lt = lsum + __shfl_xor(lsum, 32);
    if (!wave_active || myrow >= L) return;
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    __bf16 *orow = p.o + (int64_t)(start + myrow) * p.o_st + (int64_t)qh * p.o_sh;
    const __bf16 *grow = GATE ? p.g + (int64_t)(start + myrow) * p.g_st + (int64_t)qh * p.g_sh : nullptr;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const int d0 = db * 32 + 8 * jj + 4 * kg;
            store_out4<GATE>(orow + d0, GATE ? grow + d0 : nullptr, o[db][4 * jj] * inv,
                             o[db][4 * jj + 1] * inv, o[db][4 * jj + 2] * inv, o[db][4 * jj + 3] * inv);
        }
}

}  // namespace pe
