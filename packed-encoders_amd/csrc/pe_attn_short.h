// LDS-resident packed attention for short segments (length <= SK <= 128), gfx950 MFMA.
//
// One workgroup = 4 waves = one segment x HPW query heads. The segment's whole K (row-major)
// and V (transposed) tiles of every head in the group are staged in LDS once; Q rows go
// straight to registers as MFMA B operands. Each wave owns one head and walks that head's
// 32-row query blocks (4 / HPW waves share a head). A query block sees every key of the
// segment at once, so the softmax is exact, with no online rescaling: the row maximum and sum
// are per-lane scalars combined with the partner lane through one wavefront shuffle.
//
// Segments longer than short_max, or empty, leave the workgroup at once, which is what lets
// one launch of this kernel and one of the tiled kernel split a mixed batch per segment with
// no host read of cu_seqlens.
#pragma once

#include "pe_attn_device.h"

namespace pe {

template <int D, int SK, int HPW, bool GATE>
__global__ __launch_bounds__(256) void short_attn_kernel(AttnParams p) {
    static_assert(SK % 32 == 0 && SK <= 128 && (4 % HPW) == 0, "short tile shape");
    constexpr int KP = D + 8;
    constexpr int VP = SK + 8;
    constexpr int NB = SK / 32;
    constexpr int DC = D / 16;
    constexpr int DB = D / 32;
    constexpr int WSTEP = 4 / HPW;  // waves sharing one head

    __shared__ __attribute__((aligned(16))) __bf16 Ks[HPW][SK * KP];
    __shared__ __attribute__((aligned(16))) __bf16 Vt[HPW][D * VP];

    const int seg = blockIdx.x;
    const int start = p.cu[seg];
    const int L = p.cu[seg + 1] - start;
    if (L <= 0 || L > p.short_max) return;
    const int h0 = blockIdx.y * HPW;
    const int nkb = (L + 31) >> 5;
    const int kcap = nkb * 32;
    const int tid = threadIdx.x;

    // Stage K and V^T of every head of the group (keys >= L zero-filled up to the block edge).
#pragma unroll
    for (int s = 0; s < HPW; ++s) {
        const int qh = h0 + s;
        if (qh >= p.hq) break;
        const int kvh = qh / p.group;
        const __bf16 *kb = p.k + (int64_t)start * p.k_st + (int64_t)kvh * p.k_sh;
        const __bf16 *vb = p.v + (int64_t)start * p.v_st + (int64_t)kvh * p.v_sh;
        for (int c = tid; c < kcap * (D / 8); c += 256) {
            const int key = c / (D / 8), dc = c - key * (D / 8);
            st_s16(&Ks[s][key * KP + dc * 8], key < L ? ld_g16(kb + (int64_t)key * p.k_st + dc * 8) : zero8());
        }
        for (int c = tid; c < (kcap / 4) * (D / 8); c += 256) {
            const int kq = c / (D / 8), dc = c - kq * (D / 8);
            bf16x8 rows[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int key = 4 * kq + r;
                rows[r] = key < L ? ld_g16(vb + (int64_t)key * p.v_st + dc * 8) : zero8();
            }
            store_vt_chunk(&Vt[s][(dc * 8) * VP + vperm(4 * kq)], VP, rows);
        }
    }
    __syncthreads();

    const int lane = tid & 63, wave = tid >> 6;
    const int col = lane & 31, kg = lane >> 5;
    const int s = wave % HPW;
    const int qh = h0 + s;
    if (qh >= p.hq) return;

    for (int qb = wave / HPW; qb * 32 < L; qb += WSTEP) {
        const int r0 = qb * 32, r1 = min(L, r0 + 32);
        const int myrow = r0 + col;
        bf16x8 qf[DC];
        {
            const __bf16 *qrow = p.q + (int64_t)(start + myrow) * p.q_st + (int64_t)qh * p.q_sh + kg * 8;
            const bool ok = myrow < L;
#pragma unroll
            for (int c = 0; c < DC; ++c) qf[c] = ok ? ld_g16(qrow + c * 16) : zero8();
        }
        f32x16 sc[NB];
        bool live[NB];
        float mx = kNegInf;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int kb0 = 32 * b;
            live[b] = b < nkb && block_live(kb0, L, r0, r1, p.wl, p.wr);
            if (live[b]) {
#pragma unroll
                for (int j = 0; j < 16; ++j) sc[b][j] = 0.0f;
                const __bf16 *ka = &Ks[s][(kb0 + col) * KP + kg * 8];
#pragma unroll
                for (int c = 0; c < DC; ++c) sc[b] = mfma32(ld_s16(ka + c * 16), qf[c], sc[b]);
                if (!block_full(kb0, L, r0, r1, p.wl, p.wr)) {
#pragma unroll
                    for (int j = 0; j < 16; ++j) {
                        const int key = kb0 + acc_key(j, kg);
                        const bool ok = key < L && (p.wl < 0 || myrow - key <= p.wl) &&
                                        (p.wr < 0 || key - myrow <= p.wr);
                        sc[b][j] = ok ? sc[b][j] : kNegInf;
                    }
                }
#pragma unroll
                for (int j = 0; j < 16; ++j) mx = fmaxf(mx, sc[b][j]);
            }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float muse = mx == kNegInf ? 0.0f : mx * p.c;
        float ts = 0.0f;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (live[b]) {
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const float e = exp2_fast(fmaf(sc[b][j], p.c, -muse));
                    sc[b][j] = e;
                    ts += e;
                }
            }
        }
        f32x16 o[DB];
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int j = 0; j < 16; ++j) o[db][j] = 0.0f;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (live[b]) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const bf16x8 pb = to_bf16x8(sc[b], 8 * h);
                    const __bf16 *va = &Vt[s][col * VP + 32 * b + 16 * h + 8 * kg];
#pragma unroll
                    for (int db = 0; db < DB; ++db) o[db] = mfma32(ld_s16(va + db * 32 * VP), pb, o[db]);
                }
            }
        }
        const float lt = ts + __shfl_xor(ts, 32);
        if (myrow < L) {
            const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
            __bf16 *orow = p.o + (int64_t)(start + myrow) * p.o_st + (int64_t)qh * p.o_sh;
            const __bf16 *grow = GATE ? p.g + (int64_t)(start + myrow) * p.g_st + (int64_t)qh * p.g_sh : nullptr;
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const int d0 = db * 32 + 8 * jj + 4 * kg;
                    store_out4<GATE>(orow + d0, GATE ? grow + d0 : nullptr, o[db][4 * jj] * inv,
                                     o[db][4 * jj + 1] * inv, o[db][4 * jj + 2] * inv,
                                     o[db][4 * jj + 3] * inv);
                }
        }
    }
}

}  // namespace pe
