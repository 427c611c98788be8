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
// no host read of cu_seqlens. Global accesses go through buffer resources bounded by the
// segment: rows past its end read as zero and are never written.
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
    const int k_row = (int)p.k_st * 2, v_row = (int)p.v_st * 2;

    // Stage K and V^T of every head of the group (keys >= L read as zero up to the block edge).
#pragma unroll
    for (int s = 0; s < HPW; ++s) {
        const int qh = h0 + s;
        if (qh >= p.hq) break;
        const int kvh = qh / p.group;
        const __amdgpu_buffer_rsrc_t k_rs = make_rsrc(p.k + (int64_t)start * p.k_st + (int64_t)kvh * p.k_sh, rows_bytes(L, p.k_st, D));
        const __amdgpu_buffer_rsrc_t v_rs = make_rsrc(p.v + (int64_t)start * p.v_st + (int64_t)kvh * p.v_sh, rows_bytes(L, p.v_st, D));
        for (int c = tid; c < kcap * (D / 8); c += 256) {
            const int key = c / (D / 8), dc = c - key * (D / 8);
            st_s16(&Ks[s][key * KP + dc * 8], buf_ld16(k_rs, key * k_row + dc * 16, 0));
        }
        // 2-key x 8-dim chunks, key pair fastest across threads.
        const int npairs = kcap / 2;
        for (int c = tid; c < npairs * (D / 8); c += 256) {
            const int kp = c % npairs, dc = c / npairs;
            const bf16x8 a = buf_ld16(v_rs, 2 * kp * v_row + dc * 16, 0);
            const bf16x8 b = buf_ld16(v_rs, (2 * kp + 1) * v_row + dc * 16, 0);
            typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
            __bf16 *dst = &Vt[s][(dc * 8) * VP + vperm(2 * kp)];
#pragma unroll
            for (int dd = 0; dd < 8; ++dd) {
                bf16x2 t;
                t[0] = a[dd];
                t[1] = b[dd];
                *reinterpret_cast<bf16x2 *>(dst + dd * VP) = t;
            }
        }
    }
    __syncthreads();

    const int lane = tid & 63;
    const int wave = uniform(tid >> 6);
    const int col = lane & 31, kg = lane >> 5;
    const int s = wave % HPW;
    const int qh = h0 + s;
    if (qh >= p.hq) return;
    const int wl = p.wl, wr = p.wr;
    const float c2 = p.c;
    const __amdgpu_buffer_rsrc_t q_rs = make_rsrc(p.q + (int64_t)start * p.q_st + (int64_t)qh * p.q_sh, rows_bytes(L, p.q_st, D));
    const __amdgpu_buffer_rsrc_t o_rs = make_rsrc(p.o + (int64_t)start * p.o_st + (int64_t)qh * p.o_sh, rows_bytes(L, p.o_st, D));
    __amdgpu_buffer_rsrc_t g_rs = o_rs;
    if constexpr (GATE) g_rs = make_rsrc(p.g + (int64_t)start * p.g_st + (int64_t)qh * p.g_sh, rows_bytes(L, p.g_st, D));

    for (int qb = wave / HPW; qb * 32 < L; qb += WSTEP) {
        const int r0 = qb * 32, r1 = min(L, r0 + 32);
        const int myrow = r0 + col;
        bf16x8 qf[DC];
        {
            const int qoff = myrow * (int)p.q_st * 2 + kg * 16;
#pragma unroll
            for (int c = 0; c < DC; ++c) qf[c] = buf_ld16(q_rs, qoff + c * 32, 0);
        }
        f32x16 sc[NB];
        bool live[NB];
        float mx = kNegInf;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int kb0 = 32 * b;
            live[b] = b < nkb && block_live(kb0, L, r0, r1, wl, wr);
            if (live[b]) {
                const __bf16 *ka = &Ks[s][(kb0 + col) * KP + kg * 8];
                f32x16 acc;
#pragma unroll
                for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
#pragma unroll
                for (int c = 0; c < DC; ++c) acc = mfma32(ld_s16(ka + c * 16), qf[c], acc);
                if (!block_full(kb0, L, r0, r1, wl, wr)) {
#pragma unroll
                    for (int j = 0; j < 16; ++j) {
                        const int key = kb0 + acc_key(j, kg);
                        const bool ok = (key < L) & ((wl < 0) | (myrow - key <= wl)) & ((wr < 0) | (key - myrow <= wr));
                        acc[j] = ok ? acc[j] : kNegInf;
                    }
                }
                sc[b] = acc;
#pragma unroll
                for (int j = 0; j < 16; ++j) mx = fmaxf(mx, acc[j]);
            }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float muse = mx == kNegInf ? 0.0f : mx * c2;
        float ts = 0.0f;
        f32x16 o[DB];
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int j = 0; j < 16; ++j) o[db][j] = 0.0f;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (live[b]) {
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const float e = exp2_fast(fmaf(sc[b][j], c2, -muse));
                    sc[b][j] = e;
                    ts += e;
                }
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
}

}  // namespace pe
