// LDS-resident packed attention for short segments (length <= SK <= 128), gfx950 MFMA.
//
// One workgroup = 4 waves = one segment x HPW query heads. The segment's whole K and V tiles
// of every head in the group are staged in LDS once, row-major with the 16-byte units of a row
// XOR-swizzled (swz), by direct global-to-LDS loads; the wave's query blocks go straight to
// registers as MFMA B operands. Every load of the workgroup — query blocks first, then all K/V
// tiles — is issued before the one wait, so a workgroup pays the memory latency once. Each
// wave owns one head and walks that head's 32-row query blocks (4 / HPW waves share a head).
// S^T = K.Q^T reads K with ds_read_b128 and O^T = V^T.P^T reads V^T with ds_read_b64_tr_b16,
// as the tiled kernels do. A query block sees every key of the segment at once, so the softmax
// is exact, with no online rescaling: the row maximum and sum are per-lane scalars combined
// with the partner lane through one wavefront shuffle.
//
// Segments longer than short_max, or empty, leave the workgroup at once, which is what lets
// one launch of this kernel and one of the tiled kernel split a mixed batch per segment with
// no host read of cu_seqlens. Global accesses go through buffer resources bounded by the
// segment: rows past its end read as zero and are never written.
//
// ROPE: q and k are unrotated projection rows and the workgroup applies split-half RoPE itself
// (pe_attn_args.rope_cos / rope_sin; rope8, the RoPE kernel's rounding). The segment's cos and
// sin rows are staged in LDS with the K/V tiles (same loads, same swizzle, before the one
// wait): the keys are then rotated once in LDS, each thread taking (key, 16-byte column pair)
// items of every head of the group, behind one more barrier, and every wave rotates its query
// fragment in registers (a lane's dims 16 c + 8 kg .. + 7, c < D / 16, hold both halves of every
// rotation pair (c, c + D / 32)), reading the table values at the K operand's offsets.
#pragma once

#include "pe_attn_stage.h"
#include "pe_rope.h"

namespace pe {

// Waves per SIMD the compiler is asked to fit: a head_dim 64 workgroup of capacity 64 and at most
// two heads takes 16 or 32 KB of LDS, so five fit a CU once its registers allow five waves per
// SIMD (84 VGPRs instead of 105, no spills); the others are bound by LDS first.
template <int D, int SK, int HPW, bool ROPE>
constexpr int short_waves_per_eu() {
    return D == 64 && SK == 64 && HPW <= 2 && !ROPE ? 5 : 1;
}

template <int D, int SK, int HPW, bool GATE, bool ROPE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(short_waves_per_eu<D, SK, HPW, ROPE>())))
void short_attn_kernel(AttnParams p) {
    static_assert(SK % 32 == 0 && SK <= 128 && (4 % HPW) == 0, "short tile shape");
    constexpr int NB = SK / 32;
    constexpr int DC = D / 16;
    constexpr int DB = D / 32;
    constexpr int CPR = D / 8;                    // 16-byte units per row
    constexpr int WSTEP = 4 / HPW;                // waves sharing one head
    constexpr int NQ = (NB + WSTEP - 1) / WSTEP;  // query blocks per wave, at most
    constexpr int TILE = SK * D;                  // elements of one K (or V) tile
    constexpr int UPT = TILE / 8 / 256;           // 16-byte units per thread and tile
    static_assert(UPT >= 1 && TILE % (8 * 256) == 0, "a tile must split into 1 KB wave loads");

    __shared__ __attribute__((aligned(16))) __bf16 kv[HPW][2][TILE];
    // ROPE: the cos and sin rows of the segment's keys (= its query rows), laid out and
    // swizzled as a K tile, so the key pass and the query fragments read them at K's offsets.
    __shared__ __attribute__((aligned(16))) __bf16 tab[ROPE ? 2 : 1][ROPE ? TILE : 8];

    const int seg = blockIdx.x;
    const int start = p.cu[seg];
    const int L = p.cu[seg + 1] - start;  // query rows
    const int kstart = p.cuk[seg];
    const int Lk = p.cuk[seg + 1] - kstart;  // keys
    if (L <= 0 || Lk < 0 || max(L, Lk) > p.short_max) return;
    const int off = Lk - L;  // key position of query row 0 (queries end-aligned to their keys)
    const int h0 = blockIdx.y * HPW;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = uniform(tid >> 6);
    const int col = lane & 31, kg = lane >> 5;
    const int s = wave % HPW;
    const int qh = h0 + s;
    const bool wave_head = qh < p.hq;

    // The wave's query blocks as B operands (zero beyond the segment), issued first.
    const __amdgpu_buffer_rsrc_t q_rs = make_rsrc(p.q + (int64_t)start * p.q_st + (int64_t)min(qh, p.hq - 1) * p.q_sh,
                                                  rows_bytes(L, p.q_st, D));
    bf16x8 qf[NQ][DC];
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
        const int qoff = (32 * (wave / HPW + i * WSTEP) + col) * (int)p.q_st * 2 + kg * 16;
#pragma unroll
        for (int c = 0; c < DC; ++c) qf[i][c] = buf_ld16(q_rs, qoff + c * 32, 0);
    }
    // K and V of every head of the group: unit u = (j * 4 + wave) * 64 + lane of a tile holds
    // key u / CPR, global column (u % CPR) ^ swz(key); keys >= Lk read as zero.
    const int k_row = (int)p.k_st * 2, v_row = (int)p.v_st * 2;
    const uint32_t kv_base = uniform((int)lds_addr(&kv[0][0][0]));
#pragma unroll
    for (int hs = 0; hs < HPW; ++hs) {
        const int h = h0 + hs;
        if (h >= p.hq) break;
        const int kvh = h / p.group;
        const __amdgpu_buffer_rsrc_t k_rs = make_rsrc(p.k + (int64_t)kstart * p.k_st + (int64_t)kvh * p.k_sh, rows_bytes(Lk, p.k_st, D));
        const __amdgpu_buffer_rsrc_t v_rs = make_rsrc(p.v + (int64_t)kstart * p.v_st + (int64_t)kvh * p.v_sh, rows_bytes(Lk, p.v_st, D));
#pragma unroll
        for (int j = 0; j < UPT; ++j) {
            const int u = (j * 4 + wave) * 64 + lane;
            const int key = u / CPR, ch = (u % CPR) ^ swz<CPR>(key);
            const uint32_t dst = kv_base + (uint32_t)((hs * 2 * TILE) * 2 + (j * 4 + wave) * 1024);
            dma16(dst, key * k_row + ch * 16, k_rs);
            dma16(dst + TILE * 2, key * v_row + ch * 16, v_rs);
        }
    }
    if constexpr (ROPE) {
        // Table rows of keys 0..SK-1 (row (kstart + key) % rrows), unit for unit as the K tile;
        // keys past the segment take void loads (zeros, no traffic).
        const uint32_t tbytes = (uint32_t)((int64_t)p.rrows * p.rst * 2);
        const __amdgpu_buffer_rsrc_t c_rs = make_rsrc(p.rcos, tbytes), s_rs = make_rsrc(p.rsin, tbytes);
        const uint32_t tab_base = uniform((int)lds_addr(&tab[0][0]));
#pragma unroll
        for (int j = 0; j < UPT; ++j) {
            const int u = (j * 4 + wave) * 64 + lane;
            const int key = u / CPR, ch = (u % CPR) ^ swz<CPR>(key);
            const int row = (int)(((int64_t)kstart + key) % p.rrows);
            const int off = key < Lk ? row * (int)p.rst * 2 + ch * 16 : kVoidOffset;
            const uint32_t dst = (uint32_t)uniform((int)(tab_base + (uint32_t)((j * 4 + wave) * 1024)));
            dma16(dst, off, c_rs);
            dma16(dst + TILE * 2, off, s_rs);
        }
    }
    wait_vmcnt<0>();
    __syncthreads();
    if constexpr (ROPE) {
        // Rotate every head's keys in place, thread by (key, column pair (j, j + CPR / 2))
        // items (column c of key r sits at unit c ^ swz(r) of its row, in the K tile and the
        // tables alike), then let every wave see all of them.
        constexpr int HALF = CPR / 2, ITEMS = (SK * HALF + 255) / 256;
#pragma unroll
        for (int it = 0; it < ITEMS; ++it) {
            const int item = it * 256 + tid, key = item / HALF, j = item % HALF;
            if (key >= Lk) continue;
            const int lo_off = key * D + ((j ^ swz<CPR>(key)) * 8);
            const int hi_off = key * D + (((j + HALF) ^ swz<CPR>(key)) * 8);
            const bf16x8 cl = ld_s16(&tab[0][lo_off]), ch = ld_s16(&tab[0][hi_off]);
            const bf16x8 sl = ld_s16(&tab[1][lo_off]), sh = ld_s16(&tab[1][hi_off]);
#pragma unroll
            for (int hs = 0; hs < HPW; ++hs) {
                if (h0 + hs >= p.hq) break;
                __bf16 *kt_hs = &kv[hs][0][0];
                bf16x8 lo = ld_s16(kt_hs + lo_off), hi = ld_s16(kt_hs + hi_off);
                rope8(lo, hi, cl, ch, sl, sh);
                *reinterpret_cast<bf16x8 *>(kt_hs + lo_off) = lo;
                *reinterpret_cast<bf16x8 *>(kt_hs + hi_off) = hi;
            }
        }
        __syncthreads();
        // The wave's query rows (row 32 qb + col) take the same tables: their fragment units
        // 2 c + kg sit where the K operand's do (swz sees only the row's bits 0-3). Rows past
        // the segment are zero in qf and in the tables.
#pragma unroll
        for (int i = 0; i < NQ; ++i) {
            const int rbase = 32 * (wave / HPW + i * WSTEP) * D + col * D;
#pragma unroll
            for (int c = 0; c < DC / 2; ++c) {
                const int lo_off = rbase + ((2 * c + kg) ^ swz<CPR>(col)) * 8;
                const int hi_off = rbase + ((2 * (c + DC / 2) + kg) ^ swz<CPR>(col)) * 8;
                rope8(qf[i][c], qf[i][c + DC / 2], ld_s16(&tab[0][lo_off]), ld_s16(&tab[0][hi_off]),
                      ld_s16(&tab[1][lo_off]), ld_s16(&tab[1][hi_off]));
            }
        }
    }
    if (!wave_head) return;

    // Per-lane LDS offsets: K key 32b + col, unit 2c + kg; V^T as in the tiled kernels.
    int kbase_c[DC];
#pragma unroll
    for (int c = 0; c < DC; ++c) kbase_c[c] = col * D + ((2 * c + kg) ^ swz<CPR>(col)) * 8;
    const int vi = lane & 15, vg = lane >> 4;
    const int vkey0 = 4 * (vg >> 1) + (vi >> 2);
    const int vdim0 = 16 * (vg & 1) + 4 * (vi & 3);
    int vbase[2][DB];
#pragma unroll
    for (int half = 0; half < 2; ++half)
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const int key = 8 * half + vkey0, dim = 32 * db + vdim0;
            vbase[half][db] = key * D + (((dim >> 3) ^ swz<CPR>(key)) * 8) + (dim & 4);
        }
    const __bf16 *kt = &kv[s][0][0];
    const __bf16 *vt = &kv[s][1][0];

    const int wl = p.wl, wr = p.wr;
    const float c2 = p.c;
    const int nkb = (Lk + 31) >> 5;
    const __amdgpu_buffer_rsrc_t o_rs = make_rsrc(p.o + (int64_t)start * p.o_st + (int64_t)qh * p.o_sh, rows_bytes(L, p.o_st, D));
    __amdgpu_buffer_rsrc_t g_rs = o_rs;
    if constexpr (GATE) g_rs = make_rsrc(p.g + (int64_t)start * p.g_st + (int64_t)qh * p.g_sh, rows_bytes(L, p.g_st, D));

#pragma unroll
    for (int i = 0; i < NQ; ++i) {
        const int qb = wave / HPW + i * WSTEP;
        if (qb * 32 >= L) break;
        const int r0 = qb * 32, r1 = min(L, r0 + 32);
        const int myrow = r0 + col;
        f32x16 sc[NB];
        bool live[NB];
        float mx = kNegInf;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int kb0 = 32 * b;
            live[b] = b < nkb && block_live(kb0, Lk, r0 + off, r1 + off, wl, wr);
            if (live[b]) {
                f32x16 acc;
#pragma unroll
                for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
#pragma unroll
                for (int c = 0; c < DC; ++c) acc = mfma32(ld_s16(kt + kb0 * D + kbase_c[c]), qf[i][c], acc);
                if (!block_full(kb0, Lk, r0 + off, r1 + off, wl, wr)) {
                    const uint32_t km = key_mask(kb0, kg, myrow + off, Lk, wl, wr);
#pragma unroll
                    for (int j = 0; j < 16; ++j) acc[j] = mask_score(acc[j], km, acc_key(j, 0));
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
#pragma unroll
                    for (int db = 0; db < DB; ++db) {
                        const bf16x4 lo = tr16(vt + (32 * b + 16 * h) * D + vbase[0][db]);
                        const bf16x4 hi = tr16(vt + (32 * b + 16 * h) * D + vbase[1][db]);
                        const bf16x8 va = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                        o[db] = mfma32(va, pb, o[db]);
                    }
                }
            }
        }
        const float lt = ts + __shfl_xor(ts, 32);
        const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
        // With one head per wave (HPW 4) the head's K tile is read by this wave alone, so after
        // the wave's last query block it is free for the row-wise epilogue (store_rows); LDS
        // accesses of a wave complete in order, so no barrier is needed.
        const bool last = i + 1 == NQ || (qb + WSTEP) * 32 >= L;
        if (HPW == 4 && last) {
            store_rows<D, GATE>(o, inv, lane, &kv[s][0][0], o_rs, r0 * (int)p.o_st * 2, (int)p.o_st * 2, g_rs,
                                GATE ? r0 * (int)p.g_st * 2 : 0, GATE ? (int)p.g_st * 2 : 0);
        } else {
            const int ooff = myrow * (int)p.o_st * 2;
            const int goff = GATE ? myrow * (int)p.g_st * 2 : 0;
            store_block<DB, GATE>(o, inv, kg, o_rs, ooff, g_rs, goff);
        }
    }
}

}  // namespace pe
