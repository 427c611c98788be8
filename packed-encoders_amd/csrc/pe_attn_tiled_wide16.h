// Tiled packed attention for head_dim 256 on 16-row query blocks (gfx950): NW (4 or 8) waves
// per workgroup, each owning 16 query rows of one head, products on v_mfma_f32_16x16x32_bf16.
//
// Why a second wide kernel: with 32-row blocks (wide_attn_kernel) a head_dim 256 wave holds
// 128 O^T accumulators and 64 Q-fragment registers and needs about 300 registers, so one wave
// runs per SIMD and every MFMA, exponential and memory latency is exposed (counters showed a
// third of each wave's life waiting and a quarter stalled on dependencies). A 16-row block
// halves both (64 + 32 registers), so two waves share each SIMD and cover each other's
// latencies. The ring of direct global-to-LDS K/V stages, the swizzles and the plan are those
// of the 32-row kernels; a query tile is 16 NW / G rows of each of G heads. The Q fragment
// (D / 8 registers) is loaded straight into registers rather than staged through the ring:
// every ring step is a K/V step, and a workgroup's first wait covers its Q and its first
// NS K/V tiles at once (the staged form paid one memory latency for Q, then another for the
// first K/V tile, then ran a step with no products).
//
// Layouts (lane l: c16 = l % 16, g4 = l / 16). v_mfma_f32_16x16x32_bf16 takes A as 16 rows x
// 32 k (lane: row c16, k 8 g4 .. 8 g4 + 7), B as 32 k x 16 columns (lane: column c16, the same
// k) and returns C as 16 x 16 (lane: column c16, rows 4 g4 + i).
//  * S^T = K . Q^T per 16-key block kb: A = keys 16 kb + c16 by dims 32 c + 8 g4 .. (one
//    ds_read_b128 each), B = the lane's query row (Q fragment, registers). Lane l then holds, for
//    query row c16, the scores of keys 16 kb + 4 g4 + i (i = 0..3): 8 per 32-key step.
//  * O^T = V^T . P^T per 16-dim block db: B = the lane's own 8 probabilities, k-slot 8 g4 + i
//    standing for key 4 g4 + i and 8 g4 + 4 + i for key 16 + 4 g4 + i; A = V^T for the same
//    keys, two ds_read_b64_tr_b16 (lane a of a 16-lane group addresses key 4 g4 + a / 4 (+16),
//    dims 16 db + 4 (a % 4) .. + 3, and receives the four keys of dim 16 db + a).
//    Lane l accumulates dims 16 db + 4 g4 + i of query row c16.
// Row statistics combine the four lanes c16 + 16 g4 (shuffles by 16 and 32).
#pragma once

#include "pe_attn_tiled_wide.h"

namespace pe {

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Two 4-dim bf16 chunks per lane of the 16x16 accumulator layout regrouped into 8 contiguous
// dims: x holds the lane's chunk of block 2j (dims 32 j + 4 g4 ..), y of block 2j + 1, rows
// g4 = lane / 16 of 16 lanes. v_permlane32_swap exchanges rows 2-3 of x with rows 0-1 of y,
// then v_permlane16_swap rows 1 and 3 of x with rows 0 and 2 of y; row g4 then holds, in
// (x, y), the chunks of lanes (2 (g4 % 2), 2 (g4 % 2) + 1) of block 2j + g4 / 2: dims
// 32 j + 8 g4 .. + 7, 16 contiguous bytes at byte 64 j + 16 g4 of the row.
__device__ __forceinline__ bf16x8 swap16_pair(bf16x4 x, bf16x4 y) {
    typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
    u32x2 a = __builtin_bit_cast(u32x2, x), b = __builtin_bit_cast(u32x2, y);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const auto s32 = __builtin_amdgcn_permlane32_swap(a[k], b[k], false, false);
        const auto s16 = __builtin_amdgcn_permlane16_swap(s32[0], s32[1], false, false);
        a[k] = s16[0];
        b[k] = s16[1];
    }
    const bf16x4 lo = __builtin_bit_cast(bf16x4, a), hi = __builtin_bit_cast(bf16x4, b);
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// bf16(x * s) of 8 outputs x already rounded to bf16 and 8 bf16 gate factors s.
__device__ __forceinline__ bf16x8 scale8(bf16x8 x, bf16x8 s) {
    const bf16x4 lo = round4<true>((float)x[0], (float)x[1], (float)x[2], (float)x[3], bf16x4{s[0], s[1], s[2], s[3]});
    const bf16x4 hi = round4<true>((float)x[4], (float)x[5], (float)x[6], (float)x[7], bf16x4{s[4], s[5], s[6], s[7]});
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Run length of the XCD dealing for NW waves per workgroup and an NS-stage ring of 32 KB
// stages: the workgroups 32 CUs hold at once (LDS allows 160 KB / ring per CU, registers two
// waves per SIMD).
template <int NW, int NS>
__host__ __device__ inline int wide16_run(int hgroups) {
    constexpr int kByLds = 160 / (32 * NS), kByWaves = 8 / NW;
    return xcd_run<32 * (kByLds < kByWaves ? kByLds : kByWaves)>(hgroups);
}

template <int D, int NW, int G, int NS, bool GATE, bool WIN>
__global__ __launch_bounds__(64 * NW) void wide16_attn_kernel(AttnParams p) {
    static_assert(D == 256 && (NW == 4 || NW == 8) && (4 % G) == 0 && NS >= 2, "head_dim 256, 4 or 8 waves");
    constexpr int WPH = NW / G;      // waves per query head
    constexpr int BM = 16 * WPH;     // query rows per tile (the plan's tiles)
    constexpr int BN = 32;           // keys per step
    constexpr int DC = D / 32;       // 32-dim chunks of the S^T reduction
    constexpr int DB = D / 16;       // 16-dim blocks of O^T
    constexpr int CPR = D / 8;       // 16-byte units per K/V/Q row
    constexpr int TILE = BN * D;     // elements of one K (or V) tile
    constexpr int UPW = TILE / 8 / 64 / NW;  // 1 KB wave-loads per tensor per wave and step
    constexpr int LPS = 2 * UPW;     // loads per lane per step
    static_assert(LPS % 4 == 0 && UPW % 2 == 0, "loads go out four at a time");

    __shared__ __attribute__((aligned(16))) __bf16 ring[NS][2][TILE];

    // Work item: as wide_attn_kernel (each segment's tiles contiguous in the plan, runs of
    // wide16_run() items dealt to the XCDs in turn).
    const int rh = wide16_run<NW, NS>(p.hgroups);
    const int j = (int)(blockIdx.x >> 3);
    const int item = ((j / rh) * 8 + (int)(blockIdx.x & 7)) * rh + j % rh;
    const int entry = item / p.hgroups;
    const int hg = item - entry * p.hgroups;
    const WorkItem wi = load_work(p, entry);
    if (!wi.valid) return;
    const int qt_first = wi.qt_first;
    const int start = wi.start, L = wi.L;      // query rows
    const int kstart = wi.kstart, Lk = wi.Lk;  // keys
    // A segment longer than the caller's max_seqlen breaks the contract the host sized the
    // 32-bit buffer offsets by: its rows are left unwritten rather than addressed.
    if (L > p.max_seqlen || Lk > p.max_seqlen_k || Lk < 0) return;
    const int off = Lk - L;  // key position of query row 0 (queries end-aligned to their keys)
    const int nq = (L + BM - 1) / BM;
    if (qt_first >= nq) return;
    const int qt_end = min(nq, qt_first + p.strip);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = uniform(tid >> 6);
    const int c16 = lane & 15, g4 = lane >> 4;
    const int slot = wave / WPH, rb = wave - slot * WPH;
    const int qh = hg * G + slot;
    const int kvh = (hg * G) / p.group;
    const int wl = WIN ? p.wl : -1, wr = WIN ? p.wr : -1;

    const __amdgpu_buffer_rsrc_t q_rs = make_rsrc(p.q + (int64_t)start * p.q_st + (int64_t)qh * p.q_sh, rows_bytes(L, p.q_st, D));
    const __amdgpu_buffer_rsrc_t k_rs = make_rsrc(p.k + (int64_t)kstart * p.k_st + (int64_t)kvh * p.k_sh, rows_bytes(Lk, p.k_st, D));
    const __amdgpu_buffer_rsrc_t v_rs = make_rsrc(p.v + (int64_t)kstart * p.v_st + (int64_t)kvh * p.v_sh, rows_bytes(Lk, p.v_st, D));
    const __amdgpu_buffer_rsrc_t o_rs = make_rsrc(p.o + (int64_t)start * p.o_st + (int64_t)qh * p.o_sh, rows_bytes(L, p.o_st, D));
    __amdgpu_buffer_rsrc_t g_rs = o_rs;
    if constexpr (GATE) g_rs = make_rsrc(p.g + (int64_t)start * p.g_st + (int64_t)qh * p.g_sh, rows_bytes(L, p.g_st, D));
    const int q_row = (int)p.q_st * 2, k_row = (int)p.k_st * 2, v_row = (int)p.v_st * 2;

    // Key range [klo, klo + ntiles * BN) of query tile qt: the union of its rows' windows.
    auto key_range = [&](int qt, int &klo, int &ntiles) {
        const int q0 = qt * BM + off, rows_end = min(L, qt * BM + BM) + off;  // key positions
        klo = wl >= 0 ? max(0, q0 - wl) : 0;
        const int khi = wr >= 0 ? min(Lk, rows_end + wr) : Lk;
        ntiles = max(1, (khi - klo + BN - 1) / BN);
    };

    // DMA geometry. K/V: wave-load j of this wave fills units [(wave * UPW + j) * 64, +64) of a
    // tile; unit u holds key u / CPR, global 16-byte column (u % CPR) ^ swz(key).
    int koff[UPW], voff[UPW];
#pragma unroll
    for (int jj = 0; jj < UPW; ++jj) {
        const int u = (wave * UPW + jj) * 64 + lane;
        const int key = u / CPR, ch = (u % CPR) ^ swz<CPR>(key);
        koff[jj] = key * k_row + ch * 16;
        voff[jj] = key * v_row + ch * 16;
    }
    const uint32_t ring_base = uniform((int)lds_addr(&ring[0][0][0]));
    constexpr uint32_t kStageBytes = 2 * TILE * 2, kTileBytes = TILE * 2;
    // LPS loads of one step (lds[i], off[i]); the first UPW read through ra, the rest rb.
    auto dma_step = [&](const uint32_t (&lds)[LPS], const int (&off)[LPS], __amdgpu_buffer_rsrc_t ra,
                        __amdgpu_buffer_rsrc_t rb) {
#pragma unroll
        for (int g = 0; g < LPS / 4; ++g) {
            const uint32_t l4[4] = {lds[4 * g], lds[4 * g + 1], lds[4 * g + 2], lds[4 * g + 3]};
            const int o4[4] = {off[4 * g], off[4 * g + 1], off[4 * g + 2], off[4 * g + 3]};
            dma16x4(l4, o4, 4 * g < UPW ? ra : rb, 4 * g + 2 < UPW ? ra : rb);
        }
    };
    auto issue_kv = [&](int stage, int kt0) {
        const uint32_t kb = ring_base + stage * kStageBytes + wave * UPW * 1024;
        const int kbase = kt0 * k_row, vbase = kt0 * v_row;
        uint32_t lds[LPS];
        int off[LPS];
#pragma unroll
        for (int jj = 0; jj < UPW; ++jj) {
            lds[jj] = kb + jj * 1024;
            off[jj] = koff[jj] + kbase;
            lds[UPW + jj] = kb + kTileBytes + jj * 1024;
            off[UPW + jj] = voff[jj] + vbase;
        }
        dma_step(lds, off, k_rs, v_rs);
    };
    // Per-lane LDS read offsets (elements within a tile). swz<CPR>(key) = key & 15 for CPR 32.
    // K: key 16 kb + c16, unit (4 c + g4) ^ c16; with c = 4 ch + cl the XOR only touches cl,
    // so kaddr[cl] plus compile-time 16 kb D + 128 ch covers every (kb, c).
    int kaddr[4];
#pragma unroll
    for (int cl = 0; cl < 4; ++cl) kaddr[cl] = c16 * D + ((4 * cl + g4) ^ c16) * 8;
    // V^T: key 4 g4 + c16 / 4 (+16: same swizzle), dim 16 db + 4 (c16 % 4): unit
    // (2 db + (c16 % 4) / 2) ^ s with s = key & 15; with db = 8 dh + dl the XOR only touches
    // dl, so vaddr[dl] plus compile-time 128 dh (+ 16 D for the second four keys).
    const int vkey = 4 * g4 + (c16 >> 2);
    int vaddr[8];
#pragma unroll
    for (int dl = 0; dl < 8; ++dl)
        vaddr[dl] = vkey * D + (((2 * dl + ((c16 & 3) >> 1)) ^ (vkey & 15)) * 8) + 4 * (c16 & 1);

    f32x4 o[DB];
    float m;
    float ls[4];
    auto reset = [&]() {
#pragma unroll
        for (int db = 0; db < DB; ++db) o[db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        m = kNegInf;
#pragma unroll
        for (int i = 0; i < 4; ++i) ls[i] = 0.0f;
    };
    const float c2 = p.c;

    int qt = qt_first, klo, ntiles;
    key_range(qt, klo, ntiles);
    int r0 = qt * BM + rb * 16;
    int myrow = r0 + c16;
    bool wave_active = r0 < L;
    int wr1 = min(L, r0 + 16);
    bf16x8 qf[DC];
    reset();

    // Inputs of query tile qt held in registers: the Q fragment (lane (c16, g4): its row's dims
    // 32 c + 8 g4 .. + 7) and, with a gate, bf16(sigmoid(gate)) of the dims it stores after the
    // epilogue's regrouping (32 j + 8 g4 .. + 7, 16 bytes per load). The loads are the compiler's (it places the wait before the first use); the
    // empty asm makes that wait, and the sigmoids, happen here, outside the step loop: no step
    // waits on these loads, and the epilogue only scales, rounds and stores (the sigmoids run
    // while the CU's other workgroup is in its steps).
    bf16x8 sgv[GATE ? DB / 2 : 1];  // gate factors of dims 32 j + 8 g4 .. + 7 (the epilogue's layout)
    auto load_tile_inputs = [&](int qt_) {
        const int row = qt_ * BM + rb * 16 + c16;
        const int base = row * q_row + 16 * g4;
#pragma unroll
        for (int c = 0; c < DC; ++c) qf[c] = buf_ld16(q_rs, base + 64 * c, 0);
        if constexpr (GATE) {
            const int gbase = row * (int)p.g_st * 2 + 16 * g4;
#pragma unroll
            for (int j = 0; j < DB / 2; ++j) sgv[j] = buf_ld16(g_rs, gbase + 64 * j, 0);
        }
#pragma unroll
        for (int c = 0; c < DC; ++c) asm volatile("" : "+v"(qf[c]));
        if constexpr (GATE) {
#pragma unroll
            for (int j = 0; j < DB / 2; ++j) {
                const bf16x4 lo = sigmoid4(bf16x4{sgv[j][0], sgv[j][1], sgv[j][2], sgv[j][3]});
                const bf16x4 hi = sigmoid4(bf16x4{sgv[j][4], sgv[j][5], sgv[j][6], sgv[j][7]});
                sgv[j] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
            }
#pragma unroll
            for (int j = 0; j < DB / 2; ++j) asm volatile("" : "+v"(sgv[j]));
        }
    };

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

    // Prologue: every stage is free, so the first NS K/V tiles go out, then the tile's register
    // inputs (whose wait therefore covers them too: one memory latency for the workgroup's start).
    Cursor ld{qt, 0, klo, ntiles};
    int issued = 0;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        if (ld.qt < qt_end) {
            issue_kv(issued % NS, ld.klo + ld.t * BN);
            ++issued;
            adv(ld);
        }
    }
    load_tile_inputs(qt);

    int t = 0, step = 0;
    while (true) {
        // This step's loads are complete once at most the later steps' loads are in flight
        // (loads complete in issue order; other outstanding accesses only make this stricter).
        const int later = issued - step - 1;
        if (later >= 2) wait_vmcnt<2 * LPS>();
        else if (later >= 1) wait_vmcnt<LPS>();
        else wait_vmcnt<0>();
        __syncthreads();
        // Refill the stage freed by the previous step (all waves passed the barrier after it).
        if (step > 0 && ld.qt < qt_end) {
            issue_kv(issued % NS, ld.klo + ld.t * BN);
            ++issued;
            adv(ld);
        }

        const __bf16 *kt = &ring[step % NS][0][0];
        const __bf16 *vt = &ring[step % NS][1][0];
        if (wave_active) {
            const int kt0 = klo + t * BN;
            if (block_live(kt0, Lk, r0 + off, wr1 + off, wl, wr)) {
                f32x4 s[2];
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int c = 0; c < DC; ++c)
                        acc = mfma16(ld_s16(kt + 16 * kb * D + 128 * (c >> 2) + kaddr[c & 3]), qf[c], acc);
                    s[kb] = acc;
                }
                if (!block_full(kt0, Lk, r0 + off, wr1 + off, wl, wr)) {
#pragma unroll
                    for (int kb = 0; kb < 2; ++kb) {
                        const uint32_t km = key_mask(kt0 + 16 * kb, g4, myrow + off, Lk, wl, wr);
#pragma unroll
                        for (int i = 0; i < 4; ++i) s[kb][i] = mask_score(s[kb][i], km, i);
                    }
                }
                const float mx = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                                       fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
                // Each lane tests its own maximum ("some lane exceeds m" is "some row does");
                // a rescale takes the row's maximum over its four lanes.
                if (wave_any(mx * c2 > m + kLazyRescale)) {
                    float rm = fmaxf(mx, __shfl_xor(mx, 16));
                    rm = fmaxf(rm, __shfl_xor(rm, 32));
                    const float mnew = fmaxf(m, rm * c2);
                    const float alpha = mnew == kNegInf ? 1.0f : exp2_fast(m - mnew);
                    m = mnew;
#pragma unroll
                    for (int i = 0; i < 4; ++i) ls[i] *= alpha;
#pragma unroll
                    for (int db = 0; db < DB; ++db) o[db] *= alpha;
                }
                const float muse = m == kNegInf ? 0.0f : m;
                bf16x8 pb;
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int i = 0; i < 4; ++i) pb[4 * kb + i] = (__bf16)exp2_fast(fmaf(s[kb][i], c2, -muse));
                // row sums of the rounded probabilities, the values the P.V product weighs
#pragma unroll
                for (int i = 0; i < 4; ++i) ls[i] = sum2(pb, i, ls[i]);
#pragma unroll
                for (int db = 0; db < DB; ++db) {
                    const __bf16 *va = vt + 128 * (db >> 3) + vaddr[db & 7];
                    const bf16x4 lo = tr16(va);
                    const bf16x4 hi = tr16(va + 16 * D);
                    o[db] = mfma16(__builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7), pb, o[db]);
                }
            }
        }

        if (t + 1 >= ntiles) {
            // Last key tile of this query tile: normalise, apply the gate, store, reset.
            float lt = (ls[0] + ls[1]) + (ls[2] + ls[3]);
            lt += __shfl_xor(lt, 16);
            lt += __shfl_xor(lt, 32);
            if (wave_active) {
                // Lane (c16, g4) rounds its 4-dim chunks (16 db + 4 g4 ..), then for each pair of
                // 16-dim blocks (2j, 2j + 1) swap16_pair regroups the four lanes of a row so that
                // lane g4 holds dims 32 j + 8 g4 .. + 7, whose gate factors it loaded: 16
                // contiguous bytes at 64 j + 16 g4, one store per pair instead of two.
                const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
                const int ooff = myrow * (int)p.o_st * 2 + 16 * g4;
#pragma unroll
                for (int j = 0; j < DB / 2; ++j) {
                    const bf16x4 y0 = round4<false>(o[2 * j][0] * inv, o[2 * j][1] * inv, o[2 * j][2] * inv,
                                                    o[2 * j][3] * inv, bf16x4{});
                    const bf16x4 y1 = round4<false>(o[2 * j + 1][0] * inv, o[2 * j + 1][1] * inv,
                                                    o[2 * j + 1][2] * inv, o[2 * j + 1][3] * inv, bf16x4{});
                    bf16x8 z = swap16_pair(y0, y1);
                    if constexpr (GATE) z = scale8(z, sgv[j]);
                    buf_st16(o_rs, ooff + 64 * j, z);
                }
            }
            reset();
            if (qt + 1 >= qt_end) break;
            ++qt;
            key_range(qt, klo, ntiles);
            r0 = qt * BM + rb * 16;
            myrow = r0 + c16;
            wave_active = r0 < L;
            wr1 = min(L, r0 + 16);
            load_tile_inputs(qt);  // waits here (and for the ring's loads in flight): strips of several tiles only
            t = 0;
        } else {
            ++t;
        }
        ++step;
    }
}

}  // namespace pe
