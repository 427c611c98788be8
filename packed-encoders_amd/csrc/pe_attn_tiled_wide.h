// Tiled packed attention for head_dim 128 (gfx950 MFMA; head_dim 256 runs the 16-row
// wide16_attn_kernel, pe_attn_tiled_wide16.h, built on this one): the same workgroup shape,
// LDS ring, direct global-to-LDS staging, Q steps, swizzles and buffer-bounded accesses as
// tiled_attn_kernel (pe_attn_tiled.h), with a step loop shaped for the register budget of
// wide heads, whose O accumulators alone take D / 2 VGPRs per lane: one copy of the step (the
// ring stage is a register), the exact running maximum of every tile (lazy rescale above 2^8),
// and loads issued only for real steps, the wait count following how many are in flight. The
// row sums add the bf16-rounded probabilities the P.V product uses (v_dot2 with ones), as the
// head_dim 64 kernels do: under the lazily raised maximum a row's dominant probability is not
// exactly 1, and summing it unrounded would leave its bf16 rounding (up to 2^-9 relative) in
// the output. (The reference sums the unrounded values,
// packed_encoders/_kernels/triton_packed_attention.py:122-136, with a maximum that is exact per
// block.)
#pragma once

#include "pe_attn_tiled.h"

namespace pe {

// Workgroups per run that one XCD takes in a row: as many as its 32 CUs hold at once
// (RESIDENT), in whole work entries (all head groups of each). The launch rounds the grid up
// to whole rounds of 8 runs.
template <int RESIDENT>
__host__ __device__ inline int xcd_run(int hgroups) {
    return hgroups * (hgroups < RESIDENT ? RESIDENT / hgroups : 1);
}
// This kernel: two 64 KB workgroups per CU (head_dim 128).
__host__ __device__ inline int wide_run(int hgroups) { return xcd_run<64>(hgroups); }

template <int D, int G, int BN, int NS, bool GATE, bool WIN>
__global__ __launch_bounds__(256) void wide_attn_kernel(AttnParams p) {
    static_assert(D % 32 == 0 && BN % 32 == 0 && (4 % G) == 0 && NS >= 2, "tile shape");
    constexpr int WPH = 4 / G;       // waves per query head
    constexpr int BM = 32 * WPH;     // query rows per query tile
    constexpr int NB = BN / 32;      // 32-key blocks per tile
    constexpr int DC = D / 16;       // 16-dim chunks for S^T
    constexpr int DB = D / 32;       // 32-dim blocks for O^T
    constexpr int CPR = D / 8;       // 16-byte units per K/V row
    constexpr int TILE = BN * D;     // elements of one K (or V) tile
    constexpr int UPW = TILE / 8 / 64 / 4;  // 1 KB wave-loads per tensor per wave and tile
    constexpr int LPS = 2 * UPW;     // loads per lane per step (K and V, or Q)
    constexpr int QS = 64 / BN;      // Q steps per query tile
    constexpr int RQ = 32 / QS;      // query rows per wave and Q step
    static_assert(UPW >= 1 && TILE % (8 * 64 * 4) == 0, "tile must split into 1 KB wave loads");
    static_assert(64 % BN == 0 && RQ * CPR == LPS * 64, "a Q step must load as much as a K/V step");

    __shared__ __attribute__((aligned(16))) __bf16 ring[NS][2][TILE];

    // Work item: the plan lists each segment's query tiles contiguously; workgroup i runs on
    // XCD i % 8, and the runs of wide_run() consecutive items are dealt to the XCDs in turn,
    // so the tiles of a segment run side by side on one XCD and re-read its keys from that
    // XCD's L2 (dealt one item per XCD, every tile fetched them again from memory).
    const int rh = wide_run(p.hgroups);
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
    const int col = lane & 31, kg = lane >> 5;
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

    // Key range [klo, klo + ntiles * BN) of query tile qt: the union of its rows' windows
    // (never empty for a tile inside the segment: each row sees at least itself).
    auto key_range = [&](int qt, int &klo, int &ntiles) {
        const int q0 = qt * BM + off, rows_end = min(L, qt * BM + BM) + off;  // key positions
        klo = wl >= 0 ? max(0, q0 - wl) : 0;
        const int khi = wr >= 0 ? min(Lk, rows_end + wr) : Lk;
        ntiles = max(1, (khi - klo + BN - 1) / BN);
    };

    // DMA geometry. K/V: wave-load j of this wave fills units [(wave * UPW + j) * 64, +64) of a
    // tile; unit u holds key u / CPR, global 16-byte column (u % CPR) ^ swz(key). Q step i: the
    // wave's own RQ rows (rows 32 rb + RQ i + r of its head) fill its region of the stage,
    // unit j * 64 + lane holding row r = unit / CPR, column (unit % CPR) ^ swz(r).
    int koff[UPW], voff[UPW];
#pragma unroll
    for (int j = 0; j < UPW; ++j) {
        const int u = (wave * UPW + j) * 64 + lane;
        const int key = u / CPR, ch = (u % CPR) ^ swz<CPR>(key);
        koff[j] = key * k_row + ch * 16;
        voff[j] = key * v_row + ch * 16;
    }
    const uint32_t ring_base = uniform((int)lds_addr(&ring[0][0][0]));
    constexpr uint32_t kStageBytes = 2 * TILE * 2, kTileBytes = TILE * 2, kQWaveBytes = RQ * D * 2;
    static_assert(LPS % 4 == 0 && UPW % 2 == 0, "loads go out four at a time");
    // LPS loads of one step (lds[i], voff[i]); the first UPW read through ra, the rest rb.
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
        for (int j = 0; j < UPW; ++j) {
            lds[j] = kb + j * 1024;
            off[j] = koff[j] + kbase;
            lds[UPW + j] = kb + kTileBytes + j * 1024;
            off[UPW + j] = voff[j] + vbase;
        }
        dma_step(lds, off, k_rs, v_rs);
    };
    // Q offsets are recomputed at each (rare) Q step rather than held in registers: the empty
    // asm keeps the compiler from hoisting them out of the loop.
    auto issue_q = [&](int stage, int qt, int i) {
        const uint32_t qb = ring_base + stage * kStageBytes + wave * kQWaveBytes;
        const int base = (qt * BM + rb * 32 + i * RQ) * q_row;
        int ql = lane;
        asm volatile("" : "+v"(ql));
        uint32_t lds[LPS];
        int off[LPS];
#pragma unroll
        for (int j = 0; j < LPS; ++j) {
            const int u = j * 64 + ql;
            const int r = u / CPR, ch = (u % CPR) ^ swz<CPR>(r);
            lds[j] = qb + j * 1024;
            off[j] = base + r * q_row + ch * 16;
        }
        dma_step(lds, off, q_rs, q_rs);
    };

    // Per-lane LDS read offsets (elements within a tile). K: key 32b + col, unit 2c + kg (the
    // wave's Q rows use the same pattern: row col of its region). V^T (tr16): in 16-lane group
    // g = lane / 16, source lane i = lane % 16 points at key 16h + 4 * (g / 2) + i / 4 (+ 8 for
    // the second half of the operand) and dims 32 db + 16 (g % 2) + 4 (i % 4); the transpose
    // hands lane (m = dim, kg) four keys of its dim. Both swizzles depend only on bits of the
    // key below 16 (CPR 16, 32) or 32 (CPR 8) that the block / 16-key-half loops leave fixed,
    // so every address is a per-lane base plus a compile-time offset.
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

    // Current query tile; t < 0 marks its Q steps.
    int qt = qt_first, klo, ntiles;
    key_range(qt, klo, ntiles);
    int r0 = qt * BM + rb * 32;
    int myrow = r0 + col;
    bool wave_active = r0 < L;
    int wr1 = min(L, r0 + 32);
    bf16x8 qf[DC];
#pragma unroll
    for (int c = 0; c < DC; ++c) qf[c] = bf16x8{};
    reset();

    // Step bookkeeping: `adv` moves a cursor one step ahead.
    struct Cursor {
        int qt, t, klo, ntiles;
    };
    auto adv = [&](Cursor &c) {
        if (++c.t >= c.ntiles) {
            ++c.qt;
            c.t = -QS;
            if (c.qt < qt_end) key_range(c.qt, c.klo, c.ntiles);
        }
    };
    auto issue_step = [&](int stage, const Cursor &c) {
        if (c.t < 0) issue_q(stage, c.qt, c.t + QS);
        else issue_kv(stage, c.klo + c.t * BN);
    };

    // Prologue: issue the first NS - 1 steps.
    Cursor ld{qt, -QS, klo, ntiles};  // next step to issue
    int issued = 0;
#pragma unroll
    for (int s = 0; s < NS - 1; ++s) {
        if (ld.qt < qt_end) {
            issue_step(issued % NS, ld);
            ++issued;
            adv(ld);
        }
    }

    int t = -QS, step = 0;
    while (true) {
        // This step's loads are complete once at most the later steps' loads are in flight
        // (loads complete in issue order; other outstanding accesses only make this stricter).
        const int later = issued - step - 1;
        if (NS >= 3 && later >= 2) wait_vmcnt<2 * LPS>();
        else if (later >= 1) wait_vmcnt<LPS>();
        else wait_vmcnt<0>();
        __syncthreads();
        // Refill the stage freed by the previous step (all waves passed the barrier after it).
        if (ld.qt < qt_end) {
            issue_step(issued % NS, ld);
            ++issued;
            adv(ld);
        }

        const __bf16 *kt = &ring[step % NS][0][0];
        if (t < 0) {
            // Q step t + QS: lanes whose row is in this step's part read their fragments; the
            // empty asm ends the reads' scope before the next barrier frees the stage.
            const int i = t + QS;
            if (QS == 1 || col / RQ == i) {
                const __bf16 *qs = kt + wave * RQ * D - i * RQ * D;
#pragma unroll
                for (int c = 0; c < DC; ++c) qf[c] = ld_s16(qs + kbase_c[c]);
#pragma unroll
                for (int c = 0; c < DC; ++c) asm volatile("" : "+v"(qf[c]));
            }
        }

        const __bf16 *vt = &ring[step % NS][1][0];
        if (t >= 0 && wave_active) {
            const int kt0 = klo + t * BN;
            f32x16 s[NB];
            bool live[NB];
            float mp[4] = {kNegInf, kNegInf, kNegInf, kNegInf};  // partial maxima (4 chains)
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int kb0 = kt0 + 32 * b;
                live[b] = block_live(kb0, Lk, r0 + off, wr1 + off, wl, wr);
                if (live[b]) {
                    f32x16 acc;
#pragma unroll
                    for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
#pragma unroll
                    for (int c = 0; c < DC; ++c) acc = mfma32(ld_s16(kt + 32 * b * D + kbase_c[c]), qf[c], acc);
                    if (!block_full(kb0, Lk, r0 + off, wr1 + off, wl, wr)) {
                        const uint32_t km = key_mask(kb0, kg, myrow + off, Lk, wl, wr);
#pragma unroll
                        for (int j = 0; j < 16; ++j) acc[j] = mask_score(acc[j], km, acc_key(j, 0));
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
                    for (int j = 0; j < 16; ++j) s[b][j] = exp2_fast(fmaf(s[b][j], c2, -muse));
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const bf16x8 pb = to_bf16x8(s[b], 8 * h);
#pragma unroll
                        for (int i = 0; i < 4; ++i) ls[i] = sum2(pb, i, ls[i]);
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
        }

        if (t >= 0 && t + 1 >= ntiles) {
            // Last key tile of this query tile: normalise, apply the gate, store, reset.
            const float lsum = (ls[0] + ls[1]) + (ls[2] + ls[3]);
            const float lt = lsum + __shfl_xor(lsum, 32);
            if (wave_active) {
                const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
                const int ooff = myrow * (int)p.o_st * 2;
                const int goff = GATE ? myrow * (int)p.g_st * 2 : 0;
                store_block<DB, GATE>(o, inv, kg, o_rs, ooff, g_rs, goff);
            }
            reset();
            if (qt + 1 >= qt_end) break;
            ++qt;
            key_range(qt, klo, ntiles);
            r0 = qt * BM + rb * 32;
            myrow = r0 + col;
            wave_active = r0 < L;
            wr1 = min(L, r0 + 32);
            t = -QS;
        } else {
            ++t;
        }
        ++step;
    }
}

}  // namespace pe
