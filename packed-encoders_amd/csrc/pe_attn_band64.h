// Streaming band attention for head_dim 64: a symmetric-or-not bounded window whose rows each
// see five 32-key blocks (ModernBERT's +-64 local layers; any window with
// floor((31 + wr) / 32) + ceil(wl / 32) == 4), one query head per workgroup (gfx950 MFMA).
//
// Geometry. A workgroup walks a strip of consecutive 128-row query tiles of one segment and
// head; wave w holds rows 32 w .. 32 w + 31 of the tile. With keys cut into 32-key blocks
// (block j = keys 32 j .. 32 j + 31 of the segment), the rows of wave w in tile i read exactly
// the blocks F(i) + w .. F(i) + w + 4, F(i) = 4 i - ceil(wl / 32). The schedule is diagonal:
// at step s (0..4) of a tile, wave w computes block F(i) + w + s, so every wave does one block
// of work per step (a tile-major order gives some waves two blocks and others none between two
// barriers), and the blocks in use at step s are the four consecutive blocks F(i) + s ..
// F(i) + s + 3. Step 4 of tile i uses F(i) + 4 .. F(i) + 7, which are exactly the blocks of
// step 0 of tile i + 1: along a strip every key block is staged once, one new block per step,
// and the query tile is the only other traffic.
//
// Staging. Six LDS block slots (block j in slot j mod 6: the four in use plus two in flight)
// and one query buffer, filled by direct global-to-LDS loads issued two steps ahead of their
// use. Every step issues four 16-byte loads per lane (a query tile; or a K/V block plus two
// void loads; or, in the two steps that open a strip, two blocks), so "this step's loads are
// done" is one constant s_waitcnt vmcnt, as in the tiled kernel. A void load (an offset past
// every buffer range) touches no global memory but still writes its zeros to LDS, so void
// loads that pad a step land in a scratch area no one reads. The query buffer is refilled
// two steps before a tile starts, after every wave has copied the previous tile's rows into
// registers (at that tile's step 0). Blocks outside the segment are neither loaded nor
// computed; rows past its end compute nothing; buffer resources bounded by the segment make
// partial blocks read as zero. (Running loads four steps ahead in eight slots, with exact
// per-step wait counts instead of void loads, measured slower on every band workload.)
//
// Per block: S^T = K.Q^T (four 32x32x16 MFMAs), masking for blocks that cross the band's edge
// (two of the five), the lazily rescaled online softmax of the tiled kernel (log2 domain, a
// running maximum that is only a reference point, an exact re-score when a stale maximum would
// overflow), and O^T += V^T.P^T with V^T read by ds_read_b64_tr_b16.
#pragma once

#include "pe_attn_tiled.h"

namespace pe {

constexpr int kBandSlots = 6;  // K/V block slots of the band ring

// The window shapes the band kernel serves: each row spans exactly five 32-key blocks. (The
// host also requires head_dim 64, one query head per kv head group and shared key segments.)
__host__ __device__ inline bool band64_window(int wl, int wr) {
    return wl >= 0 && wr >= 0 && (31 + wr) / 32 + (wl + 31) / 32 == 4;
}

template <bool GATE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void band64_attn_kernel(AttnParams p) {
    constexpr int D = 64, BM = 128, KB = 32;  // head dim, query rows per tile, keys per block
    constexpr int DC = D / 16, DB = D / 32, CPR = D / 8;
    constexpr int BLOCK = KB * D;              // elements of one K (or V) block
    constexpr int QTILE = BM * D;              // elements of one query tile
    constexpr uint32_t kSlotBytes = 2 * BLOCK * 2, kVBytes = BLOCK * 2;
    constexpr int LPS = 4;                     // loads per lane per step
    constexpr int STEPS = 5;                   // compute steps per tile

    __shared__ __attribute__((aligned(16))) __bf16 slots[kBandSlots][2][BLOCK];
    __shared__ __attribute__((aligned(16))) __bf16 qbuf[QTILE];
    // Target of void loads (they write zeros into LDS): 1 KB per wave, never read.
    __shared__ __attribute__((aligned(16))) char vbuf[4][1024];

    // Work item, dealt to the XCDs in runs of neighbouring strips (as the tiled kernel).
    int item = blockIdx.x;
    {
        const int rh = kXcdRun * p.hgroups;
        const int j = (int)(blockIdx.x >> 3);
        item = ((j / rh) * 8 + (int)(blockIdx.x & 7)) * rh + j % rh;
    }
    const int entry = item / p.hgroups;
    const int qh = item - entry * p.hgroups;  // one query head per workgroup
    const WorkItem wi = load_work(p, entry);
    if (!wi.valid) return;
    const int start = wi.start, L = wi.L;
    if (L > p.max_seqlen || L <= 0) return;
    const int nq = (L + BM - 1) / BM;
    const int qt_first = wi.qt_first;
    if (qt_first >= nq) return;
    const int qt_end = min(nq, qt_first + p.strip);
    const int ntile = qt_end - qt_first;
    const int nblk = (L + KB - 1) / KB;        // key blocks of the segment
    const int fb0 = -((p.wl + KB - 1) / KB);   // F(i) = 4 i + fb0
    const int wl = p.wl, wr = p.wr;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = uniform(tid >> 6);
    const int col = lane & 31, kg = lane >> 5;
    const int kvh = qh / p.group;

    const __amdgpu_buffer_rsrc_t q_rs = make_rsrc(p.q + (int64_t)start * p.q_st + (int64_t)qh * p.q_sh, rows_bytes(L, p.q_st, D));
    const __amdgpu_buffer_rsrc_t k_rs = make_rsrc(p.k + (int64_t)start * p.k_st + (int64_t)kvh * p.k_sh, rows_bytes(L, p.k_st, D));
    const __amdgpu_buffer_rsrc_t v_rs = make_rsrc(p.v + (int64_t)start * p.v_st + (int64_t)kvh * p.v_sh, rows_bytes(L, p.v_st, D));
    const __amdgpu_buffer_rsrc_t o_rs = make_rsrc(p.o + (int64_t)start * p.o_st + (int64_t)qh * p.o_sh, rows_bytes(L, p.o_st, D));
    __amdgpu_buffer_rsrc_t g_rs = o_rs;
    if constexpr (GATE) g_rs = make_rsrc(p.g + (int64_t)start * p.g_st + (int64_t)qh * p.g_sh, rows_bytes(L, p.g_st, D));
    const int q_row = (int)p.q_st * 2, k_row = (int)p.k_st * 2, v_row = (int)p.v_st * 2;

    // DMA geometry. A K (or V) block is 256 16-byte units, one per lane of the workgroup: unit
    // u = 64 wave + lane holds key u / CPR, global column (u % CPR) ^ swz(key). The query tile
    // is 1024 units; wave w loads its own 32 rows, its load j (< 4) filling units
    // (4 w + j) * 64 + lane: row r = unit / CPR, column (unit % CPR) ^ swz(r).
    int koff, voff;
    {
        const int u = wave * 64 + lane;
        const int key = u / CPR, ch = (u % CPR) ^ swz<CPR>(key);
        koff = key * k_row + ch * 16;
        voff = key * v_row + ch * 16;
    }
    int qoff[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int u = (4 * wave + j) * 64 + lane;
        const int r = u / CPR, ch = (u % CPR) ^ swz<CPR>(r);
        qoff[j] = r * q_row + ch * 16;
    }
    const uint32_t slot_base = uniform((int)lds_addr(&slots[0][0][0]));
    const uint32_t q_base = uniform((int)lds_addr(&qbuf[0]));
    const uint32_t void_lds = uniform((int)lds_addr(&vbuf[0][0])) + wave * 1024;

    // The step schedule, walked identically by loader and consumer: steps 0 and 1 of a strip
    // stage blocks F(i0) .. F(i0) + 3; then tile i (0-based in the strip) runs steps
    // 2 + 5 i + s, s = 0..4. Loads for a step: s = 0 the query tile; s >= 1 block
    // F(i) + 3 + s. A block outside the segment (or a step past the strip) stages void loads.
    auto block_ok = [&](int j) { return j >= 0 && j < nblk; };
    auto issue_step = [&](int step) {
        uint32_t lds[4];
        int off[4];
        auto block_pair = [&](int j, int at) {  // K and V of block j into loads at, at + 1
            const int js = ((j % kBandSlots) + kBandSlots) % kBandSlots;
            const uint32_t sb = slot_base + js * kSlotBytes + (wave * 64) * 16;
            const bool ok = block_ok(j);
            lds[at] = ok ? sb : void_lds;
            lds[at + 1] = ok ? sb + kVBytes : void_lds;
            off[at] = ok ? koff + j * KB * k_row : kVoidOffset;
            off[at + 1] = ok ? voff + j * KB * v_row : kVoidOffset;
        };
        if (step < 2) {
            const int f = qt_first * 4 + fb0 + 2 * step;
            block_pair(f, 0);
            block_pair(f + 1, 2);
            // loads 0, 1 (K of both blocks) through k_rs, loads 2, 3 (V) through v_rs
            const uint32_t l4[4] = {lds[0], lds[2], lds[1], lds[3]};
            const int o4[4] = {off[0], off[2], off[1], off[3]};
            dma16x4(l4, o4, k_rs, v_rs);
            return;
        }
        const int t = step - 2;
        if (t >= STEPS * ntile) {
            const uint32_t l4[4] = {void_lds, void_lds, void_lds, void_lds};
            const int o4[4] = {kVoidOffset, kVoidOffset, kVoidOffset, kVoidOffset};
            dma16x4(l4, o4, k_rs, k_rs);
            return;
        }
        const int i = qt_first + t / STEPS, s = t % STEPS;
        if (s == 0) {
            const int base = i * BM * q_row;
            const uint32_t qb = q_base + (4 * wave) * 64 * 16;
            const uint32_t l4[4] = {qb, qb + 1024, qb + 2048, qb + 3072};
            const int o4[4] = {base + qoff[0], base + qoff[1], base + qoff[2], base + qoff[3]};
            dma16x4(l4, o4, q_rs, q_rs);
            return;
        }
        block_pair(4 * i + fb0 + 3 + s, 0);
        const uint32_t l4[4] = {lds[0], void_lds, lds[1], void_lds};
        const int o4[4] = {off[0], kVoidOffset, off[1], kVoidOffset};
        dma16x4(l4, o4, k_rs, v_rs);
    };
    issue_step(0);
    issue_step(1);

    // Per-lane LDS read offsets within a block (elements). K: key col, unit 2c + kg. V^T (tr16):
    // in 16-lane group g = lane / 16, source lane i = lane % 16 points at key
    // 16 h + 8 half + 4 (g / 2) + i / 4 and dims 32 db + 16 (g % 2) + 4 (i % 4).
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
    const float c2 = p.c;

    // Consumer steps: wait for this step's loads (the next step's may stay in flight), barrier,
    // then stage the step two ahead into the slots the barrier freed.
    int step = 0;
    auto begin_step = [&]() {
        wait_vmcnt<LPS>();
        __syncthreads();
        issue_step(step + 2);
    };
    begin_step();  // strip prologue: blocks F(i0), F(i0) + 1
    ++step;
    begin_step();  // F(i0) + 2, F(i0) + 3
    ++step;

    for (int i = qt_first; i < qt_end; ++i) {
        const int r0 = i * BM + wave * 32;  // the wave's first row
        const int myrow = r0 + col;
        const bool wave_active = r0 < L;
        const int a1 = min(L, r0 + 32);
        bf16x8 qf[DC];
        f32x16 o[DB];
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int j = 0; j < 16; ++j) o[db][j] = 0.0f;
        float m = kNegInf;
        float nmuse = 0.0f;  // -m, or 0 while m is -inf (a row with no key: every p is 0)
        float ls[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        bool need_exact = true;

        for (int s = 0; s < STEPS; ++s) {
            begin_step();
            if (s == 0) {
                // the wave's 32 query rows, as MFMA B operands; the empty asm ends the reads'
                // scope before a later barrier lets the buffer be refilled
                const __bf16 *qs = &qbuf[0] + wave * 32 * D;
#pragma unroll
                for (int c = 0; c < DC; ++c) qf[c] = ld_s16(qs + kbase_c[c]);
#pragma unroll
                for (int c = 0; c < DC; ++c) asm volatile("" : "+v"(qf[c]));
            }
            const int j = 4 * i + fb0 + wave + s;  // this wave's block
            if (wave_active && block_ok(j)) {
                const int js = j % kBandSlots;
                const __bf16 *kt = &slots[js][0][0];
                const __bf16 *vt = &slots[js][1][0];
                const int kb0 = j * KB;
                const bool full = block_full(kb0, L, r0, a1, wl, wr);
                f32x16 sc;
                bf16x8 pb[2];
                float st[4];
                bool exact = need_exact;
                while (true) {
#pragma unroll
                    for (int x = 0; x < 16; ++x) sc[x] = 0.0f;
#pragma unroll
                    for (int c = 0; c < DC; ++c) sc = mfma32(ld_s16(kt + kbase_c[c]), qf[c], sc);
                    if (!full) {
                        const uint32_t km = key_mask(kb0, kg, myrow, L, wl, wr);
#pragma unroll
                        for (int x = 0; x < 16; ++x) sc[x] = mask_score(sc[x], km, acc_key(x, 0));
                    }
                    if (exact) {
                        float mp[4] = {kNegInf, kNegInf, kNegInf, kNegInf};
#pragma unroll
                        for (int x = 0; x < 16; ++x) mp[x & 3] = fmaxf(mp[x & 3], sc[x]);
                        const float mx = fmaxf(fmaxf(mp[0], mp[1]), fmaxf(mp[2], mp[3]));
                        if (wave_any(mx * c2 > m + kLazyRescale)) {
                            const float mnew = fmaxf(m, fmaxf(mx, __shfl_xor(mx, 32)) * c2);
                            const float alpha = mnew == kNegInf ? 1.0f : exp2_fast(m - mnew);
                            m = mnew;
                            nmuse = mnew == kNegInf ? 0.0f : -mnew;
#pragma unroll
                            for (int x = 0; x < 4; ++x) ls[x] *= alpha;
#pragma unroll
                            for (int db = 0; db < DB; ++db)
#pragma unroll
                                for (int x = 0; x < 16; ++x) o[db][x] *= alpha;
                        }
                    }
                    f32x16 e;
#pragma unroll
                    for (int x = 0; x < 16; ++x) e[x] = exp2_fast(fmaf(sc[x], c2, nmuse));
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        pb[h] = to_bf16x8(e, 8 * h);
#pragma unroll
                        for (int x = 0; x < 4; ++x) st[x] = h == 0 ? sum2_first(pb[h], x) : sum2(pb[h], x, st[x]);
                    }
                    if (exact || !wave_any(fmaxf(fmaxf(st[0], st[1]), fmaxf(st[2], st[3])) > kOverflowGuard)) break;
                    exact = true;
                }
                if (need_exact) need_exact = wave_any((m == kNegInf) & (myrow < L));
#pragma unroll
                for (int x = 0; x < 4; ++x) ls[x] += st[x];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
#pragma unroll
                    for (int db = 0; db < DB; ++db) {
                        const bf16x4 lo = tr16(vt + (16 * h) * D + vbase[0][db]);
                        const bf16x4 hi = tr16(vt + (16 * h) * D + vbase[1][db]);
                        const bf16x8 va = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                        o[db] = mfma32(va, pb[h], o[db]);
                    }
                }
            }
            ++step;
        }

        // Normalise, apply the gate, store.
        const float lsum = (ls[0] + ls[1]) + (ls[2] + ls[3]);
        const float lt = lsum + __shfl_xor(lsum, 32);
        if (wave_active) {
            const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
            const int ooff = myrow * (int)p.o_st * 2;
            const int goff = GATE ? myrow * (int)p.g_st * 2 : 0;
            store_block<DB, GATE>(o, inv, kg, o_rs, ooff, g_rs, goff);
        }
    }
    wait_vmcnt<0>();  // the last output stores
}

}  // namespace pe
