// Tiled flash-style packed attention for long segments, head_dim 64 (gfx950 MFMA): windowed and
// causal calls (global calls run global64_attn_kernel, pe_attn_global64.h; large calls with a
// +-64-shaped band the streaming band64_attn_kernel, pe_attn_band64.h). Wider heads use
// wide_attn_kernel (head_dim 128, pe_attn_tiled_wide.h) and wide16_attn_kernel (head_dim 256,
// pe_attn_tiled_wide16.h), which share the staging below.
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
// The ring carries one flat sequence of steps: for each query tile of the strip, 64 / BN "Q
// steps" that bring the tile's query rows into a stage (each wave reads its 32 rows from there
// into registers), then one step per key tile. Every step loads the same number of 16-byte
// units per lane, so "this step's loads are done" is one constant s_waitcnt vmcnt (vmcnt 0 for
// the strip's last step, after which nothing is staged).
// No load the compiler can see remains in the loop (only the gate's), so it never inserts a
// vector-memory wait of its own that would drain the ring. Every global access goes through a
// buffer resource bounded by the segment, so rows past the segment read as zero with no
// branch. Block decisions are scalar: a key tile entirely inside every row's window takes a
// path with no per-block test; otherwise each wave skips 32-key blocks outside its rows' band
// (window / causal) and masks only blocks crossing a segment or band edge.
//
// Softmax: online, fp32, log2 domain, with a running maximum m that is only a reference
// point: numerator and denominator share it, so any m gives the same result as long as
// nothing overflows. Maxima are computed on a query tile's first key tile (and while some row
// of the wave has seen no key yet); later tiles skip them, and a key tile whose probabilities
// under the stale m sum past 2^64 on some row (scores jumping by more than ~60 in log2 units)
// is scored again exactly, raising m and rescaling the accumulators before any of it is
// added. Probabilities are rounded to
// bf16 for the P.V MFMA, and the row sums add exactly those bf16 values in fp32 (v_dot2 with
// ones), so numerator and denominator weigh every key alike; the reference sums the unrounded
// fp32 values (packed_encoders/_kernels/triton_packed_attention.py:122-136), a difference far
// inside the bf16 output rounding.
//
// Work entries (segment, first query tile of the strip) come from the device-built,
// cost-ordered list of plan_kernel; the 1-D grid walks entries with the head group fastest,
// so the most expensive strips of every head are dispatched first
// (longest-processing-time order).
#pragma once

#include "pe_attn_stage.h"

namespace pe {

constexpr float kLazyRescale = 8.0f;  // log2 of the largest unnormalised probability allowed
// Largest per-row, per-tile probability sum accepted under a stale running maximum (2^64: far
// from overflowing the bf16 probabilities, the fp32 sums or the fp32 P.V accumulators).
constexpr float kOverflowGuard = 18446744073709551616.0f;
// Consecutive work entries (all head groups of each) that one XCD takes in a row in banded
// calls, so that neighbouring query tiles meet in one L2.
constexpr int kXcdRun = 4;

// WIN: the call has a window or causal bound. Without one (global attention) every window
// test folds away at compile time, which also gives global and windowed launches distinct
// kernel names in traces.
template <int D, int G, int BN, int NS, bool GATE, bool WIN>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void tiled_attn_kernel(AttnParams p) {
    static_assert(D == 64 && BN == 64 && NS == 3, "head_dim 64 kernel (wider heads: wide_attn_kernel, wide16_attn_kernel)");
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

    // Work item of this workgroup: the list walked with the head group fastest, so that the
    // costliest strips of every head go first and the heads of one query tile, which read
    // adjacent 128-byte pieces of the same token rows, run together. Workgroup i runs on XCD
    // i % 8; a banded call re-reads each key block from the neighbouring query tile's
    // workgroups, so it deals the list to the XCDs in runs of kXcdRun entries: neighbours then
    // share one L2 instead of fetching the shared keys twice, and the dealing keeps the
    // longest-first order across XCDs (whole contiguous eighths would give one XCD all the
    // costliest tiles). The launch rounds the grid up to whole rounds of runs.
    int item = blockIdx.x;
    if (WIN && p.wl >= 0 && p.wr >= 0) {
        const int rh = kXcdRun * p.hgroups;
        const int j = (int)(blockIdx.x >> 3);
        item = ((j / rh) * 8 + (int)(blockIdx.x & 7)) * rh + j % rh;
    }
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

    // Key range [klo, klo + ntiles * BN) of query tile qt: the union of its rows' windows, in
    // key positions (at least one tile: rows that reach no key come out as zero).
    auto key_range = [&](int qt, int &klo, int &ntiles) {
        const int q0 = qt * BM + off, rows_end = min(L, qt * BM + BM) + off;
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
    // Q step geometry: the wave's RQ rows fill its region of the stage, unit j * 64 + lane
    // holding row r = unit / CPR, global column (unit % CPR) ^ swz(r).
    int qoff[LPS];
#pragma unroll
    for (int j = 0; j < LPS; ++j) {
        const int u = j * 64 + lane;
        const int r = u / CPR, ch = (u % CPR) ^ swz<CPR>(r);
        qoff[j] = r * q_row + ch * 16;
    }
    auto issue_q = [&](int stage, int qt, int i) {
        const uint32_t qb = ring_base + stage * kStageBytes + wave * kQWaveBytes;
        const int base = (qt * BM + rb * 32 + i * RQ) * q_row;
        uint32_t lds[LPS];
        int off[LPS];
#pragma unroll
        for (int j = 0; j < LPS; ++j) {
            lds[j] = qb + j * 1024;
            off[j] = base + qoff[j];
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

    const float c2 = p.c;

    // Loader: the next step to stage, walked NS - 1 steps ahead of the consumer; nothing past
    // the strip's last step. n_issued / n_begun count the steps staged and begun (wave-uniform).
    int ld_qt = qt_first, ld_t = -QS, ld_klo, ld_nt;
    key_range(ld_qt, ld_klo, ld_nt);
    int n_issued = 0, n_begun = 0;
    auto issue_next = [&](int stage) {
        if (ld_qt >= qt_end) return;
        ++n_issued;
        if (ld_t < 0) issue_q(stage, ld_qt, ld_t + QS);
        else issue_kv(stage, ld_klo + ld_t * BN);
        if (++ld_t >= ld_nt) {
            ++ld_qt;
            ld_t = -QS;
            if (ld_qt < qt_end) key_range(ld_qt, ld_klo, ld_nt);
        }
    };
#pragma unroll
    for (int st = 0; st < NS - 1; ++st) issue_next(st);

    // Consumer. Two loops, so that the O accumulators of a query tile are carried by the inner
    // (key tile) loop alone: a flat step loop whose Q steps and tile ends also pass O around
    // makes the register allocator copy all of it on every step.
    int stage = 0;  // ring stage of the current step
    // Start of a step: its loads are complete once at most the NS - 2 later steps' loads are in
    // flight (loads complete in issue order; other outstanding accesses only make the wait
    // stricter), or none when no later step was staged, so the strip's last step leaves no load
    // in flight and the workgroup ends without draining its output stores. After the barrier
    // every wave is done with the previous step's stage, which is refilled with the step NS - 1
    // ahead. The two cases are exact only for NS = 3 (at most one later step in flight): a deeper
    // ring can have fewer than NS - 2 later steps in flight near a strip's end, and would need a
    // wait sized by n_issued - n_begun - 1 instead (as the wide kernels take).
    auto begin_step = [&]() {
        if (n_issued > n_begun + 1) wait_vmcnt<(NS - 2) * LPS>();
        else wait_vmcnt<0>();
        ++n_begun;
        __syncthreads();
        issue_next(stage == 0 ? NS - 1 : stage - 1);
    };
    auto end_step = [&]() { stage = stage == NS - 1 ? 0 : stage + 1; };

    bf16x8 qf[DC];
    for (int qt = qt_first; qt < qt_end; ++qt) {
        int klo, ntiles;
        key_range(qt, klo, ntiles);
        const int r0 = qt * BM + rb * 32;
        const int myrow = r0 + col;
        const bool wave_active = r0 < L;
        const int wr1 = min(L, r0 + 32);
        const int a0 = r0 + off, a1 = wr1 + off, arow = myrow + off;  // in key positions

        // Q steps: lanes whose row is in step i's part read their fragments; the empty asm
        // ends the reads' scope before the next barrier frees the stage.
#pragma unroll
        for (int i = 0; i < QS; ++i) {
            begin_step();
            if (QS == 1 || col / RQ == i) {
                const __bf16 *qs = &ring[stage][0][0] + wave * RQ * D - i * RQ * D;
#pragma unroll
                for (int c = 0; c < DC; ++c) qf[c] = ld_s16(qs + kbase_c[c]);
#pragma unroll
                for (int c = 0; c < DC; ++c) asm volatile("" : "+v"(qf[c]));
            }
            end_step();
        }

        f32x16 o[DB];
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int j = 0; j < 16; ++j) o[db][j] = 0.0f;
        float m = kNegInf;
        float nmuse = 0.0f;  // -m, or 0 while m is -inf (a row with no key: every p is 0)
        float ls[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        bool need_exact = true;  // some row of the wave may still lack a finite running maximum

        for (int t = 0; t < ntiles; ++t) {
            begin_step();
            const __bf16 *kt = &ring[stage][0][0];
            const __bf16 *vt = &ring[stage][1][0];
            if (wave_active) {
                const int kt0 = klo + t * BN;
                // Every block of the tile live and unmasked for all of this wave's rows: the
                // common case, taken without any per-block test.
                const bool full = (kt0 + BN <= Lk) && (wl < 0 || (a1 - 1) - kt0 <= wl) && (wr < 0 || (kt0 + BN - 1) - a0 <= wr);
                // (Kept as a lambda: the register allocator then fits the kernel in 160-164 VGPRs;
                // written inline the same code spills.)
                auto kv_step = [&]() {
                    bool live[NB];
#pragma unroll
                    for (int b = 0; b < NB; ++b) live[b] = full || block_live(kt0 + 32 * b, Lk, a0, a1, wl, wr);
                    f32x16 s[NB];
                    bf16x8 pb[NB][2];
                    float st[4];
                    // The running maximum m is only a reference point: numerator and denominator
                    // share it, so any m gives the same result as long as nothing overflows.
                    // Maxima are therefore computed only while some row of the wave lacks a
                    // finite m (the first tiles of a query tile), or when this tile's
                    // probabilities under the stale m sum past kOverflowGuard on some row: the
                    // tile is then scored again exactly, m raised and the accumulators rescaled
                    // before any of it is added (a rare second pass). Otherwise a step spends no
                    // VALU on maxima.
                    bool exact = need_exact;
                    while (true) {
#pragma unroll
                        for (int b = 0; b < NB; ++b) {
                            if (!live[b]) continue;
                            // S^T = K . Q^T of 32-key block b, -inf outside the rows' windows
                            const int kb0 = kt0 + 32 * b;
                            f32x16 acc;
#pragma unroll
                            for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
#pragma unroll
                            for (int c = 0; c < DC; ++c) acc = mfma32(ld_s16(kt + 32 * b * D + kbase_c[c]), qf[c], acc);
                            if (!full && !block_full(kb0, Lk, a0, a1, wl, wr)) {
                                const uint32_t km = key_mask(kb0, kg, arow, Lk, wl, wr);
#pragma unroll
                                for (int j = 0; j < 16; ++j) acc[j] = mask_score(acc[j], km, acc_key(j, 0));
                            }
                            s[b] = acc;
                        }
                        if (exact) {
                            float mp[4] = {kNegInf, kNegInf, kNegInf, kNegInf};  // 4 partial-max chains
#pragma unroll
                            for (int b = 0; b < NB; ++b)
                                if (live[b]) {
#pragma unroll
                                    for (int j = 0; j < 16; ++j) mp[j & 3] = fmaxf(mp[j & 3], s[b][j]);
                                }
                            // Each lane tests its own maximum: the two lanes of a query row share
                            // m, so "some lane exceeds m" is "some row exceeds m"; only a rescale
                            // combines the pair.
                            const float mx = fmaxf(fmaxf(mp[0], mp[1]), fmaxf(mp[2], mp[3]));
                            if (wave_any(mx * c2 > m + kLazyRescale)) {
                                const float mnew = fmaxf(m, fmaxf(mx, __shfl_xor(mx, 32)) * c2);
                                const float alpha = mnew == kNegInf ? 1.0f : exp2_fast(m - mnew);
                                m = mnew;
                                nmuse = mnew == kNegInf ? 0.0f : -mnew;
#pragma unroll
                                for (int i = 0; i < 4; ++i) ls[i] *= alpha;
#pragma unroll
                                for (int db = 0; db < DB; ++db)
#pragma unroll
                                    for (int j = 0; j < 16; ++j) o[db][j] *= alpha;
                            }
                        }
                        // Probabilities under m: bf16 MFMA operands and fp32 sums of exactly
                        // those bf16 values.
#pragma unroll
                        for (int i = 0; i < 4; ++i) st[i] = 0.0f;
#pragma unroll
                        for (int b = 0; b < NB; ++b) {
                            if (!live[b]) continue;
                            f32x16 e;
#pragma unroll
                            for (int j = 0; j < 16; ++j) e[j] = exp2_fast(fmaf(s[b][j], c2, nmuse));
#pragma unroll
                            for (int h = 0; h < 2; ++h) {
                                pb[b][h] = to_bf16x8(e, 8 * h);
#pragma unroll
                                for (int i = 0; i < 4; ++i)
                                    st[i] = (b == 0 && h == 0) ? sum2_first(pb[b][h], i) : sum2(pb[b][h], i, st[i]);
                            }
                        }
                        if (exact || !wave_any(fmaxf(fmaxf(st[0], st[1]), fmaxf(st[2], st[3])) > kOverflowGuard)) break;
                        exact = true;
                    }
                    if (need_exact) need_exact = wave_any((m == kNegInf) & (myrow < L));
#pragma unroll
                    for (int i = 0; i < 4; ++i) ls[i] += st[i];
#pragma unroll
                    for (int b = 0; b < NB; ++b) {
                        if (!live[b]) continue;
#pragma unroll
                        for (int h = 0; h < 2; ++h) {
#pragma unroll
                            for (int db = 0; db < DB; ++db) {
                                // keys 32b + 16h + 8 half + vkey0: the swizzle sees only the bits
                                // of 8 half + vkey0 (32b + 16h changes neither)
                                const bf16x4 lo = tr16(vt + (32 * b + 16 * h) * D + vbase[0][db]);
                                const bf16x4 hi = tr16(vt + (32 * b + 16 * h) * D + vbase[1][db]);
                                const bf16x8 va = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                                o[db] = mfma32(va, pb[b][h], o[db]);
                            }
                        }
                    }
                };
                kv_step();
            }
            end_step();
        }

        // Normalise, apply the gate, store. After the strip's last step the ring is idle (its
        // loader stages nothing past the strip), and the stage of the step before the last is
        // free with no further barrier: every wave passed the last step's barrier, so is done
        // with it, and no load was issued into it. The last tile's rows leave through that
        // stage as whole rows (store_rows), each wave in its own 32-row region.
        const float lsum = (ls[0] + ls[1]) + (ls[2] + ls[3]);
        const float lt = lsum + __shfl_xor(lsum, 32);
        const bool via_lds = qt + 1 == qt_end;
        if (wave_active) {
            const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
            if (via_lds) {
                // `stage` already points past the last step's stage; the one before that is free.
                const int free_stage = stage == 0 ? NS - 2 : stage == 1 ? NS - 1 : stage - 2;
                store_rows<D, GATE>(o, inv, lane, &ring[free_stage][0][0] + wave * 32 * D, o_rs, r0 * (int)p.o_st * 2,
                                    (int)p.o_st * 2, g_rs, GATE ? r0 * (int)p.g_st * 2 : 0, GATE ? (int)p.g_st * 2 : 0);
            } else {
                const int ooff = myrow * (int)p.o_st * 2;
                const int goff = GATE ? myrow * (int)p.g_st * 2 : 0;
                store_block<DB, GATE>(o, inv, kg, o_rs, ooff, g_rs, goff);
            }
        }
    }
}

}  // namespace pe
