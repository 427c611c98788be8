// Packed global (bidirectional, unwindowed) attention for long segments, head_dim 64, on
// gfx950 MFMA: the MFMA-bound layers of a packed encoder batch (ModernBERT's global layers,
// long documents). Windowed and causal calls run tiled_attn_kernel (pe_attn_tiled.h) or, for
// large calls with a +-64-shaped band, band64_attn_kernel (pe_attn_band64.h).
//
// Work shape. One workgroup = 4 waves = one strip of query tiles of one segment for a group of
// G query heads sharing a kv head. Each wave owns 64 query rows of one head, held in VGPRs as
// two 32-row halves (A: rows 0-31, B: rows 32-63), each the B operand of
// v_mfma_f32_32x32x16_bf16. A query tile is 64 * 4 / G rows. Every K operand read from LDS
// (ds_read_b128) and every V^T operand (two ds_read_b64_tr_b16) feeds two MFMAs, one per half,
// so a wave reads 8 LDS bytes per lane and MFMA where 32-row waves read 16, and the per-block
// control is paid once per 16 MFMAs.
//
// Split tiles. A segment's last query tile often holds rows for at most half of a head's
// waves (G = 1, a 300-token segment: tiles of 256 and 44 rows). Such a tile is split by key
// block instead of leaving waves idle: waves rb and rb + WPH / 2 of a head take the same 64
// rows, the first every key tile's first 32-key block and the second its second, each with its
// own running maximum, sums and accumulators, merged through LDS at the end of the tile. Each
// step then costs a wave half a full step's MFMAs and softmax. Only segments of more than 128
// keys split: below that the merge's four barriers cost more than the shorter steps save
// (measured on equal-length batches of 8 to 128 tokens). Whether a tile splits depends on its
// segment's lengths alone.
//
// Staging is the ring of tiled_attn_kernel: NS = 3 stages of one 64-key K tile and one V tile
// (16 KB), filled by direct global-to-LDS loads issued two steps ahead, out of the compiler's
// sight, completion waited for with one constant s_waitcnt vmcnt per step; the 64 query rows
// of a wave arrive through two "Q steps" of the same ring. Rows are XOR-swizzled in 16-byte
// units (swz) so ds_read_b128 is conflict-free. All global accesses go through buffer
// resources bounded by the segment: keys past its end read as zero, rows past its end are
// never written.
//
// Softmax: online, fp32, log2 domain. The running maximum m of each row is only a reference
// point shared by numerator and denominator: it is taken exactly on the query tile's first
// 32-key block, and every later block reuses it with no max at all. A half
// block that takes some row's probability sum under the stale m past 2^64 is scored again
// exactly before its P.V product (m raised, accumulators rescaled), so no probability that
// reaches the MFMAs can overflow. Probabilities are rounded to bf16 for P.V and the row sums
// add exactly those bf16 values (v_dot2 with ones, continuing the row's sum, so that accepting
// a half block is a register rename and its check one integer max and compare).
//
// Schedule of a full key tile (two 32-key blocks b0, b1) under the stale maximum, written so
// that each wave's MFMA chain always has an independent VALU phase beside it:
//   S_A0, S_B0 = K0 . Q_A, K0 . Q_B          (8 MFMA)
//   softmax A0 (VALU)                        || S_B0 in the matrix core
//   S_A1 = K1 . Q_A ; O_A += V0^T . P_A0     (8 MFMA)
//   softmax B0                               || S_A1, O_A
//   S_B1 = K1 . Q_B ; O_B += V0^T . P_B0     (8 MFMA)
//   softmax A1                               || S_B1, O_B
//   O_A += V1^T . P_A1 ; softmax B1 ; O_B += V1^T . P_B1
// The first key tile of a query tile takes the same schedule, its maximum seeded from block
// 0's scores. The segment's last, partial tile, and the rest of a tile in which a half block's
// softmax overflowed, take the exact path: half block by half block, scores recomputed from
// the stage, the straddling block masked, the maximum raised to cover them. The hot path
// therefore holds no second copy of any operand.
#pragma once

#include "pe_attn_stage.h"

namespace pe {

// log2 of the largest unnormalised probability the exact first tile lets stand before
// rescaling, and the largest per-row probability sum a half block may leave under a stale
// maximum (2^64).
constexpr float kG64LazyRescale = 8.0f;
constexpr float kG64OverflowGuard = 18446744073709551616.0f;

// max (or sum) of x over the lane pair (l, l ^ 32) that holds one query row. Only the exact
// path and the epilogue combine a pair, so the LDS-routed shuffle costs nothing measurable.
__device__ __forceinline__ float pair_max(float x) { return fmaxf(x, __shfl_xor(x, 32)); }
__device__ __forceinline__ float pair_sum(float x) { return x + __shfl_xor(x, 32); }

template <int G, bool GATE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void global64_attn_kernel(AttnParams p) {
    static_assert(G == 1 || G == 2 || G == 4, "query heads per workgroup");
    constexpr int D = 64, BN = 64, NS = 3;
    constexpr int WPH = 4 / G;     // waves per query head
    constexpr int BM = 64 * WPH;   // query rows per query tile
    constexpr int HALF = WPH > 1 ? WPH / 2 : 1;
    constexpr int CPR = D / 8;     // 16-byte units per K/V/Q row
    constexpr int TILE = BN * D;   // elements of one K (or V) tile
    constexpr int LPS = 4;         // 16-byte loads per lane and step: K 2 + V 2, or Q 4
    constexpr uint32_t kStageBytes = 2 * TILE * 2, kTileBytes = TILE * 2;
    constexpr uint32_t kQWaveBytes = 32 * D * 2;  // a wave's 32 query rows of one Q step

    __shared__ __attribute__((aligned(16))) __bf16 ring[NS][2][TILE];
    // A split tile's helper waves hand their row maxima and sums to the primaries here (their
    // accumulators go through the ring stage the tile's last step freed).
    __shared__ float merge_ml[2][4][64];

    const int item = blockIdx.x;
    const int entry = item / p.hgroups;
    const int hg = item - entry * p.hgroups;
    const WorkItem wi = load_work(p, entry);
    if (!wi.valid) return;
    const int qt_first = wi.qt_first;
    const int start = wi.start, L = wi.L;      // query rows
    const int kstart = wi.kstart, Lk = wi.Lk;  // keys (every row reads all of them)
    // A segment longer than the caller's max_seqlen breaks the contract the host sized the
    // 32-bit buffer offsets by: its rows are left unwritten rather than addressed.
    if (L > p.max_seqlen || Lk > p.max_seqlen_k || Lk < 0) return;
    const int nq = (L + BM - 1) / BM;
    if (qt_first >= nq) return;
    const int qt_end = min(nq, qt_first + p.strip);
    const int nkt = max(1, (Lk + BN - 1) / BN);  // key tiles of every query tile

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = uniform(tid >> 6);
    const int col = lane & 31, kg = lane >> 5;
    const int slot = wave / WPH, rb = wave - slot * WPH;
    // Split tiles (see the header): split_block(qt) is this wave's key block (0 or 1) in query
    // tile qt when the tile splits, else -1; row_group(qt) the 64-row group the wave computes.
    auto split_block = [&](int qt) {
        const int groups = (L - qt * BM + 63) / 64;
        return WPH >= 2 && Lk > 2 * BN && 2 * groups <= WPH ? rb / HALF : -1;
    };
    auto row_group = [&](int qt) { return split_block(qt) < 0 ? rb : rb % HALF; };
    const int qh = hg * G + slot;
    const int kvh = (hg * G) / p.group;

    const __amdgpu_buffer_rsrc_t q_rs = make_rsrc(p.q + (int64_t)start * p.q_st + (int64_t)qh * p.q_sh, rows_bytes(L, p.q_st, D));
    const __amdgpu_buffer_rsrc_t k_rs = make_rsrc(p.k + (int64_t)kstart * p.k_st + (int64_t)kvh * p.k_sh, rows_bytes(Lk, p.k_st, D));
    const __amdgpu_buffer_rsrc_t v_rs = make_rsrc(p.v + (int64_t)kstart * p.v_st + (int64_t)kvh * p.v_sh, rows_bytes(Lk, p.v_st, D));
    const __amdgpu_buffer_rsrc_t o_rs = make_rsrc(p.o + (int64_t)start * p.o_st + (int64_t)qh * p.o_sh, rows_bytes(L, p.o_st, D));
    __amdgpu_buffer_rsrc_t g_rs = o_rs;
    if constexpr (GATE) g_rs = make_rsrc(p.g + (int64_t)start * p.g_st + (int64_t)qh * p.g_sh, rows_bytes(L, p.g_st, D));
    const int q_row = (int)p.q_st * 2, k_row = (int)p.k_st * 2, v_row = (int)p.v_st * 2;

    // DMA geometry. K/V: wave-load j (j < 2) of this wave fills units [(2 wave + j) * 64, +64) of
    // a tile; unit u holds key u / CPR, global 16-byte column (u % CPR) ^ swz(key). Q step i: the
    // wave's rows 64 rb + 32 i + r (r < 32) fill its 4 KB region of the stage, unit j * 64 + lane
    // (j < 4) holding row r = unit / CPR, column (unit % CPR) ^ swz(r).
    int koff[2], voff[2], qoff[4];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int u = (wave * 2 + j) * 64 + lane;
        const int key = u / CPR, ch = (u % CPR) ^ swz<CPR>(key);
        koff[j] = key * k_row + ch * 16;
        voff[j] = key * v_row + ch * 16;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int u = j * 64 + lane;
        const int r = u / CPR, ch = (u % CPR) ^ swz<CPR>(r);
        qoff[j] = r * q_row + ch * 16;
    }
    const uint32_t ring_base = uniform((int)lds_addr(&ring[0][0][0]));
    auto issue_kv = [&](int stage, int kt0) {
        const uint32_t kb = ring_base + stage * kStageBytes + wave * 2048;
        const uint32_t lds[4] = {kb, kb + 1024, kb + kTileBytes, kb + kTileBytes + 1024};
        const int kbase = kt0 * k_row, vbase = kt0 * v_row;
        const int off[4] = {koff[0] + kbase, koff[1] + kbase, voff[0] + vbase, voff[1] + vbase};
        dma16x4(lds, off, k_rs, v_rs);
    };
    auto issue_q = [&](int stage, int qt, int i) {
        const uint32_t qb = ring_base + stage * kStageBytes + wave * kQWaveBytes;
        const uint32_t lds[4] = {qb, qb + 1024, qb + 2048, qb + 3072};
        const int base = (qt * BM + row_group(qt) * 64 + i * 32) * q_row;
        const int off[4] = {base + qoff[0], base + qoff[1], base + qoff[2], base + qoff[3]};
        dma16x4(lds, off, q_rs, q_rs);
    };

    // Per-lane LDS read offsets (elements within a tile). K (and a wave's Q rows): key 32 b + col,
    // unit 2 c + kg. V^T (ds_read_b64_tr_b16): in 16-lane group g = lane / 16, source lane
    // i = lane % 16 points at key 16 h + 4 (g / 2) + i / 4 (+ 8 for the operand's second half)
    // and dims 32 db + 16 (g % 2) + 4 (i % 4); the transpose hands lane (dim, kg) four keys of
    // its dim. Both swizzles see only key bits the block / 16-key-half offsets leave unchanged,
    // so every read is a per-lane base plus a compile-time offset.
    int kbase_c[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) kbase_c[c] = col * D + ((2 * c + kg) ^ swz<CPR>(col)) * 8;
    const int vi = lane & 15, vg = lane >> 4;
    const int vkey0 = 4 * (vg >> 1) + (vi >> 2);
    const int vdim0 = 16 * (vg & 1) + 4 * (vi & 3);
    int vbase[2][2];  // [second 4-key half of the operand][32-dim block]
#pragma unroll
    for (int half = 0; half < 2; ++half)
#pragma unroll
        for (int db = 0; db < 2; ++db) {
            const int key = 8 * half + vkey0, dim = 32 * db + vdim0;
            vbase[half][db] = key * D + (((dim >> 3) ^ swz<CPR>(key)) * 8) + (dim & 4);
        }

    const float c2 = p.c;

    // Loader: the next step to stage, NS - 1 steps ahead of the consumer; nothing past the
    // strip's last step. n_issued / n_begun count the steps staged and begun (wave-uniform).
    int ld_qt = qt_first, ld_t = -2;
    int n_issued = 0, n_begun = 0;
    auto issue_next = [&](int stage) {
        if (ld_qt >= qt_end) return;
        ++n_issued;
        if (ld_t < 0) issue_q(stage, ld_qt, ld_t + 2);
        else issue_kv(stage, ld_t * BN);
        if (++ld_t >= nkt) {
            ++ld_qt;
            ld_t = -2;
        }
    };
#pragma unroll
    for (int st = 0; st < NS - 1; ++st) issue_next(st);

    // A step's loads are complete once at most the following step's LPS loads are in flight
    // (loads complete in issue order; outstanding output stores only make the wait stricter),
    // or none when no following step was staged: the strip's last step leaves no load in
    // flight, so the workgroup ends without draining its output stores. Exact for NS = 3, where at
    // most one following step is in flight; a deeper ring would need a wait sized by the steps
    // actually in flight.
    int stage = 0;
    auto begin_step = [&]() {
        if (n_issued > n_begun + 1) wait_vmcnt<(NS - 2) * LPS>();
        else wait_vmcnt<0>();
        ++n_begun;
        __syncthreads();
        issue_next(stage == 0 ? NS - 1 : stage - 1);
    };
    auto end_step = [&]() { stage = stage == NS - 1 ? 0 : stage + 1; };

    bf16x8 qf[2][4];
    for (int qt = qt_first; qt < qt_end; ++qt) {
        const int kb_only = split_block(qt);  // >= 0 on every wave of a split tile
        const int r0 = qt * BM + row_group(qt) * 64;  // the wave's first row
        const bool wave_active = r0 < L;

        // Q steps: half i of the wave's rows; the empty asm ends the reads' scope before the
        // next barrier frees the stage.
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            begin_step();
            const __bf16 *qs = &ring[stage][0][0] + wave * (kQWaveBytes / 2);
#pragma unroll
            for (int c = 0; c < 4; ++c) qf[i][c] = ld_s16(qs + kbase_c[c]);
#pragma unroll
            for (int c = 0; c < 4; ++c) asm volatile("" : "+v"(qf[i][c]));
            end_step();
        }

        f32x16 o[2][2];
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
            for (int db = 0; db < 2; ++db)
#pragma unroll
                for (int j = 0; j < 16; ++j) o[x][db][j] = 0.0f;
        float m[2] = {kNegInf, kNegInf};
        float nm[2] = {0.0f, 0.0f};  // -m, or 0 while m is -inf
        float ls[2][2] = {{0.0f, 0.0f}, {0.0f, 0.0f}};

        // S^T of one 32-key block for half x: K operands k4 (shared by both halves).
        auto qk = [&](const bf16x8 (&k4)[4], int x) {
            f32x16 acc;
#pragma unroll
            for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
#pragma unroll
            for (int c = 0; c < 4; ++c) acc = mfma32(k4[c], qf[x][c], acc);
            return acc;
        };
        auto load_k = [&](const __bf16 *kt, int b, bf16x8 (&k4)[4]) {
#pragma unroll
            for (int c = 0; c < 4; ++c) k4[c] = ld_s16(kt + 32 * b * D + kbase_c[c]);
        };
        // V^T operands of block b: [16-key half][32-dim block].
        auto load_v = [&](const __bf16 *vt, int b, bf16x8 (&v4)[2][2]) {
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int db = 0; db < 2; ++db) {
                    const bf16x4 lo = tr16(vt + (32 * b + 16 * h) * D + vbase[0][db]);
                    const bf16x4 hi = tr16(vt + (32 * b + 16 * h) * D + vbase[1][db]);
                    v4[h][db] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                }
        };
        auto pv = [&](const bf16x8 (&v4)[2][2], const bf16x8 (&pb)[2], int x) {
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int db = 0; db < 2; ++db) o[x][db] = mfma32(v4[h][db], pb[h], o[x][db]);
        };
        // Raise half x's maximum to cover scores s (keeping it when they stay within 2^8 of it),
        // rescaling its accumulators.
        auto raise_max = [&](const f32x16 &s, int x) {
            float mp[4] = {kNegInf, kNegInf, kNegInf, kNegInf};
#pragma unroll
            for (int j = 0; j < 16; ++j) mp[j & 3] = fmaxf(mp[j & 3], s[j]);
            const float mx = fmaxf(fmaxf(mp[0], mp[1]), fmaxf(mp[2], mp[3]));
            if (wave_any(mx * c2 > m[x] + kG64LazyRescale)) {
                const float mnew = fmaxf(m[x], pair_max(mx) * c2);
                const float alpha = mnew == kNegInf ? 1.0f : exp2_fast(m[x] - mnew);
                m[x] = mnew;
                nm[x] = mnew == kNegInf ? 0.0f : -mnew;
                ls[x][0] *= alpha;
                ls[x][1] *= alpha;
#pragma unroll
                for (int db = 0; db < 2; ++db)
#pragma unroll
                    for (int j = 0; j < 16; ++j) o[x][db][j] *= alpha;
            }
        };
        // Probabilities of scores s under half x's m, computed in place (s is consumed): bf16
        // operands pb and their fp32 sums.
        auto probs = [&](f32x16 &s, int x, bf16x8 (&pb)[2], float &st0, float &st1) {
#pragma unroll
            for (int j = 0; j < 16; ++j) s[j] = exp2_fast(fmaf(s[j], c2, nm[x]));
            pb[0] = to_bf16x8(s, 0);
            pb[1] = to_bf16x8(s, 8);
            st0 = sum2_first(pb[0], 0);
            st1 = sum2_first(pb[0], 1);
            st0 = sum2(pb[0], 2, st0);
            st1 = sum2(pb[0], 3, st1);
            st0 = sum2(pb[1], 0, st0);
            st1 = sum2(pb[1], 1, st1);
            st0 = sum2(pb[1], 2, st0);
            st1 = sum2(pb[1], 3, st1);
        };
        // The exact path, over half blocks [from, to) (2 b + x) of the stage's key tile:
        // scores recomputed from the stage (blocks past the keys skipped, the straddling block
        // masked), the maximum raised to cover them, probabilities, P.V. It serves the segment's
        // last, partial key tile (the first one too when the segment has fewer than 64 keys) and
        // the rest of a full tile whose stale-maximum softmax overflowed (whose earlier half
        // blocks are already added).
        auto exact_from = [&](const __bf16 *kt, const __bf16 *vt, int kt0, int from, int to) {
#pragma unroll 1
            for (int hb = from; hb < to; ++hb) {
                const int b = hb >> 1, x = hb & 1;
                const int kb0 = kt0 + 32 * b;
                if (kb0 >= Lk) break;
                bf16x8 k4[4], v4[2][2], px[2];
                load_k(kt, b, k4);
                f32x16 s = x ? qk(k4, 1) : qk(k4, 0);
                if (kb0 + 32 > Lk) {
                    const uint32_t km = key_mask(kb0, kg, 0, Lk, -1, -1);
#pragma unroll
                    for (int j = 0; j < 16; ++j) s[j] = mask_score(s[j], km, acc_key(j, 0));
                }
                float st0, st1;
                if (x) {
                    raise_max(s, 1);
                    probs(s, 1, px, st0, st1);
                    ls[1][0] += st0;
                    ls[1][1] += st1;
                    load_v(vt, b, v4);
                    pv(v4, px, 1);
                } else {
                    raise_max(s, 0);
                    probs(s, 0, px, st0, st1);
                    ls[0][0] += st0;
                    ls[0][1] += st1;
                    load_v(vt, b, v4);
                    pv(v4, px, 0);
                }
            }
        };
        // Half x's running maximum taken from scores s (a query tile's first block; every row
        // has a key there): the reference point of the stale softmax that follows.
        auto seed_max = [&](const f32x16 &s, int x) {
            float mp[4] = {kNegInf, kNegInf, kNegInf, kNegInf};
#pragma unroll
            for (int j = 0; j < 16; ++j) mp[j & 3] = fmaxf(mp[j & 3], s[j]);
            m[x] = pair_max(fmaxf(fmaxf(mp[0], mp[1]), fmaxf(mp[2], mp[3]))) * c2;
            nm[x] = -m[x];
        };
        // Probabilities of a half block under half x's stale m, computed in place, with the row
        // sums continued from ls[x] into st0 / st1 (ls itself kept for the check below).
        auto probs_onto = [&](f32x16 &s, int x, bf16x8 (&pb)[2], float &st0, float &st1) {
#pragma unroll
            for (int j = 0; j < 16; ++j) s[j] = exp2_fast(fmaf(s[j], c2, nm[x]));
            pb[0] = to_bf16x8(s, 0);
            pb[1] = to_bf16x8(s, 8);
            st0 = sum2_from(pb[0], 0, ls[x][0]);
            st1 = sum2_from(pb[0], 1, ls[x][1]);
            st0 = sum2(pb[0], 2, st0);
            st1 = sum2(pb[0], 3, st1);
            st0 = sum2(pb[1], 0, st0);
            st1 = sum2(pb[1], 1, st1);
            st0 = sum2(pb[1], 2, st0);
            st1 = sum2(pb[1], 3, st1);
        };
        // Softmax check of a half block: false when some row's sums with it pass the guard
        // (nothing taken: the exact path redoes the half block from ls), else they become the
        // row sums. Sums of earlier accepted half blocks stay far below the guard unless a row's
        // scores rose by ~60 log2 units, which the exact path then meets once and rescales. The
        // sums are non-negative or NaN, so their bit patterns compare as integers in the order of
        // their values (NaN above the guard): one integer max and compare, with none of the
        // canonicalising moves a float max takes.
        auto accept = [&](int x, float st0, float st1) {
            const int guard = __float_as_int(kG64OverflowGuard);
            if (wave_any(max(__float_as_int(st0), __float_as_int(st1)) > guard)) return false;
            ls[x][0] = st0;
            ls[x][1] = st1;
            return true;
        };
        // A full key tile in the pipelined order, under the stale maximum. Returns 4 when done,
        // else the half block (2 b + x) whose softmax overflowed: it and everything after it are
        // left to exact_from. Each region between checks issues its MFMAs one at a time between
        // groups of the independent softmax VALU work (sched_group_barrier: 0x008 MFMA, 0x002
        // VALU, 0x100 LDS read), so the wave keeps the matrix core fed while it computes
        // probabilities; sched_barrier fences the regions.
        auto pipelined_tile = [&](bool first, const __bf16 *kt, const __bf16 *vt) -> int {
            bf16x8 k4[4], v4[2][2], pa[2], pbb[2];
            float st0, st1;
            // R0: S_A0, then S_B0 with softmax A0 under it. A query tile's first key tile seeds
            // the stale maximum of each half from these scores (half A once S_A0 is done, half
            // B after the check), a uniform branch at the region's edges.
            load_k(kt, 0, k4);
            f32x16 sa = qk(k4, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (first) seed_max(sa, 0);
            __builtin_amdgcn_sched_barrier(0);
            f32x16 sb = qk(k4, 1);
            probs_onto(sa, 0, pa, st0, st1);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (!accept(0, st0, st1)) return 0;
            if (first) seed_max(sb, 1);
            __builtin_amdgcn_sched_barrier(0);
            // R1: S_A1, O_A += V0 P_A0; softmax B0 under them.
            load_k(kt, 1, k4);
            load_v(vt, 0, v4);
            sa = qk(k4, 0);
            pv(v4, pa, 0);
            probs_onto(sb, 1, pbb, st0, st1);
            __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 10, 0);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (!accept(1, st0, st1)) return 1;
            __builtin_amdgcn_sched_barrier(0);
            // R2: S_B1, O_B += V0 P_B0; softmax A1 under them.
            sb = qk(k4, 1);
            pv(v4, pbb, 1);
            probs_onto(sa, 0, pa, st0, st1);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (!accept(0, st0, st1)) return 2;
            __builtin_amdgcn_sched_barrier(0);
            // R3: O_A += V1 P_A1; softmax B1 under it.
            load_v(vt, 1, v4);
            pv(v4, pa, 0);
            probs_onto(sb, 1, pbb, st0, st1);
            __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 14, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 9, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (!accept(1, st0, st1)) return 3;
            __builtin_amdgcn_sched_barrier(0);
            // R4: O_B += V1 P_B1.
            pv(v4, pbb, 1);
            return 4;
        };

        // One 32-key block b of a full key tile for both halves, the split tile's share of it,
        // in the same pipelined order under the stale maximum (seeded from block b on the
        // query tile's first key tile). Returns 4 when done, else the half block whose softmax
        // overflowed.
        auto pipelined_block = [&](bool first, const __bf16 *kt, const __bf16 *vt, int b) -> int {
            bf16x8 k4[4], v4[2][2], pa[2], pbb[2];
            float st0, st1;
            load_k(kt, b, k4);
            f32x16 sa = qk(k4, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (first) seed_max(sa, 0);
            __builtin_amdgcn_sched_barrier(0);
            f32x16 sb = qk(k4, 1);
            probs_onto(sa, 0, pa, st0, st1);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (!accept(0, st0, st1)) return 2 * b;
            if (first) seed_max(sb, 1);
            __builtin_amdgcn_sched_barrier(0);
            load_v(vt, b, v4);
            pv(v4, pa, 0);
            probs_onto(sb, 1, pbb, st0, st1);
            __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 14, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 9, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (!accept(1, st0, st1)) return 2 * b + 1;
            __builtin_amdgcn_sched_barrier(0);
            pv(v4, pbb, 1);
            return 4;
        };

        if (kb_only < 0) {
            for (int t = 0; t < nkt; ++t) {
                begin_step();
                if (wave_active) {
                    const __bf16 *kt = &ring[stage][0][0];
                    const __bf16 *vt = &ring[stage][1][0];
                    const int kt0 = t * BN;
                    int from = 0;
                    if (kt0 + BN <= Lk) {
                        // A query tile's first key tile seeds the stale maximum from its first
                        // block's scores inside the pipelined schedule.
                        from = pipelined_tile(t == 0, kt, vt);
                    }
                    if (from < 4) exact_from(kt, vt, kt0, from, 4);
                }
                end_step();
            }
        } else {
            // A split tile: this wave's block of every key tile.
            for (int t = 0; t < nkt; ++t) {
                begin_step();
                if (wave_active) {
                    const __bf16 *kt = &ring[stage][0][0];
                    const __bf16 *vt = &ring[stage][1][0];
                    const int kt0 = t * BN;
                    int from = 2 * kb_only;
                    if (kt0 + BN <= Lk) from = pipelined_block(t == 0, kt, vt, kb_only);
                    if (from < 2 * kb_only + 2) exact_from(kt, vt, kt0, from, 2 * kb_only + 2);
                }
                end_step();
            }
        }

        // A split tile's halves meet: the helpers (second key block) hand their maxima, sums
        // and accumulators to the primaries through LDS, half x at a time through the stage
        // the last step read (no load is in flight to it until the next step begins, after
        // a barrier). Every wave of the workgroup takes the branch and its barriers.
        if (kb_only >= 0) {
            float *xb = reinterpret_cast<float *>(&ring[stage == 0 ? NS - 1 : stage - 1][0][0]);
            const int mg = slot * HALF + row_group(qt);  // the pair's merge buffer (< 2)
            const bool helper = wave_active && kb_only == 1;
            const bool primary = wave_active && kb_only == 0;
            __syncthreads();
            if (helper) {
                merge_ml[mg][0][lane] = m[0];
                merge_ml[mg][1][lane] = m[1];
                merge_ml[mg][2][lane] = ls[0][0] + ls[0][1];
                merge_ml[mg][3][lane] = ls[1][0] + ls[1][1];
            }
#pragma unroll
            for (int x = 0; x < 2; ++x) {
                f32x4 *buf = reinterpret_cast<f32x4 *>(xb) + mg * 512;  // 8 KB per pair
                if (helper) {
#pragma unroll
                    for (int db = 0; db < 2; ++db)
#pragma unroll
                        for (int c = 0; c < 4; ++c)
                            buf[(db * 4 + c) * 64 + lane] = f32x4{o[x][db][4 * c], o[x][db][4 * c + 1],
                                                                  o[x][db][4 * c + 2], o[x][db][4 * c + 3]};
                }
                __syncthreads();
                if (primary) {
                    const float mh = merge_ml[mg][x][lane], lh = merge_ml[mg][2 + x][lane];
                    const float mn = fmaxf(m[x], mh);
                    const float ap = m[x] > kNegInf ? exp2_fast(m[x] - mn) : 0.0f;
                    const float ah = mh > kNegInf ? exp2_fast(mh - mn) : 0.0f;
                    ls[x][0] = (ls[x][0] + ls[x][1]) * ap + lh * ah;
                    ls[x][1] = 0.0f;
#pragma unroll
                    for (int db = 0; db < 2; ++db)
#pragma unroll
                        for (int c = 0; c < 4; ++c) {
                            const f32x4 h = buf[(db * 4 + c) * 64 + lane];
#pragma unroll
                            for (int e = 0; e < 4; ++e) o[x][db][4 * c + e] = o[x][db][4 * c + e] * ap + h[e] * ah;
                        }
                }
                if (x == 0) __syncthreads();
            }
        }

        // Normalise, apply the gate, store both halves.
        if (wave_active && kb_only != 1) {
#pragma unroll
            for (int x = 0; x < 2; ++x) {
                const float lt = pair_sum(ls[x][0] + ls[x][1]);
                const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
                const int row = r0 + 32 * x + col;
                const int ooff = row * (int)p.o_st * 2;
                const int goff = GATE ? row * (int)p.g_st * 2 : 0;
                store_block<2, GATE>(o[x], inv, kg, o_rs, ooff, g_rs, goff);
            }
        }
    }
}

}  // namespace pe
