// Device-side work planning for the tiled kernel: no host read of cu_seqlens, capture-safe.
//
// One 1024-thread workgroup reads cu_seqlens, keeps the segments longer than short_max, splits
// each into BM-row query tiles grouped in strips of `strip` consecutive tiles, and writes
// (segment, first tile) entries ordered by decreasing cost (keys the strip's tiles visit: the
// whole segment, its band, or its causal prefix, per tile). Costs are bucketed at half-octave
// resolution, a counting sort in LDS, so the tiled grid dispatches the longest-running strips
// first (longest-processing-time order) and the tail is made of short strips. Consecutive
// strips of a segment with equal cost stay adjacent, so a segment's K/V is read by
// neighbouring workgroups. With `group` set, the unit of ordering is the whole segment:
// its strips are one contiguous reservation (costliest strip first), bucketed by the
// segment's total cost, so a run of neighbouring workgroups holds every query tile of a
// segment and re-reads its keys from one L2 (the head_dim 128 and 256 kernels deal such runs
// to the XCDs). Order within a bucket depends on atomics; it changes only the schedule,
// never a result: every output row is produced by exactly one workgroup.
#pragma once

#include "pe_attn_device.h"

namespace pe {

// Keys query tile t of a segment with L query rows and Lk keys visits (rows end-aligned to
// the keys: row r sits at key position r + Lk - L).
__device__ __forceinline__ int plan_tile_cost(int t, int bm, int L, int Lk, int wl, int wr) {
    const int off = Lk - L;
    const int r0 = t * bm + off, r1 = min(L, t * bm + bm) + off;
    const int klo = wl >= 0 ? max(0, r0 - wl) : 0;
    const int khi = wr >= 0 ? min(Lk, r1 + wr) : Lk;
    return max(1, khi - klo);
}

// Keys visited by query tiles [t0, t1) of a segment of nq tiles. Two shapes have a closed form:
// global (every tile visits all Lk keys) and causal with no left window (tile t visits the keys
// up to its last row, (t + 1) bm + off, the last tile up to Lk); others add tile by tile.
__device__ __forceinline__ int64_t plan_tiles_cost(int t0, int t1, int nq, int bm, int L, int Lk, int wl, int wr) {
    if (t1 <= t0) return 0;
    if (wl < 0 && wr < 0) return (int64_t)(t1 - t0) * max(1, Lk);
    const int off = Lk - L;
    if (wl < 0 && wr == 0 && off >= 0) {
        const int64_t a = t0, b = min(t1, nq - 1);  // full tiles [a, b): sum of (t + 1) bm + off
        int64_t cost = b > a ? (int64_t)bm * (b * (b + 1) / 2 - a * (a + 1) / 2) + (b - a) * off : 0;
        if (t1 >= nq) cost += Lk;  // the last tile reaches every key
        return cost;
    }
    int64_t cost = 0;
    for (int t = t0; t < t1; ++t) cost += plan_tile_cost(t, bm, L, Lk, wl, wr);
    return cost;
}

// Keys visited by the query tiles [s * strip, min(nq, (s + 1) * strip)) of a segment.
__device__ __forceinline__ int plan_strip_cost(int s, int strip, int nq, int bm, int L, int Lk, int wl, int wr) {
    const int64_t cost = plan_tiles_cost(s * strip, min(nq, (s + 1) * strip), nq, bm, L, Lk, wl, wr);
    return (int)min(cost, (int64_t)0x7fffffff);
}

// Keys visited by all strips of a segment.
__device__ __forceinline__ int plan_segment_cost(int nq, int bm, int L, int Lk, int wl, int wr) {
    return (int)min(plan_tiles_cost(0, nq, nq, bm, L, Lk, wl, wr), (int64_t)0x7fffffff);
}

// Strips [s_lo, s_hi) whose tiles all visit the same number of keys: every full tile of a global
// call, or the full tiles of a two-sided window that reach neither end of the keys
// (cost bm + wl + wr). Empty (s_lo >= s_hi) for other shapes.
__device__ __forceinline__ void plan_flat_strips(int strip, int bm, int L, int Lk, int wl, int wr, int &s_lo,
                                                 int &s_hi) {
    s_lo = s_hi = 0;
    const bool global = wl < 0 && wr < 0, band = wl >= 0 && wr >= 0;
    if (!global && !band) return;
    const int off = Lk - L;
    int t_lo = 0, t_hi = L / bm;  // full tiles: (t + 1) bm <= L
    if (band) {
        t_lo = wl - off > 0 ? (wl - off + bm - 1) / bm : 0;           // t bm + off >= wl
        t_hi = L - wr > 0 ? min(t_hi, (L - wr) / bm) : 0;              // (t + 1) bm + off + wr <= Lk
    }
    s_lo = (t_lo + strip - 1) / strip;
    s_hi = t_hi / strip;
}

__device__ __forceinline__ int plan_bucket(int cost) {
    const int lg = 31 - __clz(cost);
    const int half = lg >= 1 ? (cost >> (lg - 1)) & 1 : 0;
    return min(63, 2 * lg + half);
}

// Segments of more than kSerialStrips strips are planned by a whole wave, lanes over strips
// (a thread per segment walked a 64-strip segment serially: ~20 us for C4's 16 segments); up
// to kWaveQueue of them are queued in LDS with their lengths (a wave then reads no global
// memory per segment), and past that every segment is planned serially. Shorter segments stay
// one per thread: a wave's pass over one segment is a chain of LDS round trips (~1.5 us), so
// C5's 256 segments of up to 32 strips took 40 us by waves against 13 us by threads.
constexpr int kSerialStrips = 32;
constexpr int kWaveQueue = 2048;
constexpr int kCachedBounds = 4096;  // segments whose boundaries the plan keeps in LDS

// One entry per strip of `strip` consecutive query tiles of `bm` rows: (segment, first tile,
// the segment's first query row, its query rows), so a kernel reads a work item's bounds with
// the entry itself.
// Segment s has cu[s + 1] - cu[s] query rows and cuk[s + 1] - cuk[s] keys (cuk = cu when the
// two share boundaries); it is the short kernel's when both fit short_max. A segment longer
// than the caller's max_seqlen (or whose keys exceed max_seqlen_k) breaks the contract the
// host sized the list and the kernels' 32-bit offsets by: it takes no entry (the tiled
// kernels would skip it anyway), so it can never push a valid segment's strips out of the
// list. Pass 1 counts entries per cost bucket, pass 2 reserves contiguous runs and writes
// them; both passes plan each segment the same way (serially or by a wave), and a run's
// reservation is the same in either.
//
// count[0] receives the number of entries written, min(needed, cap); count[1] the number
// needed. They differ only when the caller's sizes break the contract that sized cap
// (cu_seqlens decreasing, or past total_tokens): the excess entries are then dropped, and
// count[1] > count[0] records it where a caller can read it.
__global__ __launch_bounds__(1024) void plan_kernel(const int32_t *cu, const int32_t *cuk, int n_seq, int short_max,
                                                    int max_seqlen, int max_seqlen_k, int bm, int strip, int wl,
                                                    int wr, int group, int4 *work, int32_t *count, int cap) {
    __shared__ int cnt[64];
    __shared__ int off[64];
    __shared__ int4 queue[kWaveQueue];  // (segment, query rows, keys, query start)
    __shared__ int queued;
    __shared__ int cu_s[kCachedBounds + 1], cuk_s[kCachedBounds + 1];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
    // The boundaries are read from global memory once, into LDS (up to kCachedBounds segments):
    // every later pass reads them there instead of paying a dependent global load each.
    const bool cached = n_seq <= kCachedBounds;
    if (cached) {
        for (int i = tid; i <= n_seq; i += blockDim.x) {
            cu_s[i] = cu[i];
            cuk_s[i] = cuk[i];
        }
    }
    if (tid < 64) cnt[tid] = 0;
    if (tid == 0) queued = 0;
    __syncthreads();
    auto bound = [&](int i) { return cached ? cu_s[i] : cu[i]; };
    auto bound_k = [&](int i) { return cached ? cuk_s[i] : cuk[i]; };

    // A segment with no query rows has nothing to plan; one outside the contract takes no entry.
    auto strips_of = [&](int seg, int &L, int &Lk, int &nq, int &ns) {
        L = bound(seg + 1) - bound(seg);
        Lk = bound_k(seg + 1) - bound_k(seg);
        nq = (L + bm - 1) / bm;
        ns = (nq + strip - 1) / strip;
        if (L <= 0 || Lk < 0 || L > max_seqlen || Lk > max_seqlen_k) return false;
        return max(L, Lk) > short_max;  // the tiled kernel's
    };
    for (int seg = tid; seg < n_seq; seg += blockDim.x) {
        int L, Lk, nq, ns;
        if (strips_of(seg, L, Lk, nq, ns) && ns > kSerialStrips) {
            const int qi = atomicAdd(&queued, 1);
            if (qi < kWaveQueue) queue[qi] = make_int4(seg, L, Lk, bound(seg));
        }
    }
    __syncthreads();
    const bool by_wave = queued <= kWaveQueue;  // else every segment serially
    const int nqueued = by_wave ? queued : 0;

    // One thread plans segment seg: pass 1 (place = false) counts, pass 2 writes.
    auto serial_segment = [&](int seg, bool place) {
        int L, Lk, nq, ns;
        if (!strips_of(seg, L, Lk, nq, ns) || (by_wave && ns > kSerialStrips)) return;
        if (group) {
            const int b = plan_bucket(plan_segment_cost(nq, bm, L, Lk, wl, wr));
            if (!place) {
                atomicAdd(&cnt[b], ns);
                return;
            }
            // Strips in decreasing cost: the causal / end-aligned prefix grows with the strip.
            const int pos = atomicAdd(&off[b], ns);
            const bool rev =
                plan_strip_cost(ns - 1, strip, nq, bm, L, Lk, wl, wr) > plan_strip_cost(0, strip, nq, bm, L, Lk, wl, wr);
            const int start = bound(seg);
            for (int i = 0; i < ns; ++i)
                if (pos + i < cap) work[pos + i] = make_int4(seg, (rev ? ns - 1 - i : i) * strip, start, L);
            return;
        }
        const int start = bound(seg);
        int s_lo, s_hi;  // strips of equal cost: a run crosses them in one step
        plan_flat_strips(strip, bm, L, Lk, wl, wr, s_lo, s_hi);
        int s = 0;
        while (s < ns) {
            // A run of consecutive strips in one cost bucket gets one contiguous reservation.
            const int b = plan_bucket(plan_strip_cost(s, strip, nq, bm, L, Lk, wl, wr));
            int e = s + 1;
            while (e < ns && plan_bucket(plan_strip_cost(e, strip, nq, bm, L, Lk, wl, wr)) == b)
                e = e >= s_lo && e < s_hi ? s_hi : e + 1;
            if (!place) {
                atomicAdd(&cnt[b], e - s);
            } else {
                const int pos = atomicAdd(&off[b], e - s);
                for (int i = 0; i < e - s; ++i)
                    if (pos + i < cap) work[pos + i] = make_int4(seg, (s + i) * strip, start, L);
            }
            s = e;
        }
    };
    // A wave plans segment seg (wave-uniform), lane i taking strips i, i + 64, ...: runs of
    // equal buckets within each 64-strip chunk are found with a ballot, one atomic per run.
    auto wave_segment = [&](int4 q, bool place) {
        const int seg = q.x, L = q.y, Lk = q.z, row0 = q.w;
        const int nq = (L + bm - 1) / bm;
        const int ns = (nq + strip - 1) / strip;
        if (group) {
            int64_t c = 0;
            for (int s = lane; s < ns; s += 64) c += plan_strip_cost(s, strip, nq, bm, L, Lk, wl, wr);
#pragma unroll
            for (int d = 32; d >= 1; d >>= 1) c += __shfl_xor(c, d);
            const int b = plan_bucket((int)min(c, (int64_t)0x7fffffff));
            int pos = 0;
            if (lane == 0) pos = place ? atomicAdd(&off[b], ns) : atomicAdd(&cnt[b], ns);
            if (!place) return;
            pos = __shfl(pos, 0);
            const bool rev =
                plan_strip_cost(ns - 1, strip, nq, bm, L, Lk, wl, wr) > plan_strip_cost(0, strip, nq, bm, L, Lk, wl, wr);
            for (int i = lane; i < ns; i += 64)
                if (pos + i < cap) work[pos + i] = make_int4(seg, (rev ? ns - 1 - i : i) * strip, row0, L);
            return;
        }
        for (int s0 = 0; s0 < ns; s0 += 64) {
            const int s = s0 + lane;
            const bool valid = s < ns;
            const int b = valid ? plan_bucket(plan_strip_cost(s, strip, nq, bm, L, Lk, wl, wr)) : -1;
            const int prev = __shfl_up(b, 1);
            const bool start = valid && (lane == 0 || b != prev);
            const uint64_t starts = __ballot(start);
            const uint64_t after = lane == 63 ? 0ull : starts >> (lane + 1);
            const int next = after ? lane + __ffsll((long long)after) : min(64, ns - s0);
            int pos = 0;
            if (start) pos = place ? atomicAdd(&off[b], next - lane) : atomicAdd(&cnt[b], next - lane);
            if (!place) continue;
            const uint64_t upto = starts & (lane == 63 ? ~0ull : (2ull << lane) - 1);
            const int rs = 63 - __clzll((long long)upto);  // this lane's run start
            const int p0 = __shfl(pos, rs);
            if (valid && p0 + (lane - rs) < cap) work[p0 + lane - rs] = make_int4(seg, s * strip, row0, L);
        }
    };

    for (int seg = tid; seg < n_seq; seg += blockDim.x) serial_segment(seg, false);
    for (int i = wave; i < nqueued; i += nwaves) wave_segment(queue[i], false);
    __syncthreads();
    // Bucket offsets, costliest bucket first: lane i of wave 0 holds bucket 63 - i, and an
    // inclusive shuffle scan over the wave gives each its start (a serial walk over the 64
    // buckets was a chain of 64 dependent LDS round trips).
    if (wave == 0) {
        const int c = cnt[63 - lane];
        int incl = c;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int up = __shfl_up(incl, d);
            if (lane >= d) incl += up;
        }
        off[63 - lane] = incl - c;
        if (lane == 63) {
            count[0] = min(incl, cap);
            count[1] = incl;
        }
    }
    __syncthreads();
    for (int seg = tid; seg < n_seq; seg += blockDim.x) serial_segment(seg, true);
    for (int i = wave; i < nqueued; i += nwaves) wave_segment(queue[i], true);
}

}  // namespace pe
