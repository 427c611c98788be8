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
// segment and re-reads its keys from one L2 (the head_dim 128 / 256 kernel deals such runs
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

// Keys visited by the query tiles [s * strip, min(nq, (s + 1) * strip)) of a segment.
__device__ __forceinline__ int plan_strip_cost(int s, int strip, int nq, int bm, int L, int Lk, int wl, int wr) {
    int64_t cost = 0;
    for (int t = s * strip; t < min(nq, (s + 1) * strip); ++t) cost += plan_tile_cost(t, bm, L, Lk, wl, wr);
    return (int)min(cost, (int64_t)0x7fffffff);
}

// Keys visited by all strips of a segment.
__device__ __forceinline__ int plan_segment_cost(int ns, int strip, int nq, int bm, int L, int Lk, int wl, int wr) {
    int64_t cost = 0;
    for (int s = 0; s < ns; ++s) cost += plan_strip_cost(s, strip, nq, bm, L, Lk, wl, wr);
    return (int)min(cost, (int64_t)0x7fffffff);
}

__device__ __forceinline__ int plan_bucket(int cost) {
    const int lg = 31 - __clz(cost);
    const int half = lg >= 1 ? (cost >> (lg - 1)) & 1 : 0;
    return min(63, 2 * lg + half);
}

// One entry per strip of `strip` consecutive query tiles of `bm` rows: (segment, first tile).
// Segment s has cu[s + 1] - cu[s] query rows and cuk[s + 1] - cuk[s] keys (cuk = cu when the
// two share boundaries); it is the short kernel's when both fit short_max.
__global__ __launch_bounds__(1024) void plan_kernel(const int32_t *cu, const int32_t *cuk, int n_seq, int short_max,
                                                    int bm, int strip, int wl, int wr, int group, int2 *work,
                                                    int32_t *count, int cap) {
    __shared__ int cnt[64];
    __shared__ int off[64];
    const int tid = threadIdx.x;
    if (tid < 64) cnt[tid] = 0;
    __syncthreads();
    for (int seg = tid; seg < n_seq; seg += blockDim.x) {
        const int L = cu[seg + 1] - cu[seg], Lk = cuk[seg + 1] - cuk[seg];
        if (max(L, Lk) <= short_max) continue;
        const int nq = (L + bm - 1) / bm;
        const int ns = (nq + strip - 1) / strip;
        if (group) {
            atomicAdd(&cnt[plan_bucket(plan_segment_cost(ns, strip, nq, bm, L, Lk, wl, wr))], ns);
            continue;
        }
        for (int s = 0; s < ns; ++s) atomicAdd(&cnt[plan_bucket(plan_strip_cost(s, strip, nq, bm, L, Lk, wl, wr))], 1);
    }
    __syncthreads();
    if (tid == 0) {
        int run = 0;
        for (int b = 63; b >= 0; --b) {
            off[b] = run;
            run += cnt[b];
        }
        *count = min(run, cap);
    }
    __syncthreads();
    for (int seg = tid; seg < n_seq; seg += blockDim.x) {
        const int L = cu[seg + 1] - cu[seg], Lk = cuk[seg + 1] - cuk[seg];
        if (max(L, Lk) <= short_max) continue;
        const int nq = (L + bm - 1) / bm;
        const int ns = (nq + strip - 1) / strip;
        if (group) {
            // Strips in decreasing cost: the causal / end-aligned prefix grows with the strip.
            const int pos = atomicAdd(&off[plan_bucket(plan_segment_cost(ns, strip, nq, bm, L, Lk, wl, wr))], ns);
            const bool rev =
                plan_strip_cost(ns - 1, strip, nq, bm, L, Lk, wl, wr) > plan_strip_cost(0, strip, nq, bm, L, Lk, wl, wr);
            for (int i = 0; i < ns; ++i)
                if (pos + i < cap) work[pos + i] = make_int2(seg, (rev ? ns - 1 - i : i) * strip);
            continue;
        }
        int s = 0;
        while (s < ns) {
            // A run of consecutive strips in one cost bucket gets one contiguous reservation.
            const int b = plan_bucket(plan_strip_cost(s, strip, nq, bm, L, Lk, wl, wr));
            int e = s + 1;
            while (e < ns && plan_bucket(plan_strip_cost(e, strip, nq, bm, L, Lk, wl, wr)) == b) ++e;
            const int pos = atomicAdd(&off[b], e - s);
            for (int i = 0; i < e - s; ++i)
                if (pos + i < cap) work[pos + i] = make_int2(seg, (s + i) * strip);
            s = e;
        }
    }
}

}  // namespace pe
