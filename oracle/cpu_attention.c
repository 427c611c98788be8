// CPU packed attention, FP32 + OpenMP — TEST INFRASTRUCTURE / CPU BASELINE ONLY (see
// oracle/__init__.py). Restates the decomposition of the reference's native CPU attention
// (packed_encoders/cpu/local_attention_x86.c:132-234, driven by cpu/attention.py:394-440):
//  - inputs head-major [heads][tokens][head_dim]; output head-major, or token-major
//    [tokens][heads * head_dim] when token_major is set;
//  - sequences delimited by lengths; one task per (head, sequence), scheduled dynamically;
//  - queries in tiles of `tile` rows; each tile copies its key window [lo, hi) transposed so a
//    row's scores are axpy sweeps over the window; a row reads keys with |i - j| <= half inside
//    its sequence, so half >= the longest length is global attention;
//  - unnormalised exponentials are accumulated into P.V and the row is scaled by 1 / sum after.
// Own code: plain loops left to the compiler's vectoriser, expf from libm, any head_dim and an
// explicit softmax scale (the reference hard-codes 64 and 0.125). Returns 0, or -1 on bad
// arguments, -3 if scratch allocation fails.
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>

static void attend_tile(const float *q, const float *k, const float *v, float *o, long ldo, int d, int length,
                        int start, int rows, int half, float scale, float *kt, float *s, float *acc) {
    const int lo = start - half < 0 ? 0 : start - half;
    const int hi = start + rows + half < length ? start + rows + half : length;
    const int cols = hi - lo;
    for (int j = 0; j < cols; ++j)
        for (int x = 0; x < d; ++x) kt[(long)x * cols + j] = k[(long)(lo + j) * d + x];
    for (int r = 0; r < rows; ++r) {
        const int i = start + r;
        const int first = (i - half > lo ? i - half : lo) - lo;
        const int last = (i + half + 1 < hi ? i + half + 1 : hi) - lo;
        for (int j = first; j < last; ++j) s[j] = 0.0f;
        for (int x = 0; x < d; ++x) {
            const float qx = q[(long)i * d + x];
            const float *kr = kt + (long)x * cols;
#pragma omp simd
            for (int j = first; j < last; ++j) s[j] += qx * kr[j];
        }
        float m = -INFINITY;
        for (int j = first; j < last; ++j) {
            s[j] *= scale;
            m = s[j] > m ? s[j] : m;
        }
        float sum = 0.0f;
        for (int j = first; j < last; ++j) {
            s[j] = expf(s[j] - m);
            sum += s[j];
        }
        for (int x = 0; x < d; ++x) acc[x] = 0.0f;
        for (int j = first; j < last; ++j) {
            const float p = s[j];
            const float *vr = v + (long)(lo + j) * d;
#pragma omp simd
            for (int x = 0; x < d; ++x) acc[x] += p * vr[x];
        }
        const float inv = 1.0f / sum;
        float *orow = o + (long)r * ldo;
        for (int x = 0; x < d; ++x) orow[x] = acc[x] * inv;
    }
}

int pe_oracle_local_attention(const float *q, const float *k, const float *v, float *out, const int32_t *lengths,
                              int tokens, int heads, int sequences, int head_dim, int tile, int half,
                              int token_major, int threads, float scale) {
    if (tokens < 1 || heads < 1 || sequences < 1 || head_dim < 1 || tile < 1 || half < 0 || threads < 1 ||
        !(scale > 0.0f))
        return -1;
    long total = 0;
    int longest = 0;
    for (int i = 0; i < sequences; ++i) {
        if (lengths[i] < 1) return -1;
        total += lengths[i];
        if (lengths[i] > longest) longest = lengths[i];
    }
    if (total != tokens) return -1;
    if (half > longest) half = longest;
    long *offsets = (long *)malloc(sizeof(long) * (size_t)sequences);
    if (!offsets) return -3;
    for (long i = 0, off = 0; i < sequences; off += lengths[i++]) offsets[i] = off;
    const int window = tile + 2 * half < longest ? tile + 2 * half : longest;
    const long ldo = token_major ? (long)heads * head_dim : head_dim;
    int failed = 0;
#pragma omp parallel num_threads(threads) reduction(| : failed)
    {
        float *kt = (float *)malloc(sizeof(float) * ((size_t)head_dim * window + window + head_dim));
        if (!kt) {
            failed = 1;
        } else {
            float *s = kt + (size_t)head_dim * window, *acc = s + window;
#pragma omp for schedule(dynamic, 1)
            for (long task = 0; task < (long)heads * sequences; ++task) {
                const int head = (int)(task / sequences), seq = (int)(task % sequences);
                const int length = lengths[seq];
                const long base = ((long)head * tokens + offsets[seq]) * head_dim;
                float *o = out + (token_major ? (offsets[seq] * heads + head) * (long)head_dim : base);
                for (int start = 0; start < length; start += tile)
                    attend_tile(q + base, k + base, v + base, o + (long)start * ldo, ldo, head_dim, length, start,
                                length - start < tile ? length - start : tile, half, scale, kt, s, acc);
            }
            free(kt);
        }
    }
    free(offsets);
    return failed ? -3 : 0;
}
