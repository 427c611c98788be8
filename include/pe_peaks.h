/*
 * pe_peaks.h — achieved-peak microbenchmarks for one MI355X (gfx950): the bf16 MFMA rate, a
 * streaming HBM read and an HBM copy, measured with the same instructions the attention kernels
 * use. They have no counterpart in the reference (packed-encoders publishes no device peaks);
 * they exist so the spec peaks a roofline fraction divides by (2.5 PFLOP/s dense bf16, 8 TB/s)
 * can be shown beside what this card sustains. Built into libpe_peaks.so; measurement only,
 * nothing in the attention path calls them.
 *
 * Every entry point launches on the caller's stream, allocates nothing and returns a status
 * (0 ok, -1 invalid argument, -4 launch failure). Timing is the caller's (HIP events).
 */
#ifndef PE_PEAKS_H
#define PE_PEAKS_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* bf16 MFMA throughput: `blocks` workgroups of 256 lanes (4 waves), each wave running four
 * independent chains of `iters` v_mfma_f32_32x32x16_bf16 (32,768 FLOP each) on operands read
 * from `operands` (at least 64 KiB of bf16: random data draws more power than zeros). Writes
 * one float per lane to `sink` (blocks * 256 floats) so no product is dead. FLOPs of a call:
 * blocks * 4 * 4 * iters * 32768. */
int pe_peak_mfma_bf16(const void *operands, float *sink, int32_t blocks, int32_t iters, hipStream_t stream);

/* Streaming read of `bytes` (a multiple of 64, 16-byte aligned) with global_load_dwordx4,
 * four loads in flight per lane; one XOR-folded int per lane to `sink` (blocks * 256 ints). */
int pe_peak_read(const void *src, size_t bytes, int32_t *sink, int32_t blocks, hipStream_t stream);

/* Copy of `bytes` (a multiple of 64, 16-byte aligned): read + write. */
int pe_peak_copy(const void *src, void *dst, size_t bytes, int32_t blocks, hipStream_t stream);

/* Direct global-to-LDS reads (buffer_load_dwordx4 ... lds, the attention kernels' staging):
 * `bytes` (a multiple of 16 KiB) streamed into a 16 KiB LDS ring per workgroup; one int per lane
 * read back from LDS to `sink` (blocks * 256 ints). */
int pe_peak_read_lds(const void *src, size_t bytes, int32_t *sink, int32_t blocks, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* PE_PEAKS_H */
