// LDS staging shared by the attention kernels (gfx950): direct global-to-LDS loads issued out
// of the compiler's sight with explicit vector-memory waits, the XOR swizzle of 16-byte row
// units that makes row-major K/V tiles conflict-free for ds_read_b128, and the transposing
// ds_read_b64_tr_b16 read of V^T operands.
#pragma once

#include "pe_attn_device.h"

namespace pe {

#define PE_LDS __attribute__((address_space(3)))

// A buffer offset past every resource's range: the load returns zeros and touches no memory.
constexpr int kVoidOffset = 0x7ffffff0;

// 16-byte unit of a row after the XOR swizzle, rows of CPR units, over 64 LDS banks of 4 bytes.
// Two reads must be conflict-free:
//  * ds_read_b128 of a K (or Q) operand serves 16 lanes per pass: 16 consecutive keys, one
//    unit column. The swizzle must be a bijection over the keys that share a bank row (the 8
//    same-parity keys of a 16-key group at head_dim 64, where two 128-byte rows fill the 64
//    banks; all 16 keys at head_dim 128).
//  * ds_read_b64_tr_b16 of a V^T operand reads 8 consecutive keys (aligned to 8) x 4 units of
//    one 32-dim block, 8 bytes per lane (512 bytes: two passes). The units after the XOR must
//    cover the row's bank span evenly: at head_dim 64 two of each parity's four keys land in
//    units 0-3 and two in units 4-7; at head_dim 128 each 4-unit block is hit by two keys.
// Head_dim 64: j = bits 1-3 of the key, then bit 0 of j folded into bit 2 (0 5 2 7 4 1 6 3).
// Head_dim 128: the key's low four bits with their two 2-bit halves exchanged. (A plain
// (key >> 1) & 7 or key & 15 serves ds_read_b128 alike but leaves half of the banks idle in
// every transposing read: four cycles instead of two.) Both depend only on key bits 0-3, so
// offsets of whole 16-key halves and 32-key blocks never change a key's swizzle. Head_dim 256
// rows span 8 bank rows and keep key & 15 (conflict-free for its 16x16 reads).
template <int CPR>
__device__ __forceinline__ int swz(int key) {
    if constexpr (CPR == 8) {
        const int j = (key >> 1) & 7;
        return j ^ ((j & 1) << 2);
    } else if constexpr (CPR == 16) {
        return ((key & 3) << 2) | ((key >> 2) & 3);
    } else {
        return key & 15;
    }
}

// Global -> LDS, 16 bytes per lane, four loads: load i's lane l data lands at lds[i] + 16 * l;
// loads 0 and 1 read through rsrc a, loads 2 and 3 through b. M0 (the LDS base register) is
// saved and restored inside the statement, so the compiler's view of it never changes.
__device__ __forceinline__ void dma16x4(const uint32_t (&lds)[4], const int (&voff)[4], __amdgpu_buffer_rsrc_t a,
                                        __amdgpu_buffer_rsrc_t b) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %5, %9, 0 offen lds\n\t"
        "s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %6, %9, 0 offen lds\n\t"
        "s_mov_b32 m0, %3\n\tbuffer_load_dwordx4 %7, %10, 0 offen lds\n\t"
        "s_mov_b32 m0, %4\n\tbuffer_load_dwordx4 %8, %10, 0 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(lds[0]), "s"(lds[1]), "s"(lds[2]), "s"(lds[3]), "v"(voff[0]), "v"(voff[1]), "v"(voff[2]), "v"(voff[3]),
          "s"(a), "s"(b)
        : "memory");
}

// One global -> LDS load of 16 bytes per lane (lane l's data lands at lds + 16 * l), M0 saved
// and restored inside the statement.
__device__ __forceinline__ void dma16(uint32_t lds, int voff, __amdgpu_buffer_rsrc_t r) {
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %2, %3, 0 offen lds\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "s"(lds), "v"(voff), "s"(r)
                 : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const PE_LDS void *)p;
}

// ds_read_b64_tr_b16 at an LDS element address: in each 16-lane group, lane j receives element
// j % 4 of the 4-element rows addressed by lanes j / 4, j / 4 + 4, j / 4 + 8 and j / 4 + 12.
__device__ __forceinline__ bf16x4 tr16(const __bf16 *p) {
    typedef __bf16 lds_bf16x4 __attribute__((ext_vector_type(4)));
    return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((PE_LDS lds_bf16x4 *)(PE_LDS void *)p);
}

// Epilogue of a wave's 32-row query block (32x32 accumulator layout, head_dim D) through its own
// LDS region of 32 rows x D (row-major, 16-byte units XOR-swizzled per row): the scaled,
// rounded rows go in as 16-byte units (swap32_pair gives each lane 8 contiguous dims) and
// come back with lane l holding unit l % (D / 8) of row l / (D / 8), so every store writes
// 64 / (D / 8) whole rows (whole 128-byte lines at D = 64) instead of 32 rows x 32 bytes. With
// a gate, its 16-byte pieces of the same units are loaded first and applied on the way out.
// The region must be idle (no other wave reading it, no load in flight into it); LDS accesses
// of one wave complete in order, so the read-back sees the lane's own wave's writes.
template <int D, bool GATE>
__device__ __forceinline__ void store_rows(const f32x16 (&o)[D / 32], float inv, int lane, __bf16 *region,
                                           __amdgpu_buffer_rsrc_t o_rs, int o_off0, int o_row,
                                           __amdgpu_buffer_rsrc_t g_rs, int g_off0, int g_row) {
    constexpr int DB = D / 32, CPR = D / 8, RPI = 64 / CPR, NR = 32 / RPI;
    const int col = lane & 31, kg = lane >> 5;
    const int urow = lane / CPR, unit = lane % CPR;
    bf16x8 g[GATE ? NR : 1];
    if constexpr (GATE) {
#pragma unroll
        for (int r = 0; r < NR; ++r) g[r] = buf_ld16(g_rs, g_off0 + (r * RPI + urow) * g_row + unit * 16, 0);
    }
#pragma unroll
    for (int q = 0; q < 2 * DB; ++q) {
        const int db = q >> 1, b = 8 * (q & 1);
        const bf16x4 x = round4<false>(o[db][b] * inv, o[db][b + 1] * inv, o[db][b + 2] * inv, o[db][b + 3] * inv,
                                       bf16x4{});
        const bf16x4 y = round4<false>(o[db][b + 4] * inv, o[db][b + 5] * inv, o[db][b + 6] * inv,
                                       o[db][b + 7] * inv, bf16x4{});
        const int u = 4 * db + 2 * (q & 1) + kg;
        *reinterpret_cast<bf16x8 *>(region + col * D + ((u ^ swz<CPR>(col)) * 8)) = swap32_pair(x, y);
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const int row = r * RPI + urow;
        bf16x8 z = *reinterpret_cast<const bf16x8 *>(region + row * D + ((unit ^ swz<CPR>(row)) * 8));
        if constexpr (GATE) z = gate8(z, g[r]);
        buf_st16(o_rs, o_off0 + row * o_row + unit * 16, z);
    }
}

}  // namespace pe
