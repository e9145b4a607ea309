// HBM -> LDS copies through gfx950's buffer-load-to-LDS path, and the LDS tile layouts of the
// attention kernels, shared by the kernels that stage their tiles this way (fmha_dma.hip,
// fmha_short.hip, linear_gemm.hip).
#pragma once

#include "fmha_device.hpp"

namespace ltx {
namespace {

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) bf16 lds_bf16;

// s_waitcnt vmcnt(0), expcnt and lgkmcnt left at their maxima: this wave's copies landed.
__device__ __forceinline__ void wait_copies() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// s_waitcnt vmcnt(N): all but this wave's N most recent copies landed (N < 64; vmcnt is split
// over bits 3:0 and 15:14 of the immediate).
template <int N>
__device__ __forceinline__ void wait_copies_but() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// A copy HBM -> LDS: every lane (all are enabled wherever the kernel copies) moves 16 bytes
// from the buffer at its offset to M0 + 16*lane. As one assembly statement the compiler sees
// no memory load, so its waits never account for these; the kernel waits for them itself
// (vmcnt). The s_nop is the wait state an M0 write needs before the load. The compiler keeps
// nothing in M0 in these kernels, so the clobber costs nothing.
__device__ __forceinline__ void copy_all(u32x4 rs, uint32_t lds_byte, int voff) {
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %1, %2, 0 offen lds"
        :
        : "s"(lds_byte), "v"(voff), "s"(rs)
        : "m0", "memory");
}

// Buffer resource words over [base, base + bytes) (raw, 32-bit format): loads past the end
// return zero.
__device__ __forceinline__ u32x4 rsrc_words(const void *base, int64_t bytes) {
    const uint64_t a = (uint64_t)base;
    const uint32_t n = bytes <= 0 ? 0u : (bytes >= 0x7fffffff ? 0x7fffffffu : (uint32_t)bytes);
    return u32x4{(uint32_t)a, (uint32_t)(a >> 32) & 0xffffu, n, (uint32_t)kRsrcWord3};
}

// Unit swizzle for gfx950's LDS (64 four-byte banks; a 16-byte access is serviced 16 lanes
// at a time): 16 consecutive rows reading the same logical unit hit 16 distinct bank groups.
// Rows of 16 units span all banks (XOR with row & 15); rows of 8 units pair up per bank
// window (XOR with (row >> 1) & 7). XOR makes the map its own inverse.
template <int UNITS>
__device__ __forceinline__ int swz(int row, int u) {
    static_assert(UNITS == 16 || UNITS == 8, "row width");
    return UNITS == 16 ? (u ^ (row & 15)) : (u ^ ((row >> 1) & 7));
}

// V tiles stay row-major (key rows of D channels) and are read through the transposing LDS
// read: 32 lanes of a ds_read_b64_tr_b16 read 4 consecutive rows x 64 bytes, so the units of
// rows r and r+1..r+3 must fall in distinct bank windows (XOR the unit with row & 3 scaled to
// a quarter row; rows of 64 channels pair up, so rows r and r+2 differ instead).
template <int UNITS>
__device__ __forceinline__ int vswz(int row, int u) {
    static_assert(UNITS == 16 || UNITS == 8, "row width");
    return UNITS == 16 ? (u ^ ((row & 3) << 2)) : (u ^ (((row >> 1) & 1) << 2));
}

typedef short i16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2 ds_read_tr(const __attribute__((address_space(3))) bf16 *p) {
    const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4 *)p);
    return __builtin_bit_cast(u32x2, v);
}

}  // namespace
}  // namespace ltx
