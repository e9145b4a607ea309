// HBM -> LDS copies through gfx950's buffer-load-to-LDS path, shared by the kernels that stage
// their tiles this way (fmha_dma.hip, linear_gemm.hip).
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

}  // namespace
}  // namespace ltx
