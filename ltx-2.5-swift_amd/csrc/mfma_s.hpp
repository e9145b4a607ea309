// S products of the attention kernels as inline assembly with VGPR results (fmha_dma.hip,
// gemma_attn.hip). A builtin MFMA in these kernels puts its result in AGPRs (their O
// accumulators need the AGPRs' room), so S would reach the softmax through one
// v_accvgpr_read per element; these statements keep S in VGPRs and take Q from AGPRs.
#pragma once

#include "fmha_device.hpp"

namespace ltx {
namespace {

// The statements:
//   mfma_s_first  S = K.Q'^T + C (fmha_dma.hip: C = -m; gemma_attn.hip: C = 0)
//   mfma_s_next   S += K.Q'^T
//   s_ready / s_defined  S usable from here on
// The compiler does not see that they are MFMAs, so the hazards it would pad are handled
// here and verified on the generated code by check_mfma_hazards.py at build time:
//   * s_ready after the last product of a chain redefines S behind 20 wait states, so no
//     instruction the compiler places afterwards (a use, a copy, a spill) touches S while
//     the MFMA is still writing it; it also keeps C allocated until then, so C is not
//     overwritten while the first product may still read it. Within a chain S is only the
//     exactly overlapping SrcC of the next product, which the hardware forwards.
//   * s_defined is the same statement without the padding, for the steady-state step, which
//     places it after the P.V products: the instructions in between are the wait states.
//   * an input written by VALU needs two wait states before the product reads it: the first
//     product of a chain (which reads C, set by VALU) has an s_nop 1 in front; the others
//     read LDS data, Q (AGPRs, written once) and their own forwarded result. The check
//     rejects any product that the compiler places closer to a VALU write of an input.
// Each statement names its registers in an assembly comment for the check.
__device__ __forceinline__ f32x16 mfma_s_first(bf16x8 a, bf16x8 b, const f32x16 &c) {
    f32x16 d;
    asm("; mfma_s %0 src %3\n\ts_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %3"
        : "=&v"(d) : "v"(a), "a"(b), "v"(c));
    return d;
}
__device__ __forceinline__ void mfma_s_next(f32x16 &acc, bf16x8 a, bf16x8 b) {
    asm("; mfma_s %0 src %0\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0"
        : "+v"(acc) : "v"(a), "a"(b));
}
// The same statements over fp16 operands (v_mfma_f32_32x32x16_f16), and s_ready for a single
// chain.
__device__ __forceinline__ f32x16 mfma_s_first(f16x8 a, f16x8 b, const f32x16 &c) {
    f32x16 d;
    asm("; mfma_s %0 src %3\n\ts_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %3"
        : "=&v"(d) : "v"(a), "a"(b), "v"(c));
    return d;
}
__device__ __forceinline__ void mfma_s_next(f32x16 &acc, f16x8 a, f16x8 b) {
    asm("; mfma_s %0 src %0\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0"
        : "+v"(acc) : "v"(a), "a"(b));
}
__device__ __forceinline__ void s_ready(f32x16 &x, const f32x16 &c0) {
    asm volatile("; s_ready %0\n\ts_nop 7\n\ts_nop 7\n\ts_nop 3" : "+v"(x) : "v"(c0));
}
__device__ __forceinline__ void s_ready(f32x16 &x, f32x16 &y, const f32x16 &c0,
                                        const f32x16 &c1) {
    asm volatile("; s_ready %0 %1\n\ts_nop 7\n\ts_nop 7\n\ts_nop 3"
                 : "+v"(x), "+v"(y) : "v"(c0), "v"(c1));
}
__device__ __forceinline__ void s_defined(f32x16 &x, f32x16 &y, const f32x16 &c0,
                                          const f32x16 &c1) {
    asm volatile("; s_defined %0 %1" : "+v"(x), "+v"(y) : "v"(c0), "v"(c1));
}

}  // namespace
}  // namespace ltx
