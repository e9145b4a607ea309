// Device-side helpers shared by the attention kernels (fmha_fwd.hip, fmha_dma.hip): bf16
// packing, raw buffer resources, the gfx950 MFMA wrapper and the Q prologue that every
// attention kernel applies in registers.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "fmha_params.hpp"

namespace ltx {
namespace {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int KT = kKeyTile;
constexpr int QW = kQueriesPerWave;
constexpr int NW = kWavesPerGroup;
constexpr int QT = kQueriesPerGroup;
constexpr int NT = NW * 64;                 // threads per workgroup
constexpr float kRebaseBound = 1.8446744e19f;  // 2^64: largest p a block may produce

__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ uint32_t pack_bf2(float a, float b) {
    bf16x2 v = {(bf16)a, (bf16)b};
    return __builtin_bit_cast(uint32_t, v);
}

// acc + both bf16 values of a packed pair, as two fp32 adds (a bf16 value is the fp32 value
// with the same upper half). Row sums use this rather than v_dot2_f32_bf16 with (1, 1), which
// is exact too but holds up the matrix cores' instruction stream several times longer.
__device__ __forceinline__ float add_bf2(float acc, uint32_t w) {
    return (acc + bf_lo(w)) + bf_hi(w);
}

// pack_bf2 whose result the compiler treats as opaque: it would otherwise rebuild the low
// half for add_bf2 with a second conversion instead of shifting the packed word.
__device__ __forceinline__ uint32_t pack_bf2_opaque(float a, float b) {
    uint32_t w = pack_bf2(a, b);
    asm volatile("" : "+v"(w));
    return w;
}

// Two floats as packed fp16, each rounded to nearest even (v_cvt_pk_f16_f32).
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
    f16x2 v = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ u32x4 pack8_f16(const float f[8]) {
    u32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = pack_f16x2(f[2 * i], f[2 * i + 1]);
    return w;
}

__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ void unpack8(const u32x4 w, float f[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = bf_lo(w[i]);
        f[2 * i + 1] = bf_hi(w[i]);
    }
}

__device__ __forceinline__ u32x4 pack8(const float f[8]) {
    u32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = pack_bf2(f[2 * i], f[2 * i + 1]);
    return w;
}

__device__ __forceinline__ u32x4 ldg16(const void *p) { return *(const u32x4 *)p; }

// Raw buffer resource over [base, base + bytes): loads past the end return zero.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kRsrcWord3 = 0x00020000;   // 32-bit data format, no swizzle (gfx9 family)

__device__ __forceinline__ rsrc_t make_rsrc(const void *base, int64_t bytes) {
    const int n = bytes <= 0 ? 0 : (bytes >= 0x7fffffff ? 0x7fffffff : (int)bytes);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, n, kRsrcWord3);
}

__device__ __forceinline__ u32x4 bload16(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

__device__ __forceinline__ f32x16 splat16(float x) {
    f32x16 v;
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = x;
    return v;
}

__device__ __forceinline__ float xlane32(float x) { return __shfl_xor(x, 32, 64); }

// Position of key k (0..63) inside a 64-key row of V^T: bits 2 and 3 swapped. A lane's B
// operand of O^T = V^T.P^T holds keys {16h + 4g + 0..3, 16h + 8 + 4g + 0..3} of the S
// registers; with this order they are the 8 contiguous positions 16h + 8g + 0..7.
__device__ __forceinline__ int vt_pos(int k) {
    return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1);
}

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Q of one wave (64 queries from q0) as MFMA B operands: load, RMS-normalise with the
// prologue's statistic and q_norm.weight (DiTAttention.swift:202-204), rotate (split-half
// RoPE, :226-237), multiply by scale*log2(e) in fp32, round to bf16 once. Lane (r, g) holds
// query 32*qb + r, channels 16c + 8g .. +7 in qf[qb][c]. Rows past Lq read as zero.
// Every load (the rows, the statistic, the weight, the table rows) is issued before any of
// the arithmetic, so an item start waits for one memory round trip, not one per kind.
template <int D>
__device__ __forceinline__ void load_q(const FmhaParams &p, int b, int h, int q0, bool active,
                                       int r, int g, bf16x8 (&qf)[2][D / 16]) {
    constexpr int NC = D / 16;
    const bf16 *Qb = (const bf16 *)p.q + (int64_t)b * p.q_bs + (int64_t)h * p.q_hs;
    const int nq = max(0, min(QW, p.Lq - q0));   // valid queries of this wave
    const rsrc_t rq = make_rsrc(Qb + (int64_t)(active ? q0 : 0) * p.q_rs,
                                (int64_t)nq * p.q_rs * 2);
    const bool norm = p.q_rstd != nullptr, rope = p.q_cos != nullptr;
    u32x4 xr[2][NC], wr[NC], cr[2][NC / 2], sr[2][NC / 2];
    float rs[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int c = 0; c < NC; ++c)
            xr[qb][c] = bload16(rq, (uint32_t)((32 * qb + r) * p.q_rs * 2 + (16 * c + 8 * g) * 2));
    if (norm) {
        const bf16 *w = (const bf16 *)p.q_w + h * D;
#pragma unroll
        for (int c = 0; c < NC; ++c) wr[c] = ldg16(w + 16 * c + 8 * g);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
            rs[qb] = p.q_rstd[(int64_t)b * p.Lq + min(q0 + 32 * qb + r, p.Lq - 1)];
    }
    if (rope) {
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
            const int qc = min(q0 + 32 * qb + r, p.Lq - 1);   // clamped index for side tables
            const int64_t toff = ((int64_t)h * p.Lq + qc) * (D / 2);
#pragma unroll
            for (int c = 0; c < NC / 2; ++c) {
                cr[qb][c] = ldg16((const bf16 *)p.q_cos + toff + 16 * c + 8 * g);
                sr[qb][c] = ldg16((const bf16 *)p.q_sin + toff + 16 * c + 8 * g);
            }
        }
    }
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        float x[NC][8];
#pragma unroll
        for (int c = 0; c < NC; ++c) unpack8(xr[qb][c], x[c]);
        if (norm) {
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                float wq[8];
                unpack8(wr[c], wq);
#pragma unroll
                for (int e = 0; e < 8; ++e) x[c][e] = (x[c][e] * rs[qb]) * wq[e];
            }
        }
        if (rope) {
#pragma unroll
            for (int c = 0; c < NC / 2; ++c) {
                float fc[8], fs[8];
                unpack8(cr[qb][c], fc);
                unpack8(sr[qb][c], fs);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float x1 = x[c][e], x2 = x[c + NC / 2][e];
                    x[c][e] = x1 * fc[e] - x2 * fs[e];
                    x[c + NC / 2][e] = x2 * fc[e] + x1 * fs[e];
                }
            }
        }
#pragma unroll
        for (int c = 0; c < NC; ++c) {
#pragma unroll
            for (int e = 0; e < 8; ++e) x[c][e] *= p.qk_scale_log2;
            qf[qb][c] = __builtin_bit_cast(bf16x8, pack8(x[c]));
        }
    }
}

// Output gate of (batch b, query q, head h): 2*sigmoid(logit) rounded to bf16, the gate
// array the reference multiplies the attention output by (DiTAttention.swift:395-399).
// 1 without a gate.
__device__ __forceinline__ float gate_factor(const void *gate, int64_t g_bs, int64_t g_rs,
                                             int64_t g_hs, int b, int q, int h) {
    if (!gate) return 1.0f;
    const float x = (float)((const bf16 *)gate)[(int64_t)b * g_bs + (int64_t)q * g_rs +
                                                (int64_t)h * g_hs];
    const float g = 2.0f / (1.0f + __builtin_amdgcn_exp2f(-x * 1.4426950408889634f));
    return (float)(bf16)g;
}

// Work item of a workgroup. Workgroup ids are dealt to the 8 XCDs round-robin; within each
// region of the grid (the leading tail splits, the whole items, the other tail splits) an XCD
// receives a contiguous range, so the query blocks (and splits) sharing one (batch, head)
// share an L2.
struct WorkItem {
    int qblk, h, b;
    int tail;          // -1 for a whole item, else the tail item's index (0-based)
    int split;         // key range of a tail item
    int t_begin, t_end;
};

__device__ __forceinline__ int xcd_major(int local, int count) {
    const int xcd = local & 7;
    return xcd * (count >> 3) + min(xcd, count & 7) + (local >> 3);
}

__device__ __forceinline__ WorkItem work_item(const FmhaParams &p) {
    const int bid = blockIdx.x;
    WorkItem w;
    int item;
    // grid order: n_lead tail splits, the whole items, the other tail splits
    const int full_local = bid - p.n_lead;
    if (full_local >= 0 && full_local < p.n_full) {
        item = xcd_major(full_local, p.n_full);
        w.tail = -1;
        w.split = 0;
    } else {
        const int tail_local = full_local < 0 ? bid : bid - p.n_full;
        const int sub = xcd_major(tail_local, p.grid - p.n_full);
        w.tail = sub / p.num_splits;
        w.split = sub % p.num_splits;
        item = p.n_full + w.tail;
    }
    w.qblk = item % p.nqblk;
    const int bh = item / p.nqblk;
    w.h = bh % p.H;
    w.b = bh / p.H;
    const int ntiles = (p.valid[w.b] + kKeyTile - 1) / kKeyTile;
    if (w.tail < 0) {
        w.t_begin = 0;
        w.t_end = ntiles;
    } else {
        w.t_begin = w.split * p.tiles_per_split;
        w.t_end = min(w.t_begin + p.tiles_per_split, ntiles);
    }
    return w;
}

}  // namespace
}  // namespace ltx
