// Device construction of the split-RoPE cos/sin tables (the GPU counterpart of
// rope_tables.cpp), following Sources/LTXModules/DiTForward.swift:455-466 (frequency grid)
// and :641-678 (rotary): one thread per (table column, 8 tokens), writing the per-head layout
// [heads][tokens][inner/2/heads] straight into the caller's device buffers. A table of the
// 12480-token stage-2 video (32 x 12480 x 64 x 2 bf16 = 102 MB per pair) is built in place
// instead of on the host and uploaded.
//
// Arithmetic matches the host builder step for step: the frequency grid in double then float,
// the patch centre, fraction and angle in float, one bf16 rounding at the end. The host builder
// takes cos and sin of the float angle in double and rounds them to float; here the device
// library's single-precision sincosf (within 4 ulp, the OpenCL bound its library meets) gives
// the same bf16 bits whenever its result lies more than kGuard ulp from a bf16 rounding
// midpoint: the double-rounded value is within 4.5 ulp of it, so no midpoint separates them.
// Closer to a midpoint (about 1 value in 2000) the angle is evaluated in double as on the
// host. The tests compare every table of the model's geometries with the host builder.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "../../include/ltx_attn.h"

namespace {

constexpr int kMaxPos = 8;   // positional dimensions (the model uses 1 or 3)
constexpr int kTok = 8;      // tokens per thread (one frequency, kTok angles)

struct RopeParams {
    const float *pos;        // [n_pos][tokens][2] patch bounds
    int32_t n_pos, tokens, half, pad, per_head, count;
    float max_pos[kMaxPos];
    double theta;
    uint16_t *cos, *sin;     // [heads][tokens][per_head] bf16 bits
};

__device__ __forceinline__ uint16_t bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// A float whose bf16 rounding could differ from that of a value within kGuard ulp of it: its
// low 16 bits are within kGuard of the midpoint 0x8000 between two bf16 neighbours.
constexpr int kGuard = 16;
__device__ __forceinline__ bool near_bf16_midpoint(float x) {
    const int low = (int)(__float_as_uint(x) & 0xffffu);
    return abs(low - 0x8000) <= kGuard;
}

__global__ __launch_bounds__(256) void rope_table_kernel(const RopeParams p) {
    const int nj = (p.half + 255) / 256;
    const int t0 = (blockIdx.x / nj) * kTok;
    const int j = (blockIdx.x % nj) * 256 + threadIdx.x;
    if (j >= p.half) return;
    const bool rot = j >= p.pad;                       // else leading identity padding
    const int jj = j - p.pad;
    const int i = rot ? jj / p.n_pos : 0, d = rot ? jj % p.n_pos : 0;  // positional dim fastest
    float f = 0.0f;
    if (rot) {
        const double e = (i == p.count - 1) ? 1.0 : (double)i * (1.0 / (double)(p.count - 1));
        f = (float)(pow(p.theta, e) * M_PI / 2);
    }
    const int hh = j / p.per_head, k = j % p.per_head;
    for (int t = t0; t < min(t0 + kTok, p.tokens); ++t) {
        float c = 1.0f, s = 0.0f;
        if (rot) {
            const float lo = p.pos[((int64_t)d * p.tokens + t) * 2];
            const float hi = p.pos[((int64_t)d * p.tokens + t) * 2 + 1];
            const float middle = (lo + hi) / 2.0f;      // patch centre
            const float frac = middle / p.max_pos[d];
            const float scaled = frac * 2.0f - 1.0f;
            const float angle = f * scaled;
            sincosf(angle, &s, &c);
            if (near_bf16_midpoint(s) || near_bf16_midpoint(c)) {
                double sd, cd;
                sincos((double)angle, &sd, &cd);
                c = (float)cd;
                s = (float)sd;
            }
        }
        const int64_t o = ((int64_t)hh * p.tokens + t) * p.per_head + k;
        p.cos[o] = bf16_rne(c);
        p.sin[o] = bf16_rne(s);
    }
}

}  // namespace

extern "C" ltx_attn_status ltx_rope_tables_device(const float *positions, int32_t n_pos,
                                                  int32_t tokens, int32_t inner,
                                                  const int32_t *max_pos, int32_t heads,
                                                  double theta, uint16_t *cos_out,
                                                  uint16_t *sin_out, void *stream) {
    if (!positions || n_pos < 1 || n_pos > kMaxPos || tokens < 1 || inner < 2 || !max_pos ||
        heads < 1 || !cos_out || !sin_out || !(theta > 0.0))
        return LTX_ATTN_EINVAL;
    if (((uintptr_t)positions & 3u) || ((uintptr_t)cos_out & 1u) || ((uintptr_t)sin_out & 1u))
        return LTX_ATTN_EINVAL;
    const int32_t half = inner / 2;
    if (half % heads != 0) return LTX_ATTN_EINVAL;
    const int32_t count = inner / (2 * n_pos);
    if (count <= 1) return LTX_ATTN_EINVAL;
    const int32_t pad = half - count * n_pos;
    if (pad < 0) return LTX_ATTN_EINVAL;
    RopeParams p{};
    p.pos = positions;
    p.n_pos = n_pos;
    p.tokens = tokens;
    p.half = half;
    p.pad = pad;
    p.per_head = half / heads;
    p.count = count;
    for (int d = 0; d < n_pos; ++d) {
        if (max_pos[d] <= 0) return LTX_ATTN_EINVAL;
        p.max_pos[d] = (float)max_pos[d];
    }
    p.theta = theta;
    p.cos = cos_out;
    p.sin = sin_out;
    const int64_t blocks = (int64_t)((tokens + kTok - 1) / kTok) * ((half + 255) / 256);
    if (blocks > 0x7fffffff) return LTX_ATTN_EUNSUPPORTED;
    hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)blocks), dim3(256), 0,
                       (hipStream_t)stream, p);
    return hipGetLastError() == hipSuccess ? LTX_ATTN_OK : LTX_ATTN_EHIP;
}
