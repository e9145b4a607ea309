// Gemma-4 text-encoder attention (Sources/LTXModules/GemmaTextEncoder.swift:158-239, mask
// :288-321) for gfx950: head dims 256 / 512, 16 query heads over 8 or 1 KV heads, causal +
// sliding-window + left-padding mask, scale 1.0, 1024 tokens per prompt.
//
// Three launches:
//   gemma_prep_kernel   one wave per (batch row, token, head) row of q or k: the per-head
//                       RMS norm (fp32, pow(mean + eps, -0.5), times the weight), rotate_half
//                       RoPE with the fp32 tables,
//                       q scaled by scale*log2(e). Writes q' as two bf16 parts (hi + lo)
//                       [B][Hq][T][D], k' [B][Hkv][T][D] (one bf16 rounding, as the
//                       reference rounds its normed k).
//   gemma_vt_kernel     v with the weightless per-head norm, written TRANSPOSED,
//                       [B][Hkv][D][T] (through an LDS tile of 64 tokens), so that the P.V
//                       operand (one channel, eight keys per lane) is two 8-byte loads.
//   gemma_attn_kernel   one workgroup of four waves per (batch row, query head, 32 queries);
//                       the waves split the head dim into four slices of D/4 channels. Per
//                       32-key block each wave forms the partial S^T = K.Q'^T over its slice
//                       (MFMA 32x32x16 over both parts of Q', K' and Q' straight from memory;
//                       the reference keeps q in fp32 after its fp32 RoPE), the four partials are
//                       added through LDS in a fixed order (every wave holds the same S), the
//                       mask and an online softmax (running max, rescale) run in every wave,
//                       and each wave accumulates O^T += V^T.P^T for its own channels with P
//                       as two bf16 parts (the reference's weights are fp32); O
//                       is written in fp32, the dtype the reference's explicit path returns.
// The key range of a query block is cut to the causal / window / padding bounds; query rows
// inside the left padding (no allowed key) attend to every key unmasked, the reference's
// rule for fully-masked rows.
#include "fmha_device.hpp"

namespace ltx {
namespace {

constexpr int kGemmaQB = 32;       // queries per workgroup

// ---- prologue ------------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void gemma_prep_kernel(const GemmaPrepParams p) {
    constexpr int E = D / 64;                       // channels per lane: 4 or 8
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int heads = p.Hq + p.Hkv;                 // q heads, then k heads, per token
    if (row >= (int64_t)p.B * p.T * heads) return;
    const int hr = (int)(row % heads);
    const int64_t bt = row / heads;
    const int t = (int)(bt % p.T), b = (int)(bt / p.T);
    const int kind = hr < p.Hq ? 0 : 1;             // q, k
    const int h = kind == 0 ? hr : hr - p.Hq;
    const bf16 *src = kind == 0 ? (const bf16 *)p.q + (int64_t)b * p.q_bs + (int64_t)t * p.q_rs
                                : (const bf16 *)p.k + (int64_t)b * p.k_bs + (int64_t)t * p.k_rs;
    src += (int64_t)h * D + lane * E;
    float x[E];
    if constexpr (E == 8) {
        unpack8(ldg16(src), x);
    } else {
        const u32x2 w = *(const u32x2 *)src;
        x[0] = bf_lo(w[0]); x[1] = bf_hi(w[0]); x[2] = bf_lo(w[1]); x[3] = bf_hi(w[1]);
    }
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) ss += x[e] * x[e];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
    const float rs = powf(ss / (float)D + p.eps, -0.5f);
    const bf16 *w = (const bf16 *)(kind == 0 ? p.q_w : p.k_w) + lane * E;
#pragma unroll
    for (int e = 0; e < E; ++e) x[e] = (x[e] * rs) * (float)w[e];
    // rotate_half pairs channel c with c +- D/2: lane l holds channels E*l ..; its partner is
    // lane l ^ 32. Table column of channel c is c mod D/2.
    const int col = (lane & 31) * E;
    const float *cs = p.cos + (int64_t)t * (D / 2) + col;
    const float *sn = p.sin + (int64_t)t * (D / 2) + col;
    const bool first = lane < 32;
    const float f = kind == 0 ? p.q_factor : 1.0f;
    float y[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const float other = __shfl_xor(x[e], 32, 64);
        const float c = cs[e], s = sn[e];
        // first half: x1 c - x2 s; second half: x2 c + x1 s
        y[e] = (first ? x[e] * c - other * s : x[e] * c + other * s) * f;
    }
    // q as two bf16 parts (hi + lo carries ~16 significant bits into the products); k as one
    auto put = [&](bf16 *dst, const float (&z)[E]) __attribute__((always_inline)) {
        if constexpr (E == 8) {
            *(u32x4 *)dst = pack8(z);
        } else {
            *(u32x2 *)dst = u32x2{pack_bf2(z[0], z[1]), pack_bf2(z[2], z[3])};
        }
    };
    const int64_t off = (((int64_t)b * (kind == 0 ? p.Hq : p.Hkv) + h) * p.T + t) * D + lane * E;
    put((bf16 *)(kind == 0 ? p.qp : p.kp) + off, y);
    if (kind == 0) {
        float lo[E];
#pragma unroll
        for (int e = 0; e < E; ++e) lo[e] = y[e] - (float)(bf16)y[e];
        put((bf16 *)p.qp_lo + off, lo);
    }
}

// v: the weightless per-head norm, stored transposed (channel rows of T keys). One workgroup
// per (batch row, KV head, 64 tokens): each wave normalises 16 token rows into an LDS tile,
// then the tile leaves as runs of 8 tokens of one channel.
template <int D>
__global__ __launch_bounds__(256) void gemma_vt_kernel(const GemmaPrepParams p) {
    constexpr int E = D / 64;
    constexpr int TT = 64;                          // tokens per workgroup
    __shared__ __attribute__((aligned(16))) bf16 tile[TT][D + 8];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ntb = (p.T + TT - 1) / TT;
    const int t0 = (int)(blockIdx.x % ntb) * TT;
    const int bh = (int)(blockIdx.x / ntb);
    const int h = bh % p.Hkv, b = bh / p.Hkv;
    for (int j = 0; j < TT / 4; ++j) {
        const int tl = wave * (TT / 4) + j, t = t0 + tl;
        if (t >= p.T) break;
        const bf16 *src = (const bf16 *)p.v + (int64_t)b * p.v_bs + (int64_t)t * p.v_rs +
                          (int64_t)h * D + lane * E;
        float x[E];
        if constexpr (E == 8) {
            unpack8(ldg16(src), x);
        } else {
            const u32x2 w = *(const u32x2 *)src;
            x[0] = bf_lo(w[0]); x[1] = bf_hi(w[0]); x[2] = bf_lo(w[1]); x[3] = bf_hi(w[1]);
        }
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) ss += x[e] * x[e];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
        const float rs = powf(ss / (float)D + p.eps, -0.5f);
#pragma unroll
        for (int e = 0; e < E; ++e) tile[tl][lane * E + e] = (bf16)(x[e] * rs);
    }
    __syncthreads();
    const int nt = min(TT, p.T - t0);               // a multiple of 4 (T is)
    for (int u = threadIdx.x; u < D * (TT / 8); u += 256) {
        const int c = u / (TT / 8), j8 = 8 * (u % (TT / 8));
        if (j8 >= nt) continue;
        float f[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = (float)tile[min(j8 + e, TT - 1)][c];
        // 8-byte stores: channel rows are T * 2 bytes apart, T a multiple of 4
        bf16 *dst = (bf16 *)p.vt + (((int64_t)b * p.Hkv + h) * D + c) * p.T + t0 + j8;
        *(u32x2 *)dst = u32x2{pack_bf2(f[0], f[1]), pack_bf2(f[2], f[3])};
        if (j8 + 8 <= nt) *(u32x2 *)(dst + 4) = u32x2{pack_bf2(f[4], f[5]), pack_bf2(f[6], f[7])};
    }
}

// ---- attention -----------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void gemma_attn_kernel(const GemmaAttnParams p) {
    constexpr int DS = D / 4;                       // channels per wave
    constexpr int NCS = DS / 16;                    // 16-channel chunks of the wave's S slice
    constexpr int NDS = DS / 32;                    // 32-channel blocks of the wave's O slice
    __shared__ float sS[2][4][16][64];              // partial S per wave, double-buffered

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 31, g = lane >> 5;
    const int nqb = (p.T + kGemmaQB - 1) / kGemmaQB;
    // heaviest (latest) query blocks first
    const int qblk = nqb - 1 - (int)(blockIdx.x % nqb);
    const int bh = (int)(blockIdx.x / nqb);
    const int h = bh % p.Hq, b = bh / p.Hq;
    const int kvh = h / (p.Hq / p.Hkv);
    const int q0 = qblk * kGemmaQB;
    const int fv = p.first_valid[b];
    const int T = p.T;

    // Q' slice of this wave: query q0 + r, channels wave*DS + 16c + 8g .. +7
    const bf16 *Qh = (const bf16 *)p.qp + ((int64_t)b * p.Hq + h) * T * D + wave * DS;
    const int qr = min(q0 + r, T - 1);
    const bf16 *Ql = (const bf16 *)p.qp_lo + ((int64_t)b * p.Hq + h) * T * D + wave * DS;
    bf16x8 qf[NCS], ql[NCS];
#pragma unroll
    for (int c = 0; c < NCS; ++c) {
        qf[c] = __builtin_bit_cast(bf16x8, ldg16(Qh + (int64_t)qr * D + 16 * c + 8 * g));
        ql[c] = __builtin_bit_cast(bf16x8, ldg16(Ql + (int64_t)qr * D + 16 * c + 8 * g));
    }
    const bf16 *Kh = (const bf16 *)p.kp + ((int64_t)b * p.Hkv + kvh) * T * D + wave * DS;
    const bf16 *Vt = (const bf16 *)p.vt + (((int64_t)b * p.Hkv + kvh) * D + wave * DS) * T;

    // Key blocks: causal / window / padding bounds; a block with rows inside the left padding
    // (their rows have no allowed key) runs over all keys, those rows unmasked.
    const int nkb = (T + 31) / 32;
    const bool has_free_rows = q0 < fv;
    int kb_lo = 0, kb_hi = nkb - 1;
    if (!has_free_rows) {
        kb_hi = min(q0 + kGemmaQB - 1, T - 1) / 32;
        int lo = fv;
        if (p.window > 0) lo = max(lo, q0 - p.window + 1);
        kb_lo = max(0, lo) / 32;
    }
    const int q = q0 + r;                           // this lane's query row
    const bool free_row = q < fv;

    f32x16 o[NDS];
#pragma unroll
    for (int db = 0; db < NDS; ++db) o[db] = splat16(0.f);
    float m = -INFINITY, l = 0.f;
    // Operands in flight: the block's K' rows are fetched one block ahead, its V'^T rows at
    // the top of the block, so their latency overlaps the products, the exchange and the
    // softmax instead of stalling each step.
    auto load_k = [&](int kb, u32x4 (&kx)[NCS]) __attribute__((always_inline)) {
        const int kr = min(kb * 32 + r, T - 1);     // keys past T read key T-1 (masked)
#pragma unroll
        for (int c = 0; c < NCS; ++c) kx[c] = ldg16(Kh + (int64_t)kr * D + 16 * c + 8 * g);
    };
    u32x4 kx[NCS];
    load_k(kb_lo, kx);
    for (int kb = kb_lo, it = 0; kb <= kb_hi; ++kb, ++it) {
        // V'^T operands of this block: channel wave*DS + 32db + r, keys 32kb + 16hf + 4g + 0..3
        // and + 8 (clamped into the row: past T only for masked keys, T a multiple of 4)
        u32x2 vx[2][NDS][2];
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            const int k0 = 32 * kb + 16 * hf + 4 * g;
#pragma unroll
            for (int db = 0; db < NDS; ++db) {
                const bf16 *vrow = Vt + (int64_t)(32 * db + r) * T;
                vx[hf][db][0] = *(const u32x2 *)(vrow + min(k0, T - 4));
                vx[hf][db][1] = *(const u32x2 *)(vrow + min(k0 + 8, T - 4));
            }
        }
        // partial S^T over this wave's channels: the hi and lo parts of q' in two chains
        f32x16 sh = splat16(0.f), sl = splat16(0.f);
#pragma unroll
        for (int c = 0; c < NCS; ++c) {
            const bf16x8 a = __builtin_bit_cast(bf16x8, kx[c]);
            sh = mfma32(a, qf[c], sh);
            sl = mfma32(a, ql[c], sl);
        }
        if (kb < kb_hi) load_k(kb + 1, kx);
        const int buf = it & 1;
#pragma unroll
        for (int i = 0; i < 16; ++i) sS[buf][wave][i][lane] = sh[i] + sl[i];
        __syncthreads();
        f32x16 s;
#pragma unroll
        for (int i = 0; i < 16; ++i)
            s[i] = ((sS[buf][0][i][lane] + sS[buf][1][i][lane]) + sS[buf][2][i][lane]) +
                   sS[buf][3][i][lane];
        // mask: key k = 32kb + 8(i>>2) + 4g + (i&3) for query q
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int k = 32 * kb + 8 * (i >> 2) + 4 * g + (i & 3);
            const bool ok = k < T && (free_row || (k <= q && k >= fv &&
                                                   (p.window <= 0 || q - k < p.window)));
            s[i] = ok ? s[i] : -INFINITY;
            mx = fmaxf(mx, s[i]);
        }
        mx = fmaxf(mx, xlane32(mx));
        const float mn = fmaxf(m, mx);
        // fp32 weights, their fp32 row sums, and P as two bf16 parts for P.V (the reference's
        // explicit path multiplies fp32 weights)
        float alpha = 1.f, ts = 0.f;
        u32x4 wh[2], wl[2];
        if (mn == -INFINITY) {                      // nothing allowed yet in this row
            wh[0] = wh[1] = wl[0] = wl[1] = u32x4{0, 0, 0, 0};
        } else {
            alpha = __builtin_amdgcn_exp2f(m - mn); // 0 when m is -inf
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float x0 = __builtin_amdgcn_exp2f(s[8 * hf + 2 * e] - mn);
                    const float x1 = __builtin_amdgcn_exp2f(s[8 * hf + 2 * e + 1] - mn);
                    ts += x0 + x1;
                    const uint32_t hi = pack_bf2_opaque(x0, x1);
                    wh[hf][e] = hi;
                    wl[hf][e] = pack_bf2(x0 - bf_lo(hi), x1 - bf_hi(hi));
                }
        }
        m = mn;
        l = l * alpha + ts;
#pragma unroll
        for (int db = 0; db < NDS; ++db) o[db] *= splat16(alpha);
        // O^T += V^T.P^T
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int db = 0; db < NDS; ++db) {
                const u32x2 lo = vx[hf][db][0], hi = vx[hf][db][1];
                const bf16x8 a = __builtin_bit_cast(bf16x8, u32x4{lo[0], lo[1], hi[0], hi[1]});
                o[db] = mfma32(a, __builtin_bit_cast(bf16x8, wh[hf]), o[db]);
                o[db] = mfma32(a, __builtin_bit_cast(bf16x8, wl[hf]), o[db]);
            }
    }

    // ---- epilogue: O / l in fp32 (the reference's dtype here), this wave's channels ------
    const float lt = l + xlane32(l);
    if (q < T) {
        const float inv = 1.0f / lt;
        float *Ob = p.out + (int64_t)b * p.o_bs + (int64_t)q * p.o_rs + (int64_t)h * D + wave * DS;
#pragma unroll
        for (int db = 0; db < NDS; ++db)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                f32x4 w;
#pragma unroll
                for (int e = 0; e < 4; ++e) w[e] = o[db][4 * i4 + e] * inv;
                *(f32x4 *)(Ob + 32 * db + 8 * i4 + 4 * g) = w;
            }
    }
}

}  // namespace

int launch_gemma_prep(const GemmaPrepParams &p, int D, void *stream) {
    const int64_t rows = (int64_t)p.B * p.T * (p.Hq + p.Hkv);
    const dim3 grid((unsigned)((rows + 3) / 4)), block(256);
    const dim3 vgrid((unsigned)((int64_t)p.B * p.Hkv * ((p.T + 63) / 64)));
    hipStream_t st = (hipStream_t)stream;
    if (D == 512) {
        hipLaunchKernelGGL(gemma_prep_kernel<512>, grid, block, 0, st, p);
        hipLaunchKernelGGL(gemma_vt_kernel<512>, vgrid, block, 0, st, p);
    } else {
        hipLaunchKernelGGL(gemma_prep_kernel<256>, grid, block, 0, st, p);
        hipLaunchKernelGGL(gemma_vt_kernel<256>, vgrid, block, 0, st, p);
    }
    return (int)hipGetLastError();
}

int launch_gemma_attn(const GemmaAttnParams &p, int D, void *stream) {
    const int nqb = (p.T + kGemmaQB - 1) / kGemmaQB;
    const dim3 grid((unsigned)((int64_t)p.B * p.Hq * nqb)), block(256);
    hipStream_t st = (hipStream_t)stream;
    if (D == 512) hipLaunchKernelGGL(gemma_attn_kernel<512>, grid, block, 0, st, p);
    else hipLaunchKernelGGL(gemma_attn_kernel<256>, grid, block, 0, st, p);
    return (int)hipGetLastError();
}

}  // namespace ltx
