// Gemma-4 text-encoder attention (Sources/LTXModules/GemmaTextEncoder.swift:158-239, mask
// :288-321) for gfx950: head dims 256 / 512, 16 query heads over 8 or 1 KV heads, causal +
// sliding-window + left-padding mask, scale 1.0, 1024 tokens per prompt.
//
// Three launches:
//   gemma_prep_kernel   one wave per (batch row, token, head) row of q or k: the per-head
//                       RMS norm (fp32, pow(mean + eps, -0.5), times the weight), rotate_half
//                       RoPE with the fp32 tables, q scaled by scale*log2(e). Rounding points:
//                       the reference's norm returns the input dtype (GemmaTextEncoder.swift
//                       :114), so its normed q and k are bf16, and its fp32 RoPE leaves both
//                       fp32. Here q is normed, rotated and scaled in fp32 without that
//                       rounding and kept as two bf16 parts (hi + lo, ~16 significant bits)
//                       [B][Hq][T][D]; k is rotated from its unrounded normed value and
//                       rounded once, after the rotation, to the single bf16 part the products
//                       take -- one rounding, as the reference's, at a different point. Both
//                       differences bring the result nearer the exact one than the
//                       reference's own arithmetic (its rounded normed q alone moves the
//                       1024-token layers' max-abs error to about 2e-2).
//                       k' is stored in MFMA operand order: per (batch row, KV head, 32-key
//                       block) D/16 units of 1 KB, lane r + 32g of unit c holding channels
//                       16c + 8g .. +7 of key r.
//   gemma_vt_kernel     v with the weightless per-head norm, transposed through an LDS tile of
//                       one 32-key block into operand order: per key half hf and 32-channel
//                       block cb one 1 KB unit, lane r + 32g holding channel 32cb + r at keys
//                       16hf + 4g + {0..3, 8..11}. Keys past T are zeros in both layouts, and
//                       every operand of the attention is one coalesced 16-byte load per lane.
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
    // 8 channels per lane: a row of D = 512 takes a wave, a row of D = 256 half a wave
    constexpr int E = 8;
    constexpr int LPR = D / E;                      // lanes per row: 64 or 32
    constexpr int RPW = 64 / LPR;                   // rows per wave
    const int lane = threadIdx.x & (LPR - 1);       // lane within the row
    const int64_t row = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW +
                        ((threadIdx.x & 63) / LPR);
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
    unpack8(ldg16(src), x);
    // the reductions and the partner exchange stay within the row's lanes (offsets < LPR)
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) ss += x[e] * x[e];
#pragma unroll
    for (int off = LPR / 2; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
    const float rs = powf(ss / (float)D + p.eps, -0.5f);
    const bf16 *w = (const bf16 *)(kind == 0 ? p.q_w : p.k_w) + lane * E;
#pragma unroll
    for (int e = 0; e < E; ++e) x[e] = (x[e] * rs) * (float)w[e];
    // rotate_half pairs channel c with c +- D/2: lane l holds channels E*l ..; its partner is
    // lane l ^ LPR/2. Table column of channel c is c mod D/2.
    const int col = (lane & (LPR / 2 - 1)) * E;
    const float *cs = p.cos + (int64_t)t * (D / 2) + col;
    const float *sn = p.sin + (int64_t)t * (D / 2) + col;
    const bool first = lane < LPR / 2;
    const float f = kind == 0 ? p.q_factor : 1.0f;
    float y[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const float other = __shfl_xor(x[e], LPR / 2, 64);
        const float c = cs[e], s = sn[e];
        // first half: x1 c - x2 s; second half: x2 c + x1 s
        y[e] = (first ? x[e] * c - other * s : x[e] * c + other * s) * f;
    }
    // q as two bf16 parts (hi + lo carries ~16 significant bits into the products); k as one
    auto put = [&](bf16 *dst, const float (&z)[E]) __attribute__((always_inline)) {
        *(u32x4 *)dst = pack8(z);
    };
    if (kind == 1) {
        // k' in operand order: 32-key block t/32, 16-channel chunk c, lane (t%32) + 32g holds
        // channels 16c + 8g .. +7 of key t
        const int ch = lane * E, c = ch >> 4, g = (ch >> 3) & 1;
        const int nkb = (p.T + 31) / 32;
        const int64_t off = ((((int64_t)b * p.Hkv + h) * nkb + (t >> 5)) * (D / 16) + c) * 512 +
                            ((t & 31) + 32 * g) * 8 + (ch & 7);
        put((bf16 *)p.kp + off, y);
    } else {
        const int64_t off = (((int64_t)b * p.Hq + h) * p.T + t) * D + lane * E;
        put((bf16 *)p.qp + off, y);
        float lo[E];
#pragma unroll
        for (int e = 0; e < E; ++e) lo[e] = y[e] - (float)(bf16)y[e];
        put((bf16 *)p.qp_lo + off, lo);
    }
}

// v: the weightless per-head norm, stored transposed in operand order. One workgroup per
// (batch row, KV head, 32-key block): each wave loads its 8 token rows at once, normalises
// them into an LDS tile, then the tile leaves as the block's P.V operand units.
template <int D>
__global__ __launch_bounds__(256) void gemma_vt_kernel(const GemmaPrepParams p) {
    constexpr int E = D / 64;
    constexpr int TT = 32;                          // tokens per workgroup: one key block
    constexpr int RW = TT / 4;                      // rows per wave
    __shared__ __attribute__((aligned(16))) bf16 tile[TT][D + 8];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nkb = (p.T + TT - 1) / TT;
    const int kb = (int)(blockIdx.x % nkb), t0 = kb * TT;
    const int bh = (int)(blockIdx.x / nkb);
    const int h = bh % p.Hkv, b = bh / p.Hkv;
    float x[RW][E];
#pragma unroll
    for (int j = 0; j < RW; ++j) {
        const int t = t0 + wave * RW + j;
#pragma unroll
        for (int e = 0; e < E; ++e) x[j][e] = 0.f;
        if (t < p.T) {
            const bf16 *src = (const bf16 *)p.v + (int64_t)b * p.v_bs + (int64_t)t * p.v_rs +
                              (int64_t)h * D + lane * E;
            if constexpr (E == 8) {
                unpack8(ldg16(src), x[j]);
            } else {
                const u32x2 w = *(const u32x2 *)src;
                x[j][0] = bf_lo(w[0]); x[j][1] = bf_hi(w[0]);
                x[j][2] = bf_lo(w[1]); x[j][3] = bf_hi(w[1]);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < RW; ++j) {
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) ss += x[j][e] * x[j][e];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
        const float rs = powf(ss / (float)D + p.eps, -0.5f);
#pragma unroll
        for (int e = 0; e < E; ++e) tile[wave * RW + j][lane * E + e] = (bf16)(x[j][e] * rs);
    }
    __syncthreads();
    // Operand units of the block: per key half hf and 32-channel block cb one 1 KB unit whose
    // lane r + 32g holds channel 32cb + r at keys 32kb + 16hf + 4g + {0..3, 8..11}. Keys past T
    // are written as zeros (their weights are 0, and 0 * 0 keeps the products finite); the
    // last block's k' rows past T are zeroed too.
    bf16 *vbase = (bf16 *)p.vt + (((int64_t)b * p.Hkv + h) * nkb + kb) * (D * 32);
    for (int u = threadIdx.x; u < 2 * (D / 32) * 64; u += 256) {
        const int l = u & 63, rest = u >> 6;
        const int cb = rest % (D / 32), hf = rest / (D / 32);
        const int r = l & 31, g = l >> 5;
        float f[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int tl = 16 * hf + 4 * g + (e & 3) + 8 * (e >> 2);
            f[e] = t0 + tl < p.T ? (float)tile[tl][32 * cb + r] : 0.f;
        }
        *(u32x4 *)(vbase + ((int64_t)hf * (D / 32) + cb) * 512 + l * 8) = pack8(f);
    }
    if ((p.T & 31) && kb == nkb - 1) {
        bf16 *kbase = (bf16 *)p.kp + (((int64_t)b * p.Hkv + h) * nkb + kb) * (D * 32);
        for (int u = threadIdx.x; u < (D / 16) * 64; u += 256) {
            const int l = u & 63;
            if (t0 + (l & 31) >= p.T) *(u32x4 *)(kbase + u * 8) = u32x4{0, 0, 0, 0};
        }
    }
}

// ---- attention -----------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void gemma_attn_kernel(const GemmaAttnParams p) {
    constexpr int DS = D / 4;                       // channels per wave
    constexpr int NCS = DS / 16;                    // 16-channel chunks of the wave's S slice
    constexpr int NDS = DS / 32;                    // 32-channel blocks of the wave's O slice
    // partial S per wave, double-buffered; 20-float lane rows keep the 16-byte accesses of
    // 16 lanes on distinct banks
    __shared__ __attribute__((aligned(16))) float sS[2][4][64][20];

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
    // K' and V'^T of this KV head in operand order: per 32-key block, one 1 KB unit (64 lanes x
    // 16 bytes) per operand, so each operand is one coalesced 16-byte load per lane.
    const int nkb_all = (T + 31) / 32;
    const bf16 *Kt = (const bf16 *)p.kp + ((int64_t)b * p.Hkv + kvh) * nkb_all * (D * 32) +
                     (wave * NCS) * 512 + lane * 8;
    const bf16 *Vt = (const bf16 *)p.vt + ((int64_t)b * p.Hkv + kvh) * nkb_all * (D * 32) +
                     (wave * NDS) * 512 + lane * 8;

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
    // The row's allowed keys as one range [k_lo, k_hi]: all keys for a row inside the left
    // padding, else causal (k <= q), past the padding (k >= fv) and inside the window
    // (q - k < window); k_hi <= T - 1 also masks the keys past T of the last block.
    const int k_lo = free_row ? 0 : max(fv, p.window > 0 ? q - p.window + 1 : 0);
    const int k_hi = free_row ? T - 1 : min(q, T - 1);

    f32x16 o[NDS];
#pragma unroll
    for (int db = 0; db < NDS; ++db) o[db] = splat16(0.f);
    float m = -INFINITY, l = 0.f;
    // Operands in flight: the block's K' rows are fetched one block ahead, its V'^T rows at
    // the top of the block, so their latency overlaps the products, the exchange and the
    // softmax instead of stalling each step.
    auto load_k = [&](int kb, u32x4 (&kx)[NCS]) __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < NCS; ++c) kx[c] = ldg16(Kt + ((int64_t)kb * (D / 16) + c) * 512);
    };
    // V'^T operand units of a block: channel block wave*NDS + db, key half hf
    auto load_v = [&](int kb, u32x4 (&vx)[2][NDS]) __attribute__((always_inline)) {
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int db = 0; db < NDS; ++db)
                vx[hf][db] = ldg16(Vt + (((int64_t)kb * 2 + hf) * (D / 32) + db) * 512);
    };
    // D = 256 has the registers to hold the next block's V'^T as well (one block ahead, like
    // K', in two buffers that alternate by block parity); D = 512 loads it at the top of its
    // block.
    constexpr bool kVAhead = D <= 256;
    u32x4 kx[NCS];
    u32x4 va[2][NDS], vb[2][NDS];
    load_k(kb_lo, kx);
    if constexpr (kVAhead) load_v(kb_lo, va);
    // One 32-key block; `buf` selects the LDS exchange buffer, vc holds this block's V'^T
    // (when loaded ahead) and vn receives the next block's.
    auto block = [&](int kb, auto bufc, u32x4 (&vc)[2][NDS], u32x4 (&vn)[2][NDS])
        __attribute__((always_inline)) {
        constexpr int buf = decltype(bufc)::value;
        u32x4 vl[2][NDS];
        if constexpr (!kVAhead) load_v(kb, vl);
        u32x4 (&vx)[2][NDS] = kVAhead ? vc : vl;
        // partial S^T over this wave's channels: the hi and lo parts of q' in two chains
        f32x16 sh = splat16(0.f), sl = splat16(0.f);
#pragma unroll
        for (int c = 0; c < NCS; ++c) {
            const bf16x8 a = __builtin_bit_cast(bf16x8, kx[c]);
            sh = mfma32(a, qf[c], sh);
            sl = mfma32(a, ql[c], sl);
        }
        if (kb < kb_hi) {
            load_k(kb + 1, kx);
            if constexpr (kVAhead) load_v(kb + 1, vn);
        }
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4)
            *(f32x4 *)&sS[buf][wave][lane][4 * i4] =
                f32x4{sh[4 * i4] + sl[4 * i4], sh[4 * i4 + 1] + sl[4 * i4 + 1],
                      sh[4 * i4 + 2] + sl[4 * i4 + 2], sh[4 * i4 + 3] + sl[4 * i4 + 3]};
        __syncthreads();
        f32x16 s;
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
            const f32x4 p0 = *(const f32x4 *)&sS[buf][0][lane][4 * i4];
            const f32x4 p1 = *(const f32x4 *)&sS[buf][1][lane][4 * i4];
            const f32x4 p2 = *(const f32x4 *)&sS[buf][2][lane][4 * i4];
            const f32x4 p3 = *(const f32x4 *)&sS[buf][3][lane][4 * i4];
#pragma unroll
            for (int e = 0; e < 4; ++e) s[4 * i4 + e] = ((p0[e] + p1[e]) + p2[e]) + p3[e];
        }
        // mask: key k = 32kb + 8(i>>2) + 4g + (i&3) for query q
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int k = 32 * kb + 8 * (i >> 2) + 4 * g + (i & 3);
            s[i] = ((k >= k_lo) & (k <= k_hi)) ? s[i] : -INFINITY;
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
                const bf16x8 a = __builtin_bit_cast(bf16x8, vx[hf][db]);
                o[db] = mfma32(a, __builtin_bit_cast(bf16x8, wh[hf]), o[db]);
                o[db] = mfma32(a, __builtin_bit_cast(bf16x8, wl[hf]), o[db]);
            }
    };
    for (int kb = kb_lo; kb <= kb_hi; kb += 2) {
        block(kb, std::integral_constant<int, 0>{}, va, vb);
        if (kb + 1 <= kb_hi) block(kb + 1, std::integral_constant<int, 1>{}, vb, va);
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
    // rows per workgroup: four waves of one (D = 512) or two (D = 256) rows
    const int64_t rows = (int64_t)p.B * p.T * (p.Hq + p.Hkv);
    const int64_t rows_wg = D == 512 ? 4 : 8;
    const dim3 grid((unsigned)((rows + rows_wg - 1) / rows_wg)), block(256);
    const dim3 vgrid((unsigned)((int64_t)p.B * p.Hkv * ((p.T + 31) / 32)));
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
