// Attention kernel for short key ranges: text cross-attention over its valid keys, and the
// cross-modal call of the video queries over the audio keys (Sources/LTXModules/
// DiTBlock.swift:390-415, :470-508). The whole K and V of a (batch, head) stay resident in
// LDS and every wave streams blocks of 32 queries past them.
//
// These calls move far more bytes than they compute (Q in and O out per query, a few KB of
// K/V per head): HBM bounds them, and what matters is keeping loads in flight. A workgroup of
// eight waves (twelve at D = 64) owns one (batch, head) and 1/G of its query blocks. It copies
// the head's K and V into LDS once (LDS DMA, the tile layout of fmha_dma.hip: K rows swizzled
// for 16-byte operand reads, V rows for transposing reads), then each wave walks its own
// query blocks with no further barrier. At D = 128 a wave loads the next block's Q, statistic
// and RoPE table rows into registers while it computes the current one, two waves per SIMD;
// at D = 64 three waves per SIMD overlap one another's loads instead. Per block: S^T = K.Q'^T
// on the matrix cores (Q' normalised, rotated and scaled by scale*log2(e) in fp32, rounded
// once), the first 32-key block sets the row max, p = exp2(s - m) rounded to bf16 with row
// sums of those bf16 weights, O^T += V^T.P^T, then O * gate / l is staged in the wave's LDS
// area and stored as whole 16-byte units of the output rows.
#include "lds_copy.hpp"

namespace ltx {
namespace {

// Waves of 32-query blocks, several per SIMD, so that one wave's arithmetic overlaps the
// others' loads (four waves of 64-query blocks, one per SIMD, reached 2.9-3.6 TB/s on the
// block set's calls against 3.8-5.0 TB/s with two waves of 32). At D = 128 a workgroup holds
// eight waves, each prefetching its next block into registers; at D = 64 it holds twelve,
// three per SIMD, which load their blocks when they reach them (the prefetch registers do not
// fit three waves; this shape took the 3120x126 video-over-audio call from 20 to 16 us). The
// per-group arrays below are indexed by the 32-query group of the wave block (QB of them).
constexpr int short_waves(int D) { return D == 64 ? 12 : 8; }

template <int D, bool ROPE>
__global__ __attribute__((amdgpu_flat_work_group_size(short_waves(D) * 64, short_waves(D) * 64),
                          amdgpu_waves_per_eu(short_waves(D) / 4, short_waves(D) / 4)))
void fmha_short_kernel(const FmhaParams p) {
    constexpr int NC = D / 16, NDB = D / 32, KU = D / 8;
    constexpr int QB = 1;                             // 32-query groups per wave block
    constexpr int SQW = 32 * QB;                      // queries per wave block
    constexpr int SNW = short_waves(D);               // waves per workgroup
    constexpr bool PREFETCH = SNW == 8;               // next block's loads during this one
    constexpr int TE = KT * D;                        // elements of a 64-key tile
    constexpr int TILES = short_max_keys(D) / KT;     // resident tiles
    constexpr int CPT = TE / 512;                     // 1 KB copies per tile
    __shared__ __attribute__((aligned(16))) bf16 sK[TILES * TE];
    __shared__ __attribute__((aligned(16))) bf16 sV[TILES * TE];
    __shared__ __attribute__((aligned(16))) bf16 sO[SNW * SQW * D];
    __shared__ __attribute__((aligned(16))) bf16 sW[D];   // q_norm.weight of the head

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 31;
    const int g = lane >> 5;
    // At D = 64 the row sums of P run on the matrix cores: read as a 16x16x32 B operand, lane
    // L of P holds 8 weights of query (L & 15) + 16 * ((L >> 4) & 1); row m of this 0/1
    // selector takes the lanes of query (L & 15) + 16 * (m >= 8), so rows 0-7 of the 16x16
    // sums hold queries 0-15 of the block and rows 8-15 queries 16-31 (5-8% faster there; at
    // D = 128, whose eight waves already fill the register file, the VALU adds stay: 1-3%
    // faster than the products).
    constexpr bool MSUM = D == 64;
    bf16x8 rsel;
    {
        const uint32_t one2 = (((lane >> 4) & 1) == ((lane & 15) >= 8 ? 1 : 0)) ? 0x3f803f80u : 0u;
        rsel = __builtin_bit_cast(bf16x8, u32x4{one2, one2, one2, one2});
    }
    const int G = p.short_groups;
    const int bh = blockIdx.x / G, gi = blockIdx.x - bh * G;
    const int h = bh % p.H, b = bh / p.H;
    const int n_valid = p.valid[b];                   // 1 .. short_max_keys(D) (host)
    const int ntiles = (n_valid + KT - 1) / KT;
    const int nkb = (n_valid + 31) / 32;
    const bool ragged = (n_valid & 31) != 0;

    // ---- the head's K and V into LDS -------------------------------------------------
    {
        const bf16 *Kb = (const bf16 *)p.k + (int64_t)b * p.k_bs + (int64_t)h * p.k_hs;
        const bf16 *Vb = (const bf16 *)p.v + (int64_t)b * p.v_bs + (int64_t)h * p.v_hs;
        const int krow = (int)(p.k_rs * 2), vrow = (int)(p.v_rs * 2);
        // rows past the valid keys arrive as zeros
        const u32x4 rk = rsrc_words(Kb, (int64_t)n_valid * krow);
        const u32x4 rv = rsrc_words(Vb, (int64_t)n_valid * vrow);
        for (int t = 0; t < ntiles; ++t)
            for (int c = wave; c < CPT; c += SNW) {
                const int q = c * 64 + lane;          // 16-byte unit of the tile
                const int row = q / KU, slot = q % KU;
                const int key = t * KT + row;
                copy_all(rk, (uint32_t)(uintptr_t)((lds_bf16 *)sK + t * TE + c * 512),
                         key * krow + 16 * swz<KU>(row, slot));
                copy_all(rv, (uint32_t)(uintptr_t)((lds_bf16 *)sV + t * TE + c * 512),
                         key * vrow + 16 * vswz<KU>(row, slot));
            }
        if (p.q_rstd && tid < D / 8)
            *(u32x4 *)(sW + 8 * tid) = ldg16((const bf16 *)p.q_w + h * D + 8 * tid);
        wait_copies();
        __syncthreads();
    }
    const lds_bf16 *Ks = (const lds_bf16 *)sK;
    const lds_bf16 *Vs = (const lds_bf16 *)sV;
    // K operand of S^T: key row 32*kb + r, channels 16c + 8g .. +7.
    auto k_opnd = [&](int kb, int c) __attribute__((always_inline)) {
        const int row = kb * 32 + r;
        return *(const __attribute__((address_space(3))) bf16x8 *)(Ks + row * D + 8 * swz<KU>(row, 2 * c + g));
    };
    // V^T operand of keys 16*t4 .. +15 (t4 counts 16-key groups from key 0), channels
    // 32*db .. +31, in the key order of P's registers (as in fmha_dma.hip).
    const int i16 = lane & 15;
    const int hsel = (lane >> 4) & 1;
    auto v_opnd = [&](int t4, int db) __attribute__((always_inline)) {
        const int row0 = 16 * t4 + 4 * g + (i16 >> 2);
        const int u = 4 * db + 2 * hsel + ((i16 & 3) >> 1);
        const int half = 4 * (i16 & 1);
        const u32x2 lo = ds_read_tr(Vs + row0 * D + 8 * vswz<KU>(row0, u) + half);
        const u32x2 hi = ds_read_tr(Vs + (row0 + 8) * D + 8 * vswz<KU>(row0 + 8, u) + half);
        return __builtin_bit_cast(bf16x8, u32x4{lo[0], lo[1], hi[0], hi[1]});
    };

    // ---- Q blocks of this wave -------------------------------------------------------
    const int nqb = (p.Lq + SQW - 1) / SQW;
    const int stride = G * SNW;
    const bf16 *Qb = (const bf16 *)p.q + (int64_t)b * p.q_bs + (int64_t)h * p.q_hs;
    const rsrc_t rq = make_rsrc(Qb, (int64_t)p.Lq * p.q_rs * 2);   // rows past Lq read zero
    const int qrow = (int)(p.q_rs * 2);
    const bool norm = p.q_rstd != nullptr;
    struct Raw {
        u32x4 x[QB][NC];
        u32x4 cs[QB][ROPE ? NC / 2 : 1], sn[QB][ROPE ? NC / 2 : 1];
        float rs[QB];
    };
    auto fetch = [&](int j, Raw &f) __attribute__((always_inline)) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            const int qi = j * SQW + 32 * qb + r;
            const int qc = min(qi, p.Lq - 1);
#pragma unroll
            for (int c = 0; c < NC; ++c)
                f.x[qb][c] = bload16(rq, (uint32_t)(qi * qrow + (16 * c + 8 * g) * 2));
            f.rs[qb] = norm ? p.q_rstd[(int64_t)b * p.Lq + qc] : 1.0f;
            if constexpr (ROPE) {
                const int64_t toff = ((int64_t)h * p.Lq + qc) * (D / 2);
#pragma unroll
                for (int c = 0; c < NC / 2; ++c) {
                    f.cs[qb][c] = ldg16((const bf16 *)p.q_cos + toff + 16 * c + 8 * g);
                    f.sn[qb][c] = ldg16((const bf16 *)p.q_sin + toff + 16 * c + 8 * g);
                }
            }
        }
    };
    // The Q prologue of load_q (fmha_device.hpp): norm with the statistic and the weight,
    // split-half rotation, scale*log2(e), one bf16 rounding.
    auto convert = [&](const Raw &f, bf16x8 (&qf)[QB][NC]) __attribute__((always_inline)) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            float x[NC][8];
#pragma unroll
            for (int c = 0; c < NC; ++c) unpack8(f.x[qb][c], x[c]);
            if (norm) {
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    float w[8];
                    unpack8(*(const u32x4 *)(sW + 16 * c + 8 * g), w);
#pragma unroll
                    for (int e = 0; e < 8; ++e) x[c][e] = (x[c][e] * f.rs[qb]) * w[e];
                }
            }
            if constexpr (ROPE) {
#pragma unroll
                for (int c = 0; c < NC / 2; ++c) {
                    float fc[8], fs[8];
                    unpack8(f.cs[qb][c], fc);
                    unpack8(f.sn[qb][c], fs);
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
    };

    bf16 *Os = sO + wave * SQW * D;                   // this wave's staging area
    bf16 *Ob = (bf16 *)p.o + (int64_t)b * p.o_bs + (int64_t)h * p.o_hs;
    int j = gi * SNW + wave;
    Raw cur;
    if (PREFETCH && j < nqb) fetch(j, cur);
    for (; j < nqb; j += stride) {
        bf16x8 qf[QB][NC];
        if (!PREFETCH) fetch(j, cur);
        convert(cur, qf);
        if (PREFETCH && j + stride < nqb) fetch(j + stride, cur);  // in flight during this block

        f32x16 o[NDB][QB];
        float l[QB];
        f32x16 negm[QB];
        f32x4 lsum[QB];              // MSUM: the row sums' accumulators
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
            for (int db = 0; db < NDB; ++db) o[db][qb] = splat16(0.f);
            l[qb] = 0.f;
            negm[qb] = splat16(0.f);
            lsum[qb] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        bool over = false;
        // S of key block kb, accumulated from C = init; keys past the valid ones -> -inf.
        auto s_block = [&](int kb, f32x16 (&s)[QB]) __attribute__((always_inline)) {
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const bf16x8 a = k_opnd(kb, c);
#pragma unroll
                for (int qb = 0; qb < QB; ++qb)
                    s[qb] = mfma32(a, qf[qb][c], c == 0 ? negm[qb] : s[qb]);
            }
            if (ragged && kb == nkb - 1) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int key = 32 * kb + 8 * (i >> 2) + 4 * g + (i & 3);
#pragma unroll
                    for (int qb = 0; qb < QB; ++qb)
                        if (key >= n_valid) s[qb][i] = -INFINITY;
                }
            }
        };
        // P = exp2(S) in bf16, the row sums of those weights, O^T += V^T.P^T.
        auto p_block = [&](const f32x16 (&s)[QB], int kb) __attribute__((always_inline)) {
            bf16x8 pn[QB][2];
            float ts[QB];
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) ts[qb] = 0.f;
#pragma unroll
            for (int qb = 0; qb < QB; ++qb)
#pragma unroll
                for (int hf = 0; hf < 2; ++hf) {
                    u32x4 w;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float x0 = __builtin_amdgcn_exp2f(s[qb][8 * hf + 2 * e]);
                        const float x1 = __builtin_amdgcn_exp2f(s[qb][8 * hf + 2 * e + 1]);
                        if constexpr (MSUM) {
                            w[e] = pack_bf2(x0, x1);
                        } else {
                            w[e] = pack_bf2_opaque(x0, x1);
                            ts[qb] = add_bf2(ts[qb], w[e]);
                        }
                    }
                    pn[qb][hf] = __builtin_bit_cast(bf16x8, w);
                    if constexpr (MSUM)
                        lsum[qb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(rsel, pn[qb][hf],
                                                                           lsum[qb], 0, 0, 0);
                }
            if constexpr (!MSUM) {
#pragma unroll
                for (int qb = 0; qb < QB; ++qb) {
                    over |= !(ts[qb] <= kRebaseBound);
                    l[qb] += ts[qb];
                }
            }
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                for (int db = 0; db < NDB; ++db) {
                    const bf16x8 a = v_opnd(2 * kb + hf, db);
#pragma unroll
                    for (int qb = 0; qb < QB; ++qb) o[db][qb] = mfma32(a, pn[qb][hf], o[db][qb]);
                }
        };
        // Pass 0: the first block's row max is the reference for all blocks (softmax is
        // exact under any shift) while no block's weights exceed 2^64. Pass 1, only when some
        // row outgrew it (pathological inputs): the true row max first, every weight <= 1.
        for (int pass = 0; pass < 2; ++pass) {
            if (pass == 1) {
                float mt[QB];
#pragma unroll
                for (int qb = 0; qb < QB; ++qb) {
                    mt[qb] = -INFINITY;
                    negm[qb] = splat16(0.f);
                }
                for (int kb = 0; kb < nkb; ++kb) {
                    f32x16 s[QB];
                    s_block(kb, s);
#pragma unroll
                    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
                        for (int i = 0; i < 16; ++i) mt[qb] = fmaxf(mt[qb], s[qb][i]);
                }
#pragma unroll
                for (int qb = 0; qb < QB; ++qb) {
                    negm[qb] = splat16(-fmaxf(mt[qb], xlane32(mt[qb])));
#pragma unroll
                    for (int db = 0; db < NDB; ++db) o[db][qb] = splat16(0.f);
                    l[qb] = 0.f;
                    lsum[qb] = f32x4{0.f, 0.f, 0.f, 0.f};
                }
                over = false;
            }
            for (int kb = 0; kb < nkb; ++kb) {
                f32x16 s[QB];
                s_block(kb, s);
                if (pass == 0 && kb == 0) {
#pragma unroll
                    for (int qb = 0; qb < QB; ++qb) {
                        float mx = s[qb][0];
#pragma unroll
                        for (int i = 1; i < 16; ++i) mx = fmaxf(mx, s[qb][i]);
                        mx = fmaxf(mx, xlane32(mx));
                        negm[qb] = splat16(-mx);
                        s[qb] -= splat16(mx);
                    }
                }
                p_block(s, kb);
            }
            if constexpr (MSUM) {
                // lane (r, g) takes query r's sum from the accumulator lane that holds it, in
                // the g = 0 lane so that l + xlane32(l) is the sum; a sum past 2^64 sends the
                // block to pass 1
#pragma unroll
                for (int qb = 0; qb < QB; ++qb) {
                    const float full = __shfl(lsum[qb][0], (r & 15) + 32 * (r >> 4), 64);
                    over |= !(full <= kRebaseBound);
                    l[qb] = g == 0 ? full : 0.f;
                }
            }
            if (__builtin_amdgcn_ballot_w64(over) == 0) break;
        }

        // ---- epilogue: O * gate / l, staged in LDS, whole 16-byte units stored ---------
        const int q0 = j * SQW;
        float inv[QB];
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
            inv[qb] = gate_factor(p.gate, p.g_bs, p.g_rs, p.g_hs, b, min(q0 + 32 * qb + r, p.Lq - 1), h) /
                      (l[qb] + xlane32(l[qb]));
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int i4 = 0; i4 < 4; ++i4) {
                    const int row = 32 * qb + r;
                    u32x2 w;
                    w[0] = pack_bf2(o[db][qb][4 * i4 + 0] * inv[qb], o[db][qb][4 * i4 + 1] * inv[qb]);
                    w[1] = pack_bf2(o[db][qb][4 * i4 + 2] * inv[qb], o[db][qb][4 * i4 + 3] * inv[qb]);
                    *(u32x2 *)(Os + row * D + 8 * swz<KU>(row, 4 * db + i4) + 4 * g) = w;
                }
        // The wave's LDS operations complete in order: the reads below see the writes above,
        // and the next block's writes come after these reads.
#pragma unroll
        for (int it = 0; it < SQW * KU / 64; ++it) {
            const int u = lane + 64 * it;
            const int row = u / KU, c = u % KU;
            const int q = q0 + row;
            if (q < p.Lq)
                *(u32x4 *)(Ob + (int64_t)q * p.o_rs + 8 * c) =
                    *(const u32x4 *)(Os + row * D + 8 * swz<KU>(row, c));
        }
    }
}

}  // namespace

int launch_fmha_short(const FmhaParams &p, int D, void *stream) {
    const dim3 grid(p.grid), block(short_waves(D) * 64);
    hipStream_t st = (hipStream_t)stream;
    const bool rope = p.q_cos != nullptr;
    // D = 128 with RoPE does not fit the register file with a block in flight; the host plan
    // sends such calls to the other kernels.
    if (D == 128 && rope) return (int)hipErrorInvalidValue;
    if (D == 128) hipLaunchKernelGGL((fmha_short_kernel<128, false>), grid, block, 0, st, p);
    else if (rope) hipLaunchKernelGGL((fmha_short_kernel<64, true>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((fmha_short_kernel<64, false>), grid, block, 0, st, p);
    return (int)hipGetLastError();
}

}  // namespace ltx
