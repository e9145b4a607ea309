// Fused DiT attention for MI355X (gfx950): bf16 MFMA flash attention with the QK-RMSNorm and
// split RoPE of the LTX 2.5 DiT (Sources/LTXModules/DiTAttention.swift:358-381) fused into
// the Q/K loads.
//
// Work decomposition
//   One workgroup = 4 waves; each wave owns 64 queries of one (batch, head) and walks the key
//   sequence in tiles of 64 keys. K and V tiles are staged through LDS (double buffered, with
//   the next tile prefetched into registers while the current one is computed).
//
// MFMA mapping (v_mfma_f32_32x32x16_bf16; C/D element i of lane l sits at column l%32,
// row 8*(i/4) + 4*(l/32) + i%4)
//   S^T = K . Q'^T   A = K rows from LDS (key x d), B = Q' from registers (d x query).
//                    Each lane therefore holds ONE query and 16 keys of every 32x32 block, so
//                    the softmax row statistics are lane-local plus one exchange with lane^32.
//   O^T = V^T . P^T  A = V^T from LDS (d x key), B = P^T taken straight from the S registers
//                    (converted to bf16), so P never leaves the registers.
//   The reduction index of an MFMA can be permuted freely as long as A and B agree; V^T is
//   stored with bits 2 and 3 of the key index swapped so the 8 keys a lane supplies for P are
//   contiguous in LDS and every A operand is a single 16-byte LDS read.
//
// Softmax
//   Q is pre-multiplied by scale*log2(e) (in fp32, before its one bf16 rounding), so
//   p = exp2(s - m). The running max m is taken from the first tile and then kept as long as
//   no p of a later tile would exceed 2^64 (checked on the tile's bf16 row sum); the MFMA
//   accumulator is initialised with -m, so the subtraction costs nothing. When a tile does
//   overflow the bound the wave rebases (rescales O and l) and recomputes that tile's p --
//   exact, and rare. The row sum is accumulated from the bf16-rounded p that feed P.V, so the
//   weights applied are exactly the weights normalised.
#include <type_traits>

#include "fmha_device.hpp"

namespace ltx {
namespace {

// ------------------------------------------------------------------------------------------
// Main kernel
// ------------------------------------------------------------------------------------------
template <int D, bool KFUSED>
struct FmhaTile {
    static constexpr int NC = D / 16;       // 16-wide reduction chunks of Q.K^T
    static constexpr int NDB = D / 32;      // 32-row blocks of O^T
    static constexpr int KS = D + 8;        // K LDS row stride (elements)
    static constexpr int VS = KT + 8;       // V^T LDS row stride (elements)
    static constexpr int K_ELEMS = KT * KS;
    static constexpr int V_ELEMS = D * VS;
    static constexpr int STAGE = K_ELEMS + V_ELEMS;
    static constexpr int OS = D + 8;        // epilogue staging row stride
    static constexpr int LDS_ELEMS =
        (2 * STAGE > NW * QW * OS) ? 2 * STAGE : NW * QW * OS;

    // K staging, plain: 16-byte chunks per thread
    static constexpr int KCPR = D / 8;                  // chunks per row
    static constexpr int KCH = KT * KCPR / NT;          // chunks per thread
    static constexpr int KROWS_STEP = NT / KCPR;
    // K staging, fused: pair units (chunk c and c + D/16) per thread
    static constexpr int KPPR = D / 16;
    static constexpr int KFP = KT * KPPR / NT;
    static constexpr int KFROWS_STEP = NT / KPPR;
    // V staging: units of 4 keys x 8 channels
    static constexpr int VUNITS = (KT / 4) * (D / 8);
    static_assert(KCH >= 1 && KFP >= 1 && VUNITS <= NT, "tile geometry");
};

template <int D, bool KFUSED>
__global__ __attribute__((amdgpu_flat_work_group_size(NT, NT), amdgpu_waves_per_eu(1, 1)))
void fmha_fwd_kernel(const FmhaParams p) {
    using T = FmhaTile<D, KFUSED>;
    constexpr int NC = T::NC, NDB = T::NDB, KS = T::KS, VS = T::VS;
    __shared__ __attribute__((aligned(16))) bf16 smem[T::LDS_ELEMS];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 31;
    const int g = lane >> 5;

    const WorkItem wi = work_item(p);
    const int qblk = wi.qblk, h = wi.h, b = wi.b;
    const int n_valid = p.valid[b];
    const int t_begin = wi.t_begin, t_end = wi.t_end;

    const int q0 = qblk * QT + wave * QW;
    const bool active = q0 < p.Lq;

    const bf16 *Kb = (const bf16 *)p.k + (int64_t)b * p.k_bs + (int64_t)h * p.k_hs;
    const bf16 *Vb = (const bf16 *)p.v + (int64_t)b * p.v_bs + (int64_t)h * p.v_hs;

    // ---- Q: load, normalise, rotate, scale, round once -------------------------------
    bf16x8 qf[2][NC];
    load_q<D>(p, b, h, q0, active, r, g, qf);

    // ---- staging (global -> registers -> LDS); K runs one tile ahead of V --------------
    // Buffer loads: the resource of tile t starts at key t*KT and ends at the last valid
    // key, so rows past it read as zero without a branch.
    const int64_t krow_bytes = p.k_rs * 2, vrow_bytes = p.v_rs * 2;
    auto tile_rsrc = [&](const bf16 *base, int64_t row_elems, int tile) __attribute__((always_inline)) {
        const int rows = min(KT, n_valid - tile * KT);
        return make_rsrc(base + (int64_t)tile * KT * row_elems, (int64_t)rows * row_elems * 2);
    };
    u32x4 kreg[KFUSED ? 2 * T::KFP : T::KCH];
    u32x4 kcs[KFUSED ? T::KFP : 1], ksn[KFUSED ? T::KFP : 1];
    float krs[KFUSED ? T::KFP : 1];
    u32x4 vreg[4];
    // k_norm weights of the thread's two channel units, kept as bf16 (unpacked where used)
    u32x4 kw1p = {0u, 0u, 0u, 0u}, kw2p = {0u, 0u, 0u, 0u};
    if (KFUSED && p.k_rstd) {
        const int c = tid % T::KPPR;
        const bf16 *w = (const bf16 *)p.k_w + h * D;
        kw1p = ldg16(w + 8 * c);
        kw2p = ldg16(w + D / 2 + 8 * c);
    }
    const bool vthr = tid < T::VUNITS;
    const int vkg = tid & 15;
    const int vdc = tid >> 4;

    auto load_k = [&](int tile) __attribute__((always_inline)) {
        const rsrc_t rk = tile_rsrc(Kb, p.k_rs, tile);
        if (!KFUSED) {
            const int c = tid % T::KCPR;
#pragma unroll
            for (int i = 0; i < T::KCH; ++i) {
                const int row = tid / T::KCPR + i * T::KROWS_STEP;
                kreg[i] = bload16(rk, (uint32_t)(row * krow_bytes + 16 * c));
            }
        } else {
            const int c = tid % T::KPPR;
#pragma unroll
            for (int i = 0; i < T::KFP; ++i) {
                const int row = tid / T::KPPR + i * T::KFROWS_STEP;
                const int key = min(tile * KT + row, n_valid - 1);
                kreg[2 * i] = bload16(rk, (uint32_t)(row * krow_bytes + 16 * c));
                kreg[2 * i + 1] = bload16(rk, (uint32_t)(row * krow_bytes + D + 16 * c));
                krs[i] = p.k_rstd ? p.k_rstd[(int64_t)b * p.Lk + key] : 1.0f;
                if (p.k_cos) {
                    const int64_t toff = ((int64_t)h * p.Lk + key) * (D / 2) + 8 * c;
                    kcs[i] = ldg16((const bf16 *)p.k_cos + toff);
                    ksn[i] = ldg16((const bf16 *)p.k_sin + toff);
                }
            }
        }
    };
    auto load_v = [&](int tile) __attribute__((always_inline)) {
        if (vthr) {
            const rsrc_t rv = tile_rsrc(Vb, p.v_rs, tile);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                vreg[i] = bload16(rv, (uint32_t)((4 * vkg + i) * vrow_bytes + 16 * vdc));
        }
    };
    auto store_k = [&](int tile) __attribute__((always_inline)) {
        bf16 *Ks = smem + (tile & 1) * T::STAGE;
        if (!KFUSED) {
            const int c = tid % T::KCPR;
#pragma unroll
            for (int i = 0; i < T::KCH; ++i) {
                const int row = tid / T::KCPR + i * T::KROWS_STEP;
                *(u32x4 *)(Ks + row * KS + 8 * c) = kreg[i];
            }
        } else {
            const int c = tid % T::KPPR;
#pragma unroll
            for (int i = 0; i < T::KFP; ++i) {
                const int row = tid / T::KPPR + i * T::KFROWS_STEP;
                float x1[8], x2[8];
                unpack8(kreg[2 * i], x1);
                unpack8(kreg[2 * i + 1], x2);
                if (p.k_rstd) {
                    u32x4 w1 = kw1p, w2 = kw2p;
                    asm volatile("" : "+v"(w1), "+v"(w2));   // unpacked here, not held as fp32
                    float kw1[8], kw2[8];
                    unpack8(w1, kw1);
                    unpack8(w2, kw2);
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        x1[e] = (x1[e] * krs[i]) * kw1[e];
                        x2[e] = (x2[e] * krs[i]) * kw2[e];
                    }
                }
                if (p.k_cos) {
                    float fc[8], fs[8];
                    unpack8(kcs[i], fc);
                    unpack8(ksn[i], fs);
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float a = x1[e], bb = x2[e];
                        x1[e] = a * fc[e] - bb * fs[e];
                        x2[e] = bb * fc[e] + a * fs[e];
                    }
                }
                *(u32x4 *)(Ks + row * KS + 8 * c) = pack8(x1);
                *(u32x4 *)(Ks + row * KS + D / 2 + 8 * c) = pack8(x2);
            }
        }
    };
    auto store_v = [&](int tile) __attribute__((always_inline)) {
        bf16 *Vt = smem + (tile & 1) * T::STAGE + T::K_ELEMS;
        if (vthr) {
            const int pos = vt_pos(4 * vkg);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t w0 = vreg[0][j >> 1], w1 = vreg[1][j >> 1];
                const uint32_t w2 = vreg[2][j >> 1], w3 = vreg[3][j >> 1];
                u32x2 out;
                if ((j & 1) == 0) {
                    out[0] = (w0 & 0xffffu) | (w1 << 16);
                    out[1] = (w2 & 0xffffu) | (w3 << 16);
                } else {
                    out[0] = (w0 >> 16) | (w1 & 0xffff0000u);
                    out[1] = (w2 >> 16) | (w3 & 0xffff0000u);
                }
                *(u32x2 *)(Vt + (8 * vdc + j) * VS + pos) = out;
            }
        }
    };

    // ---- running state ----------------------------------------------------------------
    f32x16 o[NDB][2];
#pragma unroll
    for (int db = 0; db < NDB; ++db) o[db][0] = o[db][1] = splat16(0.f);
    float m[2] = {0.f, 0.f};   // running max (log2 units), identical in lanes l and l^32
    float l[2] = {0.f, 0.f};   // this lane's share of the row sum
    f32x16 negm[2] = {splat16(0.f), splat16(0.f)};

    // Software pipeline over 32-key blocks. Block s covers keys [32s, 32s+32) of tile s/2.
    // Step s issues S(s+1) = K.Q'^T - m and O += V^T.P(s-1) on the matrix cores while the
    // VALU turns S(s) into P(s). K of tile t is read by steps 2t-1 and 2t, V of tile t by
    // steps 2t+1 and 2t+2, so the window of steps {2t-1, 2t} (opened by one barrier) reads
    // only K(t) and V(t-1) and writes K(t+1) and V(t) into the other halves of the double
    // buffer.
    const int blk_begin = 2 * t_begin;
    const int blk_end = min(2 * t_end, (n_valid + 31) / 32);
    const bool ragged = (n_valid & 31) != 0;   // block blk_end-1 is partly padding
    f32x16 sc[2];            // S(s), waiting for the softmax
    bf16x8 pp[2][2];         // P(s-1) [qb][half], waiting for P.V
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        sc[qb] = splat16(0.f);
        pp[qb][0] = pp[qb][1] = __builtin_bit_cast(bf16x8, u32x4{0, 0, 0, 0});
    }

    auto qk_block = [&](int s, f32x16 (&sn)[2]) __attribute__((always_inline)) {
        const bf16 *Ks = smem + ((s >> 1) & 1) * T::STAGE;
        const int kb = s & 1;
        sn[0] = negm[0];
        sn[1] = negm[1];
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const bf16x8 a = *(const bf16x8 *)(Ks + (kb * 32 + r) * KS + 16 * c + 8 * g);
            sn[0] = mfma32(a, qf[0][c], sn[0]);
            sn[1] = mfma32(a, qf[1][c], sn[1]);
        }
    };
    auto pv_block = [&](int s) __attribute__((always_inline)) {
        const bf16 *Vt = smem + ((s >> 1) & 1) * T::STAGE + T::K_ELEMS;
        const int kb = s & 1;
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            const int t4 = 2 * kb + hf;
#pragma unroll
            for (int db = 0; db < NDB; ++db) {
                const bf16x8 a = *(const bf16x8 *)(Vt + (db * 32 + r) * VS + 16 * t4 + 8 * g);
                o[db][0] = mfma32(a, pp[0][hf], o[db][0]);
                o[db][1] = mfma32(a, pp[1][hf], o[db][1]);
            }
        }
    };
    // S(s) -> P(s) (bf16) and this lane's row-sum share ts.
    auto softmax_block = [&](const f32x16 (&sx)[2], bf16x8 (&pn)[2][2], float (&ts)[2])
        __attribute__((always_inline)) {
        ts[0] = ts[1] = 0.f;
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                u32x4 w;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    // the row sum adds exactly the bf16 weights that feed P.V
                    w[e] = pack_bf2_opaque(__builtin_amdgcn_exp2f(sx[qb][8 * hf + 2 * e]),
                                    __builtin_amdgcn_exp2f(sx[qb][8 * hf + 2 * e + 1]));
                    ts[qb] = add_bf2(ts[qb], w[e]);
                }
                pn[qb][hf] = __builtin_bit_cast(bf16x8, w);
            }
    };

    // One pipeline step. GEN: first/last blocks, ragged padding and the pipeline's fill and
    // drain; otherwise every part is present and the step is straight-line code.
    // A block whose bf16 row sum exceeds 2^64 (or is not finite) has outgrown the running max;
    // the step only records it, and the workgroup then recomputes its rows with the safe pass
    // below, so the pipelined region carries no rescaling code.
    bool overflow = false;    // wave-uniform
    // Fast step (every part present): the 2*(NC+2*NDB) matrix-core products of the step are
    // issued one at a time with a slice of the softmax of S(s) between them, and each LDS
    // operand is read two operands ahead, so the VALU work runs under the matrix cores.
    // The sched_barrier after each slice keeps the compiler from regrouping them.
    auto fast_step = [&](int s) __attribute__((always_inline)) {
        constexpr int NOP = NC + 2 * NDB;              // LDS operands per step
        constexpr int NPAIR = 16;                      // bf16 pairs of P(s) per lane
        const bf16 *Ks = smem + (((s + 1) >> 1) & 1) * T::STAGE + (((s + 1) & 1) * 32 + r) * KS + 8 * g;
        const bf16 *Vt = smem + (((s - 1) >> 1) & 1) * T::STAGE + T::K_ELEMS + r * VS
                         + 16 * (2 * ((s - 1) & 1)) + 8 * g;
        auto opnd = [&](int i) __attribute__((always_inline)) -> bf16x8 {
            if (i < NC) return *(const bf16x8 *)(Ks + 16 * i);
            const int j = i - NC, hf = j / NDB, db = j % NDB;
            return *(const bf16x8 *)(Vt + db * 32 * VS + 16 * hf);
        };
        float ts[2] = {0.f, 0.f};
        u32x4 w[2][2];
        f32x16 sn[2];
        bf16x8 a[NOP];
        a[0] = opnd(0);
        a[1] = opnd(1);
        a[2] = opnd(2);
        int pair = 0;
        auto slice = [&](int n) __attribute__((always_inline)) {
            for (int k = 0; k < n && pair < NPAIR; ++k, ++pair) {
                const int qb = pair >> 3, hf = (pair >> 2) & 1, e = pair & 3;
                w[qb][hf][e] = pack_bf2_opaque(__builtin_amdgcn_exp2f(sc[qb][8 * hf + 2 * e]),
                                        __builtin_amdgcn_exp2f(sc[qb][8 * hf + 2 * e + 1]));
                ts[qb] = add_bf2(ts[qb], w[qb][hf][e]);
            }
        };
        constexpr int PER = 2 * NOP <= NPAIR ? NPAIR / (2 * NOP) : (NPAIR + NOP - 1) / NOP;
#pragma unroll
        for (int i = 0; i < NOP; ++i) {
            if (i + 3 < NOP) a[i + 3] = opnd(i + 3);
#pragma unroll
            for (int qb = 0; qb < 2; ++qb) {
                if (i < NC) {
                    sn[qb] = mfma32(a[i], qf[qb][i], i == 0 ? negm[qb] : sn[qb]);
                } else {
                    const int j = i - NC, hf = j / NDB, db = j % NDB;
                    o[db][qb] = mfma32(a[i], pp[qb][hf], o[db][qb]);
                }
                if (qb == 1 || 2 * NOP <= NPAIR) slice(PER);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        overflow |= !(ts[0] <= kRebaseBound) || !(ts[1] <= kRebaseBound);
        l[0] += ts[0];
        l[1] += ts[1];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
            sc[qb] = sn[qb];
            pp[qb][0] = __builtin_bit_cast(bf16x8, w[qb][0]);
            pp[qb][1] = __builtin_bit_cast(bf16x8, w[qb][1]);
        }
    };

    auto step = [&](auto gen, int s) __attribute__((always_inline)) {
        constexpr bool GEN = decltype(gen)::value;
        if constexpr (!GEN) {
            fast_step(s);
            return;
        }
        const bool do_sm = !GEN || (s >= blk_begin && s < blk_end);
        const bool do_s = !GEN || (s + 1 >= blk_begin && s + 1 < blk_end);
        const bool do_pv = !GEN || (s - 1 >= blk_begin && s - 1 < blk_end);
        if (GEN && do_sm) {
            if (ragged && s == blk_end - 1) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int key = 32 * s + 8 * (i >> 2) + 4 * g + (i & 3);
                    if (key >= n_valid) sc[0][i] = sc[1][i] = -INFINITY;
                }
            }
            if (s == blk_begin) {
                // The first block of the range sets the running max.
#pragma unroll
                for (int qb = 0; qb < 2; ++qb) {
                    float mx = sc[qb][0];
#pragma unroll
                    for (int i = 1; i < 16; ++i) mx = fmaxf(mx, sc[qb][i]);
                    mx = fmaxf(mx, xlane32(mx));
                    m[qb] = mx;
                    negm[qb] = splat16(-mx);
                    sc[qb] -= splat16(mx);
                }
            }
        }
        f32x16 sn[2];
        if (do_s) qk_block(s + 1, sn);
        if (do_pv) pv_block(s - 1);
        bf16x8 pn[2][2];
        if (do_sm) {
            float ts[2];
            softmax_block(sc, pn, ts);
            overflow |= !(ts[0] <= kRebaseBound) || !(ts[1] <= kRebaseBound);
            l[0] += ts[0];
            l[1] += ts[1];
        }
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
            if (!GEN || do_s) sc[qb] = sn[qb];
            if (!GEN || do_sm) {
                pp[qb][0] = pn[qb][0];
                pp[qb][1] = pn[qb][1];
            }
        }
    };

    // ---- main loop: one barrier per 64-key tile ---------------------------------------
    // Window t = steps {2t-1, 2t}; it loads K(t+1) and V(t) and stores them after computing.
    if (t_begin < t_end) {
        load_k(t_begin);
        store_k(t_begin);
    }
    const int t_last = t_begin < t_end ? t_end : t_begin - 1;
    // Windows [t_begin, tf0) and [tf1, t_last] fill and drain the pipeline (and carry the first
    // block, the ragged block and the split edges); the windows in between are straight-line.
    int tf0 = max(t_begin, (blk_begin + 3) / 2);        // first t with 2t-2 >= blk_begin
    int tf1 = max(tf0, blk_end / 2);                     // first t with 2t+1 >= blk_end
    tf0 = min(tf0, t_last + 1);
    tf1 = min(tf1, t_last + 1);
    auto window = [&](auto gen, int t) __attribute__((always_inline)) {
        __syncthreads();
        const bool nk = t + 1 < t_end, nv = t < t_end;
        if (nk) load_k(t + 1);
        if (nv) load_v(t);
        if (active) {
            step(gen, 2 * t - 1);
            step(gen, 2 * t);
        }
        if (nk) store_k(t + 1);
        if (nv) store_v(t);
    };
    for (int t = t_begin; t < tf0; ++t) window(std::true_type{}, t);
    for (int t = tf0; t < tf1; ++t) window(std::false_type{}, t);
    for (int t = tf1; t <= t_last; ++t) window(std::true_type{}, t);

    // ---- safe pass: only when some wave's running max was outgrown -------------------
    // Tile by tile, K and V of one tile in LDS, each 32-key block rebasing O and l as soon
    // as its weights would exceed 2^64. Pathological inputs only.
    if (__syncthreads_or(overflow)) {
#pragma unroll
        for (int db = 0; db < NDB; ++db) o[db][0] = o[db][1] = splat16(0.f);
        m[0] = m[1] = l[0] = l[1] = 0.f;
        negm[0] = negm[1] = splat16(0.f);
        for (int t = t_begin; t < t_end; ++t) {
            __syncthreads();
            load_k(t);
            load_v(t);
            store_k(t);
            store_v(t);
            __syncthreads();
            if (!active) continue;
            for (int kb = 0; kb < 2; ++kb) {
                const int s = 2 * t + kb;
                if (s >= blk_end) break;
                f32x16 sx[2];
                qk_block(s, sx);           // negm is 0 until the first block sets the max
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int key = 32 * s + 8 * (i >> 2) + 4 * g + (i & 3);
                    if (key >= n_valid) sx[0][i] = sx[1][i] = -INFINITY;
                }
#pragma unroll
                for (int qb = 0; qb < 2; ++qb) {
                    float mx = sx[qb][0];
#pragma unroll
                    for (int i = 1; i < 16; ++i) mx = fmaxf(mx, sx[qb][i]);
                    mx = fmaxf(mx, xlane32(mx));
                    // first block: take its max; later blocks: move up when it is exceeded
                    const float d = (s == blk_begin) ? mx : (mx > 0.f ? mx : 0.f);
                    const float f = (s == blk_begin) ? 1.0f : __builtin_amdgcn_exp2f(-d);
                    m[qb] += d;
                    negm[qb] = splat16(-m[qb]);
                    l[qb] *= f;
#pragma unroll
                    for (int db = 0; db < NDB; ++db) o[db][qb] *= splat16(f);
                    sx[qb] -= splat16(d);
                }
                float ts[2];
                softmax_block(sx, pp, ts);
                l[0] += ts[0];
                l[1] += ts[1];
                pv_block(s);
            }
        }
    }
    __syncthreads();

    // ---- epilogue ---------------------------------------------------------------------
    float lt[2];
    lt[0] = l[0] + xlane32(l[0]);
    lt[1] = l[1] + xlane32(l[1]);

    if (wi.tail >= 0) {
        // Tail split: fp32 partial O (unnormalised), running max and row sum, for the
        // combine kernel. An empty key range leaves max -inf and sum 0.
        if (!active) return;
        const bool empty = t_begin >= t_end;
        const int64_t rowbase =
            ((int64_t)wi.split * (p.n_items - p.n_full) + wi.tail) * QT + wave * QW;
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
            const int q = q0 + 32 * qb + r;
            if (q >= p.Lq) continue;
            const int64_t row = rowbase + 32 * qb + r;
            float *po = p.part_o + row * D;
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int i4 = 0; i4 < 4; ++i4) {
                    f32x4 v;
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = o[db][qb][4 * i4 + e];
                    *(f32x4 *)(po + db * 32 + 8 * i4 + 4 * g) = v;
                }
            if (g == 0) {
                float *ml = p.part_ml + row * 2;
                ml[0] = empty ? -INFINITY : m[qb];
                ml[1] = empty ? 0.f : lt[qb];
            }
        }
        return;
    }

    // Unsplit: normalise, stage O through LDS, store coalesced 16-byte rows.
    bf16 *Os = smem + wave * QW * T::OS;
    if (active) {
        // 1/l, times the head's output gate of the query (rows past Lq are not stored)
        const float inv0 = gate_factor(p.gate, p.g_bs, p.g_rs, p.g_hs, b, min(q0 + r, p.Lq - 1), h) / lt[0];
        const float inv1 = gate_factor(p.gate, p.g_bs, p.g_rs, p.g_hs, b, min(q0 + 32 + r, p.Lq - 1), h) / lt[1];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int i4 = 0; i4 < 4; ++i4) {
                    const float inv = qb ? inv1 : inv0;
                    u32x2 w;
                    w[0] = pack_bf2(o[db][qb][4 * i4 + 0] * inv, o[db][qb][4 * i4 + 1] * inv);
                    w[1] = pack_bf2(o[db][qb][4 * i4 + 2] * inv, o[db][qb][4 * i4 + 3] * inv);
                    *(u32x2 *)(Os + (32 * qb + r) * T::OS + db * 32 + 8 * i4 + 4 * g) = w;
                }
    }
    __syncthreads();
    if (active) {
        bf16 *Ob = (bf16 *)p.o + (int64_t)b * p.o_bs + (int64_t)h * p.o_hs;
        constexpr int CPR = D / 8;
#pragma unroll
        for (int it = 0; it < QW * CPR / 64; ++it) {
            const int u = lane + 64 * it;
            const int row = u / CPR, c = u % CPR;
            const int q = q0 + row;
            if (q < p.Lq)
                *(u32x4 *)(Ob + (int64_t)q * p.o_rs + 8 * c) =
                    *(const u32x4 *)(Os + row * T::OS + 8 * c);
        }
    }
}

// ------------------------------------------------------------------------------------------
// Prologue: per-token RMS statistic over the inner dim (DiTAttention.swift:202-204), and for
// the K-prologue strategy the normalised + rotated tensor in the merged layout.
// One wave per token row, four rows per workgroup. A lane holds UPL pair units of its row
// (channels 8c .. +7 and D/2 + 8c .. +7 of a head, the two halves the rotation mixes) and
// issues all of their loads, and those of its RoPE table rows, before any arithmetic, so
// each lane has its whole share of the row in flight; the sum of squares is reduced within
// the wave.
// ------------------------------------------------------------------------------------------
constexpr int kPrepRows = NT / 64;             // token rows per workgroup

template <int D, int UPL>
__device__ __forceinline__ void qk_prep_rows(const PrepParams &p, int blk) {
    constexpr int PPH = D / 16;               // pair units per head
    const int lane = threadIdx.x & 63;
    const int rid = blk * kPrepRows + (threadIdx.x >> 6);   // output row b*L + lrow
    if (rid >= p.B * p.L) return;
    const int b = rid / p.L;
    const int lrow = rid % p.L;
    const int Lf = p.L_full > 0 ? p.L_full : p.L;
    const int64_t frow = (int64_t)b * Lf + lrow;  // row of the statistic and partials
    const int inner = p.H * D;
    const int units = p.H * PPH;
    const bf16 *row = (const bf16 *)p.x + (int64_t)b * p.bs + (int64_t)lrow * p.rs;

    u32x4 x1[UPL], x2[UPL], tc[UPL], ts[UPL];
#pragma unroll
    for (int k = 0; k < UPL; ++k) {
        const int u = lane + 64 * k;
        if (u < units) {
            const int hh = u / PPH, c = u % PPH;
            const bf16 *src = row + (int64_t)hh * p.hs;
            x1[k] = ldg16(src + 8 * c);
            x2[k] = ldg16(src + D / 2 + 8 * c);
            if (p.out && p.cos) {
                const int64_t toff = ((int64_t)hh * Lf + lrow) * (D / 2) + 8 * c;
                tc[k] = ldg16((const bf16 *)p.cos + toff);
                ts[k] = ldg16((const bf16 *)p.sin + toff);
            }
        }
    }
    float rstd = 1.0f;
    if (p.w && p.sumsq) {
        // The projection's partial sums, added in order (every lane reads the same row).
        const float *parts = p.sumsq + frow * p.ss_rs;
        float tot = 0.f;
        for (int j = 0; j < p.ss_blocks; ++j) tot += parts[j];
        rstd = 1.0f / sqrtf(tot / (float)inner + p.eps);
        if (lane == 0 && p.rstd) p.rstd[frow] = rstd;
    } else if (p.w) {
        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < UPL; ++k) {
            if (lane + 64 * k < units) {
                float a[8], c2[8];
                unpack8(x1[k], a);
                unpack8(x2[k], c2);
#pragma unroll
                for (int e = 0; e < 8; ++e) ss += a[e] * a[e] + c2[e] * c2[e];
            }
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
        rstd = 1.0f / sqrtf(ss / (float)inner + p.eps);
        if (lane == 0 && p.rstd) p.rstd[frow] = rstd;
    }
    if (!p.out) return;
    bf16 *dst = (bf16 *)p.out + (int64_t)rid * inner;
#pragma unroll
    for (int k = 0; k < UPL; ++k) {
        const int u = lane + 64 * k;
        if (u >= units) continue;
        const int hh = u / PPH, c = u % PPH;
        float a[8], c2[8];
        unpack8(x1[k], a);
        unpack8(x2[k], c2);
        if (p.w) {
            float w1[8], w2[8];
            const bf16 *w = (const bf16 *)p.w + hh * D;
            unpack8(ldg16(w + 8 * c), w1);
            unpack8(ldg16(w + D / 2 + 8 * c), w2);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                a[e] = (a[e] * rstd) * w1[e];
                c2[e] = (c2[e] * rstd) * w2[e];
            }
        }
        if (p.cos) {
            float fc[8], fs[8];
            unpack8(tc[k], fc);
            unpack8(ts[k], fs);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float x = a[e], y = c2[e];
                a[e] = x * fc[e] - y * fs[e];
                c2[e] = y * fc[e] + x * fs[e];
            }
        }
        *(u32x4 *)(dst + hh * D + 8 * c) = pack8(a);
        *(u32x4 *)(dst + hh * D + D / 2 + 8 * c) = pack8(c2);
    }
}

// One launch for one row set, or for two (the Q statistic and the K prologue of one call):
// the first blocks_a workgroups take set a, the rest set b.
template <int D, int UPL>
__global__ __launch_bounds__(NT) void qk_prep_kernel(const PrepParams a, const PrepParams b,
                                                     const int blocks_a) {
    if ((int)blockIdx.x < blocks_a) qk_prep_rows<D, UPL>(a, blockIdx.x);
    else qk_prep_rows<D, UPL>(b, blockIdx.x - blocks_a);
}

// ------------------------------------------------------------------------------------------
// RMS statistic from the projection's partial sums of squares: one thread per token row,
// partials added in order, the same formula as the prologue's.
// ------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rstd_kernel(const RstdParams p) {
    const int row = blockIdx.x * 256 + threadIdx.x;
    if (row >= p.rows) return;
    const float *parts = p.sumsq + (int64_t)row * p.rs;
    float tot = 0.f;
    for (int j = 0; j < p.blocks; ++j) tot += parts[j];
    p.rstd[row] = 1.0f / sqrtf(tot / (float)p.n + p.eps);
}

// ------------------------------------------------------------------------------------------
// Split-KV combine: O = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s, rounded to bf16.
// ------------------------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void combine_kernel(const CombineParams p) {
    constexpr int TPR = D / 4;                 // threads per row (4 channels each)
    constexpr int RPB = 256 / TPR;             // rows per block
    const int tid = threadIdx.x;
    const int64_t row = (int64_t)blockIdx.x * RPB + tid / TPR;   // (tail item, query in block)
    const int64_t rows = (int64_t)p.n_tail * QT;
    if (row >= rows) return;
    const int ti = (int)(row / QT), qi = (int)(row % QT);
    const int item = p.n_full + ti;
    const int q = (item % p.nqblk) * QT + qi;
    if (q >= p.Lq) return;
    const int bh = item / p.nqblk;
    const int hh = bh % p.H, b = bh / p.H;
    const int d = 4 * (tid % TPR);
    const int S = p.num_splits;
    // Every split's (max, sum) and partial O are loaded before any is used, so the row waits
    // for one round trip, not one per split (every range writes its partials, an empty one
    // max -inf and zeros). The sums then run in split order, skipping empty ranges.
    f32x2 ml[kMaxSplits];
    f32x4 po[kMaxSplits];
#pragma unroll
    for (int s = 0; s < kMaxSplits; ++s) {
        if (s < S) {
            ml[s] = *(const f32x2 *)(p.part_ml + (s * rows + row) * 2);
            po[s] = *(const f32x4 *)(p.part_o + (s * rows + row) * D + d);
        }
    }
    float M = -INFINITY;
#pragma unroll
    for (int s = 0; s < kMaxSplits; ++s)
        if (s < S) M = fmaxf(M, ml[s][0]);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    float den = 0.f;
#pragma unroll
    for (int s = 0; s < kMaxSplits; ++s) {
        if (s >= S || ml[s][0] == -INFINITY) continue;
        const float w = __builtin_amdgcn_exp2f(ml[s][0] - M);
        den += w * ml[s][1];
        acc += w * po[s];
    }
    const float inv = gate_factor(p.gate, p.g_bs, p.g_rs, p.g_hs, b, q, hh) / den;
    u32x2 w;
    w[0] = pack_bf2(acc[0] * inv, acc[1] * inv);
    w[1] = pack_bf2(acc[2] * inv, acc[3] * inv);
    *(u32x2 *)((bf16 *)p.o + (int64_t)b * p.o_bs + (int64_t)q * p.o_rs + (int64_t)hh * p.o_hs +
               d) = w;
}

// ------------------------------------------------------------------------------------------
// STG passthrough (DiTAttention.swift:351-356): the module's output is V itself, split into
// heads, times the gate when the module has one. One thread per 16-byte unit of a row.
// ------------------------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void passthrough_kernel(const PassParams p) {
    constexpr int U = D / 8;                   // 16-byte units per (token, head) row
    const int64_t unit = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t rows = (int64_t)p.B * p.L * p.H;
    if (unit >= rows * U) return;
    const int64_t row = unit / U;
    const int u = (int)(unit % U);
    const int hh = (int)(row % p.H);
    const int64_t bl = row / p.H;
    const int l = (int)(bl % p.L), b = (int)(bl / p.L);
    u32x4 w = ldg16((const bf16 *)p.v + (int64_t)b * p.v_bs + (int64_t)l * p.v_rs +
                    (int64_t)hh * p.v_hs + 8 * u);
    if (p.gate) {
        const float g = gate_factor(p.gate, p.g_bs, p.g_rs, p.g_hs, b, l, hh);
        float x[8];
        unpack8(w, x);
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] *= g;
        w = pack8(x);
    }
    *(u32x4 *)((bf16 *)p.o + (int64_t)b * p.o_bs + (int64_t)l * p.o_rs + (int64_t)hh * p.o_hs +
               8 * u) = w;
}

}  // namespace

int launch_passthrough(const PassParams &p, int D, void *stream) {
    const int64_t units = (int64_t)p.B * p.L * p.H * (D / 8);
    const dim3 grid((unsigned)((units + 255) / 256)), block(256);
    hipStream_t st = (hipStream_t)stream;
    if (D == 128) hipLaunchKernelGGL(passthrough_kernel<128>, grid, block, 0, st, p);
    else hipLaunchKernelGGL(passthrough_kernel<64>, grid, block, 0, st, p);
    return (int)hipGetLastError();
}

int launch_fmha(const FmhaParams &p, int D, int kind, void *stream) {
    if (kind == kDma) return launch_fmha_dma(p, D, stream);
    const dim3 grid(p.grid), block(NT);
    hipStream_t st = (hipStream_t)stream;
    const bool k_fused = kind == kRegFused;
    if (D == 128) {
        if (k_fused) hipLaunchKernelGGL((fmha_fwd_kernel<128, true>), grid, block, 0, st, p);
        else hipLaunchKernelGGL((fmha_fwd_kernel<128, false>), grid, block, 0, st, p);
    } else {
        if (k_fused) hipLaunchKernelGGL((fmha_fwd_kernel<64, true>), grid, block, 0, st, p);
        else hipLaunchKernelGGL((fmha_fwd_kernel<64, false>), grid, block, 0, st, p);
    }
    return (int)hipGetLastError();
}

int launch_rstd(const RstdParams &p, void *stream) {
    const dim3 grid((unsigned)((p.rows + 255) / 256)), block(256);
    hipLaunchKernelGGL(rstd_kernel, grid, block, 0, (hipStream_t)stream, p);
    return (int)hipGetLastError();
}

template <int D>
static void launch_prep_d(const PrepParams &a, const PrepParams &b, int blocks_a, dim3 grid,
                          hipStream_t st) {
    const int upl = (a.H * (D / 16) + 63) / 64;   // pair units per lane (inner <= 16384)
    if (upl <= 1) hipLaunchKernelGGL((qk_prep_kernel<D, 1>), grid, dim3(NT), 0, st, a, b, blocks_a);
    else if (upl <= 2) hipLaunchKernelGGL((qk_prep_kernel<D, 2>), grid, dim3(NT), 0, st, a, b, blocks_a);
    else if (upl <= 4) hipLaunchKernelGGL((qk_prep_kernel<D, 4>), grid, dim3(NT), 0, st, a, b, blocks_a);
    else if (upl <= 8) hipLaunchKernelGGL((qk_prep_kernel<D, 8>), grid, dim3(NT), 0, st, a, b, blocks_a);
    else hipLaunchKernelGGL((qk_prep_kernel<D, 16>), grid, dim3(NT), 0, st, a, b, blocks_a);
}

static int prep_blocks(const PrepParams &p) {
    return (int)(((int64_t)p.B * p.L + kPrepRows - 1) / kPrepRows);
}

int launch_prep(const PrepParams &p, int D, void *stream) {
    const int blocks = prep_blocks(p);
    hipStream_t st = (hipStream_t)stream;
    if (D == 128) launch_prep_d<128>(p, p, blocks, dim3(blocks), st);
    else launch_prep_d<64>(p, p, blocks, dim3(blocks), st);
    return (int)hipGetLastError();
}

int launch_prep2(const PrepParams &a, const PrepParams &b, int D, void *stream) {
    const int blocks_a = prep_blocks(a), blocks = blocks_a + prep_blocks(b);
    hipStream_t st = (hipStream_t)stream;
    if (D == 128) launch_prep_d<128>(a, b, blocks_a, dim3(blocks), st);
    else launch_prep_d<64>(a, b, blocks_a, dim3(blocks), st);
    return (int)hipGetLastError();
}

int launch_combine(const CombineParams &p, int D, void *stream) {
    const int64_t rows = (int64_t)p.n_tail * QT;
    const int rpb = 256 / (D / 4);
    const dim3 grid((unsigned)((rows + rpb - 1) / rpb)), block(256);
    hipStream_t st = (hipStream_t)stream;
    if (D == 128) hipLaunchKernelGGL(combine_kernel<128>, grid, block, 0, st, p);
    else hipLaunchKernelGGL(combine_kernel<64>, grid, block, 0, st, p);
    return (int)hipGetLastError();
}

}  // namespace ltx
