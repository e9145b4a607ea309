// Attention for a short query stream over a long key stream at head dim 64 (one query block
// per (batch, head): the audio queries of the cross-modal video->audio module over the video
// keys, with K's RMSNorm statistic and 1-D RoPE), split over key ranges so that the whole GPU
// streams K and V.
//
// One workgroup of eight waves per (batch, head, key range), two waves per SIMD. Wave w owns
// the 64 queries of group w >> 1 and, of every 64-key tile, the 32-key block w & 1; the two
// waves of a group merge their (max, sum, O) at the end of the range. The range's tiles are
// copied HBM -> LDS by the buffer-load-to-LDS path three tiles ahead: the raw K rows (their
// 16-byte units XOR-swizzled as the MFMA operand reads expect), V row-major, and, when K is
// normalised or rotated, the statistic of the tile's keys and their cos/sin table rows. After
// a tile lands, waves 4-7 (waves 6-7 when three query groups keep waves 4-5 busy) normalise
// and rotate its K in place in LDS (x * rstd * w, then the split-half rotation, one bf16
// rounding -- the arithmetic of the K prologue) while every wave with queries computes on
// the tile before it: S^T = K.Q'^T, the softmax with each row's max taken from its first
// block and -max as the S accumulators' start (an exact online softmax redoes the range when
// a row sum overflows), and O^T += V^T.P^T (P as bf16, or as bf16 hi + lo parts without
// RoPE). One barrier per tile separates the phases. The range's partial O, max and row sum go to the
// split-KV workspace the combine kernel merges; a call with a single range writes O directly.
#include <type_traits>

#include "lds_copy.hpp"

namespace ltx {
namespace {

constexpr int kSplitWaves = 8;
constexpr int kSplitThreads = 64 * kSplitWaves;

template <int D, bool ROPE, bool NORM>
struct SplitLayout {
    static constexpr int NC = D / 16;                // 16-wide reduction chunks of Q.K^T
    static constexpr int NDB = D / 32;               // 32-row blocks of O^T
    static constexpr int KU = D / 8;                 // 16-byte units per K or V row
    static constexpr int TILE = KT * D * 2;          // bytes of a K or V tile
    static constexpr int TAB = KT * D;               // bytes of a tile's cos (or sin) rows
    static constexpr int RSTD = 1024;                // a wave's copy of the tile's statistics
    static constexpr int KV_DMA = TILE / 1024 / kSplitWaves;   // copies per wave per K/V tile
    static constexpr int TAB_DMA = 2 * TAB / 1024 / kSplitWaves;  // per wave, cos + sin
    static_assert(KV_DMA == 1 && TAB_DMA == 1, "one copy of each kind per wave per tile");
    static constexpr int COPIES = 2 + (ROPE ? 1 : 0) + (NORM ? 1 : 0);
    // one stage: K, V, cos, sin, the eight waves' statistic copies
    static constexpr int OFF_V = TILE;
    static constexpr int OFF_COS = 2 * TILE;
    static constexpr int OFF_SIN = OFF_COS + (ROPE ? TAB : 0);
    static constexpr int OFF_R = OFF_SIN + (ROPE ? TAB : 0);
    static constexpr int STAGE = OFF_R + (NORM ? kSplitWaves * RSTD : 0);
    // Stages of the copy ring (tiles in flight: STAGES - 1). Six stages without the statistic
    // copies (everything of a 7-tile range on the way at once) measured slower than four on
    // 126 audio queries over 3120 video keys (21.9 against 20.5 us).
    static constexpr int STAGES = 4;
    // end-of-range merge: per query group, O (64 floats per lane) then (m, l) per lane, in
    // the same LDS as the stages once every wave is done with them
    static constexpr int MERGE_FLOATS = 2 * NDB * 16 + 4;
    static constexpr int MERGE_BYTES = 4 * MERGE_FLOATS * 64 * 4;
    static constexpr int BYTES = STAGES * STAGE > MERGE_BYTES ? STAGES * STAGE : MERGE_BYTES;
    static_assert(BYTES <= 160 * 1024, "LDS of one workgroup");
};

template <int D, bool ROPE, bool NORM>
__global__ __attribute__((amdgpu_flat_work_group_size(kSplitThreads, kSplitThreads),
                          amdgpu_waves_per_eu(2, 2)))
void fmha_splitk_kernel(const FmhaParams p) {
    using T = SplitLayout<D, ROPE, NORM>;
    constexpr int NC = T::NC, NDB = T::NDB, KU = T::KU, COPIES = T::COPIES;
    constexpr int AHEAD = T::STAGES - 1;
    constexpr bool KWORK = ROPE || NORM;
    // Without RoPE (the audio queries over the text keys) the reference's own arithmetic
    // rounds little (the norms), and P rounded to bf16 would be the larger part of the
    // kernel's error: P then also takes its lo part (P - bf16(P), a second product per P.V
    // operand; 4-8% on those calls). With RoPE the reference's rounded rotations dominate
    // and P stays one bf16 part.
    constexpr bool HILO = !ROPE;
    __shared__ __attribute__((aligned(16))) char smem[T::BYTES];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 31;
    const int g = lane >> 5;
    const int qg = wave >> 1, kb = wave & 1;

    // unit: (batch, head) item and key range; items are b*H + h (one query block each)
    const int unit = blockIdx.x;
    const int item = unit / p.num_splits, split = unit % p.num_splits;
    const int h = item % p.H, b = item / p.H;
    const int n_valid = p.valid[b];
    const int ntiles = (n_valid + KT - 1) / KT;
    const int t_begin = split * p.tiles_per_split;
    const int t_end = min(t_begin + p.tiles_per_split, ntiles);
    const int q0 = qg * QW;
    const bool active = q0 < p.Lq;

    auto lds = [&](int stage, int off) __attribute__((always_inline)) {
        return (__attribute__((address_space(3))) char *)smem + stage * T::STAGE + off;
    };

    // ---- copies: one K, one V copy per wave per tile; cos (waves 0-3) or sin (4-7); the
    // tile's statistics into the wave's own slot ----------------------------------------
    const bf16 *Kb = (const bf16 *)p.k + (int64_t)b * p.k_bs + (int64_t)h * p.k_hs;
    const bf16 *Vb = (const bf16 *)p.v + (int64_t)b * p.v_bs + (int64_t)h * p.v_hs;
    const int krow = (int)(p.k_rs * 2), vrow = (int)(p.v_rs * 2);
    const u32x4 rkw = rsrc_words(Kb, (int64_t)n_valid * krow);
    const u32x4 rvw = rsrc_words(Vb, (int64_t)n_valid * vrow);
    // tables [H][Lk][D/2]: a tile's rows are one contiguous block of KT*D bytes per table
    const int64_t tab_head = (int64_t)h * p.Lk * (D / 2);
    const bf16 *tab = wave < 4 ? (const bf16 *)p.k_cos : (const bf16 *)p.k_sin;
    const u32x4 rtw = rsrc_words(ROPE ? tab + tab_head : Kb, ROPE ? (int64_t)n_valid * D : 0);
    const u32x4 rrw = rsrc_words(NORM ? p.k_rstd + (int64_t)b * p.Lk : (const float *)Kb,
                                 NORM ? (int64_t)n_valid * 4 : 0);
    const int cq = wave * 64 + lane;                 // this lane's 16-byte unit of a tile
    const int crow = cq / KU;
    const int klane = crow * krow + 16 * swz<KU>(crow, cq % KU);
    const int vlane = crow * vrow + 16 * vswz<KU>(crow, cq % KU);
    auto issue = [&](int t) __attribute__((always_inline)) {
        const int st = (t - t_begin) % T::STAGES;
        copy_all(rkw, (uint32_t)(uintptr_t)lds(st, wave * 1024), t * KT * krow + klane);
        copy_all(rvw, (uint32_t)(uintptr_t)lds(st, T::OFF_V + wave * 1024),
                 t * KT * vrow + vlane);
        if constexpr (ROPE)
            copy_all(rtw, (uint32_t)(uintptr_t)lds(st, (wave < 4 ? T::OFF_COS : T::OFF_SIN) +
                                                          (wave & 3) * 1024),
                     t * T::TAB + (wave & 3) * 1024 + 16 * lane);
        if constexpr (NORM)
            copy_all(rrw, (uint32_t)(uintptr_t)lds(st, T::OFF_R + wave * T::RSTD),
                     t * KT * 4 + 16 * lane);
    };
    // wait until this wave's copies of a tile have landed, with `after` later tiles in flight
    // (at most AHEAD - 1)
    static_assert(AHEAD == 3, "at most two later tiles in flight at a wait");
    auto wait_tile = [&](int after) __attribute__((always_inline)) {
        if (after >= 2) wait_copies_but<2 * COPIES>();
        else if (after == 1) wait_copies_but<COPIES>();
        else wait_copies();
    };

    // ---- the in-place K transform: waves 4-7, or waves 6-7 when three query groups are
    // active (waves 4 and 5 then compute). A unit (row, part) of the tile is one 16-byte unit
    // of the row's first half and the unit of the second half it is rotated with; 4 units
    // per row, 256 per tile, dealt to the transform threads in turn.
    const int tw0 = (p.Lq + QW - 1) / QW == 3 ? 6 : 4;
    const bool tthread = wave >= tw0;
    const int tfirst = tid - 64 * tw0, tstride = 64 * (kSplitWaves - tw0);
    const int tpart = tid & 3;                       // the same for every unit of a thread
    float wlo[8], whi[8];                            // k norm weights of the thread's channels
    if constexpr (NORM) {
        const bf16 *w = (const bf16 *)p.k_w + h * D;
        unpack8(ldg16(w + 8 * tpart), wlo);
        unpack8(ldg16(w + D / 2 + 8 * tpart), whi);
    }
    typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
    auto transform = [&](int st) __attribute__((always_inline)) {
      for (int u = tfirst; u < KT * 4; u += tstride) {
        const int trow = u >> 2;
        float rs = 1.f;
        if constexpr (NORM)
            rs = ((__attribute__((address_space(3))) float *)lds(st, T::OFF_R + wave * T::RSTD))[trow];
        lds_bf16 *Ks = (lds_bf16 *)lds(st, 0);
        lds_u32x4 *pl = (lds_u32x4 *)(Ks + trow * D + 8 * swz<KU>(trow, tpart));
        lds_u32x4 *ph = (lds_u32x4 *)(Ks + trow * D + 8 * swz<KU>(trow, tpart + KU / 2));
        float x1[8], x2[8];
        unpack8(*pl, x1);
        unpack8(*ph, x2);
        if constexpr (NORM) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                x1[e] = (x1[e] * rs) * wlo[e];
                x2[e] = (x2[e] * rs) * whi[e];
            }
        }
        if constexpr (ROPE) {
            float fc[8], fs[8];
            unpack8(*(const lds_u32x4 *)(lds(st, T::OFF_COS) + trow * D + 16 * tpart), fc);
            unpack8(*(const lds_u32x4 *)(lds(st, T::OFF_SIN) + trow * D + 16 * tpart), fs);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float a = x1[e], c = x2[e];
                x1[e] = a * fc[e] - c * fs[e];
                x2[e] = c * fc[e] + a * fs[e];
            }
        }
        *pl = pack8(x1);
        *ph = pack8(x2);
      }
    };

    // ---- operands ------------------------------------------------------------------------
    auto k_opnd = [&](const lds_bf16 *Ks, int c) __attribute__((always_inline)) {
        const int row = kb * 32 + r;
        return *(const __attribute__((address_space(3))) bf16x8 *)(Ks + row * D +
                                                                   8 * swz<KU>(row, 2 * c + g));
    };
    const int i16 = lane & 15;
    const int hsel = (lane >> 4) & 1;
    auto v_opnd = [&](const lds_bf16 *Vs, int t4, int db) __attribute__((always_inline)) {
        const int row0 = 16 * t4 + 4 * g + (i16 >> 2);
        const int u = 4 * db + 2 * hsel + ((i16 & 3) >> 1);
        const int half = 4 * (i16 & 1);
        const u32x2 lo = ds_read_tr(Vs + row0 * D + 8 * vswz<KU>(row0, u) + half);
        const u32x2 hi = ds_read_tr(Vs + (row0 + 8) * D + 8 * vswz<KU>(row0 + 8, u) + half);
        return __builtin_bit_cast(bf16x8, u32x4{lo[0], lo[1], hi[0], hi[1]});
    };

    // ---- the pass over the range --------------------------------------------------------
    bf16x8 qf[2][NC];
    f32x16 o[NDB][2];
    float m[2], l[2];        // running max (log2 units, equal in lanes l, l^32); row-sum share
    f32x16 negm[2];          // -m as the S accumulators' start (fast pass)
    bool overflow = false;   // fast pass: some block's row sum passed 2^64
    // fast (SAFE false): each row's max is taken from the wave's first block and kept; S
    // starts at -max, so p = exp2(S) with no per-block max, subtract or rescale, and a row sum
    // above 2^64 is only recorded. SAFE: running max, rescaling O and the sum whenever a row's
    // max grows. The safe pass runs only when some wave of the range recorded an overflow.
    auto run = [&](auto safe_c) __attribute__((always_inline)) {
        constexpr bool SAFE = decltype(safe_c)::value;
#pragma unroll
        for (int i = 0; i < AHEAD; ++i)
            if (t_begin + i < t_end) issue(t_begin + i);
        if (!SAFE) load_q<D>(p, b, h, q0, active, r, g, qf);   // overlaps the first copies
#pragma unroll
        for (int db = 0; db < NDB; ++db) o[db][0] = o[db][1] = splat16(0.f);
        m[0] = m[1] = -INFINITY;
        l[0] = l[1] = 0.f;
        negm[0] = negm[1] = splat16(0.f);
        bool first = true;   // wave-uniform: the wave's next block is its first
        // tile t_begin's K is prepared before the loop; iteration t prepares tile t+1 while
        // it computes on tile t
        if constexpr (KWORK) {
            if (t_begin < t_end) {
                wait_tile(min(AHEAD - 1, t_end - 1 - t_begin));
                __syncthreads();
                if (tthread) transform(0);
            }
        }
        for (int t = t_begin; t < t_end; ++t) {
            const int st = (t - t_begin) % T::STAGES;
            // Tile t is ready once everyone is past this barrier: its copies landed (waited
            // for below in the previous iteration or above) and, with K work, its K was
            // prepared in the previous iteration. Tile t+1's copies are waited for first, so
            // that it can be prepared now; tile t-1's buffers are free for the copies of tile
            // t + AHEAD.
            if constexpr (KWORK) {
                if (t + 1 < t_end) wait_tile(min(AHEAD - 2, t_end - 2 - t));
            } else {
                wait_tile(min(AHEAD - 1, t_end - 1 - t));
            }
            __syncthreads();
            if (t + AHEAD < t_end) issue(t + AHEAD);
            if constexpr (KWORK) {
                if (tthread && t + 1 < t_end) transform((t + 1 - t_begin) % T::STAGES);
            }
            const int key0 = t * KT + kb * 32;
            if (!active || key0 >= n_valid) continue;
            const lds_bf16 *Ks = (const lds_bf16 *)lds(st, 0);
            const lds_bf16 *Vs = (const lds_bf16 *)lds(st, T::OFF_V);
            const bool fast = !SAFE && !first;
            f32x16 s[2];
            s[0] = fast ? negm[0] : splat16(0.f);
            s[1] = fast ? negm[1] : splat16(0.f);
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const bf16x8 a = k_opnd(Ks, c);
                s[0] = mfma32(a, qf[0][c], s[0]);
                s[1] = mfma32(a, qf[1][c], s[1]);
            }
            const bool ragged = key0 + 32 > n_valid;
            bf16x8 pn[2][2], pl[2][2];   // P (fp32 weights) as bf16 hi (+ lo) parts
#pragma unroll
            for (int qb = 0; qb < 2; ++qb) {
                if (ragged) {
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        if (key0 + 8 * (i >> 2) + 4 * g + (i & 3) >= n_valid)
                            s[qb][i] = -INFINITY;
                }
                if (!fast) {
                    float mx = s[qb][0];
#pragma unroll
                    for (int i = 1; i < 16; ++i) mx = fmaxf(mx, s[qb][i]);
                    mx = fmaxf(mx, xlane32(mx));           // finite: key0 < n_valid
                    if (!SAFE) {
                        // the wave's first block: its max is the row's reference from here on
                        m[qb] = mx;
                        negm[qb] = splat16(-mx);
                    } else if (__builtin_amdgcn_ballot_w64(mx > m[qb])) {
                        // some row's max grew: rescale its O and sum (alpha = 1 elsewhere, 0
                        // on the first block, where O and the sum are still 0)
                        const float mn = fmaxf(m[qb], mx);
                        const float alpha = __builtin_amdgcn_exp2f(m[qb] - mn);
                        m[qb] = mn;
                        l[qb] *= alpha;
#pragma unroll
                        for (int db = 0; db < NDB; ++db) o[db][qb] *= splat16(alpha);
                    }
                    s[qb] -= splat16(m[qb]);
                }
                float ts = 0.f;
#pragma unroll
                for (int hf = 0; hf < 2; ++hf) {
                    u32x4 w, wl;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float x0 = __builtin_amdgcn_exp2f(s[qb][8 * hf + 2 * e]);
                        const float x1 = __builtin_amdgcn_exp2f(s[qb][8 * hf + 2 * e + 1]);
                        ts += x0 + x1;
                        w[e] = pack_bf2(x0, x1);
                        if constexpr (HILO) wl[e] = pack_bf2(x0 - bf_lo(w[e]), x1 - bf_hi(w[e]));
                    }
                    pn[qb][hf] = __builtin_bit_cast(bf16x8, w);
                    if constexpr (HILO) pl[qb][hf] = __builtin_bit_cast(bf16x8, wl);
                }
                if (!SAFE) overflow |= !(ts <= kRebaseBound);
                l[qb] += ts;
            }
            first = false;
            // O += V^T.P, with P's lo part too when HILO
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                bf16x8 a[NDB];
#pragma unroll
                for (int db = 0; db < NDB; ++db) {
                    a[db] = v_opnd(Vs, 2 * kb + hf, db);
                    o[db][0] = mfma32(a[db], pn[0][hf], o[db][0]);
                    o[db][1] = mfma32(a[db], pn[1][hf], o[db][1]);
                }
                if constexpr (HILO) {
#pragma unroll
                    for (int db = 0; db < NDB; ++db) {
                        o[db][0] = mfma32(a[db], pl[0][hf], o[db][0]);
                        o[db][1] = mfma32(a[db], pl[1][hf], o[db][1]);
                    }
                }
            }
        }
        if (t_begin >= t_end) wait_copies();
    };
    run(std::false_type{});
    // Pathological inputs only: some row's scores grew past its first block's max by more
    // than the fp32 sum can hold; every wave redoes the range with the exact online softmax.
    if (__syncthreads_or(overflow)) run(std::true_type{});

    // ---- merge the two waves of each query group: the odd wave hands (O, m, l) over ------
    __syncthreads();                                 // every wave is done with the stages
    typedef __attribute__((address_space(3))) float lds_f32;
    lds_f32 *mg = (lds_f32 *)smem + qg * T::MERGE_FLOATS * 64;
    if (kb == 1 && active) {
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int qb = 0; qb < 2; ++qb)
#pragma unroll
                for (int i = 0; i < 16; ++i) mg[((db * 2 + qb) * 16 + i) * 64 + lane] = o[db][qb][i];
        mg[(2 * NDB * 16 + 0) * 64 + lane] = m[0];
        mg[(2 * NDB * 16 + 1) * 64 + lane] = m[1];
        mg[(2 * NDB * 16 + 2) * 64 + lane] = l[0];
        mg[(2 * NDB * 16 + 3) * 64 + lane] = l[1];
    }
    __syncthreads();
    if (kb == 1 || !active) return;
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        const float mb = mg[(2 * NDB * 16 + qb) * 64 + lane];
        const float lb = mg[(2 * NDB * 16 + 2 + qb) * 64 + lane];
        const float mn = fmaxf(m[qb], mb);
        // either side may be empty (-inf); both empty leaves (-inf, 0, 0)
        const float fa = mn == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m[qb] - mn);
        const float fb = mn == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mb - mn);
        m[qb] = mn;
        l[qb] = l[qb] * fa + lb * fb;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i)
                o[db][qb][i] = o[db][qb][i] * fa + mg[((db * 2 + qb) * 16 + i) * 64 + lane] * fb;
    }

    // ---- epilogue ----------------------------------------------------------------------
    float lt[2];
    lt[0] = l[0] + xlane32(l[0]);
    lt[1] = l[1] + xlane32(l[1]);
    if (p.num_splits > 1) {
        // partial O (unnormalised), running max and row sum for the combine kernel, in its
        // layout: rows (split * n_items + item) * 256 + query. An empty range leaves -inf, 0.
        const int64_t rowbase = ((int64_t)split * p.n_items + item) * QT + q0;
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
            const int q = q0 + 32 * qb + r;
            if (q >= p.Lq) continue;
            float *po = p.part_o + (rowbase + 32 * qb + r) * D;
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
                float *ml = p.part_ml + (rowbase + 32 * qb + r) * 2;
                ml[0] = m[qb];
                ml[1] = lt[qb];
            }
        }
        return;
    }
    // a single range: O / l times the gate, 8-byte stores of each lane's 4 channels
    bf16 *Ob = (bf16 *)p.o + (int64_t)b * p.o_bs + (int64_t)h * p.o_hs;
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        const int q = q0 + 32 * qb + r;
        if (q >= p.Lq) continue;
        const float inv = gate_factor(p.gate, p.g_bs, p.g_rs, p.g_hs, b, q, h) / lt[qb];
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                u32x2 w;
                w[0] = pack_bf2(o[db][qb][4 * i4 + 0] * inv, o[db][qb][4 * i4 + 1] * inv);
                w[1] = pack_bf2(o[db][qb][4 * i4 + 2] * inv, o[db][qb][4 * i4 + 3] * inv);
                *(u32x2 *)(Ob + (int64_t)q * p.o_rs + db * 32 + 8 * i4 + 4 * g) = w;
            }
    }
}

template <bool ROPE, bool NORM>
void launch_splitk_t(const FmhaParams &p, hipStream_t st) {
    hipLaunchKernelGGL((fmha_splitk_kernel<64, ROPE, NORM>), dim3(p.grid), dim3(kSplitThreads),
                       0, st, p);
}

}  // namespace

int launch_fmha_splitk(const FmhaParams &p, int D, void *stream) {
    if (D != 64) return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    const bool rope = p.k_cos != nullptr, norm = p.k_rstd != nullptr;
    if (rope) norm ? launch_splitk_t<true, true>(p, st) : launch_splitk_t<true, false>(p, st);
    else norm ? launch_splitk_t<false, true>(p, st) : launch_splitk_t<false, false>(p, st);
    return (int)hipGetLastError();
}

}  // namespace ltx
