// Gemma-4 text-encoder attention (Sources/LTXModules/GemmaTextEncoder.swift:158-239, mask
// :288-321) for gfx950: head dims 256 / 512, 16 query heads over 8 or 1 KV heads, causal +
// sliding-window + left-padding mask, scale 1.0, 1024 tokens per prompt.
//
// Three launches (the first is the whole prologue, its q/k rows and its v blocks side by side):
//   gemma_prep_kernel   one wave per (batch row, token, head) row of q or k: the per-head
//                       RMS norm (fp32, pow(mean + eps, -0.5), times the weight), rotate_half
//                       RoPE with the fp32 tables, q scaled by scale*log2(e). Rounding points:
//                       the reference's norm returns the input dtype (GemmaTextEncoder.swift
//                       :114), so its normed q and k are bf16, and its fp32 RoPE leaves both
//                       fp32. Here q and k are normed and rotated in fp32 without that
//                       rounding and rounded once, after the rotation, to fp16 (11
//                       significant bits, against bf16's 8): q' [B][Hq][T][D] and k' are the
//                       fp16 operands of the products, far inside fp16's range: the RMS norm
//                       bounds a channel, and the rotation a channel pair, by sqrt(D) times
//                       the weight (times log2(e) for q'). The single rounding, finer than the
//                       reference's, brings the result nearer the exact one than the
//                       reference's own arithmetic (its rounded normed q alone moves the
//                       1024-token layers' max-abs error to about 2e-2).
//                       k' is stored in MFMA operand order: per (batch row, KV head, 32-key
//                       block) D/16 units of 1 KB, lane r + 32g of unit c holding channels
//                       16c + 8g .. +7 of key r.
//   (same launch)       v with the weightless per-head norm, in fp16, transposed through an
//                       LDS tile of one 32-key block into operand order: per key half hf and
//                       32-channel block cb one 1 KB unit, lane r + 32g holding channel
//                       32cb + r at keys 16hf + 4g + {0..3, 8..11}. Keys past T are zeros in both layouts, and
//                       a key block's k' and v'^T are each one contiguous run of units.
//   gemma_attn_kernel   a wave owns 32 queries over 256 channels (D = 256: the whole head;
//                       D = 512: half of it, its partner wave the other half), four waves per
//                       workgroup: 128 queries at D = 256, 64 at D = 512. The key blocks of
//                       the workgroup's range are copied HBM -> LDS by the buffer-load-to-LDS
//                       path into a ring (4 blocks at D = 256, 2 at D = 512) and read from LDS
//                       by every wave. Per key block: S^T = K.Q'^T in fp16 products (inline,
//                       S in VGPRs and Q' in AGPRs; at D = 512 the two halves' partial sums are
//                       exchanged through LDS and added in a fixed order), the mask, exp2 with
//                       each row's max fixed at its first block with an allowed key, and
//                       O^T += V^T.P^T with v' and P in fp16 (the reference's weights are
//                       fp32; with the max fixed a weight stays below 2^kGemmaBound). A block
//                       whose weights would pass 2^kGemmaBound sends the workgroup to an exact
//                       pass (online max with rescaling) over its range. O is written in
//                       fp32, the dtype the reference's explicit path returns.
//   gemma_combine_kernel  the long query blocks' keys run as ranges of at most 16 blocks on
//                       separate workgroups, each writing unnormalised O and (max, sum); the
//                       merge rescales and adds them.
#include <type_traits>

#include "lds_copy.hpp"
#include "mfma_s.hpp"

namespace ltx {
namespace {

// ---- prologue ------------------------------------------------------------------------------
// q/k rows: workgroup wg of the rows' part of the launch.
// Rows per wave of the q/k part: a wave takes kPrepPasses passes of 64 / (D / 8) rows and
// issues every pass's loads (the row, its table rows) before the first use, so the launch's
// waves each wait for one round trip instead of one per row (one row per wave and pass took
// the 1024-token prologue 18-21 us, most of it waiting).
constexpr int kPrepPasses = 4;   // 8 measured slower (23.6 / 19.8 against 16.5 / 16.3 us)

template <int D>
__device__ __forceinline__ void gemma_prep_rows(const GemmaPrepParams &p, int wg) {
    // 8 channels per lane: a row of D = 512 takes a wave, a row of D = 256 half a wave
    constexpr int E = 8;
    constexpr int LPR = D / E;                      // lanes per row: 64 or 32
    constexpr int RPW = 64 / LPR;                   // rows per wave and pass
    constexpr int NP = kPrepPasses;
    const int lane = threadIdx.x & (LPR - 1);       // lane within the row
    // (row indices in 32 bits: the launch refuses 2^31 rows or more)
    const uint32_t heads = p.Hq + p.Hkv;            // q heads, then k heads, per token
    const uint32_t total = (uint32_t)p.B * p.T * heads;
    // the wave's rows: RPW * NP consecutive rows, pass j taking rows base + RPW*j + (0..RPW-1)
    const uint32_t base = ((uint32_t)wg * 4 + (threadIdx.x >> 6)) * (RPW * NP) +
                          ((threadIdx.x & 63) / LPR);
    const int col = (lane & (LPR / 2 - 1)) * E;     // table column of the lane's channels
    u32x4 raw[NP];
    f32x4 cs[NP][2], sn[NP][2];
    int hrs[NP], ts[NP], bs[NP];
#pragma unroll
    for (int j = 0; j < NP; ++j) {
        const uint32_t row = base + RPW * j;
        const uint32_t bt = row / heads;
        hrs[j] = (int)(row - bt * heads);
        bs[j] = (int)(bt / (uint32_t)p.T);
        ts[j] = (int)(bt - (uint32_t)bs[j] * p.T);
    }
#pragma unroll
    for (int j = 0; j < NP; ++j) {
        if (base + RPW * j >= total) continue;
        const int hr = hrs[j], t = ts[j], b = bs[j];
        const bf16 *src = hr < p.Hq
            ? (const bf16 *)p.q + (int64_t)b * p.q_bs + (int64_t)t * p.q_rs + (int64_t)hr * D
            : (const bf16 *)p.k + (int64_t)b * p.k_bs + (int64_t)t * p.k_rs +
                  (int64_t)(hr - p.Hq) * D;
        raw[j] = ldg16(src + lane * E);
        const float *c = p.cos + (int64_t)t * (D / 2) + col;
        const float *sv = p.sin + (int64_t)t * (D / 2) + col;
        cs[j][0] = *(const f32x4 *)c;
        cs[j][1] = *(const f32x4 *)(c + 4);
        sn[j][0] = *(const f32x4 *)sv;
        sn[j][1] = *(const f32x4 *)(sv + 4);
    }
    float wq[E], wk[E];
    unpack8(ldg16((const bf16 *)p.q_w + lane * E), wq);
    unpack8(ldg16((const bf16 *)p.k_w + lane * E), wk);
    const bool first = lane < LPR / 2;
#pragma unroll
    for (int j = 0; j < NP; ++j) {
        if (base + RPW * j >= total) continue;
        const int hr = hrs[j], t = ts[j], b = bs[j];
        const int kind = hr < p.Hq ? 0 : 1;         // q, k
        const int h = kind == 0 ? hr : hr - p.Hq;
        float x[E];
        unpack8(raw[j], x);
        // the reductions and the partner exchange stay within the row's lanes (offsets < LPR)
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) ss += x[e] * x[e];
#pragma unroll
        for (int off = LPR / 2; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
        const float rs = powf(ss / (float)D + p.eps, -0.5f);
#pragma unroll
        for (int e = 0; e < E; ++e) x[e] = (x[e] * rs) * (kind == 0 ? wq[e] : wk[e]);
        // rotate_half pairs channel c with c +- D/2: lane l holds channels E*l ..; its partner
        // is lane l ^ LPR/2. Table column of channel c is c mod D/2.
        const float f = kind == 0 ? p.q_factor : 1.0f;
        float y[E];
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const float other = __shfl_xor(x[e], LPR / 2, 64);
            const float c = cs[j][e >> 2][e & 3], s = sn[j][e >> 2][e & 3];
            // first half: x1 c - x2 s; second half: x2 c + x1 s
            y[e] = (first ? x[e] * c - other * s : x[e] * c + other * s) * f;
        }
        // q' and k' as fp16 (11 significant bits, rounded once, to nearest)
        if (kind == 1) {
            // k' in operand order: 32-key block t/32, 16-channel chunk c, lane (t%32) + 32g
            // holds channels 16c + 8g .. +7 of key t
            const int ch = lane * E, c = ch >> 4, g = (ch >> 3) & 1;
            const int nkb = (p.T + 31) / 32;
            const int64_t off =
                ((((int64_t)b * p.Hkv + h) * nkb + (t >> 5)) * (D / 16) + c) * 512 +
                ((t & 31) + 32 * g) * 8 + (ch & 7);
            *(u32x4 *)((_Float16 *)p.kp + off) = pack8_f16(y);
        } else {
            const int64_t off = (((int64_t)b * p.Hq + h) * p.T + t) * D + lane * E;
            *(u32x4 *)((_Float16 *)p.qp + off) = pack8_f16(y);
        }
    }
}

// v: the weightless per-head norm, stored transposed in operand order. One workgroup per
// (batch row, KV head, 32-key block): each wave loads its 8 token rows at once, normalises
// them into an LDS tile, then the tile leaves as the block's P.V operand units. Workgroup wg
// of the v part of the launch.
template <int D>
__device__ __forceinline__ void gemma_vt_block(const GemmaPrepParams &p, int wg,
                                               _Float16 (&tile)[32][D + 8]) {
    constexpr int E = D / 64;
    constexpr int TT = 32;                          // tokens per workgroup: one key block
    constexpr int RW = TT / 4;                      // rows per wave
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nkb = (p.T + TT - 1) / TT;
    const int kb = wg % nkb, t0 = kb * TT;
    const int bh = wg / nkb;
    const int h = bh % p.Hkv, b = bh / p.Hkv;
    // every row's load issued before the first use: a row past T loads row T - 1 and is
    // zeroed afterwards (a branch around each load would make each wait for the one before)
    float x[RW][E];
    typedef __attribute__((ext_vector_type(E / 2))) uint32_t uvec;
    uvec raw[RW];
#pragma unroll
    for (int j = 0; j < RW; ++j) {
        const int t = min(t0 + wave * RW + j, p.T - 1);
        raw[j] = *(const uvec *)((const bf16 *)p.v + (int64_t)b * p.v_bs + (int64_t)t * p.v_rs +
                                 (int64_t)h * D + lane * E);
    }
#pragma unroll
    for (int j = 0; j < RW; ++j) {
        const bool in = t0 + wave * RW + j < p.T;
#pragma unroll
        for (int e = 0; e < E; e += 2) {
            x[j][e] = in ? bf_lo(raw[j][e / 2]) : 0.f;
            x[j][e + 1] = in ? bf_hi(raw[j][e / 2]) : 0.f;
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
        for (int e = 0; e < E; ++e) tile[wave * RW + j][lane * E + e] = (_Float16)(x[j][e] * rs);
    }
    __syncthreads();
    // Operand units of the block: per key half hf and 32-channel block cb one 1 KB unit whose
    // lane r + 32g holds channel 32cb + r at keys 32kb + 16hf + 4g + {0..3, 8..11}. Keys past T
    // are written as zeros (their weights are 0, and 0 * 0 keeps the products finite); the
    // last block's k' rows past T are zeroed too.
    _Float16 *vbase = (_Float16 *)p.vt + (((int64_t)b * p.Hkv + h) * nkb + kb) * (D * 32);
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
        *(u32x4 *)(vbase + ((int64_t)hf * (D / 32) + cb) * 512 + l * 8) = pack8_f16(f);
    }
    if ((p.T & 31) && kb == nkb - 1) {
        _Float16 *kbase = (_Float16 *)p.kp + (((int64_t)b * p.Hkv + h) * nkb + kb) * (D * 32);
        for (int u = threadIdx.x; u < (D / 16) * 64; u += 256) {
            const int l = u & 63;
            if (t0 + (l & 31) >= p.T) *(u32x4 *)(kbase + u * 8) = u32x4{0, 0, 0, 0};
        }
    }
}

// The prologue as one launch: the q/k rows' workgroups, then the v blocks' (they write
// disjoint parts of k': rows below T, and the zeroed rows past T of the last block). (The v
// blocks first measured 1.5 us faster at D = 512, with 32 of them, and 1.6 us slower at
// D = 256, with 256.)
template <int D>
__global__ __launch_bounds__(256) void gemma_prep_kernel(const GemmaPrepParams p, int row_wgs) {
    __shared__ __attribute__((aligned(16))) _Float16 tile[32][D + 8];
    const int wg = blockIdx.x;
    if (wg < row_wgs) gemma_prep_rows<D>(p, wg);
    else gemma_vt_block<D>(p, wg - row_wgs, tile);
}
// ---- attention -----------------------------------------------------------------------------
// Geometry: a wave owns 32 queries over 256 channels of the head (D = 256: the whole head; D =
// 512: one half, its partner wave the other). Four waves per workgroup: 128 queries at D =
// 256, 64 at D = 512. A key block is 32 keys; its K' and V'^T operand units (D/16 and 2 * D/32
// units of 1 KB, contiguous per block in the prologue's layout) are copied HBM -> LDS by the
// buffer-load-to-LDS path into a ring of NS stages.
template <int D>
struct GemmaTile {
    static constexpr int SPLIT = D / 256;            // waves per query group
    static constexpr int QWG = 128 / SPLIT;          // queries per workgroup
    static constexpr int NCW = 256 / 16;             // Q'/K' 16-channel chunks per wave
    static constexpr int NDW = 256 / 32;             // V'^T / O 32-channel blocks per wave
    static constexpr int KBYTES = D * 32 * 2;        // K' (or V'^T) of one key block
    static constexpr int BLOCK = 2 * KBYTES;
    static constexpr int NS = D == 256 ? 4 : 2;      // key blocks resident (copies in flight)
    static constexpr int COPIES = BLOCK / 1024 / 4;  // 1 KB copies per wave per key block
    static constexpr int XBYTES = SPLIT > 1 ? 4 * 64 * 16 * 4 : 0;   // S partial exchange
};

// Key blocks of the query block [q0, q0 + nq): causal / window / padding bounds; a block with
// rows inside the left padding (their rows have no allowed key) runs over all keys, those rows
// unmasked.
struct KeyBlocks {
    int lo, hi;
};
__device__ __forceinline__ KeyBlocks gemma_key_blocks(const GemmaAttnParams &p, int q0, int nq,
                                                      int fv) {
    return KeyBlocks{gemma_key_lo(q0, fv, p.window), gemma_key_hi(p.T, q0, nq, fv)};
}

// The fast pass keeps each row's max from its first block with an allowed key; a later block
// whose weights would pass 2^kGemmaBound (log2 units over that max) sends the workgroup to
// the exact pass, which rescales O and l whenever a row's max grows.
constexpr float kGemmaBound = 15.0f;   // the fp16 weights stay below 65504

// Partial rows before query block qblk's within its head: the key ranges of the earlier query
// blocks that split (more than one range). Spread over the wave: lane j counts block j (j + 64,
// ...), and four ballots add the counts (at most kGemmaMaxChunks = 8: four bits), so the wave
// spends a few vector instructions instead of a scalar loop over every earlier block, which the
// CU's one scalar unit would run for each of its waves in turn. Every lane must be active; the
// result is uniform.
__device__ __forceinline__ int gemma_part_offset(int T, int window, int chunk, int qwg, int fv,
                                                 int qblk) {
    const int lane = (int)threadIdx.x & 63;
    int off = 0;
    for (int j0 = 0; j0 < qblk; j0 += 64) {
        const int j = j0 + lane;
        int n = j < qblk ? gemma_ranges(T, window, chunk, j * qwg, qwg, fv) : 0;
        if (n < 2) n = 0;
#pragma unroll
        for (int bit = 0; bit < 4; ++bit) off += __popcll(__ballot((n >> bit) & 1)) << bit;
    }
    return off;
}

template <int D>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void gemma_attn_kernel(const GemmaAttnParams p) {
    using G = GemmaTile<D>;
    constexpr int SPLIT = G::SPLIT, QWG = G::QWG, NCW = G::NCW, NDW = G::NDW, NS = G::NS;
    __shared__ __attribute__((aligned(16))) char smem[NS * G::BLOCK + G::XBYTES];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 31, g = lane >> 5;
    const int grp = wave / SPLIT, half = wave % SPLIT;   // query group, channel half
    const int T = p.T;
    const int nqb = (T + QWG - 1) / QWG;
    // grid layer `chunk` holds every query block's chunk-th key range; within a layer the
    // heaviest (latest) query blocks come first, each across all (batch row, head) pairs, so
    // the workgroups that the dispatcher deals to the 8 XCDs in turn carry equal work
    const int nbh = p.B * p.Hq;
    const int per_layer = nbh * nqb;
    const int chunk = (int)blockIdx.x / per_layer;
    const int rem = (int)blockIdx.x - chunk * per_layer;
    const int qblk = nqb - 1 - rem / nbh;
    const int bh = rem % nbh;
    const int h = bh % p.Hq, b = bh / p.Hq;
    const int kvh = h / (p.Hq / p.Hkv);
    const int q0 = qblk * QWG;
    const int fv = p.first_valid[b];
    const KeyBlocks kr = gemma_key_blocks(p, q0, QWG, fv);
    const int nch = gemma_ranges(T, p.window, p.chunk, q0, QWG, fv);
    if (chunk >= nch) return;                        // this block has fewer key ranges
    const int kb_lo = kr.lo + chunk * p.chunk;
    const int kb_hi = min(kb_lo + p.chunk - 1, kr.hi);
    const int nblk = kb_hi - kb_lo + 1;

    // ---- copies of key blocks into the ring ---------------------------------------------
    const int nkb_all = (T + 31) / 32;
    const int64_t head_off = ((int64_t)b * p.Hkv + kvh) * nkb_all * (D * 32);   // elements
    const u32x4 rk = rsrc_words((const bf16 *)p.kp + head_off, (int64_t)nkb_all * G::KBYTES);
    const u32x4 rv = rsrc_words((const bf16 *)p.vt + head_off, (int64_t)nkb_all * G::KBYTES);
    auto copy_block = [&](int i) __attribute__((always_inline)) {   // i-th block of the range
        const int kb = kb_lo + i;
        char *dst = smem + (i % NS) * G::BLOCK;
#pragma unroll
        for (int j = 0; j < G::COPIES; ++j) {
            const int u = wave * G::COPIES + j;          // 1 KB unit of the block: K' then V'^T
            const bool isk = u < G::KBYTES / 1024;
            const int uu = isk ? u : u - G::KBYTES / 1024;
            copy_all(isk ? rk : rv, (uint32_t)(uintptr_t)(lds_void *)(dst + u * 1024),
                     kb * G::KBYTES + uu * 1024 + lane * 16);
        }
    };
    // The first blocks' copies go out before the Q loads, so the two latencies overlap.
#pragma unroll
    for (int i = 0; i < NS - 1; ++i)
        if (i < nblk) copy_block(i);

    // ---- Q' of this wave: query q0 + 32 grp + r, channels 256 half + 16 c + 8 g .. +7 ---
    const int q = q0 + 32 * grp + r;                 // this lane's query row
    const int qr = min(q, T - 1);
    const int64_t qoff = (((int64_t)b * p.Hq + h) * T + qr) * D + 256 * half + 8 * g;
    f16x8 qh[NCW];
#pragma unroll
    for (int c = 0; c < NCW; ++c)
        qh[c] = __builtin_bit_cast(f16x8, ldg16((const _Float16 *)p.qp + qoff + 16 * c));
    // Q' is only an MFMA operand: home it in AGPRs, leaving the VGPRs to S, P and operands
#pragma unroll
    for (int c = 0; c < NCW; ++c) asm volatile("" : "+a"(qh[c]));
    // The row's allowed keys as one range [k_lo, k_hi]: all keys for a row inside the left
    // padding, else causal (k <= q), past the padding (k >= fv) and inside the window
    // (q - k < window); k_hi <= T - 1 also masks the keys past T of the last block.
    const bool free_row = q < fv;
    const int k_lo = free_row ? 0 : max(fv, p.window > 0 ? q - p.window + 1 : 0);
    const int k_hi = free_row ? T - 1 : min(q, T - 1);

    f32x16 o[NDW];
    float m, l;
    const f32x16 zero = splat16(0.f);               // the S chains' first SrcC
    float *xs = (float *)(smem + NS * G::BLOCK);     // [4 waves][4][64 lanes][4] partial S
    bool overflow = false;                           // some row's weights passed the bound

    // One pass over the range's key blocks. SAFE: the exact online softmax (O and l rescaled
    // when a row's max grows); otherwise each row's max is fixed at its first block with an
    // allowed key. `first`: the ring's first blocks are already on their way.
    auto run = [&](auto safe, bool first) __attribute__((always_inline)) {
        constexpr bool SAFE = decltype(safe)::value;
#pragma unroll
        for (int db = 0; db < NDW; ++db) o[db] = splat16(0.f);
        m = -INFINITY;
        l = 0.f;
        if (!first) {
#pragma unroll
            for (int i = 0; i < NS - 1; ++i)
                if (i < nblk) copy_block(i);
        }
        for (int i = 0; i < nblk; ++i) {
            // block i's copies have landed for this wave (later blocks' may still be in
            // flight); after the barrier for every wave, and the stage of block i - 1 is free
            if (i + NS - 2 < nblk) wait_copies_but<(NS - 2) * G::COPIES>();
            else wait_copies();
            __syncthreads();
            if (i + NS - 1 < nblk) copy_block(i + NS - 1);
            const char *Ks = smem + (i % NS) * G::BLOCK;
            const char *Vs = Ks + G::KBYTES;
            const int kb = kb_lo + i;
            // S^T over this wave's channels: one chain of inline products with S in VGPRs and
            // Q' in AGPRs (mfma_s.hpp); a product whose SrcC is the previous result issues
            // without waiting for it
            f32x16 s;
#pragma unroll
            for (int c = 0; c < NCW; ++c) {
                const f16x8 a = *(const __attribute__((address_space(3))) f16x8 *)(
                    (lds_void *)(Ks + (half * NCW + c) * 1024 + lane * 16));
                if (c == 0) s = mfma_s_first(a, qh[0], zero);
                else mfma_s_next(s, a, qh[c]);
            }
            s_ready(s, zero);
            if constexpr (SPLIT > 1) {
                // the partner wave holds the other half of the channels: exchange the partial
                // sums and add them in a fixed order, so both waves hold the same S
                // layout [wave][i4][lane][4]: a wave's 16-byte accesses are lane-contiguous,
                // free of bank conflicts
#pragma unroll
                for (int i4 = 0; i4 < 4; ++i4)
                    *(f32x4 *)(xs + ((wave * 4 + i4) * 64 + lane) * 4) =
                        f32x4{s[4 * i4], s[4 * i4 + 1], s[4 * i4 + 2], s[4 * i4 + 3]};
                __syncthreads();
#pragma unroll
                for (int i4 = 0; i4 < 4; ++i4) {
                    const f32x4 a0 = *(const f32x4 *)(xs + (((2 * grp) * 4 + i4) * 64 + lane) * 4);
                    const f32x4 a1 = *(const f32x4 *)(xs + (((2 * grp + 1) * 4 + i4) * 64 + lane) * 4);
#pragma unroll
                    for (int e = 0; e < 4; ++e) s[4 * i4 + e] = a0[e] + a1[e];
                }
            }
            // V'^T operands of the first key half, read now: they do not depend on the softmax
            // below, which hides their LDS round trip (read beside the products, two at a
            // time, each product waited for one)
            auto v_opnd = [&](int hf, int db) __attribute__((always_inline)) {
                return *(const __attribute__((address_space(3))) f16x8 *)(
                    (lds_void *)(Vs + (hf * (D / 32) + half * NDW + db) * 1024 + lane * 16));
            };
            f16x8 va0[NDW];
#pragma unroll
            for (int db = 0; db < NDW; ++db) va0[db] = v_opnd(0, db);
            // mask: key k = 32 kb + 8 (i >> 2) + 4 g + (i & 3) for query q. A block inside
            // every row's allowed range of the wave (most blocks of a causal or windowed range)
            // needs none: its five instructions per weight were a tenth of the block's
            // (1024 tokens, D 256: 33.1 -> 30.8 us)
            float mx = -INFINITY;
            if (__builtin_amdgcn_ballot_w64(k_lo > 32 * kb || 32 * kb + 31 > k_hi) == 0) {
#pragma unroll
                for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[e]);
            } else {
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int k = 32 * kb + 8 * (e >> 2) + 4 * g + (e & 3);
                    s[e] = ((k >= k_lo) & (k <= k_hi)) ? s[e] : -INFINITY;
                    mx = fmaxf(mx, s[e]);
                }
            }
            mx = fmaxf(mx, xlane32(mx));
            if constexpr (SAFE) {
                if (__builtin_amdgcn_ballot_w64(mx > m) != 0) {
                    const float mn = fmaxf(m, mx);
                    const float alpha = mn > m ? __builtin_amdgcn_exp2f(m - mn) : 1.0f;  // 0 from -inf
#pragma unroll
                    for (int db = 0; db < NDW; ++db) o[db] *= splat16(alpha);
                    l *= alpha;
                    m = mn;
                }
            } else {
                if (m == -INFINITY) m = mx;              // the row's first allowed keys
                overflow |= mx > m + kGemmaBound;
            }
            // fp32 weights, their fp32 row sums, and P in fp16 for P.V (11 significant bits; the
            // reference's explicit path multiplies fp32 weights); a row with no allowed key
            // so far has none
            u32x4 wh[2];
            float ts = 0.f;
            if (m == -INFINITY) {
                wh[0] = wh[1] = u32x4{0, 0, 0, 0};
            } else {
#pragma unroll
                for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float x0 = __builtin_amdgcn_exp2f(s[8 * hf + 2 * e] - m);
                        const float x1 = __builtin_amdgcn_exp2f(s[8 * hf + 2 * e + 1] - m);
                        ts += x0 + x1;
                        wh[hf][e] = pack_f16x2(x0, x1);
                    }
            }
            l += ts;
            // O^T += V^T.P^T for this wave's channels; consecutive products update different
            // accumulators (a key half over all channel blocks). The second half's operands are
            // read one before each product of the first half.
            f16x8 va1[NDW];
#pragma unroll
            for (int db = 0; db < NDW; ++db) {
                va1[db] = v_opnd(1, db);
                o[db] = mfma32(va0[db], __builtin_bit_cast(f16x8, wh[0]), o[db]);
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int db = 0; db < NDW; ++db)
                o[db] = mfma32(va1[db], __builtin_bit_cast(f16x8, wh[1]), o[db]);
        }
    };
    run(std::false_type{}, true);
    // the exact pass, for the whole workgroup, when any row outgrew its fixed max
    if (__syncthreads_or(overflow)) run(std::true_type{}, false);

    // ---- epilogue: O / l in fp32 (the reference's dtype here), this wave's channels ------
    const float lt = l + xlane32(l);
    if (nch > 1) {
        // one key range of several: unnormalised O, then (max, sum) per row, for the combine
        const int64_t row = p.part_row0[b] +
                            ((int64_t)h * p.part_chunks[b] +
                             gemma_part_offset(T, p.window, p.chunk, QWG, fv, qblk) + chunk) * QWG +
                            32 * grp + r;
        float *po = p.part_o + row * D + 256 * half;
#pragma unroll
        for (int db = 0; db < NDW; ++db)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                f32x4 w;
#pragma unroll
                for (int e = 0; e < 4; ++e) w[e] = o[db][4 * i4 + e];
                *(f32x4 *)(po + 32 * db + 8 * i4 + 4 * g) = w;
            }
        if (half == 0 && g == 0) {
            p.part_ml[row * 2] = m;
            p.part_ml[row * 2 + 1] = lt;
        }
        return;
    }
    if (q < T) {
        const float inv = 1.0f / lt;
        float *Ob = p.out + (int64_t)b * p.o_bs + (int64_t)q * p.o_rs + (int64_t)h * D + 256 * half;
#pragma unroll
        for (int db = 0; db < NDW; ++db)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                f32x4 w;
#pragma unroll
                for (int e = 0; e < 4; ++e) w[e] = o[db][4 * i4 + e] * inv;
                *(f32x4 *)(Ob + 32 * db + 8 * i4 + 4 * g) = w;
            }
    }
}

// Merge of a query block's key ranges: O = sum_c 2^(m_c - M) O_c / sum_c 2^(m_c - M) l_c over
// its ranges c (M the largest max; a range in which a row allows no key has m = -inf and adds
// nothing), written in fp32. A thread per 4 channels of kCombineRows rows (RPW rows apart);
// the workgroup's rows all belong to one query block (blocks with one range wrote their
// output themselves). The loads of a pass -- N ranges of `rows` rows, about 48 registers --
// are all issued before the first use: the merge is a chain of dependent loads otherwise, and
// several rows per thread keep the workgroups few enough that the launch runs in one round.
constexpr int kCombineRows = 4;

template <int D, int N>
__device__ __forceinline__ void gemma_merge_rows(const GemmaAttnParams &p, int64_t row0, int ch,
                                                 int q, float *out) {
    constexpr int QWG = GemmaTile<D>::QWG;
    constexpr int RPW = 256 / (D / 4);
    constexpr int PASS = N <= 2 ? kCombineRows : N <= 4 ? kCombineRows / 2 : 1;
#pragma unroll
    for (int g0 = 0; g0 < kCombineRows; g0 += PASS) {
        f32x2 ml[PASS][N];
        f32x4 oc[PASS][N];
#pragma unroll
        for (int r = 0; r < PASS; ++r)
#pragma unroll
            for (int c = 0; c < N; ++c) {
                const int64_t row = row0 + (int64_t)(g0 + r) * RPW + (int64_t)c * QWG;
                ml[r][c] = *(const f32x2 *)(p.part_ml + row * 2);
                oc[r][c] = *(const f32x4 *)(p.part_o + row * D + ch);
            }
#pragma unroll
        for (int r = 0; r < PASS; ++r) {
            if (q + (g0 + r) * RPW >= p.T) continue;   // rows past T: partials, no output
            float mx = -INFINITY;
#pragma unroll
            for (int c = 0; c < N; ++c) mx = fmaxf(mx, ml[r][c][0]);
            float lsum = 0.f;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < N; ++c) {
                const float m = ml[r][c][0];
                const float wgt = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mx);
                lsum += wgt * ml[r][c][1];
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[e] += wgt * oc[r][c][e];
            }
            const float inv = 1.0f / lsum;
            f32x4 w;
#pragma unroll
            for (int e = 0; e < 4; ++e) w[e] = acc[e] * inv;
            *(f32x4 *)(out + (int64_t)(g0 + r) * RPW * p.o_rs) = w;
        }
    }
}

template <int D>
__global__ __launch_bounds__(256) void gemma_combine_kernel(const GemmaAttnParams p) {
    constexpr int QWG = GemmaTile<D>::QWG;
    constexpr int U = D / 4;                        // threads per row
    constexpr int RPW = 256 / U;                    // rows per pass of the workgroup
    constexpr int WG_PER_QB = QWG / (RPW * kCombineRows);
    static_assert(WG_PER_QB * RPW * kCombineRows == QWG, "a query block's rows split evenly");
    const int nqb = (p.T + QWG - 1) / QWG;
    const int blk = (int)blockIdx.x / WG_PER_QB;    // (batch row, head, query block)
    const int qblk = blk % nqb;
    const int bh = blk / nqb;
    const int h = bh % p.Hq, b = bh / p.Hq;
    const int q0 = qblk * QWG;
    const int nch = gemma_ranges(p.T, p.window, p.chunk, q0, QWG, p.first_valid[b]);
    if (nch <= 1) return;
    const int off = gemma_part_offset(p.T, p.window, p.chunk, QWG, p.first_valid[b], qblk);
    const int rr = ((int)blockIdx.x % WG_PER_QB) * RPW * kCombineRows + (int)threadIdx.x / U;
    const int c4 = (int)threadIdx.x % U;
    const int q = q0 + rr;
    const int64_t row0 = p.part_row0[b] + ((int64_t)h * p.part_chunks[b] + off) * QWG + rr;
    // partial rows past T exist (a range writes all its block's rows) and are read, not merged
    float *out = p.out + (int64_t)b * p.o_bs + (int64_t)q * p.o_rs + (int64_t)h * D + 4 * c4;
    static_assert(kGemmaMaxChunks == 8, "one case per range count");
    switch (nch) {
    case 2: gemma_merge_rows<D, 2>(p, row0, 4 * c4, q, out); break;
    case 3: gemma_merge_rows<D, 3>(p, row0, 4 * c4, q, out); break;
    case 4: gemma_merge_rows<D, 4>(p, row0, 4 * c4, q, out); break;
    case 5: gemma_merge_rows<D, 5>(p, row0, 4 * c4, q, out); break;
    case 6: gemma_merge_rows<D, 6>(p, row0, 4 * c4, q, out); break;
    case 7: gemma_merge_rows<D, 7>(p, row0, 4 * c4, q, out); break;
    default: gemma_merge_rows<D, 8>(p, row0, 4 * c4, q, out); break;
    }
}

}  // namespace

int launch_gemma_prep(const GemmaPrepParams &p, int D, void *stream) {
    // rows per workgroup: four waves of kPrepPasses passes of one (D = 512) or two (D = 256)
    // rows
    const int64_t rows = (int64_t)p.B * p.T * (p.Hq + p.Hkv);
    if (rows > 0x7fffffff) return (int)hipErrorInvalidValue;   // 32-bit row indices
    const int64_t rows_wg = (D == 512 ? 4 : 8) * kPrepPasses;
    const int64_t row_wgs = (rows + rows_wg - 1) / rows_wg;
    const int64_t v_wgs = (int64_t)p.B * p.Hkv * ((p.T + 31) / 32);
    if (row_wgs + v_wgs > 0x7fffffff) return (int)hipErrorInvalidValue;
    const dim3 grid((unsigned)(row_wgs + v_wgs)), block(256);
    hipStream_t st = (hipStream_t)stream;
    if (D == 512) hipLaunchKernelGGL(gemma_prep_kernel<512>, grid, block, 0, st, p, (int)row_wgs);
    else hipLaunchKernelGGL(gemma_prep_kernel<256>, grid, block, 0, st, p, (int)row_wgs);
    return (int)hipGetLastError();
}

int launch_gemma_attn(const GemmaAttnParams &p, int D, void *stream) {
    const int qwg = D == 512 ? GemmaTile<512>::QWG : GemmaTile<256>::QWG;
    const int64_t per_layer = (int64_t)p.B * p.Hq * ((p.T + qwg - 1) / qwg);
    const dim3 grid((unsigned)(per_layer * p.nch_max)), block(256);
    hipStream_t st = (hipStream_t)stream;
    if (D == 512) hipLaunchKernelGGL(gemma_attn_kernel<512>, grid, block, 0, st, p);
    else hipLaunchKernelGGL(gemma_attn_kernel<256>, grid, block, 0, st, p);
    if (p.nch_max > 1) {
        const dim3 cgrid((unsigned)(per_layer * qwg / (256 / (D / 4) * kCombineRows)));
        if (D == 512) hipLaunchKernelGGL(gemma_combine_kernel<512>, cgrid, block, 0, st, p);
        else hipLaunchKernelGGL(gemma_combine_kernel<256>, cgrid, block, 0, st, p);
    }
    return (int)hipGetLastError();
}

int gemma_queries_per_workgroup(int D) {
    return D == 512 ? GemmaTile<512>::QWG : GemmaTile<256>::QWG;
}

}  // namespace ltx
