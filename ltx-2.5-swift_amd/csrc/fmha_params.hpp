// Kernel parameter blocks shared by the HIP kernels (fmha_fwd.hip) and the C-ABI layer
// (ltx_attn_abi.cpp). Plain data only: no HIP or torch types.
#pragma once

#include <stdarg.h>
#include <stddef.h>
#include <stdint.h>

namespace ltx {

constexpr int kMaxBatch = 64;      // per-row key lengths travel in the kernel arguments
constexpr int kKeyTile = 64;       // keys per LDS tile
constexpr int kQueriesPerWave = 64;
constexpr int kWavesPerGroup = 4;
constexpr int kQueriesPerGroup = kQueriesPerWave * kWavesPerGroup;  // 256
constexpr int kMaxSplits = 16;
// Keys of one (batch, head) the short-key kernel keeps resident in LDS.
constexpr int short_max_keys(int D) { return D == 128 ? 128 : 256; }

// Main attention kernel.
struct FmhaParams {
    const void *q, *k, *v;           // bf16
    int64_t q_bs, q_rs, q_hs;
    int64_t k_bs, k_rs, k_hs;
    int64_t v_bs, v_rs, v_hs;
    void *o;                         // bf16 output (unsplit) -- element strides below
    int64_t o_bs, o_rs, o_hs;
    int32_t B, H, Lq, Lk;

    // Q prologue, applied in registers when the wave loads its queries.
    const float *q_rstd;             // [B][Lq] or null (no norm)
    const void *q_w;                 // bf16 [H*D] (with q_rstd)
    const void *q_cos, *q_sin;       // bf16 [H][Lq][D/2] or null (no RoPE)

    // K prologue applied while staging K into LDS (KFUSED kernels only).
    const float *k_rstd;             // [B][Lk] or null
    const void *k_w;
    const void *k_cos, *k_sin;       // bf16 [H][Lk][D/2] or null

    float qk_scale_log2;             // softmax scale * log2(e), folded into Q
    int32_t nqblk;                   // ceil(Lq / 256)
    // Work items are (batch, head, query block), item = (b*H + h)*nqblk + qblk. Items
    // [0, n_full) run over all their keys; each of the n_items - n_full tail items is split
    // into num_splits key ranges of tiles_per_split tiles, whose partial results the combine
    // kernel merges. The grid is n_full + (n_items - n_full) * num_splits workgroups.
    int32_t n_items;
    int32_t n_full;
    int32_t num_splits;              // >= 1 (tail items only)
    int32_t tiles_per_split;         // key tiles per split
    int32_t grid;
    // The first n_lead workgroups run tail splits, then the whole items, then the other tail
    // splits (n_lead a multiple of 8): the CUs that start on a short split begin their whole
    // items that much later, so that the rounds' Q loads and O stores are not all at once.
    int32_t n_lead;
    float *part_o;                   // tail partials [S][n_tail][256][D] fp32
    float *part_ml;                  // [S][n_tail][256][2]: running max (log2 units), row sum
    int32_t valid[kMaxBatch];        // keys valid per batch row (Lk when unmasked)
    // Short-key kernel: workgroups per (batch, head); the grid is B * H * short_groups.
    int32_t short_groups;
    // Output gate: bf16 logits, element strides; output rows times 2*sigmoid(logit), or null.
    const void *gate;
    int64_t g_bs, g_rs, g_hs;
};

// Per-token RMS statistic over the inner dim, optionally writing the normalised and rotated
// tensor (the K prologue).
struct PrepParams {
    const void *x;                   // bf16
    int64_t bs, rs, hs;
    int32_t B, L, H;                 // rows 0 .. L-1 of each batch row are processed
    int32_t L_full;                  // rows per batch of the tables, rstd and partials (0: L)
    const void *w;                   // bf16 [H*D] or null (no norm)
    float eps;
    const void *cos, *sin;           // bf16 [H][L_full][D/2] or null
    float *rstd;                     // [B][L_full] or null
    void *out;                       // bf16 [B][L][H*D] contiguous or null
    // Statistic given as partial sums of squares (row b*L_full + l at sumsq + row*ss_rs,
    // ss_blocks partials), or null: computed from x.
    const float *sumsq;
    int64_t ss_rs;
    int32_t ss_blocks;
};

// Split-KV combine over the tail items' rows.
struct CombineParams {
    const float *part_o;
    const float *part_ml;
    void *o;
    int64_t o_bs, o_rs, o_hs;
    int32_t H, Lq, nqblk;
    int32_t n_full, n_tail, num_splits;
    const void *gate;                // as in FmhaParams
    int64_t g_bs, g_rs, g_hs;
};

// STG passthrough: out = V (x 2*sigmoid(gate logit)) per (batch, token, head) row.
struct PassParams {
    const void *v;
    int64_t v_bs, v_rs, v_hs;
    void *o;
    int64_t o_bs, o_rs, o_hs;
    int32_t B, L, H;
    const void *gate;
    int64_t g_bs, g_rs, g_hs;
};

// Projection GEMM y = x . w^T (+ bias) over 256 x 256 output tiles, with the per-row sum of
// squares of each tile's bf16 outputs (the RMS-norm statistic of the projection).
constexpr int kLinearTile = 256;
struct LinearParams {
    const void *x;                   // bf16 [M][K], row stride x_rs elements
    const void *w;                   // bf16 [N][K], row stride w_rs elements
    const void *bias;                // bf16 [N] or null
    void *y;                         // bf16 [M][N], row stride y_rs elements
    int64_t x_rs, w_rs, y_rs;
    float *sumsq;                    // [M][ceil(N/256)] (row stride ss_rs floats) or null
    int64_t ss_rs;
    int32_t M, N, K;
    int32_t tiles_m, tiles_n;
    // Tail split: tiles [n_full, tiles_m * tiles_n) of the tile order are cut into `splits`
    // ranges of `steps_per_split` 64-wide k steps; each range writes its fp32 accumulators to
    // part (256 KiB per range, tile-major) and linear_fixup_kernel sums them. splits == 1:
    // every tile whole (n_full = tiles_m * tiles_n).
    float *part;
    int32_t n_full, splits, steps_per_split;
    // Workgroups of the launch: workgroup g runs whole tiles g, g + grid, ... below n_full,
    // then tail range g (grid >= the number of ranges).
    int32_t grid;
};

// RMS statistic from partial sums of squares: rstd[row] = 1/sqrt(sum_j parts[row][j] / n + eps)
// for rows [0, rows); parts row r at sumsq + r*rs, `blocks` partials.
struct RstdParams {
    const float *sumsq;
    int64_t rs;
    int32_t rows, blocks, n;
    float eps;
    float *rstd;
};

// Gemma-4 text-encoder attention (gemma_attn.hip). The prologue normalises (per head over D),
// rotates and scales q and k into q' [B][Hq][T][D], k' [B][Hkv][T][D], and normalises v into
// v' stored transposed, [B][Hkv][D][T].
struct GemmaPrepParams {
    const void *q, *k, *v;           // bf16 projections, element strides below
    int64_t q_bs, q_rs, k_bs, k_rs, v_bs, v_rs;
    int32_t B, T, Hq, Hkv;
    const void *q_w, *k_w;           // bf16 [D]
    float eps;
    float q_factor;                  // scale * log2(e), folded into q'
    const float *cos, *sin;          // fp32 [T][D/2]
    void *qp, *kp, *vt;              // fp16 outputs (workspace)
};
constexpr int kGemmaMaxChunks = 8;  // key ranges per Gemma query block, at most

struct GemmaAttnParams {
    const void *qp, *kp, *vt;
    float *out;                      // fp32 [B][T][Hq*D], element strides below
    int64_t o_bs, o_rs;
    int32_t B, T, Hq, Hkv;
    int32_t window;                  // 0: causal only
    int32_t first_valid[kMaxBatch];  // keys below are left padding
    // Key split: a query block's key blocks (32 keys each) run in ranges of `chunk` blocks,
    // at most `nch_max` per query block; with more than one, each range writes fp32 partials
    // (unnormalised O, then the row's max and sum) that gemma_combine_kernel merges. The grid
    // is nch_max layers of B * Hq * query blocks. Partials exist only for the ranges of query
    // blocks with more than one: batch row b's start at row part_row0[b], head-major, each head
    // holding part_chunks[b] ranges of `queries` rows, a query block's ranges after those of
    // the earlier split blocks of its head.
    int32_t chunk, nch_max;          // nch_max <= kGemmaMaxChunks
    float *part_o;                   // [rows][D]
    float *part_ml;                  // [rows][2]
    int64_t part_row0[kMaxBatch];
    int32_t part_chunks[kMaxBatch];
};

// Key blocks (32 keys) [lo, hi] of the Gemma query block of nq queries from q0 in a batch row
// whose keys below fv are left padding: causal, and within the window when one is set; a block
// with rows inside the padding walks every key. Its range count, at `chunk` blocks per range.
// Shared by the host's workspace layout and the kernels (constexpr: callable from both).
constexpr int gemma_key_lo(int q0, int fv, int window) {
    return q0 < fv ? 0 : (window > 0 && q0 - window + 1 > fv ? q0 - window + 1 : fv) / 32;
}
constexpr int gemma_key_hi(int T, int q0, int nq, int fv) {
    return q0 < fv ? (T + 31) / 32 - 1 : ((q0 + nq - 1 < T - 1 ? q0 + nq - 1 : T - 1) / 32);
}
// (The count is at most kGemmaMaxChunks -- the host sizes `chunk` so -- and is taken by
// comparisons rather than an integer division, which the kernels would expand into a long
// sequence per call.)
constexpr int gemma_ranges(int T, int window, int chunk, int q0, int nq, int fv) {
    const int x = gemma_key_hi(T, q0, nq, fv) - gemma_key_lo(q0, fv, window) + chunk;
    int n = 0;
    for (int k = 1; k <= kGemmaMaxChunks; ++k) n += x >= k * chunk ? 1 : 0;
    return n;
}

// Host side: set the calling thread's error detail (ltx_attn_last_error) from a printf
// format and its va_list, and return `s`. Defined in ltx_attn_abi.cpp, not exported.
__attribute__((visibility("hidden"))) int set_error_detail(int s, const char *fmt, va_list ap);

// Launchers (fmha_fwd.hip). Return the hipError_t of the launch as int.
// Attention kernels:
//   kRegPlain  K and V staged through registers (V transposed on the way into LDS)
//   kRegFused  the same, with QK-RMSNorm + RoPE applied to K while staging
//   kDma       K (prepared or raw) and V copied HBM -> LDS by the buffer-load-to-LDS path;
//              no staging registers
enum KernelKind { kRegPlain = 0, kRegFused = 1, kDma = 2 };
int launch_fmha(const FmhaParams &p, int D, int kind, void *stream);
int launch_fmha_dma(const FmhaParams &p, int D, void *stream);   // fmha_dma.hip
int launch_fmha_short(const FmhaParams &p, int D, void *stream); // fmha_short.hip
int launch_fmha_splitk(const FmhaParams &p, int D, void *stream);  // fmha_splitk.hip
int launch_prep(const PrepParams &p, int D, void *stream);
// Two row sets in one launch (a call's Q statistic and its K prologue); same H * D.
int launch_prep2(const PrepParams &a, const PrepParams &b, int D, void *stream);
int launch_combine(const CombineParams &p, int D, void *stream);
int launch_passthrough(const PassParams &p, int D, void *stream);
int launch_rstd(const RstdParams &p, void *stream);
int launch_linear(const LinearParams &p, void *stream);           // linear_gemm.hip
int64_t linear_part_bytes(int64_t tail_tiles, int splits);          // one range: 256 KiB
int launch_gemma_prep(const GemmaPrepParams &p, int D, void *stream);   // gemma_attn.hip
int launch_gemma_attn(const GemmaAttnParams &p, int D, void *stream);
int gemma_queries_per_workgroup(int D);                              // 128 (D 256), 64 (D 512)

}  // namespace ltx
