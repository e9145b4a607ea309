// C-ABI entry points of libltx_attn.so (declared in include/ltx_attn.h).
//
// Replaces the arithmetic of Sources/LTXModules/DiTAttention.swift:358-381: the QK-RMSNorm
// (:360-361 -> :202-204), the head split (:362 -> :346-349), split RoPE (:364-367 ->
// :226-234) and MLXFast.scaledDotProductAttention (:374-376). Everything here runs on the
// host: argument validation (before any launch), the choice of K strategy and split count,
// the workspace layout, and the launches on the caller's stream.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <utility>

#include "../../include/ltx_attn.h"
#include "fmha_params.hpp"

namespace {

thread_local char g_err[512];

ltx_attn_status fail(ltx_attn_status s, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return s;
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Attention and projection workgroups resident at once: one per CU (each holds most of a CU's
// LDS). Workspace sizing and validation are pure host functions and plan for a whole gfx950
// part, 256 CUs; a call plans again for its device's CU count (device_groups) and runs that
// plan when the caller's workspace covers it, else the sized one. Both are correct; only the
// tail splitting differs.
constexpr int64_t kConcurrentGroups = 256;

// CU count of the calling thread's current device, queried once per device (the count does
// not change while the process runs); kConcurrentGroups if the runtime cannot say (the error
// of a failed query is cleared so that the launches' checks do not see it). A caller's
// resident_groups > 0 stands in for it (tests of the plans of other part sizes).
constexpr int kMaxDevices = 64;
std::atomic<int32_t> g_device_cus[kMaxDevices];   // 0 = not queried yet

int64_t device_groups(int32_t override_groups) {
    if (override_groups > 0) return override_groups;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        return kConcurrentGroups;
    }
    if (dev >= 0 && dev < kMaxDevices) {
        const int32_t known = g_device_cus[dev].load(std::memory_order_relaxed);
        if (known > 0) return known;
    }
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0) {
        (void)hipGetLastError();
        return kConcurrentGroups;
    }
    if (dev >= 0 && dev < kMaxDevices) g_device_cus[dev].store(cus, std::memory_order_relaxed);
    return cus;
}
// Charge per extra split of a tail item, in rounds: its fp32 partial O is written and read
// back by the combine kernel.
constexpr double kSplitCharge = 0.02;

// Everything ltx_attn_fwd decides from the arguments alone.
struct Plan {
    bool q_norm = false, k_norm = false;
    bool q_stat = false, k_stat = false;   // statistic from the projection's partial sums
    bool q_rope = false, k_rope = false;
    bool passthrough = false;  // STG passthrough: out = V (x gate), no attention
    bool dma = false;          // LDS-DMA kernel (K prologue when K needs work)
    bool shortk = false;       // short-key kernel: the head's keys resident in LDS
    bool splitk = false;       // split-key kernel: one query block over key ranges, K
                               // normalised/rotated in LDS
    bool k_prologue = false;   // K normalised/rotated by a separate pass into the workspace
    bool k_fused = false;      // K normalised/rotated while staging into LDS
    int nqblk = 0;
    int ntiles_max = 0;
    int kmax = 0;              // largest valid key count over the batch
    int kprep_rows = 0;        // rows per batch the K prologue prepares
    int short_groups = 0;
    int64_t n_items = 0;       // (batch, head, query block) work items
    int64_t n_full = 0;        // items run whole; the rest are split into key ranges
    int splits = 1;
    int tiles_per_split = 0;
    int32_t n_lead = 0;        // tail splits placed ahead of the whole items (multiple of 8)
    int64_t grid = 0;
    // workspace layout (byte offsets)
    size_t off_qrstd = 0, off_krstd = 0, off_kprep = 0, off_part_o = 0, off_part_ml = 0;
    size_t bytes = 0;
};

ltx_attn_status check_tensor(const char *name, const void *ptr, int64_t bs, int64_t rs,
                             int64_t hs, int B, int L, int H, int D) {
    if (!ptr) return fail(LTX_ATTN_EINVAL, "%s is NULL", name);
    if (!aligned16(ptr)) return fail(LTX_ATTN_EINVAL, "%s is not 16-byte aligned", name);
    if (bs < 0 || rs < 0 || hs < 0)
        return fail(LTX_ATTN_EINVAL, "%s has a negative stride", name);
    if ((bs % 8) || (rs % 8) || (hs % 8))
        return fail(LTX_ATTN_EINVAL,
                    "%s strides (%lld, %lld, %lld) must be multiples of 8 elements", name,
                    (long long)bs, (long long)rs, (long long)hs);
    if (H > 1 && hs < D)
        return fail(LTX_ATTN_EINVAL, "%s head stride %lld overlaps a %d-wide head", name,
                    (long long)hs, D);
    if (L > 1 && rs < D)
        return fail(LTX_ATTN_EINVAL, "%s row stride %lld is below the head dim %d", name,
                    (long long)rs, D);
    if (B > 1 && bs == 0) return fail(LTX_ATTN_EINVAL, "%s batch stride is 0", name);
    return LTX_ATTN_OK;
}

ltx_attn_status make_plan(const ltx_attn_args *a, Plan *pl,
                          int64_t groups = kConcurrentGroups) {
    g_err[0] = 0;
    if (!a) return fail(LTX_ATTN_EINVAL, "args is NULL");
    if (a->B < 1 || a->H < 1 || a->Lq < 1 || a->Lk < 1)
        return fail(LTX_ATTN_EINVAL, "B, H, Lq, Lk must be >= 1 (got %d, %d, %d, %d)", a->B,
                    a->H, a->Lq, a->Lk);
    if (a->D != 64 && a->D != 128)
        return fail(LTX_ATTN_EUNSUPPORTED, "head dim %d is not 64 or 128", a->D);
    const int B = a->B, H = a->H, D = a->D;
    if ((int64_t)H * D > 16384)
        return fail(LTX_ATTN_EUNSUPPORTED, "inner dim %lld above 16384", (long long)H * D);
    ltx_attn_status s;
    if (a->all_perturbed) {
        // STG passthrough: only V, the output and the gate take part.
        if (a->Lq != a->Lk)
            return fail(LTX_ATTN_EINVAL, "all_perturbed is self-attention only (Lq %d != Lk %d)",
                        a->Lq, a->Lk);
        if ((s = check_tensor("v", a->v, a->v_bs, a->v_rs, a->v_hs, B, a->Lk, H, D))) return s;
        if ((s = check_tensor("out", a->out, a->o_bs, a->o_rs, a->o_hs, B, a->Lq, H, D)))
            return s;
        if (a->gate_logits && (((uintptr_t)a->gate_logits & 1u) || a->g_bs < 0 || a->g_rs < 0 ||
                               a->g_hs < 0))
            return fail(LTX_ATTN_EINVAL, "gate_logits misaligned or with a negative stride");
        pl->passthrough = true;
        pl->bytes = 0;
        return LTX_ATTN_OK;
    }
    if ((s = check_tensor("q", a->q, a->q_bs, a->q_rs, a->q_hs, B, a->Lq, H, D))) return s;
    if ((s = check_tensor("k", a->k, a->k_bs, a->k_rs, a->k_hs, B, a->Lk, H, D))) return s;
    if ((s = check_tensor("v", a->v, a->v_bs, a->v_rs, a->v_hs, B, a->Lk, H, D))) return s;
    if ((s = check_tensor("out", a->out, a->o_bs, a->o_rs, a->o_hs, B, a->Lq, H, D))) return s;
    if (!(a->scale > 0.f) || !isfinite(a->scale))
        return fail(LTX_ATTN_EINVAL, "scale must be positive and finite");
    if (a->gate_logits) {
        if ((uintptr_t)a->gate_logits & 1u)
            return fail(LTX_ATTN_EINVAL, "gate_logits is not 2-byte aligned");
        if (a->g_bs < 0 || a->g_rs < 0 || a->g_hs < 0)
            return fail(LTX_ATTN_EINVAL, "gate_logits has a negative stride");
    }

    pl->q_norm = a->q_norm_w != nullptr;
    pl->k_norm = a->k_norm_w != nullptr;
    if ((pl->q_norm && !aligned16(a->q_norm_w)) || (pl->k_norm && !aligned16(a->k_norm_w)))
        return fail(LTX_ATTN_EINVAL, "norm weights must be 16-byte aligned");
    if ((pl->q_norm || pl->k_norm) && !(a->norm_eps >= 0.f && isfinite(a->norm_eps)))
        return fail(LTX_ATTN_EINVAL, "norm_eps must be finite and >= 0");
    if (a->q_sumsq || a->k_sumsq) {
        if ((a->q_sumsq && !pl->q_norm) || (a->k_sumsq && !pl->k_norm))
            return fail(LTX_ATTN_EINVAL, "a projection statistic without its norm weight");
        if (a->sumsq_blocks < 1)
            return fail(LTX_ATTN_EINVAL, "sumsq_blocks must be >= 1 (got %d)", a->sumsq_blocks);
        if (((uintptr_t)a->q_sumsq & 3u) || ((uintptr_t)a->k_sumsq & 3u))
            return fail(LTX_ATTN_EINVAL, "statistic partials must be 4-byte aligned");
        if ((a->q_sumsq && a->q_sumsq_rs < a->sumsq_blocks) ||
            (a->k_sumsq && a->k_sumsq_rs < a->sumsq_blocks))
            return fail(LTX_ATTN_EINVAL, "statistic row stride below sumsq_blocks (%d)",
                        a->sumsq_blocks);
        pl->q_stat = a->q_sumsq != nullptr;
        pl->k_stat = a->k_sumsq != nullptr;
    }

    const bool qt = a->q_cos || a->q_sin, kt = a->k_cos || a->k_sin;
    if ((a->q_cos == nullptr) != (a->q_sin == nullptr) ||
        (a->k_cos == nullptr) != (a->k_sin == nullptr))
        return fail(LTX_ATTN_EINVAL, "a rotary table pair needs both cos and sin");
    if (kt && !qt)
        return fail(LTX_ATTN_EINVAL,
                    "key rotary tables without query tables (keyRotary without rotary)");
    if (qt && !kt && a->Lq != a->Lk)
        return fail(LTX_ATTN_EINVAL,
                    "K shares Q's rotary tables but Lq (%d) != Lk (%d); pass k_cos/k_sin",
                    a->Lq, a->Lk);
    for (const void *t : {a->q_cos, a->q_sin, a->k_cos, a->k_sin})
        if (t && !aligned16(t)) return fail(LTX_ATTN_EINVAL, "rotary tables must be 16-byte aligned");
    pl->q_rope = qt;
    pl->k_rope = qt;

    if (a->k_valid_len) {
        if (B > ltx::kMaxBatch)
            return fail(LTX_ATTN_EUNSUPPORTED, "key-padding lengths need B <= %d (got %d)",
                        ltx::kMaxBatch, B);
        for (int b = 0; b < B; ++b)
            if (a->k_valid_len[b] < 1 || a->k_valid_len[b] > a->Lk)
                return fail(LTX_ATTN_EINVAL, "k_valid_len[%d] = %d outside [1, %d]", b,
                            a->k_valid_len[b], a->Lk);
    } else if (B > 65535) {
        return fail(LTX_ATTN_EUNSUPPORTED, "batch %d too large", B);
    }
    if (a->kprep < LTX_ATTN_KPREP_AUTO || a->kprep > LTX_ATTN_KPREP_PROLOGUE)
        return fail(LTX_ATTN_EINVAL, "kprep %d is not an ltx_attn_kprep", a->kprep);
    if (a->resident_groups < 0 || a->resident_groups > 65536)
        return fail(LTX_ATTN_EINVAL, "resident_groups %d outside [0, 65536]", a->resident_groups);
    if (a->num_splits < 0 || a->num_splits > ltx::kMaxSplits)
        return fail(LTX_ATTN_EINVAL, "num_splits %d outside [0, %d]", a->num_splits,
                    ltx::kMaxSplits);

    pl->nqblk = (a->Lq + ltx::kQueriesPerGroup - 1) / ltx::kQueriesPerGroup;
    pl->kmax = a->Lk;
    if (a->k_valid_len) {
        pl->kmax = 1;
        for (int b = 0; b < B; ++b) pl->kmax = std::max(pl->kmax, (int)a->k_valid_len[b]);
    }
    pl->ntiles_max = (pl->kmax + ltx::kKeyTile - 1) / ltx::kKeyTile;
    pl->kprep_rows = a->Lk;

    // Kernel: with two or more query blocks per (batch, head) the LDS-DMA kernel reads K
    // (prepared by the K prologue when it needs norm/RoPE, one extra read+write of K) and V
    // straight into LDS. A single query block takes the register-staged kernel, fusing K's
    // norm/RoPE into its staging. The DMA kernel addresses one head's K and V rows with
    // 32-bit byte offsets up to the key length padded to whole tiles; calls past that take
    // the register-staged kernel.
    const bool k_work = pl->k_norm || pl->k_rope;
    // Short key ranges (text cross-attention over its valid keys, video queries over the
    // audio keys) take the short-key kernel: the head's K (prepared by the prologue, only
    // its valid rows, when it needs norm/RoPE) and V stay in LDS while the queries stream
    // past. It addresses a head's Q rows with 32-bit byte offsets, and has no D = 128
    // variant with RoPE (no such call in the model: text cross-attention takes no RoPE).
    const int64_t lq_pad = ((int64_t)a->Lq + ltx::kQueriesPerWave - 1) / ltx::kQueriesPerWave *
                           ltx::kQueriesPerWave;
    if (a->kprep == LTX_ATTN_KPREP_AUTO && a->num_splits == 0 && B <= ltx::kMaxBatch &&
        pl->kmax <= ltx::short_max_keys(D) && !(D == 128 && pl->q_rope) &&
        lq_pad * a->q_rs * 2 < 0x7fffffff) {
        pl->shortk = true;
        pl->k_prologue = k_work;
        pl->kprep_rows = pl->kmax;
        // Eight waves of 32-query blocks per workgroup (twelve at D = 64); one workgroup per
        // CU: B*H*G workgroups over the CUs, no more groups than a head's query blocks fill.
        const int waves = D == 64 ? 12 : 8, qw = 32;
        const int64_t heads = (int64_t)B * H;
        const int64_t nqb = (a->Lq + qw - 1) / qw;
        int64_t G = (groups + heads - 1) / heads;
        G = std::max<int64_t>(1, std::min(G, (nqb + waves - 1) / waves));
        pl->short_groups = (int)G;
        pl->n_items = pl->n_full = heads * G;
        pl->grid = heads * G;
        if (pl->grid > 0x7fffffff) return fail(LTX_ATTN_EUNSUPPORTED, "grid too large");
        size_t off = 0;
        if (pl->q_norm) {
            pl->off_qrstd = off;
            off = align_up(off + sizeof(float) * (size_t)B * a->Lq, 256);
        }
        if (pl->k_prologue) {
            pl->off_kprep = off;
            off = align_up(off + 2 * (size_t)B * pl->kprep_rows * H * D, 256);
        }
        pl->bytes = off;
        return LTX_ATTN_OK;
    }
    const int64_t lk_pad = ((int64_t)a->Lk + ltx::kKeyTile - 1) / ltx::kKeyTile * ltx::kKeyTile;
    const int64_t k_rs_eff = k_work ? (int64_t)H * D : a->k_rs;
    const bool dma_fits = lk_pad * k_rs_eff * 2 < 0x7fffffff && lk_pad * a->v_rs * 2 < 0x7fffffff;
    if (a->kprep == LTX_ATTN_KPREP_PROLOGUE) pl->dma = dma_fits;
    else if (a->kprep == LTX_ATTN_KPREP_AUTO) pl->dma = dma_fits && pl->nqblk >= 2;
    if (pl->dma) pl->k_prologue = k_work;
    else pl->k_fused = k_work;
    // One query block per (batch, head) over a key stream read once, at head dim 64 (the
    // audio queries over the video keys): the split-key kernel streams K (raw), its statistic
    // and table rows, and V through LDS by LDS DMA, three tiles ahead, over key ranges spread
    // across the whole GPU. Its copies address a head's raw K and V rows with 32-bit byte
    // offsets.
    const int64_t raw_k_bytes = lk_pad * a->k_rs * 2;
    if (a->kprep == LTX_ATTN_KPREP_AUTO && !pl->dma && pl->nqblk == 1 && D == 64 &&
        B <= ltx::kMaxBatch &&
        raw_k_bytes < 0x7fffffff && lk_pad * a->v_rs * 2 < 0x7fffffff)
        pl->splitk = true;

    // Work decomposition. One workgroup per CU runs at once. The whole rounds of items run
    // unsplit; the items of a last round that would leave most CUs idle are split into key
    // ranges so that they finish in a fraction of a round (split-KV, merged by the combine
    // kernel).
    // A split count S costs ceil(rem*S/256)/S rounds for the rem tail items plus a small
    // per-split charge for the partial results. A caller-fixed num_splits splits every item.
    // Calls beyond one argument table of batches (B > kMaxBatch, sliced launches) run whole.
    const int64_t N = (int64_t)B * H * pl->nqblk;
    int64_t n_full = N;
    int splits = 1;
    if (pl->splitk) {
        // about one key range per CU (measured best for 32 heads over 3120 keys and 2 x 32
        // over 15360: more ranges add start-ups and partials faster than they add overlap),
        // none shorter than two tiles
        splits = a->num_splits > 0
                     ? a->num_splits
                     : (int)std::min<int64_t>(ltx::kMaxSplits,
                                              (groups + N - 1) / N);
        splits = std::max(1, std::min(splits, (pl->ntiles_max + 1) / 2));
        n_full = 0;
    } else if (a->num_splits > 0) {
        splits = a->num_splits;
        n_full = 0;
    } else if (B <= ltx::kMaxBatch) {
        const int64_t rounds = N / groups, rem = N - rounds * groups;
        // A last round on at most half the CUs is split; a fuller one is not: with fewer
        // workgroups resident each runs its tiles faster (measured at 3120 tokens: the 160
        // tail items unsplit finish as fast as split three ways, without the combine).
        if (rem > 0 && 2 * rem <= groups) {
            double best = 1.0;
            for (int sp = 2; sp <= ltx::kMaxSplits && sp <= pl->ntiles_max; ++sp) {
                const double c =
                    (double)((rem * sp + groups - 1) / groups) / sp +
                    kSplitCharge * (sp - 1);
                if (c < best - 1e-9) {
                    best = c;
                    splits = sp;
                }
            }
            if (splits > 1) n_full = rounds * groups;
        }
    }
    splits = std::max(1, std::min(splits, pl->ntiles_max));
    pl->tiles_per_split = (pl->ntiles_max + splits - 1) / splits;
    pl->splits = (pl->ntiles_max + pl->tiles_per_split - 1) / pl->tiles_per_split;
    if (pl->splits == 1) n_full = N;
    pl->n_items = N;
    pl->n_full = n_full;
    pl->grid = n_full + (N - n_full) * pl->splits;
    // Half the tail splits (a multiple of 8: every XCD the same share) lead the grid when
    // whole rounds precede them.
    pl->n_lead = n_full > 0 && n_full < N ? (int32_t)(((N - n_full) * pl->splits / 2) & ~7ll) : 0;
    if (pl->grid > 0x7fffffff)
        return fail(LTX_ATTN_EUNSUPPORTED, "grid too large");

    size_t off = 0;
    if (pl->q_norm) {
        pl->off_qrstd = off;
        off = align_up(off + sizeof(float) * (size_t)B * a->Lq, 256);
    }
    if (pl->k_norm && pl->k_fused) {
        pl->off_krstd = off;
        off = align_up(off + sizeof(float) * (size_t)B * a->Lk, 256);
    }
    if (pl->k_prologue) {
        pl->off_kprep = off;
        off = align_up(off + 2 * (size_t)B * a->Lk * H * D, 256);
    }
    if (pl->n_full < pl->n_items) {
        const size_t rows = (size_t)pl->splits * (pl->n_items - pl->n_full) * ltx::kQueriesPerGroup;
        pl->off_part_o = off;
        off = align_up(off + sizeof(float) * rows * D, 256);
        pl->off_part_ml = off;
        off = align_up(off + sizeof(float) * rows * 2, 256);
    }
    pl->bytes = off;
    return LTX_ATTN_OK;
}

// Gemma-4 text-encoder attention: validation and workspace layout.

struct GemmaPlan {
    size_t off_q = 0, off_k = 0, off_v = 0, off_po = 0, off_pml = 0, bytes = 0;
    int32_t chunk = 0, nch_max = 1;
    int64_t part_row0[ltx::kMaxBatch] = {};   // first partial row of each batch row
    int32_t part_chunks[ltx::kMaxBatch] = {}; // split ranges per head of each batch row
};

// Key blocks (32 keys) per range of a Gemma query block. The latest query blocks of a causal
// layer walk every key block while the earliest walk a few; ranges of at most 16 blocks spread
// the long ones over several CUs at the price of fp32 partials and a merge. Measured at 1024
// tokens (MI355X, attention + merge): ranges of 16 blocks 45 + 7 us (D 256, 128-query
// workgroups) and 79 + 11 us (D 512, 64-query workgroups), of 8 blocks 53 + 10 and 99 + 17 us.
// Longer prompts take longer ranges, so that a query block never has more than the merge's
// kGemmaMaxChunks.
int32_t gemma_chunk_blocks(int32_t T) {
    const int nkb = (T + 31) / 32;
    return std::max(std::min(nkb, 16), (nkb + ltx::kGemmaMaxChunks - 1) / ltx::kGemmaMaxChunks);
}

ltx_attn_status gemma_plan(const ltx_gemma_attn_args *a, GemmaPlan *pl) {
    g_err[0] = 0;
    if (!a) return fail(LTX_ATTN_EINVAL, "args is NULL");
    if (a->B < 1 || a->T < 4 || a->Hq < 1 || a->Hkv < 1)
        return fail(LTX_ATTN_EINVAL, "B, Hq, Hkv must be >= 1 and T >= 4 (got %d, %d, %d, %d)",
                    a->B, a->Hq, a->Hkv, a->T);
    if (a->D != 256 && a->D != 512)
        return fail(LTX_ATTN_EUNSUPPORTED, "head dim %d is not 256 or 512", a->D);
    if (a->T % 4)
        return fail(LTX_ATTN_EUNSUPPORTED, "T (%d) must be a multiple of 4", a->T);
    if (a->Hq % a->Hkv)
        return fail(LTX_ATTN_EINVAL, "Hq (%d) is not a multiple of Hkv (%d)", a->Hq, a->Hkv);
    if (a->B > ltx::kMaxBatch)
        return fail(LTX_ATTN_EUNSUPPORTED, "batch %d above %d", a->B, ltx::kMaxBatch);
    const int64_t D = a->D;
    struct T3 { const char *n; const void *p; int64_t bs, rs; int64_t H; };
    for (const T3 &t : {T3{"q", a->q, a->q_bs, a->q_rs, a->Hq}, T3{"k", a->k, a->k_bs, a->k_rs, a->Hkv},
                        T3{"v", a->v, a->v_bs, a->v_rs, a->Hkv}}) {
        if (!t.p) return fail(LTX_ATTN_EINVAL, "%s is NULL", t.n);
        if (!aligned16(t.p)) return fail(LTX_ATTN_EINVAL, "%s is not 16-byte aligned", t.n);
        if (t.bs < 0 || t.rs < t.H * D || (t.bs % 8) || (t.rs % 8) || (a->B > 1 && t.bs == 0))
            return fail(LTX_ATTN_EINVAL, "%s strides (%lld, %lld) must be multiples of 8 with a "
                        "row of at least %lld elements", t.n, (long long)t.bs, (long long)t.rs,
                        (long long)(t.H * D));
    }
    if (!a->q_norm_w || !a->k_norm_w || !aligned16(a->q_norm_w) || !aligned16(a->k_norm_w))
        return fail(LTX_ATTN_EINVAL, "q_norm_w and k_norm_w must be given, 16-byte aligned");
    if (!a->cos || !a->sin || ((uintptr_t)a->cos & 3u) || ((uintptr_t)a->sin & 3u))
        return fail(LTX_ATTN_EINVAL, "cos and sin tables must be given, 4-byte aligned");
    if (!(a->eps >= 0.f) || !isfinite(a->eps) || !(a->scale > 0.f) || !isfinite(a->scale))
        return fail(LTX_ATTN_EINVAL, "eps must be finite and >= 0, scale positive and finite");
    if (a->window < 0) return fail(LTX_ATTN_EINVAL, "window %d is negative", a->window);
    if (a->first_valid)
        for (int b = 0; b < a->B; ++b)
            if (a->first_valid[b] < 0 || a->first_valid[b] > a->T)
                return fail(LTX_ATTN_EINVAL, "first_valid[%d] = %d outside [0, %d]", b,
                            a->first_valid[b], a->T);
    if (!a->out || !aligned16(a->out) || a->o_rs < a->Hq * D || (a->o_rs % 4) ||
        a->o_bs < 0 || (a->o_bs % 4) || (a->B > 1 && a->o_bs == 0))
        return fail(LTX_ATTN_EINVAL, "out must be 16-byte aligned with strides that are "
                    "multiples of 4 and a row of at least Hq*D");
    const size_t qn = 2 * (size_t)a->B * a->Hq * a->T * D;
    // k' and v'^T are stored by whole 32-key blocks (operand order), the last one zero-padded
    const size_t kn = 2 * (size_t)a->B * a->Hkv * ((a->T + 31) / 32 * 32) * D;
    pl->off_q = 0;
    pl->off_k = align_up(qn, 256);
    pl->off_v = pl->off_k + align_up(kn, 256);
    pl->bytes = pl->off_v + align_up(kn, 256);
    const int qwg = ltx::gemma_queries_per_workgroup(a->D);
    const int nkb = (a->T + 31) / 32, nqb = (a->T + qwg - 1) / qwg;
    pl->chunk = gemma_chunk_blocks(a->T);
    pl->nch_max = (nkb + pl->chunk - 1) / pl->chunk;
    if (pl->nch_max > 1) {
        // partials only for the ranges of query blocks that have more than one, laid out per
        // batch row (its padding decides which blocks split), head-major
        size_t rows = 0;
        for (int b = 0; b < a->B; ++b) {
            const int fv = a->first_valid ? a->first_valid[b] : 0;
            int chunks = 0;
            for (int j = 0; j < nqb; ++j) {
                const int n = ltx::gemma_ranges(a->T, a->window, pl->chunk, j * qwg, qwg, fv);
                if (n > 1) chunks += n;
            }
            pl->part_row0[b] = (int64_t)rows;
            pl->part_chunks[b] = chunks;
            rows += (size_t)a->Hq * chunks * qwg;
        }
        pl->off_po = pl->bytes;
        pl->off_pml = pl->off_po + align_up(rows * D * 4, 256);
        pl->bytes = pl->off_pml + align_up(rows * 2 * 4, 256);
    }
    return LTX_ATTN_OK;
}

}  // namespace

namespace ltx {
int set_error_detail(int s, const char *fmt, va_list ap) {
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    return s;
}
}  // namespace ltx

extern "C" {

void ltx_attn_args_init(ltx_attn_args *a) {
    if (!a) return;
    memset(a, 0, sizeof *a);
    a->norm_eps = 1e-6f;
    a->kprep = LTX_ATTN_KPREP_AUTO;
    a->num_splits = 0;
}

size_t ltx_attn_workspace_bytes(const ltx_attn_args *a) {
    Plan pl;
    if (make_plan(a, &pl) != LTX_ATTN_OK) return 0;
    return pl.bytes;
}

ltx_attn_status ltx_attn_validate(const ltx_attn_args *a) {
    Plan pl;
    ltx_attn_status s = make_plan(a, &pl);
    if (s) return s;
    if (pl.bytes > 0) {
        if (!a->workspace || a->workspace_bytes < pl.bytes)
            return fail(LTX_ATTN_EWORKSPACE, "workspace of %zu bytes needed (got %zu at %p)",
                        pl.bytes, a->workspace_bytes, a->workspace);
        if ((uintptr_t)a->workspace & 255u)
            return fail(LTX_ATTN_EINVAL, "workspace must be 256-byte aligned");
    }
    return LTX_ATTN_OK;
}

ltx_attn_status ltx_attn_fwd(const ltx_attn_args *a, void *stream) {
    ltx_attn_status s = ltx_attn_validate(a);
    if (s) return s;
    Plan pl;
    // the device's own plan when the workspace covers it (and is aligned for it), else the
    // one it was sized for, which ltx_attn_validate has checked
    const int64_t groups = device_groups(a->resident_groups);
    make_plan(a, &pl, groups);
    if (groups != kConcurrentGroups && pl.bytes > 0 &&
        (!a->workspace || pl.bytes > a->workspace_bytes || ((uintptr_t)a->workspace & 255u)))
        make_plan(a, &pl);
    char *ws = (char *)a->workspace;
    const int B = a->B, H = a->H, D = a->D;

    if (pl.passthrough) {
        ltx::PassParams pp{};
        pp.v = a->v; pp.v_bs = a->v_bs; pp.v_rs = a->v_rs; pp.v_hs = a->v_hs;
        pp.o = a->out; pp.o_bs = a->o_bs; pp.o_rs = a->o_rs; pp.o_hs = a->o_hs;
        pp.B = B; pp.L = a->Lq; pp.H = H;
        pp.gate = a->gate_logits;
        pp.g_bs = a->g_bs; pp.g_rs = a->g_rs; pp.g_hs = a->g_hs;
        if (int e = ltx::launch_passthrough(pp, D, stream))
            return fail(LTX_ATTN_EHIP, "passthrough launch: %s", hipGetErrorString((hipError_t)e));
        return LTX_ATTN_OK;
    }

    // 1. prologue passes: statistics (and, for the K prologue, the prepared K). A call that
    // takes both its Q statistic and its K pass from the inputs runs them as one launch.
    ltx::PrepParams qpp{}, kpp{};
    bool q_pass = false, k_pass = false;
    if (pl.q_stat) {
        ltx::RstdParams rp{};
        rp.sumsq = a->q_sumsq; rp.rs = a->q_sumsq_rs;
        rp.rows = B * a->Lq; rp.blocks = a->sumsq_blocks; rp.n = H * D; rp.eps = a->norm_eps;
        rp.rstd = (float *)(ws + pl.off_qrstd);
        if (int e = ltx::launch_rstd(rp, stream))
            return fail(LTX_ATTN_EHIP, "q statistic launch: %s", hipGetErrorString((hipError_t)e));
    } else if (pl.q_norm) {
        qpp.x = a->q; qpp.bs = a->q_bs; qpp.rs = a->q_rs; qpp.hs = a->q_hs;
        qpp.B = B; qpp.L = a->Lq; qpp.H = H;
        qpp.w = a->q_norm_w; qpp.eps = a->norm_eps;
        qpp.rstd = (float *)(ws + pl.off_qrstd);
        q_pass = true;
    }
    const void *kptr = a->k;
    int64_t k_bs = a->k_bs, k_rs = a->k_rs, k_hs = a->k_hs;
    if (pl.k_fused && pl.k_stat) {
        ltx::RstdParams rp{};
        rp.sumsq = a->k_sumsq; rp.rs = a->k_sumsq_rs;
        rp.rows = B * a->Lk; rp.blocks = a->sumsq_blocks; rp.n = H * D; rp.eps = a->norm_eps;
        rp.rstd = (float *)(ws + pl.off_krstd);
        if (int e = ltx::launch_rstd(rp, stream))
            return fail(LTX_ATTN_EHIP, "k statistic launch: %s", hipGetErrorString((hipError_t)e));
    } else if (pl.k_prologue || (pl.k_fused && pl.k_norm)) {
        kpp.x = a->k; kpp.bs = a->k_bs; kpp.rs = a->k_rs; kpp.hs = a->k_hs;
        kpp.B = B; kpp.L = pl.k_prologue ? pl.kprep_rows : a->Lk; kpp.L_full = a->Lk; kpp.H = H;
        kpp.w = a->k_norm_w; kpp.eps = a->norm_eps;
        if (pl.k_stat) {
            kpp.sumsq = a->k_sumsq; kpp.ss_rs = a->k_sumsq_rs; kpp.ss_blocks = a->sumsq_blocks;
        }
        if (pl.k_prologue) {
            kpp.out = ws + pl.off_kprep;
            kpp.cos = a->k_cos ? a->k_cos : a->q_cos;
            kpp.sin = a->k_sin ? a->k_sin : a->q_sin;
            kptr = ws + pl.off_kprep;
            k_bs = (int64_t)pl.kprep_rows * H * D; k_rs = (int64_t)H * D; k_hs = D;
        } else {
            kpp.rstd = (float *)(ws + pl.off_krstd);
        }
        k_pass = true;
    }
    if (q_pass && k_pass) {
        if (int e = ltx::launch_prep2(qpp, kpp, D, stream))
            return fail(LTX_ATTN_EHIP, "q/k prologue launch: %s", hipGetErrorString((hipError_t)e));
    } else if (q_pass || k_pass) {
        if (int e = ltx::launch_prep(q_pass ? qpp : kpp, D, stream))
            return fail(LTX_ATTN_EHIP, "%s prologue launch: %s", q_pass ? "q" : "k",
                        hipGetErrorString((hipError_t)e));
    }

    const int kind = pl.dma ? ltx::kDma : pl.k_fused ? ltx::kRegFused : ltx::kRegPlain;
    (void)kind;

    // 2. attention
    ltx::FmhaParams fp{};
    fp.q = a->q; fp.q_bs = a->q_bs; fp.q_rs = a->q_rs; fp.q_hs = a->q_hs;
    fp.k = kptr; fp.k_bs = k_bs; fp.k_rs = k_rs; fp.k_hs = k_hs;
    fp.v = a->v; fp.v_bs = a->v_bs; fp.v_rs = a->v_rs; fp.v_hs = a->v_hs;
    fp.o = a->out; fp.o_bs = a->o_bs; fp.o_rs = a->o_rs; fp.o_hs = a->o_hs;
    fp.B = B; fp.H = H; fp.Lq = a->Lq; fp.Lk = a->Lk;
    if (pl.q_norm) { fp.q_rstd = (const float *)(ws + pl.off_qrstd); fp.q_w = a->q_norm_w; }
    if (pl.q_rope) { fp.q_cos = a->q_cos; fp.q_sin = a->q_sin; }
    if (pl.k_fused) {
        if (pl.k_norm) { fp.k_rstd = (const float *)(ws + pl.off_krstd); fp.k_w = a->k_norm_w; }
        if (pl.k_rope) {
            fp.k_cos = a->k_cos ? a->k_cos : a->q_cos;
            fp.k_sin = a->k_sin ? a->k_sin : a->q_sin;
        }
    }
    fp.qk_scale_log2 = (float)((double)a->scale * 1.4426950408889634);
    fp.gate = a->gate_logits;
    fp.g_bs = a->g_bs; fp.g_rs = a->g_rs; fp.g_hs = a->g_hs;
    fp.nqblk = pl.nqblk;
    fp.n_items = (int32_t)pl.n_items;
    fp.n_full = (int32_t)pl.n_full;
    fp.num_splits = pl.splits;
    fp.tiles_per_split = pl.tiles_per_split;
    fp.grid = (int32_t)pl.grid;
    fp.n_lead = pl.n_lead;
    fp.short_groups = pl.short_groups;
    if (pl.n_full < pl.n_items) {
        fp.part_o = (float *)(ws + pl.off_part_o);
        fp.part_ml = (float *)(ws + pl.off_part_ml);
    }
    for (int b = 0; b < std::min(B, ltx::kMaxBatch); ++b)
        fp.valid[b] = a->k_valid_len ? a->k_valid_len[b] : a->Lk;
    if (!a->k_valid_len && B > ltx::kMaxBatch) {
        // Unmasked batches beyond the argument table are launched in slices of kMaxBatch.
        for (int b0 = 0; b0 < B; b0 += ltx::kMaxBatch) {
            ltx::FmhaParams sp = fp;
            const int nb = std::min(ltx::kMaxBatch, B - b0);
            sp.B = nb;
            sp.q = (const char *)a->q + 2 * (int64_t)b0 * a->q_bs;
            sp.k = (const char *)kptr + 2 * (int64_t)b0 * k_bs;
            sp.v = (const char *)a->v + 2 * (int64_t)b0 * a->v_bs;
            sp.o = (char *)a->out + 2 * (int64_t)b0 * a->o_bs;
            if (sp.gate) sp.gate = (const char *)a->gate_logits + 2 * (int64_t)b0 * a->g_bs;
            if (sp.q_rstd) sp.q_rstd += (int64_t)b0 * a->Lq;
            if (sp.k_rstd) sp.k_rstd += (int64_t)b0 * a->Lk;
            sp.n_items = sp.n_full = sp.grid = nb * H * pl.nqblk;
            sp.n_lead = 0;
            sp.num_splits = 1;
            if (a->ev_attn_start && b0 == 0)
                if (hipError_t e = hipEventRecord((hipEvent_t)a->ev_attn_start, (hipStream_t)stream))
                    return fail(LTX_ATTN_EHIP, "event record: %s", hipGetErrorString(e));
            if (int e = ltx::launch_fmha(sp, D, kind, stream))
                return fail(LTX_ATTN_EHIP, "attention launch: %s", hipGetErrorString((hipError_t)e));
        }
        if (a->ev_attn_stop)
            if (hipError_t e = hipEventRecord((hipEvent_t)a->ev_attn_stop, (hipStream_t)stream))
                return fail(LTX_ATTN_EHIP, "event record: %s", hipGetErrorString(e));
        return LTX_ATTN_OK;
    }
    if (a->ev_attn_start)
        if (hipError_t e = hipEventRecord((hipEvent_t)a->ev_attn_start, (hipStream_t)stream))
            return fail(LTX_ATTN_EHIP, "event record: %s", hipGetErrorString(e));
    if (int e = pl.shortk   ? ltx::launch_fmha_short(fp, D, stream)
                : pl.splitk ? ltx::launch_fmha_splitk(fp, D, stream)
                            : ltx::launch_fmha(fp, D, kind, stream))
        return fail(LTX_ATTN_EHIP, "attention launch: %s", hipGetErrorString((hipError_t)e));
    if (a->ev_attn_stop)
        if (hipError_t e = hipEventRecord((hipEvent_t)a->ev_attn_stop, (hipStream_t)stream))
            return fail(LTX_ATTN_EHIP, "event record: %s", hipGetErrorString(e));

    // 3. split-KV combine
    if (pl.n_full < pl.n_items) {
        ltx::CombineParams cp{};
        cp.part_o = fp.part_o; cp.part_ml = fp.part_ml;
        cp.o = a->out; cp.o_bs = a->o_bs; cp.o_rs = a->o_rs; cp.o_hs = a->o_hs;
        cp.H = H; cp.Lq = a->Lq; cp.nqblk = pl.nqblk;
        cp.n_full = (int32_t)pl.n_full;
        cp.n_tail = (int32_t)(pl.n_items - pl.n_full);
        cp.num_splits = pl.splits;
        cp.gate = a->gate_logits;
        cp.g_bs = a->g_bs; cp.g_rs = a->g_rs; cp.g_hs = a->g_hs;
        if (int e = ltx::launch_combine(cp, D, stream))
            return fail(LTX_ATTN_EHIP, "combine launch: %s", hipGetErrorString((hipError_t)e));
    }
    return LTX_ATTN_OK;
}

size_t ltx_gemma_attn_workspace_bytes(const ltx_gemma_attn_args *a) {
    GemmaPlan pl;
    return gemma_plan(a, &pl) == LTX_ATTN_OK ? pl.bytes : 0;
}

ltx_attn_status ltx_gemma_attn_fwd(const ltx_gemma_attn_args *a, void *stream) {
    GemmaPlan pl;
    if (ltx_attn_status s = gemma_plan(a, &pl)) return s;
    if (!a->workspace || a->workspace_bytes < pl.bytes)
        return fail(LTX_ATTN_EWORKSPACE, "workspace of %zu bytes needed (got %zu at %p)",
                    pl.bytes, a->workspace_bytes, a->workspace);
    if ((uintptr_t)a->workspace & 255u)
        return fail(LTX_ATTN_EINVAL, "workspace must be 256-byte aligned");
    char *ws = (char *)a->workspace;
    ltx::GemmaPrepParams pp{};
    pp.q = a->q; pp.k = a->k; pp.v = a->v;
    pp.q_bs = a->q_bs; pp.q_rs = a->q_rs; pp.k_bs = a->k_bs; pp.k_rs = a->k_rs;
    pp.v_bs = a->v_bs; pp.v_rs = a->v_rs;
    pp.B = a->B; pp.T = a->T; pp.Hq = a->Hq; pp.Hkv = a->Hkv;
    pp.q_w = a->q_norm_w; pp.k_w = a->k_norm_w;
    pp.eps = a->eps;
    pp.q_factor = (float)((double)a->scale * 1.4426950408889634);
    pp.cos = a->cos; pp.sin = a->sin;
    pp.qp = ws + pl.off_q; pp.kp = ws + pl.off_k;
    pp.vt = ws + pl.off_v;
    if (int e = ltx::launch_gemma_prep(pp, a->D, stream))
        return fail(LTX_ATTN_EHIP, "gemma prologue launch: %s", hipGetErrorString((hipError_t)e));
    ltx::GemmaAttnParams ap{};
    ap.qp = pp.qp; ap.kp = pp.kp; ap.vt = pp.vt;
    ap.out = a->out; ap.o_bs = a->o_bs; ap.o_rs = a->o_rs;
    ap.B = a->B; ap.T = a->T; ap.Hq = a->Hq; ap.Hkv = a->Hkv; ap.window = a->window;
    for (int b = 0; b < a->B; ++b) ap.first_valid[b] = a->first_valid ? a->first_valid[b] : 0;
    ap.chunk = pl.chunk;
    ap.nch_max = pl.nch_max;
    ap.part_o = (float *)(ws + pl.off_po);
    ap.part_ml = (float *)(ws + pl.off_pml);
    for (int b = 0; b < a->B; ++b) {
        ap.part_row0[b] = pl.part_row0[b];
        ap.part_chunks[b] = pl.part_chunks[b];
    }
    if (int e = ltx::launch_gemma_attn(ap, a->D, stream))
        return fail(LTX_ATTN_EHIP, "gemma attention launch: %s", hipGetErrorString((hipError_t)e));
    return LTX_ATTN_OK;
}

const char *ltx_attn_status_string(ltx_attn_status s) {
    switch (s) {
    case LTX_ATTN_OK: return "ok";
    case LTX_ATTN_EINVAL: return "invalid argument";
    case LTX_ATTN_EUNSUPPORTED: return "unsupported configuration";
    case LTX_ATTN_EHIP: return "HIP runtime error";
    case LTX_ATTN_EWORKSPACE: return "workspace too small";
    }
    return "unknown status";
}

const char *ltx_attn_last_error(void) { return g_err; }

const char *ltx_attn_provenance(void) {
    return "hip-gfx950 fused flash attention v2 (bf16 mfma_f32_32x32x16, online fp32 softmax, "
           "QK-RMSNorm+RoPE fused; K/V tiles by LDS DMA for multi-block queries)";
}

int32_t ltx_attn_abi_version(void) { return LTX_ATTN_ABI_VERSION; }

size_t ltx_attn_args_size(void) { return sizeof(ltx_attn_args); }

int32_t ltx_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n;
}

ltx_attn_status ltx_device_query(int32_t ordinal, ltx_device_info *out) {
    g_err[0] = 0;
    if (!out) return fail(LTX_ATTN_EINVAL, "out is NULL");
    const int32_t n = ltx_device_count();
    if (ordinal < 0 || ordinal >= n)
        return fail(LTX_ATTN_EINVAL, "device %d outside [0, %d)", ordinal, n);
    hipDeviceProp_t prop;
    if (hipError_t e = hipGetDeviceProperties(&prop, ordinal))
        return fail(LTX_ATTN_EHIP, "hipGetDeviceProperties: %s", hipGetErrorString(e));
    memset(out, 0, sizeof *out);
    out->ordinal = ordinal;
    out->compute_units = prop.multiProcessorCount;
    out->memory_bytes = (int64_t)prop.totalGlobalMem;
    out->clock_khz = prop.clockRate;
    out->lds_bytes_per_cu = (int32_t)prop.maxSharedMemoryPerMultiProcessor;
    snprintf(out->name, sizeof out->name, "%.127s", prop.name);
    snprintf(out->arch, sizeof out->arch, "%.63s", prop.gcnArchName);
    out->supported = strncmp(prop.gcnArchName, "gfx950", 6) == 0 &&
                     (prop.gcnArchName[6] == 0 || prop.gcnArchName[6] == ':');
    return LTX_ATTN_OK;
}

int32_t ltx_linear_sumsq_blocks(int32_t N) {
    return N <= 0 ? 0 : (N + LTX_LINEAR_SUMSQ_COLS - 1) / LTX_LINEAR_SUMSQ_COLS;
}

}  // extern "C"

namespace {

// Tail split of a projection: the tiles past the last whole round of `groups` resident
// workgroups, when they fill at most half a round, are cut into k ranges of at least two
// 64-wide steps, at most as many as fill one round. The count minimises the tail's time: a
// range's k steps (about 1.3 us each) against its fp32 partials (256 KiB per range and tile,
// written and read back by the fixup, about 0.116 us at 4.5 TB/s). Measured at 12480 x 4096 x
// 4096 (16 tail tiles): 8 ranges 0.373 ms, 16 ranges (every CU busy) 0.382 ms. Pure host
// arithmetic.
struct LinearSplit {
    int64_t tiles = 0, n_full = 0;
    int32_t splits = 1, steps_per_split = 0;
    size_t bytes = 0;
};

LinearSplit linear_split(int64_t M, int64_t N, int64_t K,
                         int64_t groups = kConcurrentGroups) {
    LinearSplit ls;
    const int64_t T = ((M + ltx::kLinearTile - 1) / ltx::kLinearTile) *
                      ((N + ltx::kLinearTile - 1) / ltx::kLinearTile);
    const int64_t nsteps = K / 64;
    ls.tiles = ls.n_full = T;
    ls.steps_per_split = (int32_t)nsteps;
    const int64_t rem = T % groups;
    if (T == 0 || rem == 0 || 2 * rem > groups || nsteps < 4) return ls;
    const int64_t s_max = std::min<int64_t>(groups / rem, nsteps / 2);
    constexpr double kStepUs = 1.3, kPartUs = 0.116;
    int64_t s = 1, per = nsteps;
    double best = 0.0;
    for (int64_t c = 2; c <= s_max; ++c) {
        const int64_t cp = (nsteps + c - 1) / c;
        const int64_t cs = (nsteps + cp - 1) / cp;   // no empty range
        const double t = (double)cp * kStepUs + (double)(rem * cs) * kPartUs;
        if (s == 1 || t < best - 1e-9) {
            best = t;
            s = cs;
            per = cp;
        }
    }
    if (s < 2) return ls;
    ls.n_full = T - rem;
    ls.splits = (int32_t)s;
    ls.steps_per_split = (int32_t)per;
    ls.bytes = (size_t)ltx::linear_part_bytes(rem, (int)s);
    return ls;
}

}  // namespace

extern "C" {

size_t ltx_linear_workspace_bytes(const ltx_linear_args *a) {
    g_err[0] = 0;
    if (!a || a->M < 0 || a->N < 8 || a->K < 64 || (a->K % 64)) {
        fail(LTX_ATTN_EINVAL, "ltx_linear_workspace_bytes: invalid M, N or K");
        return 0;
    }
    return linear_split(a->M, a->N, a->K).bytes;
}

ltx_attn_status ltx_linear(const ltx_linear_args *a, void *stream) {
    g_err[0] = 0;
    if (!a) return fail(LTX_ATTN_EINVAL, "args is NULL");
    if (a->M < 0 || a->N < 8 || a->K < 64)
        return fail(LTX_ATTN_EINVAL, "need M >= 0, N >= 8, K >= 64 (got %d, %d, %d)", a->M,
                    a->N, a->K);
    if (a->N % 8) return fail(LTX_ATTN_EINVAL, "N (%d) must be a multiple of 8", a->N);
    if (a->K % 64) return fail(LTX_ATTN_EUNSUPPORTED, "K (%d) is not a multiple of 64", a->K);
    if (!a->w || (a->M > 0 && (!a->x || !a->y)))
        return fail(LTX_ATTN_EINVAL, "w, and x and y unless M is 0, must be given");
    if (!aligned16(a->x) || !aligned16(a->w))
        return fail(LTX_ATTN_EINVAL, "x and w must be 16-byte aligned");
    if (((uintptr_t)a->y & 7u) || ((uintptr_t)a->bias & 7u))
        return fail(LTX_ATTN_EINVAL, "y and bias must be 8-byte aligned");
    if (a->x_rs < a->K || a->w_rs < a->K || (a->x_rs % 8) || (a->w_rs % 8))
        return fail(LTX_ATTN_EINVAL, "x_rs and w_rs must be >= K and multiples of 8");
    if (a->y_rs < a->N || (a->y_rs % 4))
        return fail(LTX_ATTN_EINVAL, "y_rs must be >= N and a multiple of 4");
    // The kernel addresses a 256-row tile of x or w with 32-bit byte offsets.
    const int64_t max_rs = 0x7fffffff / (2 * (int64_t)ltx::kLinearTile);
    if (a->x_rs > max_rs || a->w_rs > max_rs)
        return fail(LTX_ATTN_EUNSUPPORTED, "row strides above %lld elements", (long long)max_rs);
    const int32_t blocks = ltx_linear_sumsq_blocks(a->N);
    if (a->sumsq && (((uintptr_t)a->sumsq & 3u) || a->sumsq_rs < blocks))
        return fail(LTX_ATTN_EINVAL, "sumsq must be 4-byte aligned with a row stride >= %d",
                    blocks);
    const int64_t tiles_m = ((int64_t)a->M + ltx::kLinearTile - 1) / ltx::kLinearTile;
    const int64_t tiles_n = ((int64_t)a->N + ltx::kLinearTile - 1) / ltx::kLinearTile;
    if (tiles_m * tiles_n > 0x7fffffff) return fail(LTX_ATTN_EUNSUPPORTED, "grid too large");
    if (a->M == 0) return LTX_ATTN_OK;
    // y must not overlap its inputs: the tiles read x and w while others write y.
    auto span = [](const void *p, int64_t rows, int64_t rs, int64_t cols, size_t elem) {
        const uintptr_t b = (uintptr_t)p;
        return std::pair<uintptr_t, uintptr_t>(b, b + ((rows - 1) * rs + cols) * elem);
    };
    const auto yb = span(a->y, a->M, a->y_rs, a->N, 2);
    for (const auto &in : {span(a->x, a->M, a->x_rs, a->K, 2), span(a->w, a->N, a->w_rs, a->K, 2)})
        if (yb.first < in.second && in.first < yb.second)
            return fail(LTX_ATTN_EINVAL, "y overlaps x or w");
    if (a->sumsq) {
        const auto sb = span(a->sumsq, a->M, a->sumsq_rs, blocks, 4);
        if (sb.first < yb.second && yb.first < sb.second)
            return fail(LTX_ATTN_EINVAL, "sumsq overlaps y");
    }
    ltx::LinearParams p{};
    p.x = a->x; p.w = a->w; p.bias = a->bias; p.y = a->y;
    p.x_rs = a->x_rs; p.w_rs = a->w_rs; p.y_rs = a->y_rs;
    p.sumsq = a->sumsq; p.ss_rs = a->sumsq_rs;
    p.M = a->M; p.N = a->N; p.K = a->K;
    p.tiles_m = (int32_t)tiles_m; p.tiles_n = (int32_t)tiles_n;
    // the device's own tail split when the workspace covers it, else the one it was sized for
    if (a->resident_groups < 0 || a->resident_groups > 65536)
        return fail(LTX_ATTN_EINVAL, "resident_groups %d outside [0, 65536]", a->resident_groups);
    const int64_t groups = device_groups(a->resident_groups);
    LinearSplit ls = linear_split(a->M, a->N, a->K, groups);
    if (groups != kConcurrentGroups && ls.splits > 1 &&
        (!a->workspace || a->workspace_bytes < ls.bytes))
        ls = linear_split(a->M, a->N, a->K);
    p.n_full = (int32_t)ls.tiles;
    p.splits = 1;
    p.steps_per_split = a->K / 64;
    if (ls.splits > 1 && a->workspace && a->workspace_bytes >= ls.bytes) {
        if ((uintptr_t)a->workspace & 255u)
            return fail(LTX_ATTN_EINVAL, "linear workspace must be 256-byte aligned");
        const uintptr_t wb = (uintptr_t)a->workspace, we = wb + ls.bytes;
        auto overlaps = [&](std::pair<uintptr_t, uintptr_t> r) {
            return wb < r.second && r.first < we;
        };
        if (overlaps(yb) || overlaps(span(a->x, a->M, a->x_rs, a->K, 2)) ||
            overlaps(span(a->w, a->N, a->w_rs, a->K, 2)) ||
            (a->sumsq && overlaps(span(a->sumsq, a->M, a->sumsq_rs, blocks, 4))))
            return fail(LTX_ATTN_EINVAL, "linear workspace overlaps x, w, y or sumsq");
        p.part = (float *)a->workspace;
        p.n_full = (int32_t)ls.n_full;
        p.splits = ls.splits;
        p.steps_per_split = ls.steps_per_split;
    }
    // One workgroup per resident slot walks the whole tiles; the tail ranges were planned to
    // fill the slots the last round leaves.
    const int64_t n_ranges = (tiles_m * tiles_n - p.n_full) * (p.splits > 1 ? p.splits : 0);
    p.grid = (int32_t)std::max<int64_t>(std::min<int64_t>(groups, p.n_full), n_ranges);
    if (p.grid < 1) p.grid = 1;
    if (int e = ltx::launch_linear(p, stream))
        return fail(LTX_ATTN_EHIP, "linear launch: %s", hipGetErrorString((hipError_t)e));
    return LTX_ATTN_OK;
}

}  // extern "C"
