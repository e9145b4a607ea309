/*
 * ltx_attn.h -- C ABI of the MI355X (gfx950) fused DiT attention library.
 *
 * One shared library, libltx_attn.so, replaces the arithmetic of the LTX 2.5 DiT attention
 * hot path: QK-RMSNorm over the inner dim, the head split, split-half RoPE and scaled
 * dot-product attention. In the reference that is
 *
 *     Sources/LTXModules/DiTAttention.swift:358-381   (inside DiTAttention.callAsFunction,
 *                                                     declared at :315-318)
 *       q = rmsNorm(q, q_norm.weight); k = rmsNorm(k, k_norm.weight)   :360-361 (-> :202-204)
 *       qh = split(q); kh = split(k)                                   :362 (-> :346-349)
 *       qh = applySplitRoPE(qh, rotary); kh = applySplitRoPE(kh, keyRotary ?? rotary)
 *                                                                      :364-367 (-> :226-234)
 *       out = MLXFast.scaledDotProductAttention(qh, kh, vh, scale, mask: .none)  :374-376
 *
 * and the rotary-table builders of Sources/LTXModules/DiTForward.swift:455-738.
 *
 * Everything is plain C: pointers, sizes and status codes. Device buffers are HIP device
 * pointers; `stream` is a hipStream_t passed as void* (NULL = the default stream).
 *
 * Contract of ltx_attn_fwd (all of it checked on the host before anything is launched):
 *   - no allocation: scratch memory is the caller's `workspace`, sized by
 *     ltx_attn_workspace_bytes() for the same arguments;
 *   - no hidden global mutable state; reentrant across streams and threads (the detail
 *     string of the last failure is thread-local, like dlerror);
 *   - sizing and validation (ltx_attn_workspace_bytes, ltx_attn_validate) are pure host
 *     functions that do not touch the HIP runtime;
 *   - asynchronous on `stream`; inputs must stay valid until the stream reaches the call.
 */
#ifndef LTX_ATTN_H
#define LTX_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LTX_ATTN_ABI_VERSION 8

/* Status codes. The reference throws `DiTAttention.Failure` for structural errors
 * (DiTAttention.swift:107-121); a Swift wrapper maps these onto thrown errors. */
typedef enum {
    LTX_ATTN_OK = 0,
    LTX_ATTN_EINVAL = 1,       /* bad shape, stride, alignment, pointer or valid length   */
    LTX_ATTN_EUNSUPPORTED = 2, /* head dim other than 64/128, or a batch above the limit  */
    LTX_ATTN_EHIP = 3,         /* a HIP runtime call or kernel launch failed               */
    LTX_ATTN_EWORKSPACE = 4    /* workspace missing or smaller than ltx_attn_workspace_bytes */
} ltx_attn_status;

/* How K gets its norm + RoPE (when a K norm weight or K tables are given), and with it the
 * attention kernel. AUTO: calls whose valid keys fit in LDS (<= 128 at D=128 without RoPE,
 * <= 256 at D=64) take the short-key kernel (the prologue prepares only the valid K rows);
 * other calls the prologue when K is re-read by >= 2 query blocks, else the fused staging.
 * FUSED and PROLOGUE force the register-staged and the LDS-DMA kernel. Results agree within
 * the stated tolerance, not bit for bit, across kernels. */
typedef enum {
    LTX_ATTN_KPREP_AUTO = 0,     /* pick by cost (above)                                          */
    LTX_ATTN_KPREP_FUSED = 1,    /* normalise + rotate K inside the attention kernel's LDS staging */
    LTX_ATTN_KPREP_PROLOGUE = 2  /* one pass writes normed+rotated K (bf16) into the workspace     */
} ltx_attn_kprep;

/* Largest batch for which per-row key-padding lengths may be given. */
#define LTX_ATTN_MAX_BATCH 64

/*
 * One attention call. Element strides (not bytes). Token l of batch row b, head h, channel d
 * of q lives at q + b*q_bs + l*q_rs + h*q_hs + d. The reference's merged projection layout
 * [B, L, H*D] is q_bs = L*H*D, q_rs = H*D, q_hs = D; its split layout [B, H, L, D]
 * (DiTAttention.swift:346-349) is q_bs = H*L*D, q_hs = L*D, q_rs = D.
 * `out` uses the same scheme; the merged layout [B, Lq, H*D] is what `to_out` consumes
 * after the gate (DiTAttention.swift:402-404), which the call can apply (gate_logits).
 */
typedef struct ltx_attn_args {
    int32_t B, H, Lq, Lk, D;      /* D in {64, 128}; H*D = inner (4096 video, 2048 audio/cross) */

    const void *q, *k, *v;        /* bf16 device pointers, 16-byte aligned                  */
    int64_t q_bs, q_rs, q_hs;     /* strides: multiples of 8 elements; q_hs >= D              */
    int64_t k_bs, k_rs, k_hs;
    int64_t v_bs, v_rs, v_hs;

    /* QK-RMSNorm (DiTAttention.swift:190-204, :360-361): bf16 [H*D] weights, statistic over
     * all H*D channels of a token (not per head; channel (h, d) is inner index h*D + d).
     * NULL = that input is already normalised. */
    const void *q_norm_w, *k_norm_w;
    float norm_eps;               /* 1e-6 in the reference (DiTAttention.swift:66)           */

    /* Split RoPE (DiTAttention.swift:206-234): bf16 cos/sin tables [H, L, D/2] contiguous,
     * broadcast over the batch (the reference's [1, H, L, D/2]). q tables NULL = no RoPE.
     * k tables NULL with q tables given = K uses q's tables (`keyRotary ?? rotary`, :366),
     * which needs Lq == Lk. k tables without q tables is EINVAL. */
    const void *q_cos, *q_sin;
    const void *k_cos, *k_sin;

    /* Key padding: HOST pointer to B int32 counts; batch row b attends to keys [0, n_b).
     * NULL = every key valid. 1 <= n_b <= Lk (0 is EINVAL, as TextConditioningLayout.swift:65
     * rejects an empty mask). Fully padded tiles are skipped, not computed. */
    const int32_t *k_valid_len;

    float scale;                  /* softmax scale; 1/sqrt(D) in the reference (:372)        */

    void *out;                    /* bf16 device pointer, 16-byte aligned                   */
    int64_t o_bs, o_rs, o_hs;

    void *workspace;              /* device scratch, 256-byte aligned, or NULL if 0 bytes needed */
    size_t workspace_bytes;

    int32_t kprep;                /* ltx_attn_kprep                                            */
    int32_t num_splits;           /* 0 = auto; >= 1 forces that many key splits (split-KV)    */

    /* Optional timing hook: hipEvent_t handles (as void*) recorded on `stream` immediately
     * before and after the attention kernel itself (not the norm/RoPE prologue or the
     * split-KV combine). NULL = not recorded. */
    void *ev_attn_start, *ev_attn_stop;

    /* Per-head output gate (DiTAttention.swift:385-399): bf16 logits [B, Lq, H] from the
     * caller's `to_gate_logits(x)` (x = the query stream, :387-391), element strides below
     * (the linear's output [B, Lq, H] is g_bs = Lq*H, g_rs = H, g_hs = 1). Each output row of
     * head h is multiplied by 2*sigmoid(logit) (the bf16 gate the reference builds at :396)
     * before its bf16 rounding. NULL = no gate (the modules without to_gate_logits). */
    const void *gate_logits;      /* bf16 device pointer, 2-byte aligned                     */
    int64_t g_bs, g_rs, g_hs;     /* non-negative element strides                             */

    /* STG passthrough (DiTAttention.swift:351-356, `allPerturbed`): nonzero = the module is
     * fully perturbed, so out = V (times the gate, if given) per head, with no attention, no
     * norm and no RoPE: q, k, their norm weights and tables are ignored and may be NULL, and
     * no workspace is needed. Self-attention only (Lq == Lk). */
    int32_t all_perturbed;

    /* RMS statistic from the projection (ltx_linear's sumsq output): fp32 partial sums of
     * squares of each token's q (k) values, row b*Lq + l (b*Lk + l) at q_sumsq + row*q_sumsq_rs,
     * `sumsq_blocks` partials per row whose sum covers all H*D channels. Given with q_norm_w
     * (k_norm_w), the norm takes its statistic from them instead of a pass over q (k).
     * NULL = statistic computed here. The partials must describe the q (k) being passed. */
    const float *q_sumsq, *k_sumsq;
    int64_t q_sumsq_rs, k_sumsq_rs;   /* >= sumsq_blocks                                  */
    int32_t sumsq_blocks;             /* >= 1 when either pointer is given                */

    /* Work planning. 0 (the default) = plan the tail splits for the current device's CU count
     * (queried once per device); n > 0 = plan as if n workgroups were resident at once instead
     * (a test of the plan of another part size; at most 65536). Results agree within the
     * fp32 merge order whatever the plan. */
    int32_t resident_groups;
} ltx_attn_args;

/* Fill `a` with defaults: zero sizes and pointers, norm_eps = 1e-6, kprep AUTO, splits auto. */
void ltx_attn_args_init(ltx_attn_args *a);

/* Bytes of workspace ltx_attn_fwd needs for these arguments (0 if none). Pure host function;
 * returns 0 and sets the thread's error detail if the arguments are invalid. It plans for a
 * whole gfx950 part (256 CUs); on a device with another CU count (or with resident_groups
 * set) ltx_attn_fwd plans its tail splits for that count when the given workspace covers that
 * plan and is 256-byte aligned, else runs the sized one. */
size_t ltx_attn_workspace_bytes(const ltx_attn_args *a);

/* Check the arguments without launching anything (the first step of ltx_attn_fwd). */
ltx_attn_status ltx_attn_validate(const ltx_attn_args *a);

/* Run norm -> split -> RoPE -> SDPA (-> gate) asynchronously on `stream` (a hipStream_t or
 * NULL). Replaces DiTAttention.swift:360-381 (MLXFast.scaledDotProductAttention at :374-376)
 * and, with gate_logits, the gate multiply of :395-399. */
ltx_attn_status ltx_attn_fwd(const ltx_attn_args *a, void *stream);

/* Bytes of the device scratch ltx_attn_fwd_static holds (128 MiB per device). */
#define LTX_ATTN_STATIC_SCRATCH_BYTES ((size_t)128 << 20)

/* ltx_attn_fwd for callers that cannot allocate device memory -- code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc. No counterpart in the
 * reference (whose MLX arrays are allocated by MLX). The caller passes inputs and outputs;
 * `workspace` / `workspace_bytes` are ignored: the call's scratch (statistics, prepared K,
 * split-KV partials) is a file-scope device array of LTX_ATTN_STATIC_SCRATCH_BYTES per
 * device, looked up on the first call on each device and held until the process ends. Same
 * plan, kernels and results as ltx_attn_fwd given a workspace of exactly
 * ltx_attn_workspace_bytes for the same arguments. Calls needing more scratch than that (see
 * ltx_attn_workspace_bytes) return LTX_ATTN_EUNSUPPORTED before anything is launched. The
 * array is shared by every call on a device: calls that overlap on one device race, so the
 * caller serialises them. Allocates nothing. */
ltx_attn_status ltx_attn_fwd_static(const ltx_attn_args *a, void *stream);

/* Static text for a status code. */
const char *ltx_attn_status_string(ltx_attn_status s);

/* Detail of the calling thread's last failure ("" if none). */
const char *ltx_attn_last_error(void);

/* Provenance string recorded beside a render, like `attentionPath` in the reference's
 * .provenance.json (Sources/LTXPipeline/Renderer.swift:477-490). */
const char *ltx_attn_provenance(void);

/* ABI version of the loaded library (LTX_ATTN_ABI_VERSION it was built with). */
int32_t ltx_attn_abi_version(void);

/* sizeof(ltx_attn_args) as compiled into the library, so an FFI mirror of the struct
 * (Swift, ctypes, ...) can verify its layout at load time. */
size_t ltx_attn_args_size(void);

/* ----------------------------------------------------------------------------------------
 * Projection GEMM: `linear` of DiTAttention.swift:178-188, y = x . w^T (+ bias), with the
 * RMS-norm statistic of y from the epilogue (the q_norm / k_norm that follow, :202-204).
 * -------------------------------------------------------------------------------------- */

/* Columns of y covered by one partial sum of squares. */
#define LTX_LINEAR_SUMSQ_COLS 256

typedef struct ltx_linear_args {
    int32_t M, N, K;              /* y [M, N] = x [M, K] . w [N, K]^T; N % 8 == 0, K % 64 == 0 */
    const void *x;                /* bf16 device pointer, 16-byte aligned; row stride x_rs
                                     (x and y may be NULL when M is 0)                        */
    const void *w;                /* bf16 [N, K], the checkpoint's [out, in] layout; 16-byte   */
    const void *bias;             /* bf16 [N] (8-byte aligned), or NULL                       */
    void *y;                      /* bf16, 8-byte aligned, row stride y_rs; must not overlap x/w */
    int64_t x_rs, w_rs, y_rs;     /* element strides: x_rs, w_rs >= K, multiples of 8;
                                     y_rs >= N, a multiple of 4                                */
    /* NULL, or fp32 [M][ltx_linear_sumsq_blocks(N)] at row stride sumsq_rs (4-byte aligned):
     * partial j of row m = sum of y[m][n]^2 (the bf16 outputs, in fp32) over the columns
     * n in [256 j, 256 j + 256). Column ranges that start at a multiple of 256 (q, k of a
     * fused projection) have their own partials. */
    float *sumsq;
    int64_t sumsq_rs;
    /* Device scratch for the fp32 partial tiles of a split tail (see
     * ltx_linear_workspace_bytes), 256-byte aligned, or NULL. With less than that the tail
     * tiles run whole: same result up to fp32 summation order, slower. */
    void *workspace;
    size_t workspace_bytes;
    /* 0 = split the tail for the current device's CU count; n > 0 = for n resident workgroups
     * (as in ltx_attn_args). */
    int32_t resident_groups;
} ltx_linear_args;

/* ceil(N / LTX_LINEAR_SUMSQ_COLS): partial sums per row of y. */
int32_t ltx_linear_sumsq_blocks(int32_t N);

/* Bytes of workspace that let ltx_linear split its tail: the 256 x 256 tiles past the last
 * whole round of 256 (one per CU) are cut along K into ranges (at most as many as fill the
 * CUs; the count weighs a range's k steps against its partials' round trip), and a
 * fixup launch sums each tile's ranges (256 KiB of fp32 per range; 0 when the tiles fill
 * whole rounds or the tail is more than half a round). Pure host function; 0 for invalid
 * arguments. Sized for a whole gfx950 part (256 CUs): on a device with another CU count
 * ltx_linear splits by that count when the workspace covers it, else as sized. No
 * counterpart in the reference, whose matmul (MLX) manages its own scratch. */
size_t ltx_linear_workspace_bytes(const ltx_linear_args *a);

/* Run the projection asynchronously on `stream` (a hipStream_t or NULL). The fp32
 * accumulator is rounded to bf16, then the bias is added in fp32 and rounded again, as the
 * reference's matmul and add do (:180, :186). M == 0 launches nothing. LoRA deltas (:183-185)
 * are not applied here. */
ltx_attn_status ltx_linear(const ltx_linear_args *a, void *stream);

/* ----------------------------------------------------------------------------------------
 * RoPE table construction (host side, no GPU): the reference builds these once per forward
 * and hands them to every block (DiTForward.swift:680-738).
 * -------------------------------------------------------------------------------------- */

/* frequencyGrid (DiTForward.swift:455-466): n = inner/(2*nPos) values,
 * f_i = theta^(i/(n-1)) * pi/2 in double, endpoint exponent exactly 1, stored as float.
 * Returns the count written to `out` (capacity `cap`), or -1 on bad arguments. */
int32_t ltx_rope_frequency_grid(double theta, int32_t n_pos, int32_t inner, float *out,
                                int32_t cap);

/* videoPositions (DiTForward.swift:486-520): patch bounds [3][tokens][2] (float, seconds for
 * time with the causal correction, pixels for space); tokens = frames*height*width in
 * (t, y, x) order. Returns tokens, or -1. */
int32_t ltx_rope_video_positions(int32_t latent_frames, int32_t latent_height,
                                 int32_t latent_width, int32_t temporal_scale,
                                 int32_t spatial_scale, double frame_rate, float *out,
                                 int64_t cap);

/* An in-context reference clip appended to the video stream (IC-LoRA references, the
 * Multiple-Subject-Reference slots): DiTForward.Geometry.Reference (DiTForward.swift:220-252). */
typedef struct ltx_rope_reference {
    int32_t latent_frames, latent_height, latent_width;
    int32_t downscale_factor;       /* target-over-reference spatial ratio (2: x2 upscaler)   */
    int32_t temporal_scale_factor;  /* target-over-reference temporal ratio (1: spatial only) */
    int32_t frame_offset;           /* time shift in PIXEL frames, added before the divide by */
                                    /* the frame rate; MSR slot i of n: -(n - i); 0 otherwise */
} ltx_rope_reference;

/* referencePositions (DiTForward.swift:553-593): the reference's own patch grid built at frame
 * rate 1 (time in pixel frames), + frame_offset, / float(frame_rate / temporal_scale_factor),
 * then for temporal_scale_factor != 1 max(t - (factor - 1) * target_first_end, 0), and the
 * spatial axes times downscale_factor. `target_first_end` is the target grid's first patch
 * end ([0][0][1] of its positions). Writes bounds [3][tokens][2] with a token stride
 * `row_tokens` >= tokens: (dim, token, side) at out[(dim*row_tokens + token)*2 + side].
 * Returns tokens, or -1 (also when both frame_offset and temporal_scale_factor != 1 are set:
 * the reference refuses that combination, :564-567). */
int32_t ltx_rope_reference_positions(const ltx_rope_reference *ref, int32_t temporal_scale,
                                     int32_t spatial_scale, double frame_rate,
                                     float target_first_end, float *out, int64_t row_tokens);

/* The video grid of a render with references (rotaries(geometry:dtype:), DiTForward.swift
 * :698-711): the target's grid, then each reference's in order, every reference shifted
 * against the target's own grid. [3][total][2], total = target tokens + all reference tokens
 * (`videoTokensWithReference`); cap in floats. Returns total, or -1. */
int32_t ltx_rope_video_positions_with_references(int32_t latent_frames, int32_t latent_height,
                                                 int32_t latent_width, int32_t temporal_scale,
                                                 int32_t spatial_scale, double frame_rate,
                                                 const ltx_rope_reference *refs,
                                                 int32_t n_refs, float *out, int64_t cap);

/* audioPositions (DiTForward.swift:606-619): bounds [1][tokens][2] in seconds. */
int32_t ltx_rope_audio_positions(int32_t tokens, int32_t hop_length, int32_t sample_rate,
                                 int32_t downsample, float *out, int64_t cap);

/* rotary(positions:innerDim:maxPos:heads:theta:dtype:) (DiTForward.swift:641-678):
 * positions [n_pos][tokens][2] -> bf16 bit patterns cos/sin [heads][tokens][inner/2/heads].
 * Returns 0 or -1. */
int32_t ltx_rope_tables(const float *positions, int32_t n_pos, int32_t tokens, int32_t inner,
                        const int32_t *max_pos, int32_t heads, double theta, uint16_t *cos_out,
                        uint16_t *sin_out);

/* The same tables built on the GPU, asynchronously on `stream` (a hipStream_t or NULL):
 * `positions` ([n_pos][tokens][2] float, 4-byte aligned) and `cos_out` / `sin_out` ([heads]
 * [tokens][inner/2/heads] bf16 bit patterns) are DEVICE pointers; `max_pos` is a host array
 * of n_pos (<= 8) counts. Same bits as ltx_rope_tables for the same positions. Arguments are
 * checked before anything is launched (LTX_ATTN_EINVAL); LTX_ATTN_EHIP if the launch fails. */
ltx_attn_status ltx_rope_tables_device(const float *positions, int32_t n_pos, int32_t tokens,
                                       int32_t inner, const int32_t *max_pos, int32_t heads,
                                       double theta, uint16_t *cos_out, uint16_t *sin_out,
                                       void *stream);

/* ----------------------------------------------------------------------------------------
 * Gemma-4 text-encoder attention (Sources/LTXModules/GemmaTextEncoder.swift:158-239 with the
 * mask of :288-321), from the q/k/v projections to the merged output before o_proj.
 * Replaces, per layer: q = rope(q_norm(q_proj)), k = rope(k_norm(k_proj)), v = v_norm(v_proj
 * or the PRE-norm k_proj on the K-shares-V layers), the KV-head repeat (GQA), and the SDPA
 * with scale 1.0 under the causal / sliding-window / padding mask (rows with no allowed key
 * attend to every key, :306-319). Norms per head over D: x * pow(mean(x^2) + eps, -0.5) *
 * weight (no 1 + weight), fp32; v's norm has no weight. The sliding layers are D = 256,
 * 16 query heads over 8 KV heads, window 1024, theta 1e4; the full layers D = 512, 16 query
 * heads over 1 KV head with V from K, partial ("proportional") rotation, theta 1e6.
 * -------------------------------------------------------------------------------------- */
typedef struct ltx_gemma_attn_args {
    int32_t B, T;                 /* batch rows (prompts), tokens (queries = keys)             */
    int32_t Hq, Hkv, D;           /* D in {256, 512}; Hq a multiple of Hkv                     */
    const void *q;                /* bf16 [B, T, Hq*D] (q_proj output), element strides below  */
    const void *k;                /* bf16 [B, T, Hkv*D] (k_proj output)                        */
    const void *v;                /* bf16 [B, T, Hkv*D] (v_proj output), or == k: V = v_norm of */
                                  /* the pre-norm K projection (the K-shares-V layers)          */
    int64_t q_bs, q_rs, k_bs, k_rs, v_bs, v_rs;
    const void *q_norm_w, *k_norm_w;  /* bf16 [D]                                              */
    float eps;                    /* rms_norm_eps (1e-6)                                       */
    const float *cos, *sin;       /* fp32 [T, D/2], positions 0..T-1 (ltx_gemma_rope_tables)   */
    int32_t window;               /* sliding window (keys q - window < k <= q), 0 = causal only */
    const int32_t *first_valid;   /* HOST [B]: keys < first_valid[b] are left padding, or NULL */
    float scale;                  /* logit scale: GemmaAttentionSpec.attentionScaling = 1.0     */
    float *out;                   /* fp32 [B, T, Hq*D] (the reference's explicit path returns   */
                                  /* fp32: its q is promoted by the fp32 RoPE tables, :224-239) */
    int64_t o_bs, o_rs;           /* element strides                                           */
    void *workspace;              /* device, 256-byte aligned, >= ltx_gemma_attn_workspace_bytes */
    size_t workspace_bytes;
} ltx_gemma_attn_args;

/* Workspace for the prepared q, k (normed, rotated) and v^T (fp16 MFMA operands) and the key
 * split's partials; 0 on bad args. */
size_t ltx_gemma_attn_workspace_bytes(const ltx_gemma_attn_args *a);

/* Validate, then run asynchronously on `stream`: the per-head prologue, then the attention.
 * Same status convention as ltx_attn_fwd; nothing is launched on an error. */
ltx_attn_status ltx_gemma_attn_fwd(const ltx_gemma_attn_args *a, void *stream);

/* GemmaAttentionSpec.inverseFrequencies (GemmaAttentionSpec.swift:88-121) in double, then the
 * tables of GemmaTextEncoder.positionEmbeddings (:135-145): fp32 angle = position * float(inv),
 * fp32 cos/sin, [tokens][head_dim/2]. `proportional` != 0: the denominator is the full head dim
 * and only partial_factor*head_dim/2 frequencies are non-zero; else the denominator is the
 * rotated width head_dim*partial_factor. Returns 0 or -1 on bad arguments. */
int32_t ltx_gemma_rope_tables(int32_t tokens, int32_t head_dim, double theta,
                              double partial_factor, int32_t proportional, float *cos_out,
                              float *sin_out);

/* ----------------------------------------------------------------------------------------
 * The HIP device. The reference measures its machine rather than assuming it
 * (Sources/LTXHardware/Machine.swift:12-30, Machine.detect()); a host that selects the HIP
 * attention path explicitly describes the device it selected with these.
 * -------------------------------------------------------------------------------------- */
typedef struct ltx_device_info {
    int32_t ordinal;
    int32_t compute_units;        /* CUs (256 on an MI355X, the count the work split of the   */
                                  /* attention kernels is planned for: one workgroup per CU)  */
    int64_t memory_bytes;         /* device memory (HBM) capacity                              */
    int32_t clock_khz;            /* peak shader clock                                         */
    int32_t lds_bytes_per_cu;     /* LDS per CU (160 KiB on gfx950)                            */
    int32_t supported;            /* 1 if the device is gfx950, the architecture the library's */
                                  /* kernels are built for; 0 otherwise                        */
    char name[128];               /* marketing name                                            */
    char arch[64];                /* gcnArchName, e.g. "gfx950:sramecc+:xnack-"               */
} ltx_device_info;

/* Visible HIP devices (0 when there is none or the runtime cannot start). */
int32_t ltx_device_count(void);

/* Describe device `ordinal` (LTX_ATTN_EINVAL for a bad ordinal or NULL, LTX_ATTN_EHIP if the
 * runtime fails). Does not change the current device. */
ltx_attn_status ltx_device_query(int32_t ordinal, ltx_device_info *out);

#ifdef __cplusplus
}
#endif

#endif /* LTX_ATTN_H */
