// C++ host mirror of the reference's attention call surface over the C ABI of libltx_attn.so.
//
// Mirrors Sources/LTXModules/DiTAttention.swift:
//   Variant (with takesRotary)              :69-90
//   Rotary (the cos/sin pair)               :92-105
//   Failure (missing / shape / rotaryWithoutPosition), thrown                :107-122
//   the replaced unit of callAsFunction:    :358-381  (norm -> split -> RoPE -> SDPA)
// and MLXFast.scaledDotProductAttention(queries:keys:values:scale:mask:.none) (:374-376).
// The projections, the per-head gate and to_out stay with the caller (:342, :358-359,
// :385-404). Device memory is the caller's; nothing here allocates except the workspace
// helper, which the caller may bypass by passing its own buffer.
#pragma once

#include <cmath>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "../../include/ltx_attn.h"

namespace ltx {

// DiTAttention.Failure. `status` carries the C-ABI code behind it.
class Failure : public std::runtime_error {
public:
    Failure(ltx_attn_status status, const std::string &what)
        : std::runtime_error(what), status_(status) {}
    ltx_attn_status status() const { return status_; }

private:
    ltx_attn_status status_;
};

class DiTAttention {
public:
    static constexpr int heads = 32;             // DiTAttention.heads (:64)
    static constexpr float normEpsilon = 1e-6f;  // DiTAttention.normEpsilon (:66)

    // The six variants as the checkpoint's weight stems (:69-75).
    enum class Variant { videoSelf, videoCross, audioSelf, audioCross, audioToVideo, videoToAudio };

    static const char *rawValue(Variant v) {
        switch (v) {
        case Variant::videoSelf: return "attn1";
        case Variant::videoCross: return "attn2";
        case Variant::audioSelf: return "audio_attn1";
        case Variant::audioCross: return "audio_attn2";
        case Variant::audioToVideo: return "audio_to_video_attn";
        case Variant::videoToAudio: return "video_to_audio_attn";
        }
        return "?";
    }

    // attn2 / audio_attn2 are never rotated (:84-89).
    static bool takesRotary(Variant v) {
        return v != Variant::videoCross && v != Variant::audioCross;
    }

    // One rotary embedding: bf16 cos/sin, each [heads, tokens, D/2] on the device.
    struct Rotary {
        const void *cos = nullptr;
        const void *sin = nullptr;
    };

    // A bf16 device tensor in the merged projection layout [B, L, H*D] (element strides).
    struct Stream {
        const void *data = nullptr;
        int64_t batch_stride = 0, row_stride = 0;
        int32_t tokens = 0;
    };

    // q_norm.weight / k_norm.weight of the module: bf16 [H*D] device pointers.
    DiTAttention(const void *q_norm_weight, const void *k_norm_weight)
        : q_norm_(q_norm_weight), k_norm_(k_norm_weight) {}

    // norm -> split -> RoPE -> SDPA for one module call. q = to_q(x), k = to_k(context),
    // v = to_v(context) (pre-norm); `rotary` is `pe`, `keyRotary` is `k_pe` (nullptr means
    // "use pe for both", :310-314). `out` receives [B, Lq, H*D] bf16. With `gate_logits`
    // (bf16 [B, Lq, H] contiguous: to_gate_logits(x)) each head's rows are multiplied by
    // 2*sigmoid(logit), as the module's gate does (:395-399). `allPerturbed` is the STG
    // passthrough (:351-356): out = V per head (times the gate); q and k are not read (their
    // `data` may be null, `tokens` still gives Lq). `q_sumsq` / `k_sumsq`: the statistic
    // partials ltx_linear wrote for q / k ([B*L][sumsq_blocks]), which replace the norm's own
    // statistic pass. Throws Failure.
    void operator()(int32_t batch, int32_t inner, const Stream &q, const Stream &k,
                    const Stream &v, void *out, int64_t out_batch_stride,
                    int64_t out_row_stride, Variant variant, const Rotary *rotary,
                    const Rotary *keyRotary, void *workspace, size_t workspace_bytes,
                    void *stream, const int32_t *k_valid_len = nullptr,
                    const void *gate_logits = nullptr, bool allPerturbed = false,
                    const float *q_sumsq = nullptr, const float *k_sumsq = nullptr,
                    int32_t sumsq_blocks = 0) const {
        if (rotary && !takesRotary(variant))
            throw Failure(LTX_ATTN_EINVAL,
                          std::string(rawValue(variant)) +
                              " takes no rotary embedding; supplying one would rotate a "
                              "stream that has no latent position");
        if (keyRotary && !rotary)
            throw Failure(LTX_ATTN_EINVAL, "keyRotary without rotary");
        if (inner % heads != 0)
            throw Failure(LTX_ATTN_EINVAL, "inner dim " + std::to_string(inner) +
                                               " is not a multiple of " +
                                               std::to_string(heads) + " heads");
        ltx_attn_args a = args(batch, inner, q, k, v, out, out_batch_stride, out_row_stride,
                               rotary, keyRotary, k_valid_len);
        a.workspace = workspace;
        a.workspace_bytes = workspace_bytes;
        a.all_perturbed = allPerturbed ? 1 : 0;
        if (gate_logits) {
            a.gate_logits = gate_logits;
            a.g_bs = (int64_t)q.tokens * heads;
            a.g_rs = heads;
            a.g_hs = 1;
        }
        if (q_sumsq || k_sumsq) {
            // the projections' statistic partials (ltx_linear), [B*L][sumsq_blocks] each
            a.q_sumsq = q_sumsq;
            a.k_sumsq = k_sumsq;
            a.q_sumsq_rs = a.k_sumsq_rs = a.sumsq_blocks = sumsq_blocks;
        }
        check(ltx_attn_fwd(&a, stream));
    }

    // Workspace the same call needs (0 if none).
    size_t workspaceBytes(int32_t batch, int32_t inner, const Stream &q, const Stream &k,
                          const Stream &v, Variant, const Rotary *rotary,
                          const Rotary *keyRotary, const int32_t *k_valid_len = nullptr,
                          bool allPerturbed = false) const {
        if (allPerturbed) return 0;
        // The output only has to be a valid-looking tensor for sizing; q's geometry is used.
        ltx_attn_args a = args(batch, inner, q, k, v, const_cast<void *>(q.data),
                               q.batch_stride, q.row_stride, rotary, keyRotary, k_valid_len);
        return ltx_attn_workspace_bytes(&a);
    }

    static void check(ltx_attn_status s) {
        if (s != LTX_ATTN_OK)
            throw Failure(s, std::string(ltx_attn_status_string(s)) + ": " +
                                 ltx_attn_last_error());
    }

private:
    ltx_attn_args args(int32_t batch, int32_t inner, const Stream &q, const Stream &k,
                       const Stream &v, void *out, int64_t obs, int64_t ors,
                       const Rotary *rotary, const Rotary *keyRotary,
                       const int32_t *k_valid_len) const {
        ltx_attn_args a;
        ltx_attn_args_init(&a);
        const int32_t D = inner / heads;
        a.B = batch;
        a.H = heads;
        a.D = D;
        a.Lq = q.tokens;
        a.Lk = k.tokens;
        a.q = q.data; a.q_bs = q.batch_stride; a.q_rs = q.row_stride; a.q_hs = D;
        a.k = k.data; a.k_bs = k.batch_stride; a.k_rs = k.row_stride; a.k_hs = D;
        a.v = v.data; a.v_bs = v.batch_stride; a.v_rs = v.row_stride; a.v_hs = D;
        a.out = out; a.o_bs = obs; a.o_rs = ors; a.o_hs = D;
        a.q_norm_w = q_norm_;
        a.k_norm_w = k_norm_;
        a.norm_eps = normEpsilon;
        if (rotary) { a.q_cos = rotary->cos; a.q_sin = rotary->sin; }
        if (keyRotary) { a.k_cos = keyRotary->cos; a.k_sin = keyRotary->sin; }
        a.k_valid_len = k_valid_len;
        a.scale = (float)(1.0 / std::sqrt((double)D));   // :372
        return a;
    }

    const void *q_norm_;
    const void *k_norm_;
};

}  // namespace ltx
