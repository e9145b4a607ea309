// The whole attention module, DiTAttention.callAsFunction (Sources/LTXModules/DiTAttention.swift:
// 315-405), over libltx_attn.so:
//   v = to_v(kv)                               :341        ltx_linear
//   q = to_q(x), k = to_k(kv)                  :358-359    ltx_linear, emitting the RMS statistic
//   norm -> split -> RoPE -> SDPA              :360-381    ltx_attn_fwd, statistic from the partials
//   gate = 2*sigmoid(to_gate_logits(x))        :385-399    ltx_linear; applied inside ltx_attn_fwd
//   to_out.0(merged)                           :402-404    ltx_linear
// with kv = context ?? x (:327) and the STG passthrough (:351-356), which projects only v (and
// the gate logits). Everything runs on the caller's stream in the caller's workspace (sized by
// workspaceBytes); nothing is allocated here. LoRA deltas (:183-185) are not applied.
#pragma once

#include <algorithm>
#include <string>

#include "dit_attention.hpp"

namespace ltx {

class DiTAttentionModule {
public:
    using Variant = DiTAttention::Variant;
    using Rotary = DiTAttention::Rotary;
    static constexpr int heads = DiTAttention::heads;

    // One `linear` of the module: bf16 weight [out, in] (the checkpoint's layout) and bias
    // [out] (nullptr = none). A null weight means the module has no such linear (only
    // to_gate_logits may be absent).
    struct Linear {
        const void *weight = nullptr, *bias = nullptr;
        int32_t out = 0, in = 0;
    };
    struct Weights {
        Linear to_q, to_k, to_v, to_gate_logits, to_out;
        const void *q_norm = nullptr, *k_norm = nullptr;   // bf16 [inner]
    };
    // Token rows of one stream: bf16 [batch, tokens, width], rows `row_stride` elements apart
    // and the batch rows contiguous (batch stride tokens * row_stride).
    struct Input {
        const void *data = nullptr;
        int32_t tokens = 0;
        int64_t row_stride = 0;
    };

    explicit DiTAttentionModule(const Weights &w) : w_(w), core_(w.q_norm, w.k_norm) {
        const int32_t inner = w.to_q.out;
        auto need = [](bool ok, const std::string &what) {
            if (!ok) throw Failure(LTX_ATTN_EINVAL, "module weights: " + what);
        };
        need(w.to_q.weight && w.to_k.weight && w.to_v.weight && w.to_out.weight,
             "to_q, to_k, to_v and to_out.0 are required");
        need(inner > 0 && inner % heads == 0, "to_q.weight rows must be k * 32 heads");
        need(w.to_k.out == inner && w.to_v.out == inner, "to_k / to_v rows must equal to_q's");
        need(w.to_k.in == w.to_v.in, "to_k and to_v read the same context width");
        need(w.to_out.in == inner, "to_out.0 must read the inner width");
        need(w.q_norm && w.k_norm, "q_norm.weight and k_norm.weight are required");
        if (w.to_gate_logits.weight)
            need(w.to_gate_logits.out == heads && w.to_gate_logits.in == w.to_q.in,
                 "to_gate_logits.weight must be [32, queryDim]");
    }

    int32_t inner() const { return w_.to_q.out; }

    // out: bf16 [batch, Lq, to_out.out] contiguous. `context` nullptr = self-attention.
    // `rotary` / `keyRotary` / `k_valid_len` as DiTAttention's. Throws Failure.
    void operator()(int32_t batch, const Input &x, const Input *context, Variant variant,
                    const Rotary *rotary, const Rotary *keyRotary, const int32_t *k_valid_len,
                    bool allPerturbed, void *out, void *workspace, size_t workspace_bytes,
                    void *stream) const {
        // Everything the reference refuses is refused here, before the first launch.
        if (rotary && !DiTAttention::takesRotary(variant))
            throw Failure(LTX_ATTN_EINVAL,
                          std::string(DiTAttention::rawValue(variant)) +
                              " takes no rotary embedding; supplying one would rotate a "
                              "stream that has no latent position");
        if (keyRotary && !rotary) throw Failure(LTX_ATTN_EINVAL, "keyRotary without rotary");
        if (!x.data || (context && !context->data) || !out)
            throw Failure(LTX_ATTN_EINVAL, "x, context (when given) and out must be given");
        if (x.row_stride < w_.to_q.in || (context && context->row_stride < w_.to_k.in) ||
            (!context && w_.to_k.in != w_.to_q.in))
            throw Failure(LTX_ATTN_EINVAL, "input widths do not match the projections");
        const Input &kv = context ? *context : x;
        const Layout L = layout(batch, x, kv, variant, rotary, keyRotary, k_valid_len,
                                allPerturbed);
        if (workspace_bytes < L.bytes || (L.bytes && !workspace))
            throw Failure(LTX_ATTN_EWORKSPACE, "module workspace of " + std::to_string(L.bytes) +
                                                   " bytes needed");
        if (reinterpret_cast<uintptr_t>(workspace) & 255u)
            throw Failure(LTX_ATTN_EINVAL, "module workspace must be 256-byte aligned");
        char *ws = static_cast<char *>(workspace);
        const int32_t n = inner(), blocks = ltx_linear_sumsq_blocks(n);
        void *v = ws + L.v, *q = ws + L.q, *k = ws + L.k, *gate = ws + L.gate;
        void *merged = ws + L.merged;
        float *qs = reinterpret_cast<float *>(ws + L.qparts);
        float *ks = reinterpret_cast<float *>(ws + L.kparts);
        const int32_t Mq = batch * x.tokens, Mk = batch * kv.tokens;
        void *scratch = ws + L.attn;
        const size_t sb = L.lin_bytes;
        project(w_.to_v, kv.data, kv.row_stride, Mk, v, n, nullptr, scratch, sb, stream);
        if (!allPerturbed) {
            project(w_.to_q, x.data, x.row_stride, Mq, q, n, qs, scratch, sb, stream);
            project(w_.to_k, kv.data, kv.row_stride, Mk, k, n, ks, scratch, sb, stream);
        }
        const bool gated = w_.to_gate_logits.weight != nullptr;
        if (gated)
            project(w_.to_gate_logits, x.data, x.row_stride, Mq, gate, heads, nullptr, scratch,
                    sb, stream);
        const DiTAttention::Stream sq{allPerturbed ? nullptr : q, (int64_t)x.tokens * n, n, x.tokens};
        const DiTAttention::Stream sk{allPerturbed ? nullptr : k, (int64_t)kv.tokens * n, n, kv.tokens};
        const DiTAttention::Stream sv{v, (int64_t)kv.tokens * n, n, kv.tokens};
        core_(batch, n, sq, sk, sv, merged, (int64_t)x.tokens * n, n, variant, rotary, keyRotary,
              ws + L.attn, L.attn_bytes, stream, k_valid_len, gated ? gate : nullptr,
              allPerturbed, allPerturbed ? nullptr : qs, allPerturbed ? nullptr : ks, blocks);
        project(w_.to_out, merged, n, Mq, out, w_.to_out.out, nullptr, scratch, sb, stream);
    }

    size_t workspaceBytes(int32_t batch, const Input &x, const Input *context, Variant variant,
                          const Rotary *rotary, const Rotary *keyRotary,
                          const int32_t *k_valid_len, bool allPerturbed) const {
        return layout(batch, x, context ? *context : x, variant, rotary, keyRotary, k_valid_len,
                      allPerturbed)
            .bytes;
    }

private:
    struct Layout {
        size_t v = 0, q = 0, k = 0, qparts = 0, kparts = 0, gate = 0, merged = 0, attn = 0;
        size_t attn_bytes = 0, lin_bytes = 0, bytes = 0;
    };

    static size_t up(size_t x) { return (x + 255) / 256 * 256; }

    Layout layout(int32_t batch, const Input &x, const Input &kv, Variant variant,
                  const Rotary *rotary, const Rotary *keyRotary, const int32_t *k_valid_len,
                  bool allPerturbed) const {
        if (batch < 1 || x.tokens < 1 || kv.tokens < 1)
            throw Failure(LTX_ATTN_EINVAL, "batch and token counts must be >= 1");
        const size_t n = (size_t)inner(), blocks = (size_t)ltx_linear_sumsq_blocks(inner());
        const size_t Mq = (size_t)batch * x.tokens, Mk = (size_t)batch * kv.tokens;
        Layout L;
        size_t off = 0;
        auto take = [&](size_t bytes) { const size_t at = off; off = up(off + bytes); return at; };
        L.v = take(2 * Mk * n);
        if (!allPerturbed) {
            L.q = take(2 * Mq * n);
            L.k = take(2 * Mk * n);
            L.qparts = take(4 * Mq * blocks);
            L.kparts = take(4 * Mk * blocks);
        }
        if (w_.to_gate_logits.weight) L.gate = take(2 * Mq * heads);
        L.merged = take(2 * Mq * n);
        // The attention call's own workspace, sized with the geometry it will see.
        const int32_t ni = inner();
        const DiTAttention::Stream sq{allPerturbed ? nullptr : reinterpret_cast<void *>(256),
                                      (int64_t)x.tokens * ni, ni, x.tokens};
        const DiTAttention::Stream sk{reinterpret_cast<void *>(256), (int64_t)kv.tokens * ni, ni,
                                      kv.tokens};
        L.attn_bytes = core_.workspaceBytes(batch, ni, allPerturbed ? sk : sq, sk, sk, variant,
                                            rotary, keyRotary, k_valid_len, allPerturbed);
        if (!allPerturbed && L.attn_bytes == 0) {
            // 0 is also the answer for invalid arguments: surface the library's reason.
            const char *why = ltx_attn_last_error();
            if (why && *why) throw Failure(LTX_ATTN_EINVAL, why);
        }
        // The projections' split-tail scratch shares that region: they run before and after
        // the attention call on the same stream.
        auto lin = [](const Linear &l, size_t M) {
            ltx_linear_args a{};
            a.M = (int32_t)M; a.N = l.out; a.K = l.in;
            return l.weight ? ltx_linear_workspace_bytes(&a) : (size_t)0;
        };
        L.lin_bytes = std::max({lin(w_.to_v, Mk), lin(w_.to_q, Mq), lin(w_.to_k, Mk),
                                lin(w_.to_gate_logits, Mq), lin(w_.to_out, Mq)});
        L.attn = take(std::max(L.attn_bytes, L.lin_bytes));
        L.bytes = off;
        return L;
    }

    // y [M, out] = x [M, in] . w^T (+ b), rows of x `x_rs` apart; `sumsq` optional partials;
    // `scratch` the split tail's partial tiles.
    static void project(const Linear &l, const void *x, int64_t x_rs, int32_t M, void *y,
                        int32_t y_rs, float *sumsq, void *scratch, size_t scratch_bytes,
                        void *stream) {
        ltx_linear_args a{};
        a.M = M; a.N = l.out; a.K = l.in;
        a.x = x; a.w = l.weight; a.bias = l.bias; a.y = y;
        a.x_rs = x_rs; a.w_rs = l.in; a.y_rs = y_rs;
        a.sumsq = sumsq;
        a.sumsq_rs = ltx_linear_sumsq_blocks(l.out);
        a.workspace = scratch;
        a.workspace_bytes = scratch_bytes;
        DiTAttention::check(ltx_linear(&a, stream));
    }

    Weights w_;
    DiTAttention core_;
};

}  // namespace ltx
