// The six attention calls of one DiT block, in the reference's order, over libltx_attn.so.
//
// Mirrors the attention part of Sources/LTXModules/DiTBlock.swift:343-438:
//   phase 1  attn1 (video self), audio_attn1 (audio self)            :343-368
//            each may be fully perturbed (STG passthrough, DiTForward.swift:1009-1010)
//   phase 2  attn2 (video <- text), audio_attn2 (audio <- text)      :370-381
//            text K/V (the modulated connector features, all 1024 tokens), never rotated.
//            The reference attends over every text token with no mask (DiTForward.swift:38-42
//            passes none; DiTAttention.swift:374-376 runs mask: .none), so a caller matching
//            it passes text_valid_len = nullptr. Per-row valid lengths are an extension of
//            this library (key padding, e.g. prompts whose padding was never modulated) and
//            give different outputs from the reference's.
//   phase 3  audio_to_video, then video_to_audio                     :383-435
//            queries and contexts from the pre-cross-modal snapshot of both streams; pe is
//            the query stream's cross grid, k_pe the other stream's (crossed over)
// Between phases the reference updates the residual streams (adaLN, residual adds, norms) and
// projects the next modules' inputs; those steps and the projections stay with the caller,
// who hands each phase the projections it computed (so the snapshot rule of phase 3 is the
// caller's: both directions' inputs come from the streams as they stood before a2v).
//
// One stream, calls in block order, one workspace shared by every call (sized by
// workspaceBytes for the largest); nothing is allocated here. Two streams measured no gain:
// each call of a pair already fills the GPU.
#pragma once

#include <algorithm>

#include "dit_attention.hpp"

namespace ltx {

class DiTBlockAttention {
public:
    using Variant = DiTAttention::Variant;
    using Stream = DiTAttention::Stream;
    using Rotary = DiTAttention::Rotary;

    // q_norm.weight / k_norm.weight (bf16 [inner] device pointers) of one module.
    struct Norms {
        const void *q = nullptr, *k = nullptr;
    };

    // One module's inputs and output: the pre-norm projections q = to_q(x), k = to_k(ctx),
    // v = to_v(ctx) in the merged layout [B, L, inner], the output [B, Lq, inner] and, for
    // modules with to_gate_logits, the logits [B, Lq, heads] (contiguous).
    struct Call {
        int32_t inner = 0;
        Stream q, k, v;
        void *out = nullptr;
        int64_t out_batch_stride = 0, out_row_stride = 0;
        const void *gate_logits = nullptr;
    };

    // The four tables DiTForward.rotaries(geometry:dtype:) builds (DiTForward.swift:698-738).
    struct Rotaries {
        Rotary videoSelf, audioSelf, videoCross, audioCross;
    };

    DiTBlockAttention(Norms attn1, Norms audio_attn1, Norms attn2, Norms audio_attn2,
                      Norms audio_to_video, Norms video_to_audio)
        : m_{DiTAttention(attn1.q, attn1.k), DiTAttention(audio_attn1.q, audio_attn1.k),
             DiTAttention(attn2.q, attn2.k), DiTAttention(audio_attn2.q, audio_attn2.k),
             DiTAttention(audio_to_video.q, audio_to_video.k),
             DiTAttention(video_to_audio.q, video_to_audio.k)} {}

    // Phase 1: video and audio self-attention (:343-368).
    void selfAttention(int32_t batch, const Call &video, const Call &audio, const Rotaries &r,
                       bool videoPerturbed, bool audioPerturbed, void *workspace,
                       size_t workspace_bytes, void *stream) const {
        run(kAttn1, batch, video, Variant::videoSelf, &r.videoSelf, nullptr, nullptr,
            videoPerturbed, workspace, workspace_bytes, stream);
        run(kAudioAttn1, batch, audio, Variant::audioSelf, &r.audioSelf, nullptr, nullptr,
            audioPerturbed, workspace, workspace_bytes, stream);
    }

    // Phase 2: text cross-attention of both streams (:370-381). `text_valid_len`: null for
    // the reference's arithmetic (every text token attended, no mask); or a host array of
    // `batch` counts when the caller wants key padding (keys past the count ignored).
    void textCross(int32_t batch, const Call &video, const Call &audio,
                   const int32_t *text_valid_len, void *workspace, size_t workspace_bytes,
                   void *stream) const {
        run(kAttn2, batch, video, Variant::videoCross, nullptr, nullptr, text_valid_len, false,
            workspace, workspace_bytes, stream);
        run(kAudioAttn2, batch, audio, Variant::audioCross, nullptr, nullptr, text_valid_len,
            false, workspace, workspace_bytes, stream);
    }

    // Phase 3: audio -> video, then video -> audio (:383-435), from the snapshot.
    void crossModal(int32_t batch, const Call &a2v, const Call &v2a, const Rotaries &r,
                    void *workspace, size_t workspace_bytes, void *stream) const {
        run(kA2V, batch, a2v, Variant::audioToVideo, &r.videoCross, &r.audioCross, nullptr,
            false, workspace, workspace_bytes, stream);
        run(kV2A, batch, v2a, Variant::videoToAudio, &r.audioCross, &r.videoCross, nullptr,
            false, workspace, workspace_bytes, stream);
    }

    // Workspace for all six calls (the largest; calls on one stream reuse it in turn).
    size_t workspaceBytes(int32_t batch, const Call &video_self, const Call &audio_self,
                          const Call &video_text, const Call &audio_text, const Call &a2v,
                          const Call &v2a, const Rotaries &r, const int32_t *text_valid_len,
                          bool videoPerturbed = false, bool audioPerturbed = false) const {
        size_t need = 0;
        auto take = [&](int i, const Call &c, Variant v, const Rotary *pe, const Rotary *kpe,
                        const int32_t *vl, bool perturbed) {
            need = std::max(need, m_[i].workspaceBytes(batch, c.inner, c.q, c.k, c.v, v, pe,
                                                       kpe, vl, perturbed));
        };
        take(kAttn1, video_self, Variant::videoSelf, &r.videoSelf, nullptr, nullptr,
             videoPerturbed);
        take(kAudioAttn1, audio_self, Variant::audioSelf, &r.audioSelf, nullptr, nullptr,
             audioPerturbed);
        take(kAttn2, video_text, Variant::videoCross, nullptr, nullptr, text_valid_len, false);
        take(kAudioAttn2, audio_text, Variant::audioCross, nullptr, nullptr, text_valid_len,
             false);
        take(kA2V, a2v, Variant::audioToVideo, &r.videoCross, &r.audioCross, nullptr, false);
        take(kV2A, v2a, Variant::videoToAudio, &r.audioCross, &r.videoCross, nullptr, false);
        return need;
    }

private:
    enum { kAttn1, kAudioAttn1, kAttn2, kAudioAttn2, kA2V, kV2A };

    void run(int i, int32_t batch, const Call &c, Variant v, const Rotary *pe, const Rotary *kpe,
             const int32_t *valid, bool perturbed, void *ws, size_t ws_bytes,
             void *stream) const {
        m_[i](batch, c.inner, c.q, c.k, c.v, c.out, c.out_batch_stride, c.out_row_stride, v, pe,
              kpe, ws, ws_bytes, stream, valid, c.gate_logits, perturbed);
    }

    DiTAttention m_[6];
};

}  // namespace ltx
