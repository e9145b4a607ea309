// Host-side construction of the split-RoPE cos/sin tables the DiT hands to every attention
// call, following Sources/LTXModules/DiTForward.swift:440-738. Pure C++ (no GPU); exported
// through the C ABI declared in include/ltx_attn.h.
//
// Precision follows the reference step by step: the frequency grid in double then float
// (:455-466), positions and angles in float (:486-520, :606-619, :641-678), cos/sin in float,
// one round-to-nearest-even cast to bf16 at the end (:676-677).
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <vector>

#include "../../include/ltx_attn.h"

namespace {

uint16_t bf16_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

}  // namespace

extern "C" {

int32_t ltx_rope_frequency_grid(double theta, int32_t n_pos, int32_t inner, float *out,
                                int32_t cap) {
    if (n_pos < 1 || inner < 1) return -1;
    const int32_t count = inner / (2 * n_pos);
    if (count <= 1 || !out || cap < count) return -1;
    const double step = 1.0 / (double)(count - 1);
    for (int32_t i = 0; i < count; ++i) {
        // i * step, except the endpoint, which is written as exactly 1 (DiTForward.swift:462).
        const double e = (i == count - 1) ? 1.0 : (double)i * step;
        out[i] = (float)(pow(theta, e) * M_PI / 2);
    }
    return count;
}

int32_t ltx_rope_video_positions(int32_t latent_frames, int32_t latent_height,
                                 int32_t latent_width, int32_t temporal_scale,
                                 int32_t spatial_scale, double frame_rate, float *out,
                                 int64_t cap) {
    if (latent_frames < 1 || latent_height < 1 || latent_width < 1 || temporal_scale < 1 ||
        spatial_scale < 1 || !(frame_rate > 0) || !out)
        return -1;
    const int64_t tokens = (int64_t)latent_frames * latent_height * latent_width;
    if (tokens > INT32_MAX || cap < 3 * tokens * 2) return -1;
    const int32_t scales[3] = {temporal_scale, spatial_scale, spatial_scale};
    const float fr = (float)frame_rate;
    int64_t tok = 0;
    for (int32_t t = 0; t < latent_frames; ++t)
        for (int32_t y = 0; y < latent_height; ++y)
            for (int32_t x = 0; x < latent_width; ++x, ++tok) {
                const int32_t start[3] = {t, y, x};
                for (int dim = 0; dim < 3; ++dim) {
                    // Integer pixel bounds, then the causal correction, then the float
                    // conversion, then (time only) the divide by the frame rate.
                    int64_t lo = (int64_t)start[dim] * scales[dim];
                    int64_t hi = (int64_t)(start[dim] + 1) * scales[dim];
                    if (dim == 0) {
                        lo = lo + 1 - temporal_scale;
                        hi = hi + 1 - temporal_scale;
                        if (lo < 0) lo = 0;
                        if (hi < 0) hi = 0;
                    }
                    float lof = (float)lo, hif = (float)hi;
                    if (dim == 0) {
                        lof /= fr;
                        hif /= fr;
                    }
                    out[(dim * tokens + tok) * 2] = lof;
                    out[(dim * tokens + tok) * 2 + 1] = hif;
                }
            }
    return (int32_t)tokens;
}

int32_t ltx_rope_reference_positions(const ltx_rope_reference *r, int32_t temporal_scale,
                                     int32_t spatial_scale, double frame_rate,
                                     float target_first_end, float *out, int64_t row_tokens) {
    if (!r || !out || !(frame_rate > 0) || r->downscale_factor < 1 ||
        r->temporal_scale_factor < 1)
        return -1;
    // An offset and a sparse-reference shift do not compose: the shift clamps time at zero
    // and would erase the negative times the offset creates (DiTForward.swift:570-573).
    if (r->frame_offset != 0 && r->temporal_scale_factor != 1) return -1;
    const int64_t tokens = (int64_t)r->latent_frames * r->latent_height * r->latent_width;
    if (r->latent_frames < 1 || r->latent_height < 1 || r->latent_width < 1 ||
        tokens > INT32_MAX || row_tokens < tokens)
        return -1;
    // 1. the reference's own patch grid at frame rate 1: time stays in pixel frames (the
    //    divide by 1.0f is exact, so the no-offset grid keeps its bits)
    std::vector<float> grid((size_t)tokens * 6);
    if (ltx_rope_video_positions(r->latent_frames, r->latent_height, r->latent_width,
                                 temporal_scale, spatial_scale, 1.0, grid.data(),
                                 (int64_t)grid.size()) != (int32_t)tokens)
        return -1;
    // 2.-3. the offset in pixel frames, then the reference's own time spacing
    //       fps / temporalScaleFactor, the divisor rounded to float once
    const float offset = (float)r->frame_offset;
    const float spacing = (float)(frame_rate / (double)r->temporal_scale_factor);
    // 4. a temporally sparse reference slides forward so its last patch ends where the
    //    target's does: shift = (factor - 1) * the target's first patch end, clamped at 0
    const float shift = (float)(r->temporal_scale_factor - 1) * target_first_end;
    const float down = (float)r->downscale_factor;
    for (int64_t tok = 0; tok < tokens; ++tok)
        for (int side = 0; side < 2; ++side) {
            float t = grid[(size_t)tok * 2 + side];
            if (r->frame_offset != 0) t = t + offset;
            t = t / spacing;
            if (r->temporal_scale_factor != 1) {
                t = t - shift;
                if (t < 0.0f) t = 0.0f;                       // maximum(t, 0)
            }
            out[(0 * row_tokens + tok) * 2 + side] = t;
            for (int dim = 1; dim < 3; ++dim) {
                float x = grid[((size_t)dim * tokens + tok) * 2 + side];
                // 5. the spatial axes scaled by the target-over-reference ratio
                if (r->downscale_factor != 1) x = x * down;
                out[(dim * row_tokens + tok) * 2 + side] = x;
            }
        }
    return (int32_t)tokens;
}

int32_t ltx_rope_video_positions_with_references(int32_t latent_frames, int32_t latent_height,
                                                 int32_t latent_width, int32_t temporal_scale,
                                                 int32_t spatial_scale, double frame_rate,
                                                 const ltx_rope_reference *refs,
                                                 int32_t n_refs, float *out, int64_t cap) {
    if (n_refs < 0 || (n_refs > 0 && !refs) || !out) return -1;
    const int64_t target = (int64_t)latent_frames * latent_height * latent_width;
    if (latent_frames < 1 || latent_height < 1 || latent_width < 1) return -1;
    int64_t total = target;
    for (int32_t i = 0; i < n_refs; ++i)
        total += (int64_t)refs[i].latent_frames * refs[i].latent_height * refs[i].latent_width;
    if (total > INT32_MAX || cap < 3 * total * 2) return -1;
    std::vector<float> grid((size_t)target * 6);
    if (ltx_rope_video_positions(latent_frames, latent_height, latent_width, temporal_scale,
                                 spatial_scale, frame_rate, grid.data(),
                                 (int64_t)grid.size()) != (int32_t)target)
        return -1;
    for (int dim = 0; dim < 3; ++dim)
        memcpy(out + (size_t)dim * total * 2, grid.data() + (size_t)dim * target * 2,
               sizeof(float) * target * 2);
    // every reference reads the shift from the generated grid itself, never from the growing
    // concatenation (DiTForward.swift:707-711): the target's first patch end, [0][0][1]
    const float first_end = grid[1];
    int64_t at = target;
    for (int32_t i = 0; i < n_refs; ++i) {
        const int32_t n = ltx_rope_reference_positions(&refs[i], temporal_scale, spatial_scale,
                                                       frame_rate, first_end, out + at * 2,
                                                       total);
        if (n < 0) return -1;
        at += n;
    }
    return (int32_t)total;
}

int32_t ltx_rope_audio_positions(int32_t tokens, int32_t hop_length, int32_t sample_rate,
                                 int32_t downsample, float *out, int64_t cap) {
    if (tokens < 1 || hop_length < 1 || sample_rate < 1 || downsample < 1 || !out ||
        cap < (int64_t)tokens * 2)
        return -1;
    auto seconds = [&](int32_t i) {
        float frame = (float)((int64_t)i * downsample);
        frame = frame + 1.0f - (float)downsample;
        if (frame < 0.0f) frame = 0.0f;
        // `* hop` then `/ sampleRate`, two roundings (DiTForward.swift:604-611).
        return frame * (float)hop_length / (float)sample_rate;
    };
    for (int32_t i = 0; i < tokens; ++i) {
        out[2 * i] = seconds(i);
        out[2 * i + 1] = seconds(i + 1);
    }
    return tokens;
}

int32_t ltx_rope_tables(const float *positions, int32_t n_pos, int32_t tokens, int32_t inner,
                        const int32_t *max_pos, int32_t heads, double theta, uint16_t *cos_out,
                        uint16_t *sin_out) {
    if (!positions || n_pos < 1 || tokens < 1 || inner < 2 || !max_pos || heads < 1 ||
        !cos_out || !sin_out)
        return -1;
    if ((inner / 2) % heads != 0) return -1;
    for (int d = 0; d < n_pos; ++d)
        if (max_pos[d] <= 0) return -1;
    const int32_t count = inner / (2 * n_pos);
    if (count <= 1) return -1;
    std::vector<float> freqs(count);
    if (ltx_rope_frequency_grid(theta, n_pos, inner, freqs.data(), count) != count) return -1;
    const int32_t used = count * n_pos;
    const int32_t half = inner / 2;
    const int32_t pad = half - used;
    if (pad < 0) return -1;
    const int32_t per_head = half / heads;

    std::vector<float> frac(n_pos);
    for (int32_t t = 0; t < tokens; ++t) {
        for (int d = 0; d < n_pos; ++d) {
            const float lo = positions[((int64_t)d * tokens + t) * 2];
            const float hi = positions[((int64_t)d * tokens + t) * 2 + 1];
            const float middle = (lo + hi) / 2.0f;                 // patch centre
            frac[d] = middle / (float)max_pos[d];
        }
        for (int32_t j = 0; j < half; ++j) {
            float c = 1.0f, s = 0.0f;                               // leading identity pad
            if (j >= pad) {
                const int32_t jj = j - pad;
                const int32_t i = jj / n_pos, d = jj % n_pos;        // positional dim fastest
                const float scaled = frac[d] * 2.0f - 1.0f;
                const float angle = freqs[i] * scaled;
                c = cosf(angle);
                s = sinf(angle);
            }
            // [tokens, heads, per_head] -> [heads, tokens, per_head]
            const int32_t hh = j / per_head, k = j % per_head;
            const int64_t o = ((int64_t)hh * tokens + t) * per_head + k;
            cos_out[o] = bf16_bits(c);
            sin_out[o] = bf16_bits(s);
        }
    }
    return 0;
}

// GemmaAttentionSpec.inverseFrequencies (GemmaAttentionSpec.swift:88-121), in double, then
// GemmaTextEncoder.positionEmbeddings (GemmaTextEncoder.swift:135-145): the frequencies are
// narrowed to float, the angle is the float product position * inv, and cos/sin are taken of
// that float angle in float.
int32_t ltx_gemma_rope_tables(int32_t tokens, int32_t head_dim, double theta,
                              double partial_factor, int32_t proportional, float *cos_out,
                              float *sin_out) {
    if (tokens < 1 || head_dim < 2 || (head_dim & 1) || !(theta > 0.0) ||
        !(partial_factor > 0.0 && partial_factor <= 1.0) || !cos_out || !sin_out)
        return -1;
    const int32_t half = head_dim / 2;
    std::vector<double> inv(half, 0.0);
    if (proportional) {
        // denominator: the full head dim; int(factor * headDim / 2) real angles
        const int32_t n = (int32_t)(partial_factor * (double)head_dim / 2.0);
        for (int32_t i = 0; i < n && i < half; ++i)
            inv[i] = 1.0 / pow(theta, (double)(2 * i) / (double)head_dim);
    } else {
        // denominator: the rotated width; its frequencies, zero beyond
        const int32_t dim = (int32_t)((double)head_dim * partial_factor);
        for (int32_t i = 0; i < dim / 2 && i < half; ++i)
            inv[i] = 1.0 / pow(theta, (double)(2 * i) / (double)dim);
    }
    for (int32_t t = 0; t < tokens; ++t)
        for (int32_t i = 0; i < half; ++i) {
            const float angle = (float)t * (float)inv[i];
            cos_out[(int64_t)t * half + i] = cosf(angle);
            sin_out[(int64_t)t * half + i] = sinf(angle);
        }
    return 0;
}

}  // extern "C"
