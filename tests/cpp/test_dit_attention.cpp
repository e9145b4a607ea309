// Host-side behaviour of the C++ DiTAttention mirror (no GPU needed): the reference's
// structural failures are thrown before anything reaches the device.
#include <cstdio>
#include <cstdint>
#include <string>

#include "../../ltx-2.5-swift_amd/host/dit_attention.hpp"

static int failures = 0;
#define EXPECT(cond, msg)                                                   \
    do {                                                                    \
        if (!(cond)) { std::printf("FAIL: %s\n", msg); ++failures; }       \
        else std::printf("ok: %s\n", msg);                                  \
    } while (0)

int main() {
    using ltx::DiTAttention;
    // Fake, aligned device addresses: validation never dereferences them.
    auto fake = [](uintptr_t i) { return reinterpret_cast<void *>((uintptr_t)0x7f0000000000ull + (i << 32)); };
    const int T = 3120, inner = 4096;
    DiTAttention::Stream q{fake(1), (int64_t)T * inner, inner, T};
    DiTAttention::Stream k{fake(2), (int64_t)T * inner, inner, T};
    DiTAttention::Stream v{fake(3), (int64_t)T * inner, inner, T};
    DiTAttention attn(fake(4), fake(5));
    DiTAttention::Rotary pe{fake(6), fake(7)};

    // rotaryWithoutPosition on attn2 (DiTAttention.swift:319-321)
    bool threw = false;
    try {
        attn(1, inner, q, k, v, fake(8), (int64_t)T * inner, inner,
             DiTAttention::Variant::videoCross, &pe, nullptr, nullptr, 0, nullptr);
    } catch (const ltx::Failure &f) {
        threw = std::string(f.what()).find("attn2 takes no rotary") != std::string::npos;
    }
    EXPECT(threw, "rotary on attn2 is refused");

    threw = false;
    try {
        attn(1, inner, q, k, v, fake(8), (int64_t)T * inner, inner,
             DiTAttention::Variant::videoSelf, nullptr, &pe, nullptr, 0, nullptr);
    } catch (const ltx::Failure &f) {
        threw = f.status() == LTX_ATTN_EINVAL;
    }
    EXPECT(threw, "keyRotary without rotary is refused");

    // head dim 96 (inner 3072 over 32 heads) is not a fused-path head dim
    threw = false;
    try {
        attn(1, 3072, q, k, v, fake(8), (int64_t)T * inner, inner,
             DiTAttention::Variant::videoSelf, nullptr, nullptr, nullptr, 0, nullptr);
    } catch (const ltx::Failure &f) {
        threw = f.status() == LTX_ATTN_EUNSUPPORTED;
    }
    EXPECT(threw, "head dim 96 is unsupported");

    // self-attention with norm + RoPE at 3120 tokens needs workspace; without it: EWORKSPACE
    const size_t need = attn.workspaceBytes(1, inner, q, k, v, DiTAttention::Variant::videoSelf,
                                            &pe, nullptr);
    EXPECT(need > 0, "workspace is sized");
    threw = false;
    try {
        attn(1, inner, q, k, v, fake(8), (int64_t)T * inner, inner,
             DiTAttention::Variant::videoSelf, &pe, nullptr, nullptr, 0, nullptr);
    } catch (const ltx::Failure &f) {
        threw = f.status() == LTX_ATTN_EWORKSPACE;
    }
    EXPECT(threw, "missing workspace is refused");

    // an empty key-padding mask is refused (TextConditioningLayout.swift:65)
    const int32_t lens[1] = {0};
    threw = false;
    try {
        attn(1, inner, q, k, v, fake(8), (int64_t)T * inner, inner,
             DiTAttention::Variant::videoCross, nullptr, nullptr, fake(9), 1 << 30, nullptr, lens);
    } catch (const ltx::Failure &f) {
        threw = f.status() == LTX_ATTN_EINVAL;
    }
    EXPECT(threw, "empty key mask is refused");

    EXPECT(DiTAttention::takesRotary(DiTAttention::Variant::audioToVideo), "a2v takes rotary");
    EXPECT(!DiTAttention::takesRotary(DiTAttention::Variant::audioCross), "audio_attn2 does not");
    std::printf("%d failure(s)\n", failures);
    return failures ? 1 : 0;
}
