// Host-side behaviour of the C++ block driver (no GPU needed): workspace sizing over the six
// calls, STG passthrough needing none, and the reference's failures thrown before any launch.
#include <cstdio>
#include <cstdint>
#include <string>

#include "../../ltx-2.5-swift_amd/host/dit_block.hpp"

static int failures = 0;
#define EXPECT(cond, msg)                                                   \
    do {                                                                    \
        if (!(cond)) { std::printf("FAIL: %s\n", msg); ++failures; }       \
        else std::printf("ok: %s\n", msg);                                  \
    } while (0)

int main() {
    using ltx::DiTBlockAttention;
    using ltx::DiTAttention;
    auto fake = [](uintptr_t i) { return reinterpret_cast<void *>((uintptr_t)0x7f0000000000ull + (i << 32)); };
    const int B = 2, Tv = 15360, Ta = 152, Tt = 1024;
    auto stream_of = [&](uintptr_t id, int T, int inner) {
        return DiTAttention::Stream{fake(id), (int64_t)T * inner, inner, T};
    };
    auto call = [&](int inner, DiTAttention::Stream q, DiTAttention::Stream kv, uintptr_t out) {
        DiTBlockAttention::Call c;
        c.inner = inner; c.q = q; c.k = kv; c.v = kv; c.out = fake(out);
        c.out_batch_stride = (int64_t)q.tokens * inner; c.out_row_stride = inner;
        return c;
    };
    const auto v4 = stream_of(1, Tv, 4096), a2 = stream_of(2, Ta, 2048), t4 = stream_of(3, Tt, 4096),
               t2 = stream_of(4, Tt, 2048), v2 = stream_of(5, Tv, 2048);
    DiTBlockAttention::Call vs = call(4096, v4, v4, 20), as = call(2048, a2, a2, 21),
                            vt = call(4096, v4, t4, 22), at = call(2048, a2, t2, 23),
                            a2v = call(2048, v2, a2, 24), v2a = call(2048, a2, v2, 25);
    DiTBlockAttention::Norms n{fake(30), fake(31)};
    DiTBlockAttention block(n, n, n, n, n, n);
    DiTBlockAttention::Rotaries r{{fake(40), fake(41)}, {fake(42), fake(43)},
                                  {fake(44), fake(45)}, {fake(46), fake(47)}};
    const int32_t valid[2] = {94, 11};

    // the block's workspace is the largest single call's
    using V = DiTAttention::Variant;
    DiTAttention m(fake(30), fake(31));
    const size_t w_vs = m.workspaceBytes(B, 4096, v4, v4, v4, V::videoSelf, &r.videoSelf, nullptr);
    const size_t w_as = m.workspaceBytes(B, 2048, a2, a2, a2, V::audioSelf, &r.audioSelf, nullptr);
    const size_t w_vt = m.workspaceBytes(B, 4096, v4, t4, t4, V::videoCross, nullptr, nullptr, valid);
    const size_t w_at = m.workspaceBytes(B, 2048, a2, t2, t2, V::audioCross, nullptr, nullptr, valid);
    const size_t w_av = m.workspaceBytes(B, 2048, v2, a2, a2, V::audioToVideo, &r.videoCross,
                                         &r.audioCross);
    const size_t w_va = m.workspaceBytes(B, 2048, a2, v2, v2, V::videoToAudio, &r.audioCross,
                                         &r.videoCross);
    const size_t others = std::max({w_as, w_vt, w_at, w_av, w_va});
    const size_t need = block.workspaceBytes(B, vs, as, vt, at, a2v, v2a, r, valid);
    EXPECT(w_vs > 0 && need == std::max(w_vs, others), "workspace = the largest call's");
    // a perturbed video self-attention needs none
    const size_t need_p = block.workspaceBytes(B, vs, as, vt, at, a2v, v2a, r, valid, true, false);
    EXPECT(need_p == others, "perturbed self-attention needs no workspace");

    // an empty text row (CFG with an empty prompt) is refused before anything runs
    const int32_t empty[2] = {94, 0};
    bool threw = false;
    try {
        block.textCross(B, vt, at, empty, fake(50), need, nullptr);
    } catch (const ltx::Failure &f) {
        threw = f.status() == LTX_ATTN_EINVAL;
    }
    EXPECT(threw, "empty text row is refused");

    // the phases pass every call's arguments through the same validation: a workspace that is
    // too small fails the first call that needs more
    threw = false;
    try {
        block.selfAttention(B, vs, as, r, false, false, fake(50), 16, nullptr);
    } catch (const ltx::Failure &f) {
        threw = f.status() == LTX_ATTN_EWORKSPACE;
    }
    EXPECT(threw, "short workspace is refused");

    std::printf("%d failure(s)\n", failures);
    return failures ? 1 : 0;
}
