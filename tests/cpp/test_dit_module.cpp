// Host-side behaviour of the C++ module driver (no GPU needed): weight-shape checks, the
// workspace layout (projections, statistic partials, gate logits, merged output and the
// attention call's own workspace) and failures thrown before anything is launched.
#include <algorithm>
#include <cstdio>
#include <cstdint>
#include <string>

#include "../../ltx-2.5-swift_amd/host/dit_module.hpp"

static int failures = 0;
#define EXPECT(cond, msg)                                                   \
    do {                                                                    \
        if (!(cond)) { std::printf("FAIL: %s\n", msg); ++failures; }       \
        else std::printf("ok: %s\n", msg);                                  \
    } while (0)

int main() {
    using ltx::DiTAttentionModule;
    using ltx::DiTAttention;
    auto fake = [](uintptr_t i) { return reinterpret_cast<void *>((uintptr_t)0x7f0000000000ull + (i << 32)); };
    auto lin = [&](uintptr_t id, int out, int in) {
        return DiTAttentionModule::Linear{fake(id), fake(id + 100), out, in};
    };
    DiTAttentionModule::Weights w;
    w.to_q = lin(1, 4096, 4096); w.to_k = lin(2, 4096, 4096); w.to_v = lin(3, 4096, 4096);
    w.to_gate_logits = lin(4, 32, 4096); w.to_out = lin(5, 4096, 4096);
    w.q_norm = fake(6); w.k_norm = fake(7);
    DiTAttentionModule m(w);
    EXPECT(m.inner() == 4096, "inner width from to_q");

    // shape checks at construction
    auto rejects = [&](DiTAttentionModule::Weights bad) {
        try { DiTAttentionModule x(bad); } catch (const ltx::Failure &f) { return f.status() == LTX_ATTN_EINVAL; }
        return false;
    };
    auto bad = w; bad.to_q.out = 4000;
    EXPECT(rejects(bad), "to_q rows not a multiple of 32 heads");
    bad = w; bad.to_k.out = 2048;
    EXPECT(rejects(bad), "to_k rows differ from to_q's");
    bad = w; bad.to_gate_logits.out = 16;
    EXPECT(rejects(bad), "to_gate_logits must have 32 rows");
    bad = w; bad.to_out.weight = nullptr;
    EXPECT(rejects(bad), "to_out.0 is required");
    bad = w; bad.to_gate_logits.weight = nullptr;
    EXPECT(!rejects(bad), "to_gate_logits is optional");

    // workspace: projections + partials + gate + merged + the attention call's own
    const int B = 1, T = 12480;
    DiTAttentionModule::Input x{fake(8), T, 4096};
    DiTAttention::Rotary pe{fake(9), fake(10)};
    using V = DiTAttention::Variant;
    const size_t need = m.workspaceBytes(B, x, nullptr, V::videoSelf, &pe, nullptr, nullptr, false);
    auto up = [](size_t v) { return (v + 255) / 256 * 256; };
    const size_t proj = 3 * up(2ull * T * 4096) + 2 * up(4ull * T * 16) + up(2ull * T * 32) +
                        up(2ull * T * 4096);
    EXPECT(need > proj, "workspace holds the projections and the attention's own");
    const size_t need_p = m.workspaceBytes(B, x, nullptr, V::videoSelf, &pe, nullptr, nullptr, true);
    // the projections' split-tail scratch, the larger of to_v / to_out (12480 x 4096 x 4096:
    // 16 tail tiles in 8 k ranges) and to_gate_logits (12480 x 32 x 4096: 49 tiles in 4)
    ltx_linear_args la{};
    la.M = T; la.N = 4096; la.K = 4096;
    const size_t scratch_v = ltx_linear_workspace_bytes(&la);
    EXPECT(scratch_v == 16ull * 8 * 256 * 256 * 4, "linear scratch: 16 tail tiles x 8 k ranges");
    la.N = 32;
    const size_t scratch_g = ltx_linear_workspace_bytes(&la);
    EXPECT(scratch_g == 49ull * 4 * 256 * 256 * 4, "gate logits scratch: 49 tiles x 4 k ranges");
    const size_t scratch = std::max(scratch_v, scratch_g);
    EXPECT(need_p == up(2ull * T * 4096) + up(2ull * T * 32) + up(2ull * T * 4096) + up(scratch),
           "perturbed: v, gate logits, the merged output and the projections' scratch only");

    // failures before any launch
    try {
        DiTAttention::Rotary none{};
        (void)none;
        m(B, x, nullptr, V::videoCross, &pe, nullptr, nullptr, false, fake(11), fake(12), need,
          nullptr);
        EXPECT(false, "rotary on attn2 is refused");
    } catch (const ltx::Failure &f) {
        EXPECT(f.status() == LTX_ATTN_EINVAL &&
                   std::string(f.what()).find("no rotary") != std::string::npos,
               "rotary on attn2 is refused");
    }
    try {
        m(B, x, nullptr, V::videoSelf, &pe, nullptr, nullptr, false, fake(11), fake(12), need - 256,
          nullptr);
        EXPECT(false, "short workspace is refused");
    } catch (const ltx::Failure &f) {
        EXPECT(f.status() == LTX_ATTN_EWORKSPACE, "short workspace is refused");
    }
    std::printf("%d failure(s)\n", failures);
    return failures ? 1 : 0;
}
