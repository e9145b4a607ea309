"""Pins the CPU oracle (oracle/oracle.py and oracle/attn_oracle.c) before anything is checked
against it.

Each check is chosen so that a plausible mistake fails it: a dropped term, a wrong sign or
index, a transposed operand, a per-head instead of per-token norm, interleaved instead of
split RoPE, tail instead of leading RoPE padding, a wrong mask convention. None of them
re-types the oracle's own formula.
"""

import json
import math
import os

import numpy as np
import pytest

import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _bits(x):
    return O.f32_to_bf16_bits(np.asarray(x, dtype=np.float32))


# ---------------------------------------------------------------------------------------
# SDPA core
# ---------------------------------------------------------------------------------------

def test_mlx_capability_uniform_case():
    """Tests/LTXModulesTests/MLXCapabilityTests.swift:78-91: ones Q/K, V = 2 -> 2.0 +- 1e-4,
    [1, 4, 16, 64], scale 1/sqrt(64)."""
    B, H, L, D = 1, 4, 16, 64
    q = np.ones((B, L, H * D), np.float32)
    v = np.full((B, L, H * D), 2.0, np.float32)
    for mode in ("exact", "reference"):
        out = O.attention(_bits(q), _bits(q), _bits(v), H, scale=1.0 / math.sqrt(D), mode=mode)
        assert out.shape == (B, L, H * D)
        assert abs(out[0, 0, 0] - 2.0) < 1e-4
        assert np.all(np.abs(out - 2.0) < 1e-4)
    c = O.c_attention(_bits(q), _bits(q), _bits(v), H, scale=1.0 / math.sqrt(D))
    assert np.all(np.abs(c - 2.0) < 1e-4)


def _python_sdpa(q, k, v, scale):
    """Definition-level brute force with math.exp, lists only (tiny inputs)."""
    out = []
    for qi in q:
        logits = [scale * sum(a * b for a, b in zip(qi, kj)) for kj in k]
        mx = max(logits)
        w = [math.exp(x - mx) for x in logits]
        z = sum(w)
        out.append([sum(w[j] * v[j][d] for j in range(len(k))) / z for d in range(len(v[0]))])
    return out


def test_sdpa_matches_python_brute_force():
    rng = np.random.default_rng(7)
    q = rng.standard_normal((1, 1, 3, 4))
    k = rng.standard_normal((1, 1, 5, 4))
    v = rng.standard_normal((1, 1, 5, 4))
    got = O.sdpa(q, k, v, 0.37)[0, 0]
    ref = _python_sdpa(q[0, 0].tolist(), k[0, 0].tolist(), v[0, 0].tolist(), 0.37)
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)
    # a transposed K (q . k with k swapped axes) is caught
    bad = O.sdpa(q, k[..., ::-1], v, 0.37)[0, 0]
    assert np.max(np.abs(bad - np.asarray(ref))) > 1e-3


def test_sdpa_closed_forms():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((2, 3, 7, 8))
    k = rng.standard_normal((2, 3, 9, 8))
    v = rng.standard_normal((2, 3, 9, 8))
    # Lk = 1 -> O = V
    np.testing.assert_allclose(O.sdpa(q, k[:, :, :1], v[:, :, :1], 0.5),
                               np.broadcast_to(v[:, :, :1], (2, 3, 7, 8)), atol=1e-12)
    # equal keys -> O = mean(V)
    keq = np.broadcast_to(k[:, :, :1], k.shape)
    np.testing.assert_allclose(O.sdpa(q, keq, v, 0.5),
                               np.broadcast_to(v.mean(axis=2, keepdims=True), q.shape),
                               atol=1e-12)
    # scale 0 -> mean(V)
    np.testing.assert_allclose(O.sdpa(q, k, v, 0.0),
                               np.broadcast_to(v.mean(axis=2, keepdims=True), q.shape),
                               atol=1e-12)
    # permuting keys together with values leaves O unchanged
    perm = rng.permutation(9)
    np.testing.assert_allclose(O.sdpa(q, k[:, :, perm], v[:, :, perm], 0.5),
                               O.sdpa(q, k, v, 0.5), atol=1e-12)
    # permuting keys alone changes it
    assert np.max(np.abs(O.sdpa(q, k[:, :, perm], v, 0.5) - O.sdpa(q, k, v, 0.5))) > 1e-3
    # rows of P sum to 1: V = ones -> O = ones
    np.testing.assert_allclose(O.sdpa(q, k, np.ones_like(v), 0.5), np.ones(q.shape), atol=1e-12)


def test_key_padding_equals_truncation():
    """Masked SDPA over Lk keys with n valid == SDPA over K[:n], V[:n] (the additive
    -bf16max convention of TextConditioningLayout.swift:94-107 with >= 1 valid key)."""
    rng = np.random.default_rng(5)
    q = rng.standard_normal((2, 2, 6, 8))
    k = rng.standard_normal((2, 2, 10, 8))
    v = rng.standard_normal((2, 2, 10, 8))
    got = O.sdpa(q, k, v, 0.4, valid_len=[4, 1])
    np.testing.assert_allclose(got[0], O.sdpa(q[:1], k[:1, :, :4], v[:1, :, :4], 0.4)[0])
    # n = 1 -> O = V[0]
    np.testing.assert_allclose(got[1], np.broadcast_to(v[1, :, :1], (2, 6, 8)), atol=1e-12)
    # the additive -bf16max mask gives the same numbers
    logits = np.einsum("hqd,hkd->hqk", q[0], k[0]) * 0.4
    logits[:, :, 4:] += -O.BF16_MAX
    p = np.exp(logits - logits.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    np.testing.assert_allclose(got[0], p @ v[0], atol=1e-12)
    with pytest.raises(ValueError):
        O.sdpa(q, k, v, 0.4, valid_len=[0, 3])


def test_softmax_shift_invariance():
    """Adding a per-row constant to the logits leaves O unchanged: q -> q + c*k_mean-free dir
    is awkward, so shift via an extra key-independent term: equal-norm augmentation."""
    rng = np.random.default_rng(11)
    q = rng.standard_normal((1, 1, 4, 8))
    k = rng.standard_normal((1, 1, 6, 8))
    v = rng.standard_normal((1, 1, 6, 8))
    # append a dimension where every key has the same value -> adds q_extra*c to each logit
    q2 = np.concatenate([q, rng.standard_normal((1, 1, 4, 1)) * 5], -1)
    k2 = np.concatenate([k, np.full((1, 1, 6, 1), 3.0)], -1)
    v2 = v
    np.testing.assert_allclose(O.sdpa(q2, k2, v2, 0.3), O.sdpa(q, k, v, 0.3), atol=1e-12)


# ---------------------------------------------------------------------------------------
# Per-head output gate
# ---------------------------------------------------------------------------------------

def test_head_gate_closed_forms():
    """2*sigmoid is centred on 1 (DiTAttention.swift:393-394): a zero logit passes through (a
    plain sigmoid would halve it), large logits saturate at 2 and 0, g(x) + g(-x) = 2, and
    the gate is increasing."""
    x = O.f32_to_bf16_bits(np.array([0.0, 30.0, -30.0], dtype=np.float32))
    g = O.head_gate(x)
    assert g[0] == 1.0
    assert abs(g[1] - 2.0) < 1e-12 and abs(g[2]) < 1e-12
    r = O.randn_bf16_bits((2, 5, 3), 7, std=3.0)
    neg = O.f32_to_bf16_bits(-O.bf16_bits_to_f32(r))
    np.testing.assert_allclose(O.head_gate(r) + O.head_gate(neg), 2.0, atol=1e-12)
    xs = np.sort(O.bf16_bits_to_f32(r).ravel())
    gs = O.head_gate(O.f32_to_bf16_bits(xs))
    assert np.all(np.diff(gs) >= 0)
    # the reference's gate array is bf16: reference mode rounds it
    assert np.all(O.head_gate(r, "reference") == O.round_bf16(O.head_gate(r)))


def test_head_gate_scales_each_heads_rows():
    """Zero logits leave the attention output unchanged; a logit of -30 on one (token, head)
    silences exactly that head's row, and doubling comes from +30."""
    B, L, H, D = 1, 6, 3, 8
    q = O.randn_bf16_bits((B, L, H * D), 1)
    k = O.randn_bf16_bits((B, L, H * D), 2)
    v = O.randn_bf16_bits((B, L, H * D), 3)
    base = O.attention(q, k, v, H)
    zero = O.f32_to_bf16_bits(np.zeros((B, L, H), dtype=np.float32))
    np.testing.assert_array_equal(O.attention(q, k, v, H, gate_bits=zero), base)
    logits = np.zeros((B, L, H), dtype=np.float32)
    logits[0, 2, 1] = -30.0
    logits[0, 4, 2] = 30.0
    got = O.attention(q, k, v, H, gate_bits=O.f32_to_bf16_bits(logits)).reshape(B, L, H, D)
    want = base.reshape(B, L, H, D).copy()
    want[0, 2, 1] *= 0.0
    want[0, 4, 2] *= 2.0
    np.testing.assert_allclose(got, want, atol=1e-12)


# ---------------------------------------------------------------------------------------
# Projections (linear) and the whole module
# ---------------------------------------------------------------------------------------

def test_linear_matches_python_brute_force():
    """y[m][n] = sum_k x[m][k] w[n][k] + b[n]: w is [out, in] (a transposed operand or a
    dropped bias fails this), summed exactly here with math.fsum."""
    M, N, K = 3, 5, 7
    x = O.randn_bf16_bits((M, K), 11)
    w = O.randn_bf16_bits((N, K), 12)
    b = O.randn_bf16_bits((N,), 13)
    xf, wf, bf = (O.bf16_bits_to_f32(t).astype(float) for t in (x, w, b))
    want = np.array([[math.fsum([xf[m, k] * wf[n, k] for k in range(K)] + [bf[n]])
                      for n in range(N)] for m in range(M)])
    np.testing.assert_allclose(O.linear(x, w, b), want, rtol=1e-13, atol=1e-13)
    # leading axes are rows
    np.testing.assert_allclose(O.linear(x.reshape(1, M, K), w, b)[0], want, rtol=1e-13,
                               atol=1e-13)


def test_linear_reference_mode_rounds_matmul_then_bias():
    """The matmul's output is bf16 before the bias is added (DiTAttention.swift:180, :186):
    1 + 2^-9 rounds to 1, and 1 + 2^-8 is a tie that rounds to even (1), whereas one rounding
    of 1 + 2^-9 + 2^-8 gives 1 + 2^-7. An identity weight passes x through unchanged."""
    x = _bits([[1.0, 2.0 ** -9]])
    w = _bits([[1.0, 1.0]])
    b = _bits([2.0 ** -8])
    assert O.linear(x, w, b, "reference")[0, 0] == 1.0
    assert O.round_bf16(np.float32(1.0 + 2.0 ** -9 + 2.0 ** -8)) == 1.0 + 2.0 ** -7
    assert O.linear(x, w, b, "exact")[0, 0] == 1.0 + 2.0 ** -9 + 2.0 ** -8
    xi = O.randn_bf16_bits((4, 64), 3)
    eye = _bits(np.eye(64))
    np.testing.assert_array_equal(O.linear(xi, eye, None, "reference"), O.bf16_bits_to_f32(xi))


def test_sumsq_partials_blocks():
    """Partials cover [256 j, 256 j + 256); the last block is ragged, and the partials add up
    to the row's sum of squares (the rms_norm statistic times N)."""
    y = np.ones((2, 600))
    np.testing.assert_array_equal(O.sumsq_partials(y), [[256, 256, 88]] * 2)
    r = np.random.default_rng(5).standard_normal((3, 4096))
    p = O.sumsq_partials(r)
    assert p.shape == (3, 16)
    np.testing.assert_allclose(p.sum(-1), (r * r).sum(-1), rtol=1e-12)
    np.testing.assert_allclose(p[:, 3], (r[:, 768:1024] ** 2).sum(-1), rtol=1e-12)
    # the statistic the norm derives from them
    np.testing.assert_allclose(O.rms_norm(r, np.ones(4096), 0.0, "exact"),
                               r / np.sqrt(p.sum(-1, keepdims=True) / 4096), rtol=1e-12)


def _module_weights(inner, K, heads, seed, gate=True, identity=False):
    rng = np.random.default_rng(seed)
    def w(n, k, scale):
        return O.f32_to_bf16_bits((rng.standard_normal((n, k)) * scale).astype(np.float32))
    ws = {}
    for name in ("to_q", "to_k", "to_v"):
        ws[name + ".weight"] = _bits(np.eye(inner, K)) if identity else w(inner, K, K ** -0.5)
        if not identity:
            ws[name + ".bias"] = w(1, inner, 0.1)[0]
    ws["q_norm.weight"] = w(1, inner, 0.2)[0] + 0 if not identity else _bits(np.ones(inner))
    ws["k_norm.weight"] = w(1, inner, 0.2)[0] if not identity else _bits(np.ones(inner))
    ws["to_out.0.weight"] = _bits(np.eye(K, inner)) if identity else w(K, inner, inner ** -0.5)
    if gate:
        ws["to_gate_logits.weight"] = w(heads, K, K ** -0.5)
        ws["to_gate_logits.bias"] = w(1, heads, 0.5)[0]
    return ws


def test_attention_module_reduces_to_the_core():
    """With identity projections and unit norm weights the module is the replaced unit on x
    itself; fully perturbed it returns v = x (DiTAttention.swift:351-356); a gate whose
    logits are 0 passes through and one of -30 silences its head (the logits are read off x,
    :387-391: they change with x, not with the attention output)."""
    B, L, H, D = 1, 5, 2, 8
    inner = H * D
    x = O.randn_bf16_bits((B, L, inner), 21)
    ws = _module_weights(inner, inner, H, 1, gate=False, identity=True)
    core = O.round_bf16(O.attention(x, x, x, H, q_norm_w=ws["q_norm.weight"],
                                    k_norm_w=ws["k_norm.weight"], mode="reference"))
    np.testing.assert_array_equal(O.attention_module(x, ws, H), core)
    np.testing.assert_array_equal(O.attention_module(x, ws, H, all_perturbed=True),
                                  O.bf16_bits_to_f32(x))
    gw = dict(ws)
    gw["to_gate_logits.weight"] = _bits(np.zeros((H, inner)))
    np.testing.assert_array_equal(O.attention_module(x, gw, H), core)
    gw["to_gate_logits.bias"] = _bits([-30.0, 0.0])
    got = O.attention_module(x, gw, H).reshape(B, L, H, D)
    assert np.all(np.abs(got[..., 0, :]) < 1e-11)          # 2*sigmoid(-30) ~ 1.9e-13
    np.testing.assert_array_equal(got[..., 1, :], core.reshape(B, L, H, D)[..., 1, :])


def test_attention_module_context_feeds_k_and_v_only():
    """Cross-attention: q from x, k and v from the context (:327, :341, :358-359). Swapping
    which stream feeds q changes the result; the output width is to_out's."""
    B, Lq, Lk, H, D, K = 1, 4, 6, 2, 8, 32
    inner = H * D
    x = O.randn_bf16_bits((B, Lq, K), 31)
    c = O.randn_bf16_bits((B, Lk, K), 32)
    ws = _module_weights(inner, K, H, 2)
    out = O.attention_module(x, ws, H, context_bits=c)
    assert out.shape == (B, Lq, K)
    q = O.f32_to_bf16_bits(O.linear(x, ws["to_q.weight"], ws["to_q.bias"], "reference"))
    k = O.f32_to_bf16_bits(O.linear(c, ws["to_k.weight"], ws["to_k.bias"], "reference"))
    v = O.f32_to_bf16_bits(O.linear(c, ws["to_v.weight"], ws["to_v.bias"], "reference"))
    o = O.round_bf16(O.attention(q, k, v, H, q_norm_w=ws["q_norm.weight"],
                                 k_norm_w=ws["k_norm.weight"], mode="reference"))
    g = O.head_gate(O.f32_to_bf16_bits(O.linear(x, ws["to_gate_logits.weight"],
                                                ws["to_gate_logits.bias"], "reference")),
                    "reference")
    o = O.round_bf16(o.reshape(B, Lq, H, D) * g[..., None]).reshape(B, Lq, inner)
    want = O.linear(O.f32_to_bf16_bits(o), ws["to_out.0.weight"], ws["to_out.0.bias"]
                    if "to_out.0.bias" in ws else None, "reference")
    np.testing.assert_array_equal(out, want)


# ---------------------------------------------------------------------------------------
# RMSNorm over the inner dim
# ---------------------------------------------------------------------------------------

def test_rms_norm_statistic_spans_all_heads():
    rng = np.random.default_rng(2)
    H, D = 4, 8
    x = rng.standard_normal((3, H * D))
    x[:, :D] *= 10.0                       # head 0 is much louder than the others
    w = np.ones(H * D)
    y = O.rms_norm(x, w, 1e-6, "exact")
    # RMS over the whole row is 1 ...
    np.testing.assert_allclose(np.sqrt(np.mean(y * y, axis=-1)), 1.0, rtol=1e-6)
    # ... and the heads keep their relative loudness (a per-head norm would flatten it)
    per_head = np.sqrt(np.mean(y.reshape(3, H, D) ** 2, axis=-1))
    assert np.all(per_head[:, 0] > 3 * per_head[:, 1])
    # scale invariance
    np.testing.assert_allclose(O.rms_norm(7.5 * x, w, 0.0, "exact"),
                               O.rms_norm(x, w, 0.0, "exact"), rtol=1e-12)
    # the weight is per inner channel
    w2 = np.arange(1, H * D + 1, dtype=np.float64)
    np.testing.assert_allclose(O.rms_norm(x, w2, 1e-6, "exact"), y * w2, rtol=1e-12)


def test_rms_norm_reference_mode_rounds_once_to_bf16():
    rng = np.random.default_rng(4)
    x = O.bf16_bits_to_f32(O.randn_bf16_bits((5, 256), 9))
    w = O.bf16_bits_to_f32(O.randn_bf16_bits((256,), 10, 1.0, 0.02))
    r = O.rms_norm(x, w, 1e-6, "reference")
    assert np.all(O.round_bf16(r) == r)   # representable in bf16
    e = O.rms_norm(x, w, 1e-6, "exact")
    assert np.max(np.abs(r - e) / np.maximum(np.abs(e), 1e-3)) <= 2.0 ** -8


# ---------------------------------------------------------------------------------------
# Split RoPE apply
# ---------------------------------------------------------------------------------------

def test_split_rope_convention_and_invariants():
    D = 8
    x = np.arange(1, D + 1, dtype=np.float64).reshape(1, 1, 1, D)
    ang = np.array([0.3, -1.1, 2.0, 0.7])
    c, s = np.cos(ang).reshape(1, 1, 4), np.sin(ang).reshape(1, 1, 4)
    y = O.split_rope(x, c, s, "exact")[0, 0, 0]
    # hand-written: pairs are (d, d + D/2), not adjacent channels
    x1, x2 = x[0, 0, 0, :4], x[0, 0, 0, 4:]
    np.testing.assert_allclose(y[:4], x1 * np.cos(ang) - x2 * np.sin(ang))
    np.testing.assert_allclose(y[4:], x2 * np.cos(ang) + x1 * np.sin(ang))
    assert abs(y[0] - (1 * math.cos(0.3) - 5 * math.sin(0.3))) < 1e-12
    # identity when cos = 1, sin = 0 (also what the video pad channels are)
    np.testing.assert_allclose(O.split_rope(x, np.ones((1, 1, 4)), np.zeros((1, 1, 4))), x)
    # per-pair norm preserved
    np.testing.assert_allclose(y[:4] ** 2 + y[4:] ** 2, x1 ** 2 + x2 ** 2)


def test_rope_relative_position_property():
    """<R_m q, R_n k> depends only on m - n for a single 1-D frequency."""
    rng = np.random.default_rng(8)
    D = 16
    q = rng.standard_normal(D)
    k = rng.standard_normal(D)
    f = rng.uniform(0.1, 2.0, D // 2)

    def rot(x, pos):
        a = f * pos
        return O.split_rope(x.reshape(1, 1, 1, D), np.cos(a).reshape(1, 1, -1),
                            np.sin(a).reshape(1, 1, -1))[0, 0, 0]

    d1 = rot(q, 5.0) @ rot(k, 2.0)
    d2 = rot(q, 13.0) @ rot(k, 10.0)
    assert abs(d1 - d2) < 1e-10
    assert abs(d1 - rot(q, 5.0) @ rot(k, 3.0)) > 1e-6


# ---------------------------------------------------------------------------------------
# RoPE tables against the reference's own digests (tiny_v5 manifest)
# ---------------------------------------------------------------------------------------

def _digests():
    with open(os.path.join(GOLDEN, "tiny_v5_rope_digests.json")) as fh:
        return json.load(fh)


def _stats(bits):
    x = O.bf16_bits_to_f32(bits).astype(np.float64)
    return x.mean(), x.std(ddof=1), x.min(), x.max()   # torch.std is unbiased


@pytest.mark.parametrize("table,tap,tol", [
    ("videoSelf", "block_00.attn1.in.kw_pe", 1e-9),
    ("videoCross", "block_00.audio_to_video_attn.in.kw_pe", 1e-9),
    ("audioSelf", "block_00.audio_attn1.in.kw_pe", 2e-6),
    ("audioCross", "block_00.video_to_audio_attn.in.kw_pe", 2e-6),
])
def test_rope_tables_match_reference_digests(table, tap, tol):
    """320x192x25 @ 24 fps: 240 video / 26 audio tokens. The reference reports its video
    tables bit-exact against upstream and the audio grid as needing a tolerance
    (docs/FRAGILE_CONTRACTS.md, the rotary paragraph); the same split holds here."""
    dig = _digests()
    tabs = O.rotaries(25, 192, 320, 24.0)
    cos, sin = tabs[table]
    for bits, key in ((cos, tap), (sin, tap + ".el1")):
        d = dig[key]
        assert list(bits.shape) == d["shape"][1:]
        mean, std, mn, mx = _stats(bits)
        assert abs(mean - d["mean"]) < tol, (key, mean, d["mean"])
        assert abs(std - d["std"]) < tol, (key, std, d["std"])
        assert mn == d["min"] and mx == d["max"]


def test_rope_table_structure():
    # frequency grid: first pi/2, last theta*pi/2 exactly (endpoint overwritten)
    f = O.frequency_grid(10000.0, 3, 4096)
    assert f.size == 682
    assert f[0] == np.float32(math.pi / 2) and f[-1] == np.float32(10000.0 * math.pi / 2)
    # video: 2 leading identity channels (3*682 = 2046 < 2048), in head 0 only
    cos, sin = O.rotaries(25, 192, 320)["videoSelf"]
    c0 = O.bf16_bits_to_f32(cos[0])
    s0 = O.bf16_bits_to_f32(sin[0])
    assert np.all(c0[:, :2] == 1.0) and np.all(s0[:, :2] == 0.0)
    assert not np.all(c0[:, 2] == 1.0)
    assert not np.all(O.bf16_bits_to_f32(cos[31])[:, -2:] == 1.0)
    # audio token bounds: [0, 0.01) then [0.01, 0.05) (DiTForward.swift:600-602)
    a = O.audio_positions(3)
    np.testing.assert_allclose(a[0, 0, 0], [0.0, 0.01], rtol=1e-6)
    np.testing.assert_allclose(a[0, 0, 1], [0.01, 0.05], rtol=1e-6)
    # video: first token's time bounds are [0, 1) pixel frames / fps
    v = O.video_positions(2, 1, 2)
    np.testing.assert_allclose(v[0, 0, 0], [0.0, np.float32(1.0) / np.float32(24.0)])
    np.testing.assert_allclose(v[0, 0, 2], [np.float32(1.0) / np.float32(24.0),
                                            np.float32(9.0) / np.float32(24.0)])
    np.testing.assert_allclose(v[0, 2, 1], [32.0, 64.0])   # x fastest, pixels


# ---------------------------------------------------------------------------------------
# The C restatement against the float64 restatement
# ---------------------------------------------------------------------------------------

@pytest.mark.parametrize("mode", ["exact", "reference"])
def test_c_oracle_matches_numpy_oracle(mode):
    B, H, Lq, Lk, D = 2, 4, 70, 90, 64
    q = O.randn_bf16_bits((B, Lq, H * D), 1)
    k = O.randn_bf16_bits((B, Lk, H * D), 2)
    v = O.randn_bf16_bits((B, Lk, H * D), 3)
    wq = O.randn_bf16_bits((H * D,), 4, 1.0, 0.02)
    wk = O.randn_bf16_bits((H * D,), 5, 1.0, 0.02)
    cq, sq = O.rotary_tables(O.audio_positions(Lq), H * D, [20], H)
    ck, sk = O.rotary_tables(O.audio_positions(Lk), H * D, [20], H)
    kw = dict(q_norm_w=wq, k_norm_w=wk, q_cos=cq, q_sin=sq, k_cos=ck, k_sin=sk,
              valid_len=[90, 33], mode=mode)
    ref = O.attention(q, k, v, H, **kw)
    got = O.c_attention(q, k, v, H, **kw).reshape(B, Lq, H * D)
    cmp = O.compare(got, ref)
    assert cmp["rel_rms"] < 2e-6 and cmp["max_abs"] < 1e-5
    # head / query subsets agree with the full call
    sub = O.c_attention(q, k, v, H, heads_range=(1, 3), q_range=(10, 40), **kw)
    np.testing.assert_allclose(sub, got.reshape(B, Lq, H, D)[:, 10:40, 1:3], atol=1e-6)


def test_reference_rounding_points_change_the_result():
    """The reference's bf16 roundings (after the norm, after each RoPE op) are visible: the
    two modes differ by more than fp32 noise but stay within a few bf16 ulps."""
    B, H, L, D = 1, 2, 40, 64
    q = O.randn_bf16_bits((B, L, H * D), 21)
    k = O.randn_bf16_bits((B, L, H * D), 22)
    v = O.randn_bf16_bits((B, L, H * D), 23)
    w = O.randn_bf16_bits((H * D,), 24, 1.0, 0.02)
    cq, sq = O.rotary_tables(O.audio_positions(L), H * D, [20], H)
    kw = dict(q_norm_w=w, k_norm_w=w, q_cos=cq, q_sin=sq)
    e = O.attention(q, k, v, H, mode="exact", **kw)
    r = O.attention(q, k, v, H, mode="reference", **kw)
    rel = O.compare(r, e)["rel_rms"]
    assert 1e-4 < rel < 1e-2


def test_golden_fixtures_reproduce():
    """The committed golden vectors are reproduced by the oracle (regression pin)."""
    path = os.path.join(GOLDEN, "fixtures.npz")
    data = np.load(path, allow_pickle=False)
    names = sorted({k.split("/")[0] for k in data.files})
    assert names, "no fixtures"
    for name in names:
        g = {k.split("/", 1)[1]: data[k] for k in data.files if k.startswith(name + "/")}
        meta = json.loads(str(g["meta"]))
        kw = {}
        for key in ("q_norm_w", "k_norm_w", "q_cos", "q_sin", "k_cos", "k_sin"):
            if key in g:
                kw[key] = g[key]
        if "valid_len" in g:
            kw["valid_len"] = g["valid_len"]
        out = O.attention(g["q"], g["k"], g["v"], meta["heads"], mode="exact", **kw)
        np.testing.assert_allclose(out.astype(np.float32), g["out_exact"], rtol=0, atol=1e-6,
                                   err_msg=name)


# ---------------------------------------------------------------------------------------
# Gemma-4 text-encoder attention (GemmaTextEncoder.swift:158-239, mask :288-321)
# ---------------------------------------------------------------------------------------

def test_gemma_inverse_frequencies_match_reference_goldens():
    """The reference's own expected values (Tests/LTXFoundationTests/
    GemmaAttentionSpecTests.swift:37-90), to its 1e-6 relative bound."""
    sl = O.gemma_inverse_frequencies(256, 1e4, 1.0, "default")
    assert sl.size == 128 and np.all(sl > 0)
    for i, want in ((0, 1.0), (1, 0.9305720329284668), (2, 0.8659643530845642),
                    (126, 0.00011547819303814322), (127, 0.00010746077896328643)):
        assert abs(sl[i] - want) / want < 1e-6, (i, sl[i])
    assert sl[1] == 1.0 / 10000.0 ** (1.0 / 128.0)
    fu = O.gemma_inverse_frequencies(512, 1e6, 0.25, "proportional")
    assert fu.size == 256 and np.count_nonzero(fu) == 64
    for i, want in ((0, 1.0), (1, 0.9474635124206543), (62, 0.03522694483399391),
                    (63, 0.03337624669075012)):
        assert abs(fu[i] - want) / want < 1e-6, (i, fu[i])
    assert np.all(fu[64:] == 0.0)
    # the default formula on a partial spec would divide by the rotated width: far off
    assert abs(1.0 / 1e6 ** (2.0 / 128.0) - fu[1]) > 0.1


def test_gemma_mask_rules():
    """Causal, window, left padding, and rows with no allowed key un-masked entirely
    (GemmaTextEncoder.swift:288-321), against a brute-force statement of each rule."""
    T = 12
    for window, fv in ((0, 0), (4, 0), (0, 5), (3, 5), (1, 0)):
        m = O.gemma_mask(T, window, fv)
        for q in range(T):
            allowed = [k <= q and (window == 0 or q - k < window) and k >= fv for k in range(T)]
            if not any(allowed):
                allowed = [True] * T
            assert list(m[q]) == allowed, (window, fv, q)
    # at T == window the sliding mask equals the causal one (the reference's coincidence)
    assert np.array_equal(O.gemma_mask(16, 16, 3), O.gemma_mask(16, 0, 3))


def _gemma_case(B, T, Hq, Hkv, D, seed, shared=False):
    q = O.randn_bf16_bits((B, T, Hq * D), seed)
    k = O.randn_bf16_bits((B, T, Hkv * D), seed + 1)
    v = k if shared else O.randn_bf16_bits((B, T, Hkv * D), seed + 2)
    wq = O.randn_bf16_bits((D,), seed + 3, mean=1.03, std=0.02)
    wk = O.randn_bf16_bits((D,), seed + 4, mean=0.12, std=0.01)
    inv = O.gemma_inverse_frequencies(D, 1e4, 1.0, "default")
    cos, sin = O.gemma_rope_tables(T, inv)
    return q, k, v, wq, wk, cos, sin


def test_gemma_attention_brute_force():
    """The vectorised oracle against a per-(query, key) loop with math.exp on a tiny case:
    per-head norms (pow(mean + eps, -0.5), weight; none on v), rotate_half RoPE, GQA by
    head // (Hq / Hkv), the mask, scale 1."""
    import math

    B, T, Hq, Hkv, D = 1, 7, 4, 2, 8
    q, k, v, wq, wk, cos, sin = _gemma_case(B, T, Hq, Hkv, D, 11)
    got = O.gemma_attention(q, k, v, Hq, Hkv, wq, wk, cos, sin, window=3,
                            first_valid=[2]).reshape(T, Hq, D)
    qf = O.bf16_bits_to_f32(q).astype(np.float64).reshape(T, Hq, D)
    kf = O.bf16_bits_to_f32(k).astype(np.float64).reshape(T, Hkv, D)
    vf = O.bf16_bits_to_f32(v).astype(np.float64).reshape(T, Hkv, D)
    wqf, wkf = (O.bf16_bits_to_f32(w).astype(np.float64) for w in (wq, wk))

    def norm(x, w):
        ms = sum(e * e for e in x) / len(x)
        return [e * (ms + 1e-6) ** -0.5 * (1.0 if w is None else w[i]) for i, e in enumerate(x)]

    def rope(x, t):
        h = D // 2
        return ([x[i] * cos[t, i] - x[i + h] * sin[t, i] for i in range(h)] +
                [x[i + h] * cos[t, i] + x[i] * sin[t, i] for i in range(h)])

    for h in range(Hq):
        kh = h // (Hq // Hkv)
        for t in range(T):
            qq = rope(norm(qf[t, h], wqf), t)
            keys = [kk for kk in range(T) if kk <= t and t - kk < 3 and kk >= 2] or list(range(T))
            logits = [sum(a * b for a, b in zip(qq, rope(norm(kf[kk, kh], wkf), kk)))
                      for kk in keys]
            mx = max(logits)
            w = [math.exp(x - mx) for x in logits]
            want = [sum(w[j] * norm(vf[kk, kh], None)[c] for j, kk in enumerate(keys)) / sum(w)
                    for c in range(D)]
            assert np.allclose(got[t, h], want, rtol=1e-9, atol=1e-12), (h, t)


def test_gemma_attention_invariants():
    """Future keys, keys past the window and padding keys do not reach a valid row; a
    padding row attends to every key unmasked; the K-shares-V layers take V from the
    PRE-norm K projection (so V differs from the finished K)."""
    B, T, Hq, Hkv, D = 1, 40, 2, 1, 16
    q, k, v, wq, wk, cos, sin = _gemma_case(B, T, Hq, Hkv, D, 21)
    base = O.gemma_attention(q, k, v, Hq, Hkv, wq, wk, cos, sin, window=8, first_valid=[5])
    k2, v2 = k.copy(), v.copy()
    k2[0, 30:] ^= 0x0040            # perturb keys/values after query 29
    v2[0, 30:] ^= 0x0040
    k2[0, :5] ^= 0x0040             # and the padding keys
    v2[0, :5] ^= 0x0040
    k2[0, 10:12] ^= 0x0040          # and keys more than 8 behind query 20
    v2[0, 10:12] ^= 0x0040
    alt = O.gemma_attention(q, k2, v2, Hq, Hkv, wq, wk, cos, sin, window=8, first_valid=[5])
    assert np.array_equal(base[0, 20:30], alt[0, 20:30])
    # a padding row == unmasked attention over all keys
    full = O.gemma_attention(q, k, v, Hq, Hkv, wq, wk, cos, sin, window=0, first_valid=[0])
    free = O.gemma_attention(q, k, v, Hq, Hkv, wq, wk, cos, sin, window=8, first_valid=[40])
    assert not np.allclose(full[0, 3], free[0, 3])          # causal vs all keys differ
    qq = O.gemma_attention(q, k, v, Hq, Hkv, wq, wk, cos, sin, window=0, first_valid=[5])
    # rows 0..4 of first_valid=5 equal rows of a call where every row is free
    assert np.allclose(qq[0, :5], free[0, :5], rtol=0, atol=0)
    # shared K/V: V is the weightless norm of the raw K projection, not of the finished K
    sh = O.gemma_attention(q, k, k, Hq, Hkv, wq, wk, cos, sin)
    assert not np.allclose(sh, O.gemma_attention(q, k, v, Hq, Hkv, wq, wk, cos, sin))


# ---------------------------------------------------------------------------------------
# The comparison metric and the reference bench's operand stream (Sources/ltx/Bench.swift)
# ---------------------------------------------------------------------------------------

def test_compare_hand_computed_cases():
    """BenchComparison (Bench.swift:508-536): relRMS = sqrt(sum (a-b)^2 / sum b^2) over the
    reference b, maxAbs, and the fraction of equal bf16 patterns -- on cases worked by hand,
    so a dropped square root (0.5), a denominator over the candidate (sqrt(1/5)) or a mean in
    place of a maximum fails."""
    c = O.compare([1.0, 2.0], [1.0, 1.0])
    assert c["rel_rms"] == math.sqrt(0.5)
    assert c["max_abs"] == 1.0
    assert c["bit_identical"] == 0.5
    assert c["elements"] == 2
    # the reference is the denominator: swapping the operands changes the figure
    assert O.compare([1.0, 1.0], [1.0, 2.0])["rel_rms"] == math.sqrt(1.0 / 5.0)
    # a uniform 1% error is exactly 1e-2, maxAbs is the largest single difference
    c = O.compare([1.01, -2.02, 0.0], [1.0, -2.0, 0.0])
    assert abs(c["rel_rms"] - 1e-2) < 1e-12 and abs(c["max_abs"] - 0.02) < 1e-12
    # sum b^2 == 0 (Bench.swift:532-534): 0 when the candidate is 0 too, else infinity
    assert O.compare([0.0, 0.0], [0.0, 0.0])["rel_rms"] == 0.0
    assert O.compare([0.0, 1e-3], [0.0, 0.0])["rel_rms"] == math.inf
    # "bit identical" is on the bf16 patterns: values rounding to one bf16 are identical
    c = O.compare([1.0 + 2.0 ** -10, 1.0 + 2.0 ** -6], [1.0, 1.0])
    assert c["bit_identical"] == 0.5


# The standard splitmix64 generator seeded with 0 (Vigna's published sequence, the one the
# xoshiro family seeds from): its first six outputs.
SPLITMIX64_SEED0 = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F,
                    0xF88BB8A8724C81EC, 0x1B39896A51A8749B, 0x53CB9F0C747EA2EA]


def test_splitmix64_stream_matches_published_values():
    """Bench.swift:479-490 advances its state before mixing from a state that already holds
    seed + gamma: its word i is the standard output i + 1. Seeding it with -gamma therefore
    gives the standard sequence of seed 0 from its first word."""
    mask = (1 << 64) - 1
    got = O.splitmix64(6, (-O.SPLITMIX_GAMMA) & mask)
    assert [int(x) for x in got] == SPLITMIX64_SEED0
    got = O.splitmix64(5, 0)
    assert [int(x) for x in got] == SPLITMIX64_SEED0[1:]


def test_splitmix_bf16_operands():
    """Words -> [-1, 1) -> bf16 (Bench.swift:488-491): the top 24 bits m give exactly
    (m - 2^23) / 2^23. Worked by hand for the first standard word: m = 0xE220A8 = 14819496,
    value 6430888 / 8388608 = 0.76662..., whose nearest bf16 (step 2^-8 in [0.5, 1)) is
    196 / 256 = 0.765625 = 0x3F44. The whole stream stays in [-1, 1) and is within half a
    bf16 step of its exact value."""
    mask = (1 << 64) - 1
    bits = O.splitmix_bf16_bits(6, (-O.SPLITMIX_GAMMA) & mask)
    assert int(bits[0]) == 0x3F44
    bits = O.splitmix_bf16_bits(4096, 0x5EED)
    vals = O.bf16_bits_to_f32(bits).astype(np.float64)
    exact = (O.splitmix64(4096, 0x5EED) >> np.uint64(40)).astype(np.float64) / 2.0 ** 23 - 1.0
    assert np.all(vals >= -1.0) and np.all(vals <= 1.0)
    half_step = np.exp2(np.floor(np.log2(np.maximum(np.abs(exact), 2.0 ** -126))) - 8)
    assert np.all(np.abs(vals - exact) <= half_step)
    assert abs(vals.mean()) < 0.05 and 0.5 < vals.std() < 0.65   # uniform: std 1/sqrt(3)
