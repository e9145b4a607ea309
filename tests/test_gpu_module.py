"""GPU parity of the whole attention module (``DiTAttentionModule``: projections with the RMS
statistic from the q / k epilogues, the fused attention, the gate and ``to_out``) against the
oracle's ``attention_module`` (``DiTAttention.swift:315-405``) on the same bf16 weights.

Truth: the oracle computing every operation in float64 between the reference's bf16 rounding
points (each projection's output, the attention output, the gated output). The module chains
five roundings to bf16 plus the reference's in-op roundings, so its bar is relative to the
reference's own arithmetic on the same inputs (the oracle's ``mode="reference"``): relative RMS
and max-abs error each at most 1.25x the reference's (floors 2.5e-3 and 2e-2, the attention
call's bar).
"""

import numpy as np
import pytest

import ltx_attn as L
import oracle as O

from test_gpu_parity import dev, host_f32

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _weights(q_dim, kv_dim, inner, out_dim, seed, gate=True, bias=True):
    rng = np.random.default_rng(seed)

    def w(shape, scale):
        return O.f32_to_bf16_bits((rng.standard_normal(shape) * scale).astype(np.float32))

    ws = {"to_q.weight": w((inner, q_dim), q_dim ** -0.5),
          "to_k.weight": w((inner, kv_dim), kv_dim ** -0.5),
          "to_v.weight": w((inner, kv_dim), kv_dim ** -0.5),
          "q_norm.weight": O.f32_to_bf16_bits((1.0 + 0.2 * rng.standard_normal(inner))
                                              .astype(np.float32)),
          "k_norm.weight": O.f32_to_bf16_bits((1.0 + 0.2 * rng.standard_normal(inner))
                                              .astype(np.float32)),
          "to_out.0.weight": w((out_dim, inner), inner ** -0.5)}
    if bias:
        for n in ("to_q", "to_k", "to_v", "to_out.0"):
            ws[n + ".bias"] = w((ws[n + ".weight"].shape[0],), 0.1)
    if gate:
        ws["to_gate_logits.weight"] = w((32, q_dim), q_dim ** -0.5)
        ws["to_gate_logits.bias"] = w((32,), 0.5)
    return ws


def _tables(H, L, D, seed):
    ang = np.random.default_rng(seed).uniform(-3, 3, (H, L, D // 2))
    return (O.f32_to_bf16_bits(np.cos(ang).astype(np.float32)),
            O.f32_to_bf16_bits(np.sin(ang).astype(np.float32)))


CASES = {
    # name: (B, Lq, Lk, query width, context width (None = self), inner, rotary, key rotary,
    #        key lengths, perturbed)
    "self": (2, 300, 300, 2048, None, 2048, True, False, None, False),
    "self_perturbed": (2, 300, 300, 2048, None, 2048, True, False, None, True),
    "text_cross_cfg": (2, 300, 128, 2048, 2048, 2048, False, False, (94, 11), False),
    "audio_to_video": (1, 520, 152, 4096, 2048, 2048, True, True, None, False),
}


@pytest.mark.parametrize("name", list(CASES))
def test_module_matches_oracle(device, name):
    import torch

    B, Lq, Lk, qd, kd, inner, rot, krot, valid, perturbed = CASES[name]
    H, D = 32, inner // 32
    out_dim = qd
    ws = _weights(qd, kd or qd, inner, out_dim, 7)
    x = O.randn_bf16_bits((B, Lq, qd), 11)
    ctx = None if kd is None else O.randn_bf16_bits((B, Lk, kd), 12)
    qc = qs = kc = ks = None
    if rot:
        qc, qs = _tables(H, Lq, D, 13)
    if krot:
        kc, ks = _tables(H, Lk, D, 14)
    _say(f"module {name}: B={B} Lq={Lq} Lk={Lk} inner={inner}")
    m = L.DiTAttentionModule({k: dev(v, device) for k, v in ws.items()})
    variant = {"self": L.Variant.videoSelf, "self_perturbed": L.Variant.videoSelf,
               "text_cross_cfg": L.Variant.videoCross,
               "audio_to_video": L.Variant.audioToVideo}[name]
    out = m(dev(x, device), None if ctx is None else dev(ctx, device), variant=variant,
            rotary=None if qc is None else L.Rotary(dev(qc, device), dev(qs, device)),
            key_rotary=None if kc is None else L.Rotary(dev(kc, device), dev(ks, device)),
            k_valid_len=valid, all_perturbed=perturbed)
    torch.cuda.synchronize()
    got = host_f32(out)
    kw = dict(context_bits=ctx, q_cos=qc, q_sin=qs, k_cos=kc, k_sin=ks, valid_len=valid,
              all_perturbed=perturbed)
    truth = O.attention_module(x, ws, H, mode="exact", **kw)
    ref = O.attention_module(x, ws, H, mode="reference", **kw)
    assert got.shape == (B, Lq, out_dim)
    c, r = O.compare(got, truth), O.compare(ref, truth)
    _say(f"  {name}: relRMS {c['rel_rms']:.3e} (reference {r['rel_rms']:.3e}), maxAbs "
         f"{c['max_abs']:.3e} (reference {r['max_abs']:.3e})")
    assert c["rel_rms"] <= 1.25 * max(r["rel_rms"], 2.5e-3), (name, c, r)
    assert c["max_abs"] <= 1.25 * max(r["max_abs"], 2e-2), (name, c, r)
