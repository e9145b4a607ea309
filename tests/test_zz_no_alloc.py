"""ltx_attn_fwd_static: the attention entry point that allocates nothing (its scratch is the
library's per-device static array), called through the C ABI.

GPU: two calls in a row, the second smaller, each bit-identical to ltx_attn_fwd with a
caller-provided workspace on the same arguments (same plan, same kernels), and the smaller one
also within the stated tolerance of the oracle; then the first call again, to show that what
the array kept from a previous call changes nothing. CPU: refusals that happen on the host
before any device work (oversized plans, invalid arguments).
"""

import ctypes

import numpy as np
import pytest

import ltx_attn as L
import oracle as O

FAKE = 0x7F0000000000


def _say(msg):
    print(msg, flush=True)


def _fake_args(B, H, Lq, Lk, D, norm=False, rope=False):
    a = L.Args()
    L.load_library().ltx_attn_args_init(ctypes.byref(a))
    a.B, a.H, a.Lq, a.Lk, a.D = B, H, Lq, Lk, D
    inner = H * D
    a.q, a.k, a.v, a.out = FAKE, FAKE + (1 << 36), FAKE + (2 << 36), FAKE + (3 << 36)
    a.q_bs, a.q_rs, a.q_hs = Lq * inner, inner, D
    a.k_bs, a.k_rs, a.k_hs = Lk * inner, inner, D
    a.v_bs, a.v_rs, a.v_hs = Lk * inner, inner, D
    a.o_bs, a.o_rs, a.o_hs = Lq * inner, inner, D
    a.scale = D ** -0.5
    if norm:
        a.q_norm_w, a.k_norm_w = FAKE + (4 << 36), FAKE + (5 << 36)
    if rope:
        a.q_cos = a.q_sin = FAKE + (6 << 36)
    return a


def test_static_entry_refuses_oversized_plans_on_the_host():
    """The 2 x 15360-token video self-attention with norm + RoPE needs 240 MiB (prepared K and
    statistics): more than the static scratch holds, refused before any device work, with the
    sizes in the detail. The same call with the K staging fused (no prepared K) fits."""
    lib = L.load_library()
    a = _fake_args(2, 32, 15360, 15360, 128, norm=True, rope=True)
    need = lib.ltx_attn_workspace_bytes(ctypes.byref(a))
    assert need > L.STATIC_SCRATCH_BYTES
    assert lib.ltx_attn_fwd_static(ctypes.byref(a), None) == L.EUNSUPPORTED
    detail = lib.ltx_attn_last_error().decode()
    assert str(need) in detail and str(L.STATIC_SCRATCH_BYTES) in detail
    a.kprep, a.num_splits = L.KPREP_FUSED, 1
    assert 0 < lib.ltx_attn_workspace_bytes(ctypes.byref(a)) <= L.STATIC_SCRATCH_BYTES


def test_static_entry_validates_like_ltx_attn_fwd():
    lib = L.load_library()
    assert lib.ltx_attn_fwd_static(None, None) == L.EINVAL
    a = _fake_args(1, 32, 100, 100, 96)
    assert lib.ltx_attn_fwd_static(ctypes.byref(a), None) == L.EUNSUPPORTED
    a = _fake_args(1, 32, 100, 100, 128)
    a.scale = -1.0
    assert lib.ltx_attn_fwd_static(ctypes.byref(a), None) == L.EINVAL


def _call(device, q, k, v, H, wq, wk, rot, no_alloc):
    import torch

    out = L.attention_fwd(q, k, v, heads=H, q_norm_w=wq, k_norm_w=wk, rotary=rot,
                          no_alloc=no_alloc)
    torch.cuda.synchronize()
    return out.view(torch.int16).cpu().numpy().view(np.uint16)


def _inputs(device, B, H, T, D, seed):
    import torch

    def t(shape, s, mean=0.0, std=1.0):
        g = torch.Generator(device=device)
        g.manual_seed(s)
        return (torch.randn(shape, generator=g, device=device) * std + mean).to(torch.bfloat16)

    q, k, v = (t((B, T, H * D), seed + i) for i in range(3))
    wq, wk = t((H * D,), seed + 3, 1.0, 0.02), t((H * D,), seed + 4, 1.0, 0.02)
    cos, sin = L.rope_tables(L.rope_audio_positions(T), H * D, [20], H)
    to_dev = lambda b: torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).to(  # noqa: E731
        device).view(torch.bfloat16)
    rot = L.Rotary(to_dev(cos), to_dev(sin))
    return q, k, v, wq, wk, rot, (cos, sin)


@pytest.mark.gpu
def test_static_entry_matches_the_workspace_entry(device):
    import torch

    def bits(t):
        return t.view(torch.int16).cpu().numpy().view(np.uint16)

    # 1: 2 x 2100 tokens, 32 heads of 128, norm + RoPE: the statistics, the K prologue's
    #    prepared K and the split-KV partials of the last round's 64 items fill most of it
    big = (2, 32, 2100, 128)
    q, k, v, wq, wk, rot, _ = _inputs(device, *big, 0x5EED + 700)
    lib = L.load_library()
    need = lib.ltx_attn_workspace_bytes(
        ctypes.byref(_fake_args(2, 32, 2100, 2100, 128, norm=True, rope=True)))
    _say(f"no-alloc call 1: B,H,T,D = {big}, scratch {need} of {L.STATIC_SCRATCH_BYTES} bytes")
    assert need > L.STATIC_SCRATCH_BYTES // 2
    want1 = _call(device, q, k, v, 32, wq, wk, rot, False)
    got1 = _call(device, q, k, v, 32, wq, wk, rot, True)
    assert np.array_equal(got1, want1)

    # 2: smaller (8 heads of 64, 700 tokens): a different plan over the same array
    small = (2, 8, 700, 64)
    _say(f"no-alloc call 2: B,H,T,D = {small}")
    q2, k2, v2, wq2, wk2, rot2, (cos2, sin2) = _inputs(device, *small, 0x5EED + 710)
    want2 = _call(device, q2, k2, v2, 8, wq2, wk2, rot2, False)
    got2 = _call(device, q2, k2, v2, 8, wq2, wk2, rot2, True)
    assert np.array_equal(got2, want2)
    truth = O.attention(bits(q2), bits(k2), bits(v2), 8, q_norm_w=bits(wq2), k_norm_w=bits(wk2),
                        q_cos=cos2, q_sin=sin2, mode="exact")
    c = O.compare(O.bf16_bits_to_f32(got2), truth)
    _say(f"  call 2 vs oracle: relRMS {c['rel_rms']:.3e} maxAbs {c['max_abs']:.3e}")
    assert c["rel_rms"] <= 5e-3 and c["max_abs"] <= 2e-2

    # 3: the first call again, over what call 2 left in the array
    _say("no-alloc call 3: call 1 repeated")
    assert np.array_equal(_call(device, q, k, v, 32, wq, wk, rot, True), want1)
