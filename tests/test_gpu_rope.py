"""The GPU RoPE table builder (ltx_rope_tables_device) against the host builder, which the
CPU suite pins to the oracle and to the reference's own table digests: the same bf16 bits for
every table the model builds at the reference's test geometry and at the benchmark's two video
shapes, and the digests again through the GPU tables."""
import json
import os

import numpy as np
import pytest

import ltx_attn as L
import oracle as O

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _bits(t):
    import torch

    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("geometry", [
    (25, 192, 320, None),        # tiny_v5: 240 video / 26 audio tokens
    (97, 768, 1280, None),       # stage 2, 12480 video tokens
    (121, 768, 1280, 152),       # the block set: 15360 video / 152 audio tokens
])
def test_device_tables_equal_host_tables(device, geometry):
    import torch

    frames, h, w, audio = geometry
    print(f"rope tables {frames}x{h}x{w}", flush=True)
    dev_t = L.rotaries_device(frames, h, w, audio_tokens=audio)
    host_t = L.rotaries(frames, h, w, audio_tokens=audio)
    torch.cuda.synchronize()
    for name, (hc, hs) in host_t.items():
        r = dev_t[name]
        for got, want, part in ((_bits(r.cos), hc, "cos"), (_bits(r.sin), hs, "sin")):
            assert got.shape == want.shape, (name, part)
            diff = int(np.count_nonzero(got != want))
            assert diff == 0, (name, part, diff, got.size)


def test_device_tables_match_reference_digests(device):
    import torch

    with open(os.path.join(GOLDEN, "tiny_v5_rope_digests.json")) as fh:
        dig = json.load(fh)
    tabs = L.rotaries_device(25, 192, 320)
    torch.cuda.synchronize()
    for table, tap, tol in (("videoSelf", "block_00.attn1.in.kw_pe", 1e-9),
                            ("videoCross", "block_00.audio_to_video_attn.in.kw_pe", 1e-9),
                            ("audioSelf", "block_00.audio_attn1.in.kw_pe", 2e-6),
                            ("audioCross", "block_00.video_to_audio_attn.in.kw_pe", 2e-6)):
        r = tabs[table]
        for t, key in ((r.cos, tap), (r.sin, tap + ".el1")):
            x = O.bf16_bits_to_f32(_bits(t)).astype(np.float64)
            assert abs(x.mean() - dig[key]["mean"]) < tol, key
            assert abs(x.std(ddof=1) - dig[key]["std"]) < tol, key


def test_attention_with_device_tables(device):
    """The tables feed the attention call directly (no host round trip): same output as with
    the host tables uploaded."""
    import torch

    H, D = 32, 128
    dev_t = L.rotaries_device(25, 192, 320)
    host_t = L.rotaries(25, 192, 320)
    T = host_t["videoSelf"][0].shape[1]
    g = torch.Generator(device=device)
    g.manual_seed(0x5EED + 90)
    q, k, v = (torch.randn((1, T, H * D), generator=g, device=device).to(torch.bfloat16)
               for _ in range(3))
    up = [torch.from_numpy(x.view(np.int16)).to(device).view(torch.bfloat16)
          for x in host_t["videoSelf"]]
    a = L.attention_fwd(q, k, v, heads=H, rotary=dev_t["videoSelf"])
    b = L.attention_fwd(q, k, v, heads=H, rotary=L.Rotary(up[0], up[1]))
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_attention_over_a_reference_lengthened_stream(device):
    """The stage-2 upscaler's stream with an IC-LoRA reference (VideoUpscaler.swift:808-812;
    positions DiTForward.swift:553-593, :707-711) and two Multiple-Subject-Reference slots:
    3120 target tokens (13 x 12 x 20), a half-resolution reference of 13 x 6 x 10 (downscale 2)
    and two one-frame slots at -2 and -1 pixel frames: 4380 tokens. The device builder's video
    tables equal the oracle's (its own positions, its own table recipe), and the self-attention
    with norm + 3-D RoPE over the lengthened stream matches the C oracle over every head and
    row, to the stated tolerance. The device tables equal the host builder's bit for bit; the
    host positions equal the oracle's bit for bit (its tables may differ from the host's by a
    rare bf16 step: its cos/sin are numpy's float32 ones)."""
    import torch

    from test_gpu_parity import _gpu_bits, check_heads

    H, D = 32, 128
    refs = [L.Reference(13, 6, 10, downscale_factor=2)] + L.msr_slots(2, 1, 12, 20)
    tabs = L.rotaries_device(97, 384, 640, references=refs)
    torch.cuda.synchronize()
    pos = O.video_positions_with_references(
        13, 12, 20, [dict(latent_frames=13, latent_height=6, latent_width=10,
                          downscale_factor=2)] +
        [dict(latent_frames=1, latent_height=12, latent_width=20, frame_offset=-(2 - i))
         for i in range(2)], 24.0)
    host_pos = L.rope_video_positions_with_references(13, 12, 20, refs)
    assert np.array_equal(host_pos.view(np.uint32), pos[0].view(np.uint32))
    host_cos, host_sin = L.rope_tables(host_pos, H * D, [20, 2048, 2048], H)
    assert np.array_equal(_bits(tabs["videoSelf"].cos), host_cos)
    assert np.array_equal(_bits(tabs["videoSelf"].sin), host_sin)
    cos, sin = O.rotary_tables(pos, H * D, [20, 2048, 2048], H)
    T = cos.shape[1]
    print(f"reference-lengthened stream: {T} video tokens", flush=True)
    assert T == 3120 + 780 + 2 * 240
    seed = 0x5EED + 600
    tq, qb = _gpu_bits((1, T, H * D), seed, device)
    tk, kb = _gpu_bits((1, T, H * D), seed + 1, device)
    tv, vb = _gpu_bits((1, T, H * D), seed + 2, device)
    wq, wqb = _gpu_bits((H * D,), seed + 3, device, 1.0, 0.02)
    wk, wkb = _gpu_bits((H * D,), seed + 4, device, 1.0, 0.02)
    out = L.attention_fwd(tq, tk, tv, heads=H, q_norm_w=wq, k_norm_w=wk,
                          rotary=tabs["videoSelf"])
    torch.cuda.synchronize()
    kw = dict(q_norm_w=wqb, k_norm_w=wkb, q_cos=cos, q_sin=sin)
    truth = O.c_attention(qb, kb, vb, H, mode="exact", **kw)
    refm = O.round_bf16(O.c_attention(qb, kb, vb, H, mode="reference", **kw))
    got = O.bf16_bits_to_f32(_bits(out)).reshape(truth.shape)
    check_heads(got, truth, refm, "reference-lengthened self-attention")
