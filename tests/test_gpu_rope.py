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
