#!/usr/bin/env python3
"""Benchmark of the fused DiT attention path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1]

One step = one ``ltx_attn_fwd`` call (QK-RMSNorm statistic, K prologue, attention) on the
workload the headline metric is quoted on: stage-2 video self-attention at 1280x768x97
(latent 13x24x40 -> 12480 tokens), H=32, D=128, pre-norm bf16 Q/K/V [1, 12480, 4096] ~ N(0,1),
q/k norm weights ~ N(1, 0.02), 3-D RoPE tables from the reference's position recipe. FLOPs use
the reference's convention 4*Sq*Skv*H*D (Sources/ltx/BenchGEMM.swift:154-159).

Prints ONE JSON line. ``roofline`` is for the dominant kernel (the attention kernel itself),
timed with HIP events recorded by the library around that kernel on the call's stream.
``cpu_baseline`` times the C restatement of the reference's explicit fp32 path on a bounded
sample of the same workload, on this host's cores. ``secondary`` holds the other two figures
the metric names (3120-token self-attention TFLOP/s and ms per DiT-block attention set) and
the projection GEMM / whole-module figures at the 12480-token shapes.
"""

import argparse
import ctypes
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "ltx-2.5-swift_amd"), os.path.join(ROOT, "oracle")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "attention TFLOP/s + % bf16 MFMA peak at 3120/12480 tokens; ms per DiT-block attn"
PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_attn_c4.json")
# The sources the dominant kernel is built from: a traffic figure counted on another version
# of them is stale and not reported.
KERNEL_SOURCES = [os.path.join(ROOT, "ltx-2.5-swift_amd", "csrc", f) for f in
                  ("fmha_dma.hip", "fmha_device.hpp", "lds_copy.hpp", "mfma_s.hpp",
                   "fmha_params.hpp", "ltx_attn_abi.cpp")]


def kernel_source_sha256():
    import hashlib

    h = hashlib.sha256()
    for path in KERNEL_SOURCES:
        with open(path, "rb") as fh:
            h.update(os.path.basename(path).encode() + b"\0" + fh.read())
    return h.hexdigest()


class HipEvents:
    """hipEvent_t handles through the HIP runtime's C API (the library records them)."""

    def __init__(self):
        self.rt = ctypes.CDLL("libamdhip64.so")
        self.rt.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.rt.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float),
                                                ctypes.c_void_p, ctypes.c_void_p]
        self.rt.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.rt.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def create(self):
        ev = ctypes.c_void_p()
        if self.rt.hipEventCreate(ctypes.byref(ev)) != 0:
            raise RuntimeError("hipEventCreate failed")
        return ev

    def elapsed_ms(self, a, b):
        self.rt.hipEventSynchronize(b)
        ms = ctypes.c_float()
        if self.rt.hipEventElapsedTime(ctypes.byref(ms), a, b) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value

    def destroy(self, ev):
        self.rt.hipEventDestroy(ev)


def _randn(shape, seed, device, mean=0.0, std=1.0):
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(seed)
    t = torch.randn(shape, generator=g, device=device, dtype=torch.float32) * std + mean
    return t.to(torch.bfloat16)


def _dev_bits(bits, device):
    import numpy as np
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(device).view(
        torch.bfloat16)


def _host_bits(t):
    import numpy as np
    import torch

    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def c4_inputs(device):
    import ltx_attn as L

    H, D, T = 32, 128, 12480
    q = _randn((1, T, H * D), 0x5EED, device)
    k = _randn((1, T, H * D), 0x5EED + 1, device)
    v = _randn((1, T, H * D), 0x5EED + 2, device)
    wq = _randn((H * D,), 0x5EED + 3, device, 1.0, 0.02)
    wk = _randn((H * D,), 0x5EED + 4, device, 1.0, 0.02)
    cos, sin = L.rope_tables(L.rope_video_positions(13, 24, 40), H * D, [20, 2048, 2048], H)
    return dict(q=q, k=k, v=v, wq=wq, wk=wk, cos=cos, sin=sin, H=H, D=D, T=T,
                rot=L.Rotary(_dev_bits(cos, device), _dev_bits(sin, device)))


def time_steps(call, steps, warmup, hip, events_per_step=True):
    """Warmup, then exactly `steps` timed calls bracketed by synchronisation.
    Returns (wall seconds, list of attention-kernel ms from the library's event hook)."""
    import torch

    for _ in range(warmup):
        call(None)
    torch.cuda.synchronize()
    evs = [(hip.create(), hip.create()) for _ in range(steps)] if events_per_step else []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        call(evs[i] if evs else None)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kms = [hip.elapsed_ms(a, b) for a, b in evs]
    for a, b in evs:
        hip.destroy(a)
        hip.destroy(b)
    return wall, kms


def stats(samples_ms):
    """Median, min, max and spread (max - min) / median of per-call times, the reference's
    timing summary (Sources/ltx/Bench.swift:123-152)."""
    xs = sorted(samples_ms)
    n = len(xs)
    med = xs[n // 2] if n % 2 else 0.5 * (xs[n // 2 - 1] + xs[n // 2])
    return {"median_ms": round(med, 4), "min_ms": round(xs[0], 4), "max_ms": round(xs[-1], 4),
            "spread": round((xs[-1] - xs[0]) / med, 4) if med > 0 else None, "samples": n}


def per_call_ms(call, steps, hip, stream=None):
    """Each call's own time: HIP events recorded on the call's stream before and after it
    (a separate run from the aggregate timing, which records nothing between calls)."""
    import torch

    st = stream if stream is not None else torch.cuda.current_stream().cuda_stream
    rt = hip.rt
    rt.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    evs = [(hip.create(), hip.create()) for _ in range(steps)]
    torch.cuda.synchronize()
    for a, b in evs:
        rt.hipEventRecord(a, ctypes.c_void_p(st))
        call(None)
        rt.hipEventRecord(b, ctypes.c_void_p(st))
    torch.cuda.synchronize()
    ms = [hip.elapsed_ms(a, b) for a, b in evs]
    for a, b in evs:
        hip.destroy(a)
        hip.destroy(b)
    return ms


def settle(call, seconds):
    """Run `call` untimed for `seconds` of wall time: on a fresh MI355X the kernel's duration
    falls by about a quarter over its first ~25 launches (the clock ramps up under load) and
    holds after that. Returns the number of calls made."""
    import torch

    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        call(None)
        n += 1
        if n % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return n


def bench_c4(device, steps, warmup, hip, settle_s=0.0):
    import torch

    import ltx_attn as L

    x = c4_inputs(device)
    H, D, T = x["H"], x["D"], x["T"]
    out = torch.empty_like(x["q"])
    ws = torch.empty(512 << 20, dtype=torch.uint8, device=device)

    def call(ev):
        L.attention_fwd(x["q"], x["k"], x["v"], heads=H, q_norm_w=x["wq"], k_norm_w=x["wk"],
                        rotary=x["rot"], out=out, workspace=ws,
                        events=None if ev is None else (ev[0], ev[1]))

    # The whole-call figure is timed without the kernel's event records (each adds a few
    # microseconds between launches); the kernel's own duration comes from a second, equally
    # long run with them.
    settle(call, settle_s)
    wall, _ = time_steps(call, steps, warmup, hip, events_per_step=False)
    _, kms = time_steps(call, steps, 0, hip)
    cms = per_call_ms(call, steps, hip)
    flops = 4.0 * T * T * H * D
    return x, {
        "flops": flops, "wall_s": wall, "ms_per_step": wall / steps * 1e3,
        "tflops": flops * steps / wall / 1e12,
        "kernel_ms": sum(kms) / len(kms), "kernel_stats": stats(kms), "call_stats": stats(cms),
        "kernel_tflops": flops / (sum(kms) / len(kms) * 1e-3) / 1e12,
        "bytes": 4.0 * T * H * D * 2,
    }


def bench_c1(device, steps, warmup, hip):
    import torch

    import ltx_attn as L

    H, D, T = 32, 128, 3120
    q = _randn((1, T, H * D), 0x5EED + 10, device)
    k = _randn((1, T, H * D), 0x5EED + 11, device)
    v = _randn((1, T, H * D), 0x5EED + 12, device)
    out = torch.empty_like(q)

    def call(ev):
        L.attention_fwd(q, k, v, heads=H, out=out,
                        events=None if ev is None else (ev[0], ev[1]))

    wall, _ = time_steps(call, steps, warmup, hip, events_per_step=False)
    _, kms = time_steps(call, steps, 0, hip)
    cms = per_call_ms(call, steps, hip)
    flops = 4.0 * T * T * H * D
    km = sum(kms) / len(kms)
    return {"tflops": flops * steps / wall / 1e12, "ms_per_call": wall / steps * 1e3,
            "kernel_ms": km, "kernel_tflops": flops / (km * 1e-3) / 1e12,
            "pct_peak": 100.0 * flops / (km * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
            "kernel_stats": stats(kms), "call_stats": stats(cms)}


def bench_short_keys(device, steps, warmup, hip, block=True):
    """The HBM-bound calls at 640x384x97: text cross-attention (3120 video queries over 1024
    text keys, 94 valid; and the CFG pair at B=2 with 94 and 1 valid), and the cross-modal
    pair of a 4 s clip at D=64 with 1-D temporal RoPE (frame index 0..12 for the 3120 video
    tokens, 0..125 for the 126 audio tokens): video queries over audio K/V and audio queries
    over video K/V. Per call: the attention kernel's time (events the library records around
    it), the whole call's, the algorithmic bytes (Q, valid K and V, tables, O, once each) and
    the kernel's GB/s."""
    import numpy as np
    import torch

    import ltx_attn as L

    H = 32
    ws = torch.empty(64 << 20, dtype=torch.uint8, device=device)
    res = {}

    def measure(name, q, k, v, bytes_, flops, **kw):
        out = torch.empty_like(q)

        def call(ev):
            L.attention_fwd(q, k, v, heads=H, out=out, workspace=ws,
                            events=None if ev is None else (ev[0], ev[1]), **kw)

        wall, _ = time_steps(call, steps, warmup, hip, events_per_step=False)
        _, kms = time_steps(call, steps, 0, hip)
        km = sum(kms) / len(kms)
        res[name] = {"kernel_ms": round(km, 4), "call_ms": round(wall / steps * 1e3, 4),
                     "bytes": int(bytes_), "kernel_gbs": round(bytes_ / (km * 1e-3) / 1e9, 1),
                     "pct_hbm_peak": round(100 * bytes_ / (km * 1e-3) / 1e9 / PEAK_HBM_GBS, 2),
                     "gflop": round(flops / 1e9, 3)}

    Tv, Tt = 3120, 1024
    for B, valid in ((1, [94]), (2, [94, 1])):
        q = _randn((B, Tv, H * 128), 0x5EED + 20, device)
        k = _randn((B, Tt, H * 128), 0x5EED + 21, device)
        v = _randn((B, Tt, H * 128), 0x5EED + 22, device)
        nk = sum(valid)
        measure(f"text_cross_3120_B{B}", q, k, v, 2 * (2 * B * Tv + 2 * nk) * H * 128,
                4.0 * Tv * nk * H * 128, k_valid_len=valid)

    Ta, D = 126, 64
    inner = H * D

    def index_tables(idx):
        pos = np.zeros((1, len(idx), 2), dtype=np.float32)     # [n_pos, tokens, (start, end)]
        pos[0, :, 0] = idx
        pos[0, :, 1] = idx
        c, s_ = L.rope_tables(pos, inner, [20], H)
        return L.Rotary(_dev_bits(c, device), _dev_bits(s_, device))

    rv = index_tables(np.arange(Tv) // (20 * 12))
    ra = index_tables(np.arange(Ta))
    xv = _randn((1, Tv, inner), 0x5EED + 23, device)
    xa = _randn((1, Ta, inner), 0x5EED + 24, device)
    ya = _randn((1, Ta, inner), 0x5EED + 25, device)
    yv = _randn((1, Tv, inner), 0x5EED + 26, device)
    per_tok = 2 * inner          # one bf16 row of a stream, or its cos + sin table rows
    measure("cross_modal_video_q_3120x126", xv, xa, ya,
            (2 * Tv + 2 * Ta) * per_tok + (Tv + Ta) * per_tok, 4.0 * Tv * Ta * inner,
            rotary=rv, key_rotary=ra)
    measure("cross_modal_audio_q_126x3120", xa, xv, yv,
            (2 * Ta + 2 * Tv) * per_tok + (Tv + Ta) * per_tok, 4.0 * Tv * Ta * inner,
            rotary=ra, key_rotary=rv)
    if not block:
        return res

    # The block set's two large short-key calls at 1280x768x121, B=2: video->text over 94 of
    # 1024 text keys (norm on both sides) and video queries over the 152 audio keys (norm +
    # temporal RoPE); bytes are the attention kernel's own (the statistic and K passes are
    # separate launches).
    # Q, K and V are separate draws and q_norm / k_norm separate weights (separate seeds per
    # operand, as BenchGEMM.swift:627-632 draws them), as the module's projections are.
    B, Tv, Ta = 2, 15360, 152
    tabs = L.rotaries(121, 768, 1280, audio_tokens=Ta)
    rvc = L.Rotary(*(_dev_bits(t, device) for t in tabs["videoCross"]))
    rac = L.Rotary(*(_dev_bits(t, device) for t in tabs["audioCross"]))
    wq4, wk4 = (_randn((4096,), 0x5EED + 100 + i, device, 1.0, 0.02) for i in range(2))
    wq2, wk2 = (_randn((2048,), 0x5EED + 102 + i, device, 1.0, 0.02) for i in range(2))
    qv = _randn((B, Tv, 4096), 0x5EED + 50, device)
    kt = _randn((B, 1024, 4096), 0x5EED + 70, device)
    vt = _randn((B, 1024, 4096), 0x5EED + 71, device)
    measure("block_text_cross_15360_B2", qv, kt, vt, 2 * (2 * B * Tv + 2 * 188) * 4096,
            4.0 * B * Tv * 94 * 4096, q_norm_w=wq4, k_norm_w=wk4, k_valid_len=[94, 94])
    del qv, kt, vt
    qv2 = _randn((B, Tv, 2048), 0x5EED + 90, device)
    ka = _randn((B, Ta, 2048), 0x5EED + 60, device)
    va = _randn((B, Ta, 2048), 0x5EED + 61, device)
    measure("block_video_q_15360x152_B2", qv2, ka, va,
            2 * (2 * B * Tv + 2 * B * Ta) * 2048 + 2 * (Tv + Ta) * 2048,
            4.0 * B * Tv * Ta * 2048, q_norm_w=wq2, k_norm_w=wk2, rotary=rvc, key_rotary=rac)
    return res


def bench_text_cross_unmasked(device, steps, warmup, hip):
    """The text cross-attention as the DiT runs it: every one of the 1024 text tokens
    attended, no mask (DiTForward.swift:38-42 passes none; DiTAttention.swift:374-376 runs
    mask: .none). The reference bench's attn2 / audio_attn2 cases at the production shape
    (BenchGEMM.swift:478-484: B = 1, raw SDPA, 3120 video / 126 audio queries over 1024 keys),
    and the block set's pair at 1280x768x121 with CFG (B = 2, 2 x 15360 video and 2 x 152
    audio queries, q / k norm over the inner dim). Q, K, V separate draws. Per call: the
    attention kernel's median time over `steps` calls (events the library records around it),
    the whole call's, TFLOP/s (4 * Sq * Skv * H * D) and % of the dense bf16 peak."""
    import torch

    import ltx_attn as L

    H, Tt = 32, 1024
    ws = torch.empty(256 << 20, dtype=torch.uint8, device=device)
    res = {}
    cases = (("attn2_3120x1024_B1", 1, 3120, 4096, False, 200),
             ("audio_attn2_126x1024_B1", 1, 126, 2048, False, 210),
             ("attn2_15360x1024_B2_norm", 2, 15360, 4096, True, 220),
             ("audio_attn2_152x1024_B2_norm", 2, 152, 2048, True, 230))
    for name, B, Tq, inner, norm, seed in cases:
        q = _randn((B, Tq, inner), 0x5EED + seed, device)
        k = _randn((B, Tt, inner), 0x5EED + seed + 1, device)
        v = _randn((B, Tt, inner), 0x5EED + seed + 2, device)
        kw = {}
        if norm:
            kw = dict(q_norm_w=_randn((inner,), 0x5EED + seed + 3, device, 1.0, 0.02),
                      k_norm_w=_randn((inner,), 0x5EED + seed + 4, device, 1.0, 0.02))
        out = torch.empty_like(q)

        def call(ev):
            L.attention_fwd(q, k, v, heads=H, out=out, workspace=ws,
                            events=None if ev is None else (ev[0], ev[1]), **kw)

        wall, _ = time_steps(call, steps, warmup, hip, events_per_step=False)
        _, kms = time_steps(call, steps, 0, hip)
        st = stats(kms)
        fl = 4.0 * B * Tq * Tt * inner
        res[name] = {"kernel_ms": st["median_ms"], "call_ms": round(wall / steps * 1e3, 4),
                     "kernel_tflops": round(fl / (st["median_ms"] * 1e-3) / 1e12, 1),
                     "pct_peak": round(100 * fl / (st["median_ms"] * 1e-3) / 1e12
                                       / PEAK_BF16_TFLOPS, 2),
                     "gflop": round(fl / 1e9, 2), "kernel_time_stats": st}
        del q, k, v, out
    return res


def bench_connector(device, steps, warmup, hip):
    """The embeddings connector's attention at 1024 tokens (EmbeddingsConnector.swift:
    288-331), video width 4096 (32 x 128) and audio width 2048 (32 x 64): q/k norm over the
    width, the connector's 1-D RoPE, the per-head gate, no mask. ms per call (events around
    the attention kernel, and the whole call)."""
    import torch

    import ltx_attn as L

    H, T = 32, 1024
    res = {}
    ws = torch.empty(64 << 20, dtype=torch.uint8, device=device)
    for width, seed in ((4096, 300), (2048, 310)):
        q, k, v = (_randn((1, T, width), 0x5EED + seed + i, device) for i in range(3))
        w = _randn((width,), 0x5EED + seed + 3, device, 1.0, 0.02)
        gate = _randn((1, T, H), 0x5EED + seed + 4, device, 0.0, 2.0)
        rot = L.connector_rotary(T, width, H, device)
        out = torch.empty_like(q)

        def call(ev):
            L.attention_fwd(q, k, v, heads=H, q_norm_w=w, k_norm_w=w, rotary=rot,
                            gate_logits=gate, out=out, workspace=ws,
                            events=None if ev is None else (ev[0], ev[1]))

        wall, _ = time_steps(call, steps, warmup, hip, events_per_step=False)
        _, kms = time_steps(call, steps, 0, hip)
        km = sum(kms) / len(kms)
        fl = 4.0 * T * T * width
        res[f"connector_{width}"] = {"kernel_ms": round(km, 4),
                                     "call_ms": round(wall / steps * 1e3, 4),
                                     "kernel_tflops": round(fl / (km * 1e-3) / 1e12, 1)}
    return res


def bench_gemma(device, steps, warmup):
    """The Gemma-4 text encoder's attention at its 1024 tokens (GemmaTextEncoder.swift:158-239):
    a sliding layer (D 256, 16 query heads over 8 KV heads, window 1024) and a full layer
    (D 512, one KV head shared as V, partial RoPE), one prompt, no padding. ms per call (the
    per-head prologue and the attention), and TFLOP/s over the causal pairs (4 * pairs * D *
    Hq)."""
    import torch

    import ltx_attn as L

    T, res = 1024, {}
    for name, spec, seed in (("sliding", L.GEMMA_SLIDING, 500), ("full", L.GEMMA_FULL, 510)):
        D, Hq, Hkv = spec["head_dim"], spec["q_heads"], spec["kv_heads"]
        q = _randn((1, T, Hq * D), 0x5EED + seed, device)
        k = _randn((1, T, Hkv * D), 0x5EED + seed + 1, device)
        v = k if spec["shares_kv"] else _randn((1, T, Hkv * D), 0x5EED + seed + 2, device)
        wq = _randn((D,), 0x5EED + seed + 3, device, 1.03, 0.02)
        wk = _randn((D,), 0x5EED + seed + 4, device, 0.12 if D == 256 else 0.06, 0.01)
        cos, sin = (torch.from_numpy(t).to(device) for t in
                    L.gemma_rope_tables(T, D, spec["theta"], spec["partial"], spec["proportional"]))
        out = torch.empty((1, T, Hq * D), dtype=torch.float32, device=device)
        ws = torch.empty(256 << 20, dtype=torch.uint8, device=device)   # q', k', v', partials
        ms = _time_ms(lambda: L.gemma_attention_fwd(
            q, k, v, q_heads=Hq, kv_heads=Hkv, q_norm_w=wq, k_norm_w=wk, cos=cos, sin=sin,
            window=spec["window"], out=out, workspace=ws), steps, warmup)
        pairs = T * (T + 1) / 2
        res[f"gemma_{name}_1024_ms"] = round(ms, 4)
        res[f"gemma_{name}_1024_tflops"] = round(4.0 * pairs * D * Hq / (ms * 1e-3) / 1e12, 1)
    return res


def bench_c5(device, steps, warmup, hip, per_call_repeats=10):
    """The six attentions of one DiT block at 1280x768x121, B=2 (CFG), in block order
    (Sources/LTXModules/DiTBlock.swift:343-438): attn1, audio_attn1, attn2, audio_attn2,
    audio_to_video, video_to_audio. Every call's Q, K and V are separate draws and every
    module's q_norm / k_norm separate weights (separate seeds per operand, as
    BenchGEMM.swift:627-632 draws them), as the module's projections and norms are. The text
    keys have 94 valid of 1024 per row (the block-set configuration); the unmasked text cross
    the DiT runs is timed by bench_text_cross_unmasked. Per call, the attention kernel's
    median over `per_call_repeats` calls after 3 warm-up calls (the reference's protocol,
    BenchGEMM.swift:96-100)."""
    import torch

    import ltx_attn as L

    Tv, Ta, Tt, B = 15360, 152, 1024, 2
    tabs = L.rotaries(121, 768, 1280, audio_tokens=Ta)
    rot = {k: L.Rotary(_dev_bits(c, device), _dev_bits(s, device)) for k, (c, s) in tabs.items()}
    valid = [94, 94]
    # name, query stream (tokens, width), key stream, q table, k table, text valid lengths
    spec = [
        ("attn1", (Tv, 4096), (Tv, 4096), "videoSelf", None, None),
        ("audio_attn1", (Ta, 2048), (Ta, 2048), "audioSelf", None, None),
        ("attn2", (Tv, 4096), (Tt, 4096), None, None, valid),
        ("audio_attn2", (Ta, 2048), (Tt, 2048), None, None, valid),
        ("audio_to_video_attn", (Tv, 2048), (Ta, 2048), "videoCross", "audioCross", None),
        ("video_to_audio_attn", (Ta, 2048), (Tv, 2048), "audioCross", "videoCross", None),
    ]
    ops, norms, flops = {}, {}, 0.0
    for i, (name, (Lq, wq_), (Lk, wk_), _, _, vl) in enumerate(spec):
        seed = 0x5EED + 50 + 10 * i
        ops[name] = (_randn((B, Lq, wq_), seed, device), _randn((B, Lk, wk_), seed + 1, device),
                     _randn((B, Lk, wk_), seed + 2, device))
        norms[name] = (_randn((wq_,), seed + 3, device, 1.0, 0.02),
                       _randn((wk_,), seed + 4, device, 1.0, 0.02))
        flops += 4.0 * B * Lq * (Lk if vl is None else vl[0]) * wq_
    outs = {name: torch.empty_like(ops[name][0]) for name in ops}
    ws = torch.empty(512 << 20, dtype=torch.uint8, device=device)
    io = {name: ops[name] + (outs[name],) for name in ops}
    tables = {"videoSelf": rot["videoSelf"], "audioSelf": rot["audioSelf"],
              "videoCross": rot["videoCross"], "audioCross": rot["audioCross"]}
    block = L.DiTBlockAttention(norms)

    def call(ev):
        block.self_attention(io["attn1"], io["audio_attn1"], tables, workspace=ws)
        block.text_cross(io["attn2"], io["audio_attn2"], valid, workspace=ws)
        block.cross_modal(io["audio_to_video_attn"], io["video_to_audio_attn"], tables,
                          workspace=ws)

    wall, _ = time_steps(call, steps, warmup, hip, events_per_step=False)
    # per-attention kernel time: events around the attention kernel, median of the repeats
    per, per_stats = {}, {}
    for name, _, _, pe, kpe, vl in spec:
        q, k, v = ops[name]

        def one(ev, q=q, k=k, v=v, name=name, pe=pe, kpe=kpe, vl=vl):
            L.attention_fwd(q, k, v, heads=32, q_norm_w=norms[name][0],
                            k_norm_w=norms[name][1], rotary=rot[pe] if pe else None,
                            key_rotary=rot[kpe] if kpe else None, k_valid_len=vl,
                            out=outs[name], workspace=ws,
                            events=None if ev is None else (ev[0], ev[1]))

        _, kms = time_steps(one, per_call_repeats, 3, hip)
        per_stats[name] = stats(kms)
        per[name] = per_stats[name]["median_ms"]
    ms = wall / steps * 1e3
    return {"ms_per_block": ms, "tflops": flops / (ms * 1e-3) / 1e12,
            "kernel_ms": per, "kernel_time_stats": per_stats}


def bench_rope_tables(device):
    """The 12480-token video table pair (32 x 12480 x 64 cos + sin, bf16) built on the GPU,
    against the host builder plus the upload it needs."""
    import torch

    import ltx_attn as L

    pos = L.rope_video_positions(13, 24, 40)
    pos_dev = torch.from_numpy(pos).to(device)
    for _ in range(3):
        L.rope_tables_device(pos_dev, 4096, [20, 2048, 2048], 32)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    n = 20
    for _ in range(n):
        L.rope_tables_device(pos_dev, 4096, [20, 2048, 2048], 32)
    torch.cuda.synchronize()
    gpu_ms = (time.perf_counter() - t0) / n * 1e3
    t0 = time.perf_counter()
    c, s_ = L.rope_tables(pos, 4096, [20, 2048, 2048], 32)
    up = [_dev_bits(c, device), _dev_bits(s_, device)]
    torch.cuda.synchronize()
    host_ms = (time.perf_counter() - t0) * 1e3
    return {"device_ms": gpu_ms, "host_build_and_upload_ms": host_ms}


def _time_ms(fn, n, warm):
    import torch

    for _ in range(warm):
        fn()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record()
    for _ in range(n):
        fn()
    b.record()
    b.synchronize()
    return a.elapsed_time(b) / n


def bench_projection(device, x):
    """The projection GEMM with the RMS statistic from its epilogue (``ltx_linear``) at the
    12480-token video self-attention's shapes: to_q (12480 x 4096 x 4096) and to_q/to_k/to_v
    fused into one N = 12288 projection, with hipBLASLt (torch's linear, no statistic) timed
    beside it on the same shapes as a point of comparison; the attention call taking its
    statistic from the partials instead of its own pass over q; and the whole module
    (DiTAttention.callAsFunction: projections, attention with the gate, to_out) through
    ``DiTAttentionModule``."""
    import torch
    import torch.nn.functional as F

    import ltx_attn as L

    T, C = 12480, 4096
    xin = _randn((1, T, C), 0x5EED + 40, device)
    w = {n: _randn((C, C), 0x5EED + 41 + i, device, 0.0, C ** -0.5)
         for i, n in enumerate(("to_q", "to_k", "to_v", "to_out.0"))}
    wf = torch.cat([w["to_q"], w["to_k"], w["to_v"]], 0).contiguous()
    y1 = torch.empty((1, T, C), dtype=torch.bfloat16, device=device)
    y3 = torch.empty((1, T, 3 * C), dtype=torch.bfloat16, device=device)
    lws = torch.empty(max(L.linear_workspace_bytes(T, C, C), L.linear_workspace_bytes(T, 3 * C, C),
                          256), dtype=torch.uint8, device=device)
    # the clock ramps down while the host builds the RoPE tables before this: settle it first
    settle(lambda ev: L.linear(xin, wf, out=y3, sumsq=True, workspace=lws), 0.25)
    ms_q = _time_ms(lambda: L.linear(xin, w["to_q"], out=y1, sumsq=True, workspace=lws), 20, 5)
    ms_qkv = _time_ms(lambda: L.linear(xin, wf, out=y3, sumsq=True, workspace=lws), 10, 3)
    # the same without the tail split (every tile whole: one more round of 256 workgroups)
    ms_q_whole = _time_ms(lambda: L.linear(xin, w["to_q"], out=y1, sumsq=True, workspace=False),
                          20, 5)
    ms_qkv_whole = _time_ms(lambda: L.linear(xin, wf, out=y3, sumsq=True, workspace=False), 10, 3)
    ms_q_blas = _time_ms(lambda: F.linear(xin, w["to_q"]), 20, 5)
    ms_qkv_blas = _time_ms(lambda: F.linear(xin, wf), 10, 3)
    fl_q, fl_qkv = 2.0 * T * C * C, 2.0 * T * 3 * C * C

    # attention with the projection's statistic vs its own statistic pass
    out = torch.empty_like(x["q"])
    ws = torch.empty(512 << 20, dtype=torch.uint8, device=device)
    _, qs = L.linear(xin, w["to_q"], sumsq=True, workspace=lws)
    _, ks = L.linear(xin, w["to_k"], sumsq=True, workspace=lws)
    kw = dict(heads=x["H"], q_norm_w=x["wq"], k_norm_w=x["wk"], rotary=x["rot"], out=out,
              workspace=ws)
    ms_attn_own = _time_ms(lambda: L.attention_fwd(x["q"], x["k"], x["v"], **kw), 10, 3)
    ms_attn_given = _time_ms(lambda: L.attention_fwd(x["q"], x["k"], x["v"], q_sumsq=qs,
                                                     k_sumsq=ks, **kw), 10, 3)

    # the whole module
    weights = {n + ".weight": t for n, t in w.items()}
    for i, n in enumerate(("to_q", "to_k", "to_v", "to_out.0")):
        weights[n + ".bias"] = _randn((C,), 0x5EED + 50 + i, device, 0.0, 0.1)
    weights["to_gate_logits.weight"] = _randn((32, C), 0x5EED + 55, device, 0.0, C ** -0.5)
    weights["q_norm.weight"], weights["k_norm.weight"] = x["wq"], x["wk"]
    mod = L.DiTAttentionModule(weights)
    ms_mod = _time_ms(lambda: mod(xin, variant=L.Variant.videoSelf, rotary=x["rot"],
                                  workspace=ws), 5, 2)
    fl_mod = 5 * fl_q + 2.0 * T * C * 32 + 4.0 * T * T * C
    return {
        "linear_12480x4096x4096_ms": round(ms_q, 4),
        "linear_12480x4096x4096_tflops": round(fl_q / ms_q / 1e9, 1),
        "linear_12480x4096x4096_pct_peak": round(100 * fl_q / ms_q / 1e9 / PEAK_BF16_TFLOPS, 2),
        "linear_12480x4096x4096_whole_tiles_ms": round(ms_q_whole, 4),
        "linear_fused_qkv_whole_tiles_ms": round(ms_qkv_whole, 4),
        "linear_fused_qkv_12480x12288x4096_ms": round(ms_qkv, 4),
        "linear_fused_qkv_tflops": round(fl_qkv / ms_qkv / 1e9, 1),
        "linear_fused_qkv_pct_peak": round(100 * fl_qkv / ms_qkv / 1e9 / PEAK_BF16_TFLOPS, 2),
        "hipblaslt_12480x4096x4096_ms": round(ms_q_blas, 4),
        "hipblaslt_fused_qkv_ms": round(ms_qkv_blas, 4),
        "attn_12480_own_statistic_ms": round(ms_attn_own, 4),
        "attn_12480_projection_statistic_ms": round(ms_attn_given, 4),
        "video_self_module_12480_ms": round(ms_mod, 4),
        "video_self_module_12480_tflops": round(fl_mod / ms_mod / 1e9, 1),
    }


def cpu_baseline(x, budget_s):
    """The C restatement of the reference's explicit path (fp32 logits, softmax, P.V, with
    its bf16 rounding points), multithreaded, on a bounded sample of the c4 workload:
    all 12480 keys, a contiguous block of queries, some heads."""
    import oracle as O

    # Every core this process may run on, unless the host allots a smaller CPU share per GPU
    # through OMP_NUM_THREADS (the GPU hosts here give each GPU 16 threads).
    visible = len(os.sched_getaffinity(0))
    threads = visible
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        threads = min(visible, int(omp))
    H, D, T = x["H"], x["D"], x["T"]
    qb, kb, vb = _host_bits(x["q"]), _host_bits(x["k"]), _host_bits(x["v"])
    wq, wk = _host_bits(x["wq"]), _host_bits(x["wk"])
    kw = dict(q_norm_w=wq, k_norm_w=wk, q_cos=x["cos"], q_sin=x["sin"], mode="reference",
              threads=threads)
    # calibrate on two sample sizes (the K preparation is a fixed cost per call), then size
    # the sample to the budget
    def timed(nh_, nq_):
        t0 = time.perf_counter()
        O.c_attention(qb, kb, vb, H, heads_range=(0, nh_), q_range=(0, nq_), **kw)
        return time.perf_counter() - t0

    t_small = timed(1, 256)
    t_big = timed(1, 1280)
    per_row = max((t_big - t_small) / 1024.0, 1e-7)     # one query row of one head
    rows = max(1280, int((budget_s - t_small) / per_row))
    nh = max(1, min(H, rows // T))
    nq = T if rows >= T else rows
    dt = timed(nh, nq)
    flops = 4.0 * nq * T * nh * D
    cpu = "unknown"
    info = {}
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if not line.strip():
                    break                              # the first processor's block
                key, _, val = line.partition(":")
                info[key.strip()] = val.strip()
    except OSError:
        pass
    if "model name" in info:
        cpu = info["model name"]
        # a virtual machine may report only the vendor's family name: add family/model/stepping
        if not any(ch.isdigit() for ch in cpu) and "cpu family" in info:
            cpu += (f" (family {info['cpu family']}, model {info.get('model', '?')}, "
                    f"stepping {info.get('stepping', '?')})")
    return {"value": flops / dt / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": (f"{nh} head(s) x {nq} queries x {T} keys of the 12480-token workload "
                       f"(norm + 3-D RoPE + explicit fp32 SDPA), {dt:.1f} s on {threads} "
                       f"threads of {cpu}; substitute for the reference's MLX CPU path (mlx "
                       "not installed)"),
            "cpu_model": cpu, "host_cores_visible": visible, "isa": O.c_library_isa,
            "seconds": round(dt, 2)}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--settle-ms", type=float, default=250.0,
                    help="untimed calls for this long before the warmup steps, so the clock "
                         "has ramped up (reported as clock_settle_ms)")
    ap.add_argument("--cpu-budget", type=float, default=12.0,
                    help="seconds of CPU work for the cpu_baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--projection-only", action="store_true",
                    help="only run the 12480 x 4096 x 4096 projection (ltx_linear with its "
                         "statistic), --steps times (for counter passes)")
    ap.add_argument("--short-keys-only", action="store_true",
                    help="only run the short-key calls (text cross-attention, the cross-modal "
                         "pair, the block set's video->text and video->audio-keys calls), "
                         "--steps times each (for counter passes)")
    ap.add_argument("--c1-only", action="store_true",
                    help="only run the 3120-token self-attention, --steps timed calls (for "
                         "counter passes)")
    ap.add_argument("--block-only", action="store_true",
                    help="only run one DiT block's six attentions at 1280x768x121, B=2, "
                         "--steps times (for counter passes)")
    ap.add_argument("--text-cross-only", action="store_true",
                    help="only run the unmasked text cross-attention calls (3120 and 126 "
                         "queries over 1024 keys, B=1; 2 x 15360 and 2 x 152 with norm), "
                         "--steps timed calls each")
    ap.add_argument("--gemma-only", action="store_true",
                    help="only run the Gemma-4 encoder attention (sliding and full layer at "
                         "1024 tokens), --steps timed calls each")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB, --steps times "
                         "(the known-size kernel that scales FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus > 1 or world > 1:
        print("bench.py measures one MI355X: the attention path runs on a single GPU "
              "(head/query sharding over several GPUs is designed, not built); "
              f"--gpus {args.gpus} is not supported.", file=sys.stderr)
        sys.exit(2)

    import torch

    import ltx_attn as L

    L.load_library()
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    hip = HipEvents()

    if args.copy_calibration:
        n = args.copy_calibration << 20
        src = torch.empty(n, dtype=torch.uint8, device=device).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "launches": args.steps}), flush=True)
        return

    if args.projection_only:
        xin = _randn((12480, 4096), 0x5EED + 40, device)
        w = _randn((4096, 4096), 0x5EED + 41, device, 0.0, 4096 ** -0.5)
        y = torch.empty((12480, 4096), dtype=torch.bfloat16, device=device)
        lws = torch.empty(max(L.linear_workspace_bytes(12480, 4096, 4096), 256),
                          dtype=torch.uint8, device=device)
        for _ in range(args.steps):
            L.linear(xin, w, out=y, sumsq=True, workspace=lws)
        torch.cuda.synchronize()
        print(json.dumps({"projection": [12480, 4096, 4096], "launches": args.steps}), flush=True)
        return

    if args.c1_only:
        res = bench_c1(device, args.steps, args.warmup, hip)
        print(json.dumps({"video_self_3120": {k: v for k, v in res.items()}}), flush=True)
        return

    if args.block_only:
        res = bench_c5(device, args.steps, args.warmup, hip)
        print(json.dumps({"dit_block_attn": res}), flush=True)
        return

    if args.text_cross_only:
        res = bench_text_cross_unmasked(device, args.steps, args.warmup, hip)
        print(json.dumps({"text_cross_unmasked": res}), flush=True)
        return

    if args.gemma_only:
        res = bench_gemma(device, args.steps, args.warmup)
        print(json.dumps({"gemma_text_encoder_attn": res}), flush=True)
        return

    if args.short_keys_only:
        res = bench_short_keys(device, args.steps, args.warmup, hip)
        print(json.dumps({"short_key_calls": res}), flush=True)
        return

    x, c4 = bench_c4(device, args.steps, args.warmup, hip, args.settle_ms / 1e3)
    print(f"# c4: {c4['ms_per_step']:.3f} ms/step, attention kernel {c4['kernel_ms']:.3f} ms "
          f"({c4['kernel_tflops']:.1f} TFLOP/s)", file=sys.stderr, flush=True)
    secondary = {}
    if not args.no_secondary:
        c1 = bench_c1(device, 10, 3, hip)
        print(f"# c1: {c1['kernel_ms']:.3f} ms kernel, {c1['kernel_tflops']:.1f} TFLOP/s",
              file=sys.stderr, flush=True)
        short = bench_short_keys(device, 10, 3, hip)
        print("# short-key calls: " + ", ".join(f"{k} {v['kernel_ms']:.4f} ms "
                                                 f"({v['kernel_gbs']:.0f} GB/s)"
                                                 for k, v in short.items()),
              file=sys.stderr, flush=True)
        tcu = bench_text_cross_unmasked(device, 10, 3, hip)
        print("# text cross, unmasked 1024 keys: " + ", ".join(
            f"{k} {v['kernel_ms']:.4f} ms ({v['kernel_tflops']:.0f} TFLOP/s)"
            for k, v in tcu.items()), file=sys.stderr, flush=True)
        conn = bench_connector(device, 10, 3, hip)
        gemma = bench_gemma(device, 10, 3)
        c5 = bench_c5(device, 5, 2, hip)
        print(f"# c5: {c5['ms_per_block']:.3f} ms per block attention set", file=sys.stderr,
              flush=True)
        rope = bench_rope_tables(device)
        print(f"# rope tables (12480 video tokens): {rope['device_ms']:.3f} ms on the GPU, "
              f"{rope['host_build_and_upload_ms']:.1f} ms host build + upload", file=sys.stderr,
              flush=True)
        proj = bench_projection(device, x)
        print(f"# projection 12480x4096x4096: {proj['linear_12480x4096x4096_ms']:.3f} ms "
              f"({proj['linear_12480x4096x4096_tflops']} TFLOP/s; hipBLASLt "
              f"{proj['hipblaslt_12480x4096x4096_ms']:.3f} ms); video self-attention module "
              f"{proj['video_self_module_12480_ms']:.3f} ms", file=sys.stderr, flush=True)
        secondary = {
            "video_self_3120_tflops": round(c1["kernel_tflops"], 2),
            "video_self_3120_pct_peak": round(c1["pct_peak"], 2),
            "video_self_3120_ms": round(c1["kernel_ms"], 4),
            "video_self_3120_call_ms": round(c1["ms_per_call"], 4),
            "video_self_3120_call_tflops": round(c1["tflops"], 2),
            "short_key_calls": short,
            "text_cross_unmasked": tcu,
            "connector_attn_1024": conn,
            "gemma_text_encoder_attn": gemma,
            "dit_block_attn_ms": round(c5["ms_per_block"], 4),
            "dit_block_attn_tflops": round(c5["tflops"], 2),
            "dit_block_attn_kernel_ms": c5["kernel_ms"],
            "dit_block_attn_kernel_time_stats": c5["kernel_time_stats"],
            "video_self_3120_kernel_time_stats": c1["kernel_stats"],
            "video_self_3120_call_time_stats": c1["call_stats"],
            "rope_tables_12480_device_ms": round(rope["device_ms"], 4),
            "rope_tables_12480_host_build_upload_ms": round(rope["host_build_and_upload_ms"], 2),
            "projection": proj,
        }

    traffic, traffic_note = None, "no counter pass recorded"
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as fh:
            rec = json.load(fh)
        if rec.get("kernel_source_sha256") == kernel_source_sha256():
            traffic = rec.get("hbm_bytes_per_launch")
            traffic_note = (f"FETCH_SIZE x {rec.get('fetch_scale')} + WRITE_SIZE x "
                            f"{rec.get('write_scale')} per dispatch, counted on these kernel "
                            "sources (profiles/traffic_attn_video_self_12480.md)")
        else:
            traffic_note = "stale: the kernel sources changed since the last counter pass"
    achieved = c4["kernel_tflops"]
    roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                "traffic": traffic, "traffic_note": traffic_note,
                "kernel": "fmha_dma_kernel<128>",
                "kernel_avg_ms": round(c4["kernel_ms"], 4),
                "kernel_time_stats": c4["kernel_stats"],
                "flops_per_launch": c4["flops"]}
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(x, args.cpu_budget)
        # GPU whole-call throughput over the CPU restatement's, same workload and FLOP count
        cpu["speedup"] = round(c4["tflops"] / cpu["value"], 1)

    line = {
        "metric": METRIC,
        "value": round(c4["tflops"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "clock_settle_ms": args.settle_ms,
        "ms_per_step": round(c4["ms_per_step"], 4),
        "step_time_stats": c4["call_stats"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "stage-2 video self-attention 1280x768x97: 12480 tokens, "
                               "H=32, D=128, B=1, fused QK-RMSNorm (eps 1e-6) + 3-D RoPE",
                   "B": 1, "H": 32, "Lq": 12480, "Lk": 12480, "D": 128,
                   "parallelism": "single GPU"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "secondary": secondary,
        "provenance": L.provenance(),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
