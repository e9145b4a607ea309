"""GPU parity: the HIP library, called through its C ABI, against the CPU oracle.

Tolerance (stated by the target): on the bf16 outputs, relative RMS error <= 5e-3 and
max-abs error <= 2e-2 against the fp32/float64 oracle of the same seeded inputs. Each check
also asserts that the kernel is no further from the truth than the reference's own rounding
points put the reference (``mode="reference"`` of the oracle), plus a small slack.
"""

import json
import math
import os

import numpy as np
import pytest

import ltx_attn as L
import oracle as O

pytestmark = pytest.mark.gpu

REL_RMS = 5e-3
MAX_ABS = 2e-2
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _say(msg):
    print(msg, flush=True)


def dev(bits, device):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(device)
    return t.view(torch.bfloat16)


def host_bits(t):
    import torch

    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def host_f32(t):
    return O.bf16_bits_to_f32(host_bits(t))


def check(got, truth, ref_out=None, label=""):
    c = O.compare(got, truth)
    _say(f"  {label}: relRMS {c['rel_rms']:.3e} maxAbs {c['max_abs']:.3e}")
    assert c["rel_rms"] <= REL_RMS, (label, c)
    assert c["max_abs"] <= MAX_ABS, (label, c)
    if ref_out is not None:
        r = O.compare(ref_out, truth)
        _say(f"  {label}: reference arithmetic relRMS {r['rel_rms']:.3e}")
        assert c["rel_rms"] <= max(r["rel_rms"], 2.5e-3) * 1.25, (label, c, r)
    return c


def run(device, q, k, v, heads, **kw):
    """numpy bf16 bits in, numpy fp32 (bf16 values) out, merged layout."""
    import torch

    tq, tk, tv = dev(q, device), dev(k, device), dev(v, device)
    extra = {}
    for name in ("q_norm_w", "k_norm_w"):
        if kw.get(name) is not None:
            extra[name] = dev(kw.pop(name), device)
        else:
            kw.pop(name, None)
    qc, qs, kc, ks = (kw.pop(n, None) for n in ("q_cos", "q_sin", "k_cos", "k_sin"))
    if qc is not None:
        extra["rotary"] = L.Rotary(dev(qc, device), dev(qs, device))
    if kc is not None:
        extra["key_rotary"] = L.Rotary(dev(kc, device), dev(ks, device))
    if isinstance(kw.get("gate_logits"), np.ndarray):
        extra["gate_logits"] = dev(kw.pop("gate_logits"), device)
    out = L.attention_fwd(tq, tk, tv, heads=heads, **extra, **kw)
    torch.cuda.synchronize()
    return host_f32(out)


def test_device_query(device):
    """ltx_device_query describes the MI355X the tests run on (the device a Swift host
    selects explicitly, and whose CU count the work split is planned over)."""
    info = L.device_info(0)
    _say(f"device: {info}")
    assert info["supported"] and info["arch"].startswith("gfx950")
    assert info["compute_units"] == 256
    assert info["memory_bytes"] > 250e9
    assert info["lds_bytes_per_cu"] >= 160 * 1024
    assert L.load_library().ltx_device_count() >= 1
    with pytest.raises(L.Failure):
        L.device_info(L.load_library().ltx_device_count())


# ---------------------------------------------------------------------------------------
# The reference's own attention test, through MLXFast's signature
# ---------------------------------------------------------------------------------------

def test_mlx_capability_uniform_case(device):
    """MLXCapabilityTests.fusedAttention (Tests/LTXModulesTests/MLXCapabilityTests.swift:78-91)."""
    import torch

    heads, tokens, head_dim = 4, 16, 64
    q = torch.ones((1, heads, tokens, head_dim), dtype=torch.bfloat16, device=device)
    k = torch.ones_like(q)
    v = torch.ones_like(q) * 2.0
    out = L.scaled_dot_product_attention(q, k, v, scale=1.0 / math.sqrt(head_dim))
    torch.cuda.synchronize()
    assert list(out.shape) == [1, heads, tokens, head_dim]
    assert abs(out[0, 0, 0, 0].item() - 2.0) < 1e-4
    assert torch.all((out.float() - 2.0).abs() < 1e-4)


# ---------------------------------------------------------------------------------------
# Committed golden vectors
# ---------------------------------------------------------------------------------------

def _fixtures():
    data = np.load(os.path.join(GOLDEN, "fixtures.npz"), allow_pickle=False)
    names = sorted({k.split("/")[0] for k in data.files})
    return data, names


@pytest.mark.parametrize("name", _fixtures()[1])
def test_golden_fixture(device, name):
    data, _ = _fixtures()
    g = {k.split("/", 1)[1]: data[k] for k in data.files if k.startswith(name + "/")}
    meta = json.loads(str(g["meta"]))
    _say(f"golden {name} {meta}")
    kw = {key: g[key] for key in ("q_norm_w", "k_norm_w", "q_cos", "q_sin", "k_cos", "k_sin")
          if key in g}
    if "valid_len" in g:
        kw["k_valid_len"] = list(g["valid_len"])
    # AUTO picks the short-key kernel where the keys fit in LDS, else the LDS-DMA kernel
    for kprep in (L.KPREP_AUTO, L.KPREP_FUSED, L.KPREP_PROLOGUE):
        got = run(device, g["q"], g["k"], g["v"], meta["heads"], kprep=kprep, **dict(kw))
        check(got, g["out_exact"], O.bf16_bits_to_f32(g["out_ref_bf16"]),
              f"{name} kprep={kprep}")


# ---------------------------------------------------------------------------------------
# Edge shapes, small enough for the float64 oracle
# ---------------------------------------------------------------------------------------

@pytest.mark.parametrize("B,H,Lq,Lk,D,valid", [
    (1, 2, 1, 1, 64, None),
    (1, 2, 7, 5, 128, None),
    (2, 3, 65, 63, 64, None),
    (1, 2, 257, 129, 128, None),
    (2, 2, 300, 200, 128, [200, 1]),
    (2, 2, 100, 1024, 64, [94, 1]),
    (3, 1, 33, 100, 128, [64, 65, 100]),
])
def test_edge_shapes(device, B, H, Lq, Lk, D, valid):
    _say(f"edge B={B} H={H} Lq={Lq} Lk={Lk} D={D} valid={valid}")
    seed = B * 1000 + Lq * 7 + Lk
    q = O.randn_bf16_bits((B, Lq, H * D), seed)
    k = O.randn_bf16_bits((B, Lk, H * D), seed + 1)
    v = O.randn_bf16_bits((B, Lk, H * D), seed + 2)
    truth = O.attention(q, k, v, H, valid_len=valid, mode="exact")
    got = run(device, q, k, v, H, k_valid_len=valid)
    check(got, truth, None, "edge")


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("splits", [1, 2, 3, 16])
def test_split_kv_matches(device, D, splits):
    """Short query stream over a long key stream (the audio-queries case), forced splits."""
    B, H, Lq, Lk = 1, 4, 126, 1500
    _say(f"split D={D} splits={splits}")
    q = O.randn_bf16_bits((B, Lq, H * D), 11)
    k = O.randn_bf16_bits((B, Lk, H * D), 12)
    v = O.randn_bf16_bits((B, Lk, H * D), 13)
    truth = O.attention(q, k, v, H, mode="exact")
    got = run(device, q, k, v, H, num_splits=splits)
    check(got, truth, None, f"splits={splits}")


def test_split_kv_ragged_rows_with_empty_splits(device):
    """Batch rows with very different valid lengths: later splits of the short row are empty."""
    B, H, Lq, Lk, D = 2, 2, 40, 1024, 64
    q = O.randn_bf16_bits((B, Lq, H * D), 21)
    k = O.randn_bf16_bits((B, Lk, H * D), 22)
    v = O.randn_bf16_bits((B, Lk, H * D), 23)
    valid = [1000, 3]
    truth = O.attention(q, k, v, H, valid_len=valid, mode="exact")
    got = run(device, q, k, v, H, k_valid_len=valid, num_splits=8)
    check(got, truth, None, "ragged split")


def _gate_bits(shape, seed):
    """Gate logits ~ N(0, 2), with every 7th at +12 and every 11th from the 3rd at -12
    (saturated gates: x2 and ~x0)."""
    f = O.bf16_bits_to_f32(O.randn_bf16_bits(shape, seed, std=2.0)).copy()
    f.ravel()[::7] = 12.0
    f.ravel()[3::11] = -12.0
    return O.f32_to_bf16_bits(f)


@pytest.mark.parametrize("case", ["dma_whole_and_tail", "register_split", "register_whole",
                                  "short_keys", "strided_logits"])
def test_output_gate(device, case):
    """The per-head gate (DiTAttention.swift:395-399) in every epilogue: the LDS-DMA kernel's
    whole items and the combine of its split tail items (2 x 16 heads x 9 query blocks = 288
    items: 256 whole + 32 split in two), the register kernel split and unsplit, the short-key
    kernel, and logits given as a strided view."""
    import torch

    B, H, Lq, Lk, D, kw = {
        "dma_whole_and_tail": (2, 16, 2100, 128, 128, {"kprep": L.KPREP_PROLOGUE}),
        "short_keys": (2, 8, 1500, 100, 128, {}),
        "register_split": (1, 4, 126, 1500, 64, {"num_splits": 3}),
        "register_whole": (2, 4, 100, 300, 128, {"num_splits": 1}),
        "strided_logits": (1, 8, 600, 200, 128, {}),
    }[case]
    _say(f"output gate {case}: B={B} H={H} Lq={Lq} Lk={Lk} D={D} {kw}")
    seed = 0x5EED + 60
    q = O.randn_bf16_bits((B, Lq, H * D), seed)
    k = O.randn_bf16_bits((B, Lk, H * D), seed + 1)
    v = O.randn_bf16_bits((B, Lk, H * D), seed + 2)
    g = _gate_bits((B, Lq, H), seed + 3)
    if case == "strided_logits":
        wide = np.zeros((B, Lq, 2 * H), dtype=np.uint16)
        wide[:, :, 1::2] = g
        kw["gate_logits"] = dev(wide, device)[:, :, 1::2]
        assert kw["gate_logits"].stride() == (Lq * 2 * H, 2 * H, 2)
    else:
        kw["gate_logits"] = g
    truth = O.attention(q, k, v, H, gate_bits=g, mode="exact")
    got = run(device, q, k, v, H, **kw)
    check(got, truth, None, f"gate {case}")
    # The gate itself: the gated output is the ungated output times the bf16 gate, to the
    # two bf16 roundings in between (2^-8 relative), row by row.
    kw.pop("gate_logits")
    plain = run(device, q, k, v, H, **kw).reshape(B, Lq, H, D)
    want = plain * O.head_gate(g, "reference")[..., None]
    err = np.abs(got.reshape(B, Lq, H, D) - want)
    assert np.all(err <= np.abs(want) * 2.0 ** -7 + 1e-6), float(err.max())
    # rows whose gate saturates at ~0 come out ~0
    f = O.bf16_bits_to_f32(g)
    off = got.reshape(B, Lq, H, D)[f < -11.0]
    assert off.size and np.abs(off).max() < 1e-4


@pytest.mark.parametrize("gated", [False, True])
def test_stg_passthrough(device, gated):
    """A fully perturbed module (DiTAttention.swift:351-356) returns V split into heads, times
    the bf16 gate when it has one (:395-399), with no attention: out is V bit for bit, or the
    one bf16 rounding of V x gate."""
    import torch

    B, H, L_, D = 2, 32, 300, 128
    _say(f"STG passthrough gated={gated}")
    v = O.randn_bf16_bits((B, L_, H * D), 81)
    tv = dev(v, device)
    kw = {}
    g = None
    if gated:
        g = _gate_bits((B, L_, H), 82)
        kw["gate_logits"] = dev(g, device)
    core = L.DiTAttentionCore(None, None)
    out = core(None, None, tv, variant=L.Variant.videoSelf, all_perturbed=True, **kw)
    torch.cuda.synchronize()
    got = host_bits(out)
    if not gated:
        assert np.array_equal(got, v)
    else:
        want = O.f32_to_bf16_bits(O.bf16_bits_to_f32(v).reshape(B, L_, H, D) *
                                  O.head_gate(g, "reference")[..., None]).reshape(v.shape)
        assert np.array_equal(got, want)


@pytest.mark.parametrize("Lq", [40, 300])
def test_batches_beyond_one_launch(device, Lq):
    """B = 66 unmasked batch rows run as launches of 64 + 2 rows (the per-row key lengths
    travel in the kernel arguments); each launch's pointers, statistics and gate start at
    its first row. Lq = 40: register kernel; Lq = 300: LDS-DMA kernel."""
    B, H, Lk, D = 66, 2, 50, 64
    _say(f"batches beyond one launch: B={B} Lq={Lq}")
    q = O.randn_bf16_bits((B, Lq, H * D), 71)
    k = O.randn_bf16_bits((B, Lk, H * D), 72)
    v = O.randn_bf16_bits((B, Lk, H * D), 73)
    w = O.randn_bf16_bits((H * D,), 74, mean=1.0, std=0.02)
    g = _gate_bits((B, Lq, H), 75)
    truth = O.attention(q, k, v, H, q_norm_w=w, k_norm_w=w, gate_bits=g, mode="exact")
    got = run(device, q, k, v, H, q_norm_w=w, k_norm_w=w, gate_logits=g)
    check(got, truth, None, f"B={B} Lq={Lq}")


def test_rebase_path_large_logits(device):
    """Logits that grow along the key axis (up to ~190 log2 units above the first block's max)
    force the running max to be rebased several times. The scale ln(2) makes the folded factor
    scale*log2(e) exactly 1, so Q enters the MFMA unrounded and the logits are exact: what is
    checked is the rebase arithmetic, not the rounding of very large logits."""
    B, H, Lq, Lk, D = 1, 2, 64, 640, 64
    rng = np.random.default_rng(5)
    qf = rng.standard_normal((B, Lq, H * D)).astype(np.float32) * 2.0
    kf = rng.standard_normal((B, Lk, H * D)).astype(np.float32)
    kf *= (1.0 + np.arange(Lk, dtype=np.float32) / 40.0)[None, :, None]
    q, k = O.f32_to_bf16_bits(qf), O.f32_to_bf16_bits(kf)
    v = O.randn_bf16_bits((B, Lk, H * D), 6)
    scale = float(np.float32(math.log(2.0)))
    truth = O.attention(q, k, v, H, scale=scale, mode="exact")
    got = run(device, q, k, v, H, scale=scale)
    check(got, truth, None, "rebase")
    # the same through split-KV (rebases inside each split, then the combine)
    got = run(device, q, k, v, H, scale=scale, num_splits=4)
    check(got, truth, None, "rebase split")


@pytest.mark.parametrize("D,groups", [(64, 0), (128, 0), (128, 6)])
def test_dma_kernel_large_logits(device, D, groups):
    """The LDS-DMA kernel (three query blocks per head) on logits growing along the keys, far
    past the first block's max: its row sums (matrix-core products) pass 2^64, so the fast pass
    is discarded and the items redo their keys with the exact online softmax. With the
    device's CU count the six items run as split key ranges (and the combine); with six
    resident groups they run whole. scale = ln 2 folds to exactly 1, so the logits are exact."""
    B, H, Lq, Lk = 1, 2, 600, 1200
    _say(f"LDS-DMA kernel, large logits: D={D} groups={groups}")
    rng = np.random.default_rng(11 + D)
    qf = rng.standard_normal((B, Lq, H * D)).astype(np.float32) * 2.0
    kf = rng.standard_normal((B, Lk, H * D)).astype(np.float32)
    kf *= (1.0 + np.arange(Lk, dtype=np.float32) / 40.0)[None, :, None]
    q, k = O.f32_to_bf16_bits(qf), O.f32_to_bf16_bits(kf)
    v = O.randn_bf16_bits((B, Lk, H * D), 12)
    scale = float(np.float32(math.log(2.0)))
    truth = O.attention(q, k, v, H, scale=scale, mode="exact")
    got = run(device, q, k, v, H, scale=scale, resident_groups=groups)
    check(got, truth, None, f"LDS-DMA large logits D={D} groups={groups}")


@pytest.mark.parametrize("B,H,Lq,Lk,D,valid,rope", [
    (2, 4, 1000, 1024, 128, [128, 1], False),   # most keys kept at D=128; a single key
    (2, 4, 1000, 300, 64, [256, 129], True),    # most keys kept at D=64, norm + RoPE
    (2, 32, 4100, 77, 64, None, True),          # 129 query blocks of 32 per head: 4-5 per wave
    (1, 2, 1, 3, 128, None, False),             # one query
])
def test_short_key_kernel(device, B, H, Lq, Lk, D, valid, rope):
    """The short-key kernel (the head's keys resident in LDS, eight waves per workgroup each
    streaming blocks of 32 queries past them) against the oracle, and the LDS-DMA kernel on the
    same call, with norm on both sides (its gated epilogue: test_output_gate)."""
    _say(f"short keys B={B} H={H} Lq={Lq} Lk={Lk} D={D} valid={valid} rope={rope}")
    seed = 0x5EED + 90 + Lq
    q = O.randn_bf16_bits((B, Lq, H * D), seed)
    k = O.randn_bf16_bits((B, Lk, H * D), seed + 1)
    v = O.randn_bf16_bits((B, Lk, H * D), seed + 2)
    wq = O.randn_bf16_bits((H * D,), seed + 3, mean=1.0, std=0.02)
    wk = O.randn_bf16_bits((H * D,), seed + 4, mean=1.0, std=0.02)
    kw = dict(q_norm_w=wq, k_norm_w=wk)
    if rope:
        qc, qs = _index_rotary(np.arange(Lq) // 7, H * D, H)
        kc, ks = _index_rotary(np.arange(Lk) // 3, H * D, H)
        kw.update(q_cos=qc, q_sin=qs, k_cos=kc, k_sin=ks)
    truth = O.attention(q, k, v, H, valid_len=valid, mode="exact", **kw)
    ref = O.attention(q, k, v, H, valid_len=valid, mode="reference", **kw)
    for kprep in (L.KPREP_AUTO, L.KPREP_PROLOGUE):
        got = run(device, q, k, v, H, k_valid_len=valid, kprep=kprep, **dict(kw))
        check(got, truth, O.round_bf16(ref), f"short keys kprep={kprep}")


def test_short_key_kernel_large_logits(device):
    """Logits growing along the keys (up to ~100 log2 units above the first 32-key block's
    max) make the short-key kernel redo its blocks from the true row max. scale = ln 2 folds
    to exactly 1, so the logits are exact and the check is on the softmax arithmetic."""
    B, H, Lq, Lk, D = 1, 2, 200, 250, 64
    rng = np.random.default_rng(7)
    qf = rng.standard_normal((B, Lq, H * D)).astype(np.float32) * 2.0
    kf = rng.standard_normal((B, Lk, H * D)).astype(np.float32)
    kf *= (1.0 + np.arange(Lk, dtype=np.float32) / 40.0)[None, :, None]
    q, k = O.f32_to_bf16_bits(qf), O.f32_to_bf16_bits(kf)
    v = O.randn_bf16_bits((B, Lk, H * D), 8)
    scale = float(np.float32(math.log(2.0)))
    truth = O.attention(q, k, v, H, scale=scale, mode="exact")
    got = run(device, q, k, v, H, scale=scale)
    check(got, truth, None, "short keys, large logits")


@pytest.mark.parametrize("width,head_dim", [(4096, 128), (2048, 64)])
def test_connector_attention(device, width, head_dim):
    """The embeddings connector's attention (EmbeddingsConnector.swift:288-331): q/k
    RMS-normed over the full width, the connector's 1-D split RoPE (arange(1024) over
    maxPos 4096), no mask, scale 1/sqrt(head_dim), and the per-head 2*sigmoid gate from
    to_gate_logits, over 1024 tokens and 32 heads, against the oracle (whose arithmetic is the
    connector's explicit fp32 softmax). The attention is compared ungated to the stated
    tolerance and the gate as the gated output against the ungated one times the bf16 gate."""
    H, T = 32, 1024
    _say(f"connector attention width={width} head_dim={head_dim}")
    seed = 0x5EED + 200 + head_dim
    x = [O.randn_bf16_bits((1, T, width), seed + i) for i in range(3)]
    wq = O.randn_bf16_bits((width,), seed + 3, mean=1.0, std=0.02)
    wk = O.randn_bf16_bits((width,), seed + 4, mean=1.0, std=0.02)
    cos, sin = L.rope_tables(L.rope_connector_positions(T), width, [L.CONNECTOR_MAX_POS], H)
    g = _gate_bits((1, T, H), seed + 5)
    kw = dict(q_norm_w=wq, k_norm_w=wk, q_cos=cos, q_sin=sin)
    truth = O.attention(*x, H, mode="exact", **kw)
    ref = O.attention(*x, H, mode="reference", **kw)
    plain = run(device, *x, H, **dict(kw))
    check(plain, truth, O.round_bf16(ref), f"connector {width}")
    gated = run(device, *x, H, gate_logits=g, **dict(kw))
    want = plain.reshape(1, T, H, head_dim) * O.head_gate(g, "reference")[..., None]
    err = np.abs(gated.reshape(1, T, H, head_dim) - want)
    assert np.all(err <= np.abs(want) * 2.0 ** -7 + 1e-6), float(err.max())


def test_split_layout_and_strided_output(device):
    import torch

    B, H, Lq, Lk, D = 2, 4, 96, 80, 128
    q = O.randn_bf16_bits((B, H, Lq, D), 31)
    k = O.randn_bf16_bits((B, H, Lk, D), 32)
    v = O.randn_bf16_bits((B, H, Lk, D), 33)
    merged = lambda x: x.transpose(0, 2, 1, 3).reshape(B, x.shape[2], H * D)  # noqa: E731
    truth = O.attention(merged(q), merged(k), merged(v), H, mode="exact")
    tq, tk, tv = dev(q, device), dev(k, device), dev(v, device)
    out = L.scaled_dot_product_attention(tq, tk, tv, scale=1.0 / math.sqrt(D))
    torch.cuda.synchronize()
    got = host_f32(out).transpose(0, 2, 1, 3).reshape(B, Lq, H * D)
    check(got, truth, None, "split layout")
    # merged output written into a wider row: the padding must stay untouched
    big = torch.full((B, Lq, H * D + 64), 7.0, dtype=torch.bfloat16, device=device)
    view = big[:, :, 32:32 + H * D]
    L.attention_fwd(dev(merged(q), device), dev(merged(k), device), dev(merged(v), device),
                    heads=H, out=view)
    torch.cuda.synchronize()
    assert torch.all(big[:, :, :32] == 7.0) and torch.all(big[:, :, 32 + H * D:] == 7.0)
    check(host_f32(view.contiguous()), truth, None, "strided out")


def test_deterministic(device):
    B, H, L_, D = 1, 8, 700, 128
    q = O.randn_bf16_bits((B, L_, H * D), 41)
    k = O.randn_bf16_bits((B, L_, H * D), 42)
    v = O.randn_bf16_bits((B, L_, H * D), 43)
    a = run(device, q, k, v, H)
    b = run(device, q, k, v, H)
    assert np.array_equal(a, b)


def test_dit_attention_core_rules(device):
    """DiTAttentionCore mirrors DiTAttention: rotary on attn2/audio_attn2 is refused."""
    import torch

    w = torch.ones(4096, dtype=torch.bfloat16, device=device)
    core = L.DiTAttentionCore(w, w)
    x = torch.zeros((1, 8, 4096), dtype=torch.bfloat16, device=device)
    tab = torch.zeros((32, 8, 64), dtype=torch.bfloat16, device=device)
    with pytest.raises(L.RotaryWithoutPosition):
        core(x, x, x, variant=L.Variant.videoCross, rotary=L.Rotary(tab, tab))
    with pytest.raises(L.Failure):
        core(x, x, x, variant=L.Variant.videoSelf, key_rotary=L.Rotary(tab, tab))


# ---------------------------------------------------------------------------------------
# The benchmark shapes at full size: every head and every query row against the C oracle
# ---------------------------------------------------------------------------------------

def _gpu_bits(shape, seed, device, mean=0.0, std=1.0):
    """Seeded N(mean, std) bf16 drawn on the GPU (fast at full size), plus its host bits."""
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(seed)
    t = (torch.randn(shape, generator=g, device=device, dtype=torch.float32) * std + mean)
    t = t.to(torch.bfloat16)
    return t, host_bits(t)


def _index_rotary(indices, inner, heads):
    """1-D temporal tables from integer positions (frame index / audio index), built with the
    reference's rotary recipe (frequency grid, centre/maxPos, theta 1e4)."""
    pos = np.zeros((1, 1, len(indices), 2), dtype=np.float32)
    pos[0, 0, :, 0] = indices
    pos[0, 0, :, 1] = indices
    return O.rotary_tables(pos, inner, [20], heads)


def check_heads(got, truth, ref_out, label):
    """The stated tolerance per (batch row, head) -- a wrong head cannot hide in the average of
    the others -- besides the whole-output check, and per head too at most 1.25x the reference
    arithmetic's own error (floor 2.5e-3). All arrays [B, Lq, H, D]."""
    check(got, truth, ref_out, label)
    g, t, r = (np.asarray(x, dtype=np.float64) for x in (got, truth, ref_out))
    ssr = np.sum(t * t, axis=(1, 3))
    rel = np.sqrt(np.sum((g - t) ** 2, axis=(1, 3)) / ssr)
    rel_ref = np.sqrt(np.sum((r - t) ** 2, axis=(1, 3)) / ssr)
    worst = np.unravel_index(int(np.argmax(rel / np.maximum(rel_ref, 2.5e-3))), rel.shape)
    _say(f"  {label}: worst (b, h) = {tuple(int(i) for i in worst)}: relRMS {rel[worst]:.3e} "
         f"(reference arithmetic {rel_ref[worst]:.3e})")
    assert np.all(rel <= REL_RMS), (label, float(rel.max()))
    assert np.all(rel <= np.maximum(rel_ref, 2.5e-3) * 1.25), (label, worst, float(rel[worst]))


def _full_check(device, tq, tk, tv, heads, bits, kw_host, kw_dev, label, **call_kw):
    """One call on the GPU; the C oracle over all heads and query rows, exact (fp32 after
    the bf16 inputs) and with the reference's rounding points."""
    import torch

    out = L.attention_fwd(tq, tk, tv, heads=heads, **kw_dev, **call_kw)
    torch.cuda.synchronize()
    got = host_f32(out)
    qb, kb, vb = bits
    truth = O.c_attention(qb, kb, vb, heads, mode="exact", **kw_host)
    refm = O.round_bf16(O.c_attention(qb, kb, vb, heads, mode="reference", **kw_host))
    check_heads(got.reshape(truth.shape), truth, refm, label)


def test_c1_video_self_3120(device):
    _say("c1 video self-attention [1,32,3120,128]")
    shape = (1, 3120, 4096)
    tq, qb = _gpu_bits(shape, 0x5EED, device)
    tk, kb = _gpu_bits(shape, 0x5EED + 1, device)
    tv, vb = _gpu_bits(shape, 0x5EED + 2, device)
    _full_check(device, tq, tk, tv, 32, (qb, kb, vb), {}, {}, "c1")


def test_c1_splitmix_operands(device):
    """The 3120-token self-attention on the reference bench's own operand stream (splitmix64
    -> uniform [-1, 1) -> bf16, Bench.swift:479-493; seeds 0x5EED + k as BenchGEMM.swift
    :627-632) instead of N(0, 1) draws."""
    shape = (1, 3120, 4096)
    n = int(np.prod(shape))
    bits = [O.splitmix_bf16_bits(n, 0x5EED + i).reshape(shape) for i in range(3)]
    _say("c1 with splitmix64 operands")
    tq, tk, tv = (dev(b, device) for b in bits)
    _full_check(device, tq, tk, tv, 32, tuple(bits), {}, {}, "c1 splitmix")


@pytest.mark.parametrize("B,valid", [(1, [94]), (2, [94, 1])])
def test_c2_text_cross_masked(device, B, valid):
    _say(f"c2 text cross B={B} valid={valid}")
    tq, qb = _gpu_bits((B, 3120, 4096), 0x5EED + 10, device)
    tk, kb = _gpu_bits((B, 1024, 4096), 0x5EED + 11, device)
    tv, vb = _gpu_bits((B, 1024, 4096), 0x5EED + 12, device)
    _full_check(device, tq, tk, tv, 32, (qb, kb, vb), {"valid_len": valid},
                {"k_valid_len": valid}, "c2")


@pytest.mark.parametrize("kprep", [L.KPREP_PROLOGUE, L.KPREP_FUSED])
def test_whole_and_tail_items_ragged(device, kprep):
    """2 x 32 heads x 9 query blocks = 576 items: two whole rounds of 256 items run over all
    their keys, the last 64 items (batch 1, heads 24-31) are split into key ranges of 12 tiles
    and merged by the combine kernel. Batch 1 has 700 valid keys (11 tiles), so three of the
    four ranges of each of its tail items are empty."""
    _say(f"whole + tail items, ragged keys, kprep={kprep}")
    B, H, Lq, Lk, valid = 2, 32, 2100, 3000, [3000, 700]
    tq, qb = _gpu_bits((B, Lq, H * 128), 0x5EED + 40, device)
    tk, kb = _gpu_bits((B, Lk, H * 128), 0x5EED + 41, device)
    tv, vb = _gpu_bits((B, Lk, H * 128), 0x5EED + 42, device)
    _full_check(device, tq, tk, tv, H, (qb, kb, vb), {"valid_len": valid},
                {"k_valid_len": valid}, "whole+tail", kprep=kprep)


@pytest.mark.parametrize("H,T,groups", [(12, 1300, 32), (12, 1300, 100), (12, 1300, 200),
                                         (16, 2400, 150)])
def test_plans_for_other_part_sizes(device, H, T, groups):
    """A call plans its tail splits for the device's CU count (the resident_groups argument
    stands in for it) when the workspace covers that plan, and runs the plan the workspace was sized
    for (256 CUs) otherwise. 12 heads x 6 query blocks = 72 items: 32 groups split the 8 tail
    items four ways, 100 run all 72 whole, 200 split every item two ways (the sized plan: three
    ways; both fit its workspace). 16 heads x 10 query blocks = 160 items: 150 groups split the
    10 tail items, which the sized plan (no split, no workspace) cannot hold, so that call runs
    the sized plan; with a large workspace it runs its own. Every head and row against the C
    oracle."""
    import torch

    tq, qb = _gpu_bits((1, T, H * 128), 0x5EED + 70, device)
    tk, kb = _gpu_bits((1, T, H * 128), 0x5EED + 71, device)
    tv, vb = _gpu_bits((1, T, H * 128), 0x5EED + 72, device)
    _say(f"{H} heads x {T} tokens, plan for {groups} resident groups, sized workspace")
    _full_check(device, tq, tk, tv, H, (qb, kb, vb), {}, {}, f"groups {groups} sized",
                resident_groups=groups)
    _say(f"{H} heads x {T} tokens, plan for {groups} resident groups, large workspace")
    ws = torch.empty(64 << 20, dtype=torch.uint8, device=device)
    _full_check(device, tq, tk, tv, H, (qb, kb, vb), {}, {"workspace": ws}, f"groups {groups} own",
                resident_groups=groups)


@pytest.mark.parametrize("direction", ["video_q", "audio_q"])
def test_c3_cross_modal(device, direction):
    _say(f"c3 cross-modal {direction}")
    Tv, Ta, H, D = 3120, 126, 32, 64
    vid_idx = np.arange(Tv) // (20 * 12)           # latent frame index 0..12
    aud_idx = np.arange(Ta)                        # 0..125
    vc, vs = _index_rotary(vid_idx, H * D, H)
    ac, as_ = _index_rotary(aud_idx, H * D, H)
    if direction == "video_q":
        Lq, Lk, qt, kt = Tv, Ta, (vc, vs), (ac, as_)
    else:
        Lq, Lk, qt, kt = Ta, Tv, (ac, as_), (vc, vs)
    tq, qb = _gpu_bits((1, Lq, H * D), 0x5EED + 20, device)
    tk, kb = _gpu_bits((1, Lk, H * D), 0x5EED + 21, device)
    tv, vb = _gpu_bits((1, Lk, H * D), 0x5EED + 22, device)
    kw_host = dict(q_cos=qt[0], q_sin=qt[1], k_cos=kt[0], k_sin=kt[1])
    kw_dev = dict(rotary=L.Rotary(dev(qt[0], device), dev(qt[1], device)),
                  key_rotary=L.Rotary(dev(kt[0], device), dev(kt[1], device)))
    _full_check(device, tq, tk, tv, H, (qb, kb, vb), kw_host, kw_dev, f"c3 {direction}")


@pytest.mark.parametrize("Lq", [40, 126, 152, 230])
def test_split_key_kernel_query_groups(device, Lq):
    """The split-key kernel (one query block over a long key stream, D 64, K's norm and RoPE
    applied in LDS) with 1, 2, 3 and 4 active 64-query groups: the K transform runs on the
    waves without queries (waves 4-7, or 6-7 with three groups) or beside the products (four
    groups). B = 2 with a ragged key length in each row."""
    H, D, Lk = 4, 64, 2500
    seed = 0x5EED + 700 + Lq
    _say(f"split-key kernel Lq={Lq} Lk={Lk} H={H}")
    qt = _index_rotary(np.arange(Lq), H * D, H)
    kt = _index_rotary(np.arange(Lk) // 7, H * D, H)
    tq, qb = _gpu_bits((2, Lq, H * D), seed, device)
    tk, kb = _gpu_bits((2, Lk, H * D), seed + 1, device)
    tv, vb = _gpu_bits((2, Lk, H * D), seed + 2, device)
    wq, wqb = _gpu_bits((H * D,), seed + 3, device, 1.0, 0.02)
    wk, wkb = _gpu_bits((H * D,), seed + 4, device, 1.0, 0.02)
    valid = [Lk - 37, 1601]
    kw_host = dict(q_norm_w=wqb, k_norm_w=wkb, q_cos=qt[0], q_sin=qt[1], k_cos=kt[0],
                   k_sin=kt[1], valid_len=valid)
    kw_dev = dict(q_norm_w=wq, k_norm_w=wk, k_valid_len=valid,
                  rotary=L.Rotary(dev(qt[0], device), dev(qt[1], device)),
                  key_rotary=L.Rotary(dev(kt[0], device), dev(kt[1], device)))
    _full_check(device, tq, tk, tv, H, (qb, kb, vb), kw_host, kw_dev, f"split-key Lq={Lq}")


def test_split_key_ranges_reuse_and_graph_replay(device):
    """The split-key kernel's key ranges and their merge: 2, 5 and 16 ranges against the
    oracle; repeated calls on one workspace, and a workspace filled with arbitrary bytes
    beforehand, give the first call's bits; a HIP graph of the call (kernel and merge launch)
    replayed several times, with eager work and eager calls between the replays, gives them
    on every replay."""
    import torch

    H, D, Lq, Lk = 8, 64, 126, 3120
    seed = 0x5EED + 800
    _say(f"split-key ranges, reuse and graph replay Lq={Lq} Lk={Lk} H={H}")
    qt = _index_rotary(np.arange(Lq), H * D, H)
    kt = _index_rotary(np.arange(Lk) // 240, H * D, H)
    tq, qb = _gpu_bits((1, Lq, H * D), seed, device)
    tk, kb = _gpu_bits((1, Lk, H * D), seed + 1, device)
    tv, vb = _gpu_bits((1, Lk, H * D), seed + 2, device)
    kw_host = dict(q_cos=qt[0], q_sin=qt[1], k_cos=kt[0], k_sin=kt[1])
    kw_dev = dict(rotary=L.Rotary(dev(qt[0], device), dev(qt[1], device)),
                  key_rotary=L.Rotary(dev(kt[0], device), dev(kt[1], device)))
    for splits in (2, 5, 16):
        _full_check(device, tq, tk, tv, H, (qb, kb, vb), kw_host, kw_dev,
                    f"split-key {splits} ranges", num_splits=splits)

    ws = torch.empty(8 << 20, dtype=torch.uint8, device=device)   # more than the call needs
    out = torch.empty_like(tq)

    def call():
        L.attention_fwd(tq, tk, tv, heads=H, num_splits=5, out=out, workspace=ws, **kw_dev)

    call()
    torch.cuda.synchronize()
    first = out.clone()
    for _ in range(3):
        out.zero_()
        call()
        torch.cuda.synchronize()
        assert torch.equal(out, first)
    ws.copy_(torch.randint(0, 256, ws.shape, dtype=torch.uint8, device=device))
    out.zero_()
    call()
    torch.cuda.synchronize()
    assert torch.equal(out, first)

    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        call()                       # warm the capture stream's path
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    torch.cuda.synchronize()
    scratch = torch.zeros(1 << 20, device=device)
    for i in range(4):
        out.zero_()
        scratch.add_(1.0)            # eager work between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, first), f"replay {i}"
        call()                       # an eager call between replays
        torch.cuda.synchronize()
        assert torch.equal(out, first), f"eager after replay {i}"


@pytest.mark.parametrize("kprep", [L.KPREP_PROLOGUE, L.KPREP_FUSED])
def test_c4_stage2_self_12480_norm_rope(device, kprep):
    _say(f"c4 12480 self-attention, norm + 3-D RoPE, kprep={kprep}")
    H, D, T = 32, 128, 12480
    tq, qb = _gpu_bits((1, T, H * D), 0x5EED + 30, device)
    tk, kb = _gpu_bits((1, T, H * D), 0x5EED + 31, device)
    tv, vb = _gpu_bits((1, T, H * D), 0x5EED + 32, device)
    wq, wqb = _gpu_bits((H * D,), 0x5EED + 33, device, 1.0, 0.02)
    wk, wkb = _gpu_bits((H * D,), 0x5EED + 34, device, 1.0, 0.02)
    cos, sin = L.rope_tables(L.rope_video_positions(13, 24, 40), H * D, [20, 2048, 2048], H)
    kw_host = dict(q_norm_w=wqb, k_norm_w=wkb, q_cos=cos, q_sin=sin)
    kw_dev = dict(q_norm_w=wq, k_norm_w=wk, rotary=L.Rotary(dev(cos, device), dev(sin, device)))
    _full_check(device, tq, tk, tv, H, (qb, kb, vb), kw_host, kw_dev, "c4", kprep=kprep)


AUDIO_101_CASES = [
    # label, (query tokens, width), (key tokens, width), q table, k table
    ("audio_attn1", ("a", 2048), ("a", 2048), "audioSelf", None),
    ("audio_attn2", ("a", 2048), ("t", 2048), None, None),
    ("audio_to_video", ("v", 2048), ("a", 2048), "videoCross", "audioCross"),
    ("video_to_audio", ("a", 2048), ("v", 2048), "audioCross", "videoCross"),
]


@pytest.mark.parametrize("case", AUDIO_101_CASES, ids=[c[0] for c in AUDIO_101_CASES])
def test_audio_stream_at_formula_token_count(device, case):
    """The audio stream's attentions at the token count the geometry formula gives for 97
    frames at 24 fps (LatentGeometry.swift:128-132: round(97 / 24 * 25) = 101, against the 126
    of 121 frames) beside 3120 video tokens (640x384) and 1024 unmasked text tokens, with the
    tables rotaries builds for that clip and separate q / k norm weights."""
    label, (qs, qw), (ks, kwid), qtab, ktab = case
    H, D = 32, 64
    Ta = L.audio_latent_count(97, 24.0)
    assert Ta == 101
    tokens = {"v": 3120, "a": Ta, "t": 1024}
    seed = 0x5EED + 400 + 10 * AUDIO_101_CASES.index(case)
    _say(f"audio stream at 101 tokens, {label}: Lq {tokens[qs]} Lk {tokens[ks]}")
    tq, qb = _gpu_bits((1, tokens[qs], qw), seed, device)
    tk, kb = _gpu_bits((1, tokens[ks], kwid), seed + 1, device)
    tv, vb = _gpu_bits((1, tokens[ks], kwid), seed + 2, device)
    wq, wqb = _gpu_bits((qw,), seed + 3, device, 1.0, 0.02)
    wk, wkb = _gpu_bits((kwid,), seed + 4, device, 1.0, 0.02)
    kw_host = dict(q_norm_w=wqb, k_norm_w=wkb)
    kw_dev = dict(q_norm_w=wq, k_norm_w=wk)
    tabs = L.rotaries(97, 384, 640)
    assert tabs["audioSelf"][0].shape[1] == Ta and tabs["videoCross"][0].shape[1] == 3120
    for name, host_keys, dev_key in ((qtab, ("q_cos", "q_sin"), "rotary"),
                                     (ktab, ("k_cos", "k_sin"), "key_rotary")):
        if name:
            kw_host.update({host_keys[0]: tabs[name][0], host_keys[1]: tabs[name][1]})
            kw_dev[dev_key] = L.Rotary(dev(tabs[name][0], device), dev(tabs[name][1], device))
    assert H * D == qw
    _full_check(device, tq, tk, tv, H, (qb, kb, vb), kw_host, kw_dev, f"audio101 {label}")


C5_CASES = [
    # label, query stream (tokens, width), key stream, D, q table, k table, text keys valid
    ("attn1", ("v", 4096), ("v", 4096), 128, "videoSelf", None, None),
    ("audio_attn1", ("a", 2048), ("a", 2048), 64, "audioSelf", None, None),
    ("attn2", ("v", 4096), ("t", 4096), 128, None, None, [94, 94]),
    ("audio_attn2", ("a", 2048), ("t", 2048), 64, None, None, [94, 94]),
    ("audio_to_video", ("v", 2048), ("a", 2048), 64, "videoCross", "audioCross", None),
    ("video_to_audio", ("a", 2048), ("v", 2048), 64, "audioCross", "videoCross", None),
]


@pytest.mark.parametrize("case", C5_CASES, ids=[c[0] for c in C5_CASES])
def test_c5_block_set(device, case):
    """One DiT block's six attentions at B=2 (15360 video, 152 audio, 1024 text tokens of
    which 94 valid), with norm + RoPE where the reference applies it (DiTBlock.swift:343-438).
    Q, K and V are separate draws and q_norm / k_norm separate weights, as the module's
    projections and norms are, so an operand mix-up changes the output."""
    import torch

    label, (qs, qw), (ks, kwid), D, qtab, ktab, vl = case
    H = 32
    tokens = {"v": 15360, "a": 152, "t": 1024}
    seed = 0x5EED + 50 + 10 * C5_CASES.index(case)
    _say(f"c5 {label}: Lq {tokens[qs]} Lk {tokens[ks]} D {D}")
    tq, qb = _gpu_bits((2, tokens[qs], qw), seed, device)
    tk, kb = _gpu_bits((2, tokens[ks], kwid), seed + 1, device)
    tv, vb = _gpu_bits((2, tokens[ks], kwid), seed + 2, device)
    wq, wqb = _gpu_bits((qw,), seed + 3, device, 1.0, 0.02)
    wk, wkb = _gpu_bits((kwid,), seed + 4, device, 1.0, 0.02)
    kw_host = dict(q_norm_w=wqb, k_norm_w=wkb)
    kw_dev = dict(q_norm_w=wq, k_norm_w=wk)
    if qtab or ktab:
        vt = L.rotaries(121, 768, 1280, audio_tokens=tokens["a"])
    if qtab:
        kw_host.update(q_cos=vt[qtab][0], q_sin=vt[qtab][1])
        kw_dev["rotary"] = L.Rotary(dev(vt[qtab][0], device), dev(vt[qtab][1], device))
    if ktab:
        kw_host.update(k_cos=vt[ktab][0], k_sin=vt[ktab][1])
        kw_dev["key_rotary"] = L.Rotary(dev(vt[ktab][0], device), dev(vt[ktab][1], device))
    if vl:
        kw_host["valid_len"] = vl
        kw_dev["k_valid_len"] = vl
    _full_check(device, tq, tk, tv, H, (qb, kb, vb), kw_host, kw_dev, f"c5 {label}")
    torch.cuda.synchronize()


def test_text_cross_unmasked_as_the_dit_calls_it(device):
    """The DiT's attn2 / audio_attn2 attend over every text token with no mask
    (DiTForward.swift:38-42 passes no mask; DiTAttention.swift:374-376 runs mask: .none):
    the block driver's text_cross with no valid lengths over 1024 modulated connector
    tokens, B = 2, against the oracle's unmasked attention over all 1024 keys."""
    import torch

    B, Tv, Ta, Tt, H = 2, 3120, 126, 1024, 32
    _say(f"text cross, unmasked: {Tv} video / {Ta} audio queries over {Tt} text keys")
    seed = 0x5EED + 300
    wv, wvb = _gpu_bits((4096,), seed, device, 1.0, 0.02)
    wa, wab = _gpu_bits((2048,), seed + 1, device, 1.0, 0.02)
    wkv, wkvb = _gpu_bits((4096,), seed + 2, device, 1.0, 0.02)
    wka, wkab = _gpu_bits((2048,), seed + 3, device, 1.0, 0.02)
    streams = {}
    for name, (T, inner, s) in {"vq": (Tv, 4096, 4), "tk4": (Tt, 4096, 5), "tv4": (Tt, 4096, 6),
                                "aq": (Ta, 2048, 7), "tk2": (Tt, 2048, 8),
                                "tv2": (Tt, 2048, 9)}.items():
        streams[name] = _gpu_bits((B, T, inner), seed + s, device)
    norms = {v.value: (wv, wkv) if v in (L.Variant.videoSelf, L.Variant.videoCross)
             else (wa, wka) for v in L.Variant}
    blk = L.DiTBlockAttention(norms)
    vo = torch.empty_like(streams["vq"][0])
    ao = torch.empty_like(streams["aq"][0])
    blk.text_cross((streams["vq"][0], streams["tk4"][0], streams["tv4"][0], vo),
                   (streams["aq"][0], streams["tk2"][0], streams["tv2"][0], ao))
    torch.cuda.synchronize()
    for label, out, (q, k, v), (w1, w2) in (("attn2", vo, ("vq", "tk4", "tv4"), (wvb, wkvb)),
                                            ("audio_attn2", ao, ("aq", "tk2", "tv2"),
                                             (wab, wkab))):
        bits = tuple(streams[n][1] for n in (q, k, v))
        kw = dict(q_norm_w=w1, k_norm_w=w2)
        truth = O.c_attention(*bits, H, mode="exact", **kw)
        refm = O.round_bf16(O.c_attention(*bits, H, mode="reference", **kw))
        check_heads(host_f32(out).reshape(truth.shape), truth, refm, f"unmasked {label}")


def test_block_driver_matches_single_calls(device):
    """The block driver (DiTBlock.swift:343-438 order, one workspace) gives each module's
    output bit for bit as its own call does, with every call's Q, K and V separate draws and
    every module's q_norm / k_norm separate weights, so a Q/K/V or q_norm/k_norm mix-up inside
    the driver changes the output: CFG rows with different text lengths, a gated
    audio->video call, both self-attentions computed and then both perturbed (STG
    passthrough). The driver's self-attention and cross-modal outputs are also checked
    against the oracle over every head and row."""
    import torch

    B, Ta, Tt, H = 2, 152, 1024, 32
    rot = L.rotaries_device(25, 320, 480, audio_tokens=Ta)
    Tv = rot["videoSelf"].cos.shape[1]
    _say(f"block driver: {Tv} video / {Ta} audio / {Tt} text tokens, B={B}")
    seeds = iter(range(0x5EED + 900, 0x5EED + 1000))

    def t(shape, mean=0.0, std=1.0):
        return _gpu_bits(shape, next(seeds), device, mean, std)

    video = (L.Variant.videoSelf, L.Variant.videoCross)
    norms = {v.value: tuple(t((4096 if v in video else 2048,), 1.0, 0.02) for _ in range(2))
             for v in L.Variant}
    shapes = {                                   # (query stream, key stream)
        "attn1": ((Tv, 4096), (Tv, 4096)),
        "audio_attn1": ((Ta, 2048), (Ta, 2048)),
        "attn2": ((Tv, 4096), (Tt, 4096)),
        "audio_attn2": ((Ta, 2048), (Tt, 2048)),
        "audio_to_video_attn": ((Tv, 2048), (Ta, 2048)),
        "video_to_audio_attn": ((Ta, 2048), (Tv, 2048)),
    }
    ops = {n: tuple(t((B,) + s) for s in (qs, ks, ks)) for n, (qs, ks) in shapes.items()}
    gate = t((B, Tv, H), 0.0, 2.0)
    valid = [94, 11]

    def io(name, gated=False):
        q, k, v = (x[0] for x in ops[name])
        out = torch.full_like(q, 7.0)
        return (q, k, v, out, gate[0]) if gated else (q, k, v, out)

    calls = {n: io(n, n == "audio_to_video_attn") for n in shapes}
    ws = torch.empty(256 << 20, dtype=torch.uint8, device=device)
    blk = L.DiTBlockAttention({k: (w[0][0], w[1][0]) for k, w in norms.items()})
    blk.self_attention(calls["attn1"], calls["audio_attn1"], rot, workspace=ws)
    blk.text_cross(calls["attn2"], calls["audio_attn2"], valid, workspace=ws)
    blk.cross_modal(calls["audio_to_video_attn"], calls["video_to_audio_attn"], rot,
                    workspace=ws)
    perturbed = {n: io(n) for n in ("attn1", "audio_attn1")}
    blk.self_attention(perturbed["attn1"], perturbed["audio_attn1"], rot,
                       video_perturbed=True, audio_perturbed=True, workspace=ws)
    torch.cuda.synchronize()

    tables = {
        "attn1": ("videoSelf", None), "audio_attn1": ("audioSelf", None),
        "attn2": (None, None), "audio_attn2": (None, None),
        "audio_to_video_attn": ("videoCross", "audioCross"),
        "video_to_audio_attn": ("audioCross", "videoCross"),
    }

    def single(name):
        q, k, v = (x[0] for x in ops[name])
        wq, wk = (w[0] for w in norms[name])
        pe, kpe = tables[name]
        kw = dict(q_norm_w=wq, k_norm_w=wk)
        if pe:
            kw["rotary"] = rot[pe]
        if kpe:
            kw["key_rotary"] = rot[kpe]
        if name in ("attn2", "audio_attn2"):
            kw["k_valid_len"] = valid
        if name == "audio_to_video_attn":
            kw["gate_logits"] = gate[0]
        return L.attention_fwd(q, k, v, heads=H, **kw)

    for name in shapes:
        assert torch.equal(calls[name][3], single(name)), name
    for name in ("attn1", "audio_attn1"):                  # passthrough: V itself
        assert torch.equal(perturbed[name][3], ops[name][2][0]), name

    # the driver's outputs against the oracle (exact, and with the reference's rounding
    # points), every head and row
    for name in ("attn1", "audio_attn1", "audio_to_video_attn", "video_to_audio_attn"):
        bits = tuple(x[1] for x in ops[name])
        kw = dict(q_norm_w=norms[name][0][1], k_norm_w=norms[name][1][1])
        pe, kpe = tables[name]
        if pe:
            kw.update(q_cos=host_bits(rot[pe].cos), q_sin=host_bits(rot[pe].sin))
        if kpe:
            kw.update(k_cos=host_bits(rot[kpe].cos), k_sin=host_bits(rot[kpe].sin))
        truth = O.c_attention(*bits, H, mode="exact", **kw)
        refm = O.round_bf16(O.c_attention(*bits, H, mode="reference", **kw))
        if name == "audio_to_video_attn":
            truth = truth * O.head_gate(gate[1])[..., None]
            refm = O.round_bf16(refm * O.head_gate(gate[1], "reference")[..., None])
        got = host_f32(calls[name][3]).reshape(truth.shape)
        check_heads(got, truth, refm, f"block driver {name}")
