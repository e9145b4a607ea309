"""GPU parity of the Gemma-4 text-encoder attention (``ltx_gemma_attn_fwd``) against the
oracle's restatement of GemmaTextEncoder.swift:158-239 with the mask of :288-321.

Tolerance (the target's): relative RMS error <= 5e-3 and max-abs <= 2e-2 on the outputs
(fp32 here, the dtype of the reference's explicit path) against the float64 oracle of the same
inputs; in addition the kernel may be at most 1.25x as far from the truth as the reference's
own arithmetic (``mode="reference"``: bf16 norms, fp32 RoPE and softmax), with a 2.5e-3
floor. Stress cases with logits far beyond the checkpoint's take only the relative bound.
"""

import os

import numpy as np
import pytest

import ltx_attn as L
import oracle as O

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _dev(bits, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(device).view(
        torch.bfloat16)


def _run(device, case):
    import torch

    B, T, kind, fv, seed = case["B"], case["T"], case["kind"], case["fv"], case["seed"]
    spec = dict(L.GEMMA_SLIDING if kind == "sliding" else L.GEMMA_FULL)
    if "window" in case:
        spec["window"] = case["window"]
    D, Hq, Hkv = spec["head_dim"], spec["q_heads"], spec["kv_heads"]
    q = O.randn_bf16_bits((B, T, Hq * D), seed)
    k = O.randn_bf16_bits((B, T, Hkv * D), seed + 1)
    v = k if spec["shares_kv"] else O.randn_bf16_bits((B, T, Hkv * D), seed + 2)
    # weights at the checkpoint's magnitudes: q_norm ~1.03, k_norm ~0.12 (D 256) / ~0.06 (D 512)
    wq = O.randn_bf16_bits((D,), seed + 3, mean=1.03, std=0.02)
    wk = O.randn_bf16_bits((D,), seed + 4, mean=case.get("wk_mean", 0.12 if D == 256 else 0.06),
                           std=0.01)
    cos, sin = L.gemma_rope_tables(T, D, spec["theta"], spec["partial"], spec["proportional"])
    tq, tk = _dev(q, device), _dev(k, device)
    tv = tk if spec["shares_kv"] else _dev(v, device)
    out = L.gemma_attention_fwd(tq, tk, tv, q_heads=Hq, kv_heads=Hkv,
                                q_norm_w=_dev(wq, device), k_norm_w=_dev(wk, device),
                                cos=torch.from_numpy(cos).to(device),
                                sin=torch.from_numpy(sin).to(device),
                                window=spec["window"], first_valid=fv)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    kw = dict(window=spec["window"], first_valid=fv)
    truth = O.gemma_attention(q, k, v, Hq, Hkv, wq, wk, cos, sin, mode="exact", **kw)
    if case.get("absolute_only"):
        return got, truth, None
    ref = O.gemma_attention(q, k, v, Hq, Hkv, wq, wk, cos, sin, mode="reference", **kw)
    return got, truth, ref


CASES = {
    # the layers at the encoder's 1024 tokens: 94 real tokens left-padded to 1024, and none
    "sliding_1024_pad930": dict(B=1, T=1024, kind="sliding", fv=[930], seed=0x5EED + 400),
    "full_1024_pad930": dict(B=1, T=1024, kind="full", fv=[930], seed=0x5EED + 410),
    "sliding_1024_nopad": dict(B=1, T=1024, kind="sliding", fv=[0], seed=0x5EED + 420),
    "full_1024_nopad": dict(B=1, T=1024, kind="full", fv=[0], seed=0x5EED + 430),
    # a window shorter than the sequence, ragged T, two prompts with different padding
    "sliding_window40_T100_B2": dict(B=2, T=100, kind="sliding", fv=[0, 37], window=40,
                                     seed=0x5EED + 440),
    "full_T68_B2": dict(B=2, T=68, kind="full", fv=[67, 3], seed=0x5EED + 450),
    # a fully padded prompt (first_valid == T): no row has an allowed key, so every row
    # attends to all keys unmasked (GemmaTextEncoder.swift:306-319)
    "sliding_T100_fully_padded": dict(B=1, T=100, kind="sliding", fv=[100], seed=0x5EED + 460),
    "full_T64_B2_one_fully_padded": dict(B=2, T=64, kind="full", fv=[64, 10],
                                         seed=0x5EED + 470),
    # windows below one 32-key block: the key range starts and ends inside a block
    "sliding_window1_T92": dict(B=1, T=92, kind="sliding", fv=[0], window=1, seed=0x5EED + 480),
    "sliding_window17_T92_B2": dict(B=2, T=92, kind="sliding", fv=[0, 50], window=17,
                                    seed=0x5EED + 490),
    # 8 KV heads at a ragged length with a window and padding in the same prompt
    "sliding_window17_T76_pad5": dict(B=1, T=76, kind="sliding", fv=[5], window=17,
                                      seed=0x5EED + 500),
    # prompts longer than 32 key blocks: the latest query blocks' keys run as up to four
    # ranges of 16 blocks merged afterwards, with padding and (sliding) a window inside them
    "sliding_window700_T1600_pad200": dict(B=1, T=1600, kind="sliding", fv=[200], window=700,
                                           seed=0x5EED + 510),
    "full_T1600_pad200": dict(B=1, T=1600, kind="full", fv=[200], seed=0x5EED + 520),
    # two rows that split differently (the second's padding leaves fewer key blocks): each
    # row's partials sit at their own offset
    "full_T1600_B2_pad0_900": dict(B=2, T=1600, kind="full", fv=[0, 900], seed=0x5EED + 550),
    # 65 query blocks of 64: the split blocks before the last number more than a wave's 64
    # lanes, so the partial offset is counted over two passes of the wave. The float64 truth
    # only (the bound relative to the reference's arithmetic would double the oracle's time).
    "full_T4160": dict(B=1, T=4160, kind="full", fv=[0], seed=0x5EED + 560, absolute_only=True),
    # k_norm weights 25x the checkpoint's: logits with a spread of ~70 (log2 units), so later
    # key blocks pass a row's first-block max by more than 2^15 and the workgroups rerun their
    # range with the exact online softmax. Logits that large amplify the inputs' bf16
    # rounding (the reference's own arithmetic is ~2e-2 off), so only the bound relative to
    # the reference's arithmetic applies.
    "sliding_1024_large_logits": dict(B=1, T=1024, kind="sliding", fv=[0], wk_mean=3.0,
                                      seed=0x5EED + 530, relative_only=True),
    "full_1024_large_logits": dict(B=1, T=1024, kind="full", fv=[0], wk_mean=3.0,
                                   seed=0x5EED + 540, relative_only=True),
}




def _random_case(i):
    """Seeded draws of batch, prompt length (a multiple of 4, as the call requires), layer
    kind, window and left padding per row (padding up to the whole prompt), for shapes no
    hand-written case names."""
    rng = np.random.default_rng(0x5EED + 7000 + i)
    B = int(rng.choice([1, 2]))
    T = 4 * max(1, int(np.exp(rng.uniform(np.log(4), np.log(1400)))) // 4)   # a multiple of 4
    kind = str(rng.choice(["sliding", "full"]))
    case = dict(B=B, T=T, kind=kind, seed=int(rng.integers(1, 1 << 30)),
                fv=[int(rng.integers(0, T + 1)) if rng.random() < 0.5 else 0 for _ in range(B)])
    if kind == "sliding" and rng.random() < 0.5:
        case["window"] = int(rng.integers(1, T + 1))
    return case


# 8 cases by default; LTX_GEMMA_RANDOM_CASES=n runs the first n seeds of the same sequence.
CASES.update({f"random_{i}": _random_case(i)
              for i in range(int(os.environ.get("LTX_GEMMA_RANDOM_CASES", "8")))})


@pytest.mark.parametrize("name", sorted(CASES))
def test_gemma_attention(device, name):
    _say(f"gemma {name}")
    got, truth, ref = _run(device, CASES[name])
    c = O.compare(got, truth)
    if ref is None:
        _say(f"  relRMS {c['rel_rms']:.3e} maxAbs {c['max_abs']:.3e}")
    else:
        r = O.compare(ref, truth)
        _say(f"  relRMS {c['rel_rms']:.3e} maxAbs {c['max_abs']:.3e} "
             f"(reference arithmetic relRMS {r['rel_rms']:.3e})")
    if not CASES[name].get("relative_only"):
        assert c["rel_rms"] <= 5e-3, c
        assert c["max_abs"] <= 2e-2, c
    if ref is not None:
        assert c["rel_rms"] <= max(r["rel_rms"], 2.5e-3) * 1.25, (c, r)
