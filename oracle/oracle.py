"""CPU oracle for the LTX 2.5 DiT attention path (QK-RMSNorm -> split RoPE -> SDPA).

TEST INFRASTRUCTURE ONLY. Nothing in the shipped library imports, links or calls this
module; only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
use it, and only as the parity reference. The product path is the HIP library in
``ltx-2.5-swift_amd/``.

This is a numpy restatement of the reference's arithmetic:

* ``rms_norm``       -- ``Sources/LTXModules/DiTAttention.swift:190-204`` (statistic over the
                        whole inner dim ``H*D`` per token, eps 1e-6, weight cast to bf16),
                        fp32 statistic per ``Sources/LTXModules/DiTBlock.swift:219-221``.
* head split         -- ``DiTAttention.swift:346-349`` (head ``h`` = channels ``[h*D,(h+1)*D)``).
* ``split_rope``     -- ``DiTAttention.swift:206-234`` (contiguous halves, not interleaved;
                        bf16 x bf16 elementwise, each op rounded, no upcast).
* ``sdpa``           -- the explicit path ``DiTAttention.swift:377-381``: fp32 logits
                        ``Q.K^T * scale``, fp32 softmax, fp32 ``P.V``, cast to bf16. The fused
                        path (``:374-376``) computes the same function.
* key padding        -- additive ``-finfo(bf16).max`` per ``Sources/LTXFoundation/
                        TextConditioningLayout.swift:94-107``; with at least one valid key it
                        equals SDPA restricted to the valid keys, which is what ``sdpa``
                        computes. Zero valid keys is rejected (``TextConditioningLayout.swift:65``
                        throws ``emptyMask``).
* ``linear``         -- ``DiTAttention.swift:178-188``: ``x . w^T`` in the weight's dtype
                        (bf16 out of an fp32 accumulation), then ``+ bias`` as a bf16 add.
* ``sumsq_partials`` -- the RMS statistic of a projection's bf16 output, summed per block of
                        256 columns (what ``ltx_linear`` emits for ``rms_norm``).
* ``attention_module`` -- ``DiTAttention.callAsFunction`` (``:315-405``): projections, the
                        replaced unit, the gate from ``x`` and ``to_out``.
* RoPE tables        -- ``Sources/LTXModules/DiTForward.swift:455-466`` (``frequencyGrid``),
                        ``:486-520`` (``videoPositions``), ``:553-593``
                        (``referencePositions``, IC-LoRA / MSR reference clips),
                        ``:606-619`` (``audioPositions``),
                        ``:641-678`` (``rotary``), ``:698-738`` (``rotaries``).

Gemma-4 text-encoder attention (``Sources/LTXModules/GemmaTextEncoder.swift``):

* ``gemma_inverse_frequencies`` -- ``Sources/LTXFoundation/GemmaAttentionSpec.swift:88-121``
                        (``default`` divides by the rotated width, ``proportional`` by the full
                        head dim and zero-pads the non-rotating tail).
* ``gemma_rope_tables`` -- ``GemmaTextEncoder.swift:135-145``: fp32 angles ``position *
                        inv_freq``, fp32 cos/sin, per token, shared by the heads.
* ``gemma_attention``   -- ``GemmaTextEncoder.swift:158-239`` (per-head q/k RMS norm with
                        ``pow(mean + eps, -0.5)`` and the weight, no ``1 +``; ``rotate_half``
                        RoPE; V normed by a weightless norm and never rotated, taken from the
                        pre-norm K projection on the K-shares-V layers; GQA by repeating KV
                        heads; scale 1.0; the explicit fp32 path) with the mask of
                        ``:288-321`` (causal, sliding window, key padding, fully-masked rows
                        un-masked).

Two arithmetic modes:

* ``mode="exact"``     float64 everywhere from the bf16 inputs (norm, RoPE and SDPA in
                        float64, nothing rounded) -- the truth the tolerance is measured against.
* ``mode="reference"`` the reference's rounding points: normed q/k rounded to bf16, each
                        RoPE multiply/add rounded to bf16, logits/softmax/PV in fp32
                        (accumulated here in float64, which is fp32 with exact summation).

Pinning (each function is checked in ``tests/test_oracle.py`` against something other than
its own formula): closed forms (MLXCapabilityTests' uniform case, Lk=1 -> V, equal keys ->
mean V, scale 0 -> mean V, masked == truncated), invariants (key/value permutation, row
shift, per-pair RoPE norm, relative-position property of the rotation), a pure-Python
brute-force SDPA on tiny inputs, the independent C restatement in ``attn_oracle.c``, and the
tiny_v5 manifest digests of the reference's RoPE tables
(``Tests/Fixtures/goldens/tiny_v5/manifest.json``, keys ``block_00.*.in.kw_pe*``).
``compare`` (the pass/fail gate of every GPU test) is pinned by hand-worked cases including
the zero-reference branch; ``splitmix64`` by the published splitmix64 outputs for seed 0 and
``splitmix_bf16_bits`` by a hand-rounded word and the half-step bound.
"""

from __future__ import annotations

import math

import numpy as np

__all__ = [
    "f32_to_bf16_bits", "bf16_bits_to_f32", "round_bf16", "randn_bf16_bits",
    "splitmix64", "splitmix_bf16_bits", "rms_norm", "split_rope", "sdpa", "head_gate", "attention",
    "linear", "sumsq_partials", "attention_module",
    "frequency_grid", "video_positions", "reference_positions",
    "video_positions_with_references", "audio_positions", "rotary_tables",
    "rotaries", "compare",
]

BF16_MAX = float(np.float32(3.3895313892515355e38))


# --------------------------------------------------------------------------------------
# bf16 helpers (round-to-nearest-even, as Sources/ltx/Bench.swift:462-469)
# --------------------------------------------------------------------------------------

def f32_to_bf16_bits(x) -> np.ndarray:
    """RNE fp32 -> bf16 bit pattern (``BenchOperand.bf16Bits``, ``Bench.swift:462-469``)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = (u + np.uint32(0x7FFF) + ((u >> 16) & 1)) >> 16
    r = np.where(nan, (u >> 16) | 0x40, r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b) -> np.ndarray:
    """bf16 bit pattern -> fp32 (``BenchOperand.float(ofBf16:)``, ``Bench.swift:471-473``)."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x) -> np.ndarray:
    """Round to bf16 and back to fp32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(x, dtype=np.float32)))


def randn_bf16_bits(shape, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """Seeded N(mean, std) draws rounded to bf16 -- the synthetic operands of every config."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(size=shape, dtype=np.float32) * np.float32(std) + np.float32(mean)
    return f32_to_bf16_bits(x)


SPLITMIX_GAMMA = 0x9E3779B97F4A7C15


def splitmix64(count: int, seed: int) -> np.ndarray:
    """The 64-bit words behind the reference bench's operands (``Bench.swift:479-490``).

    The state starts at ``seed + gamma`` and is advanced by ``gamma`` BEFORE each word is
    mixed, so word ``i`` is the standard splitmix64 output ``i + 1`` of a generator seeded
    with ``seed`` (the first output of the standard generator is skipped).
    """
    # state before mixing word i: seed + (i + 2) * gamma, modulo 2^64 (uint64 arithmetic
    # wraps exactly that way)
    with np.errstate(over="ignore"):
        z = (np.uint64(seed % (1 << 64)) + np.uint64(SPLITMIX_GAMMA) *
             (np.arange(count, dtype=np.uint64) + np.uint64(2)))
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def splitmix_bf16_bits(count: int, seed: int) -> np.ndarray:
    """The reference bench's operand stream: splitmix64 -> uniform [-1, 1) -> bf16.

    Restates ``BenchOperand.bits(count:seed:)`` (``Sources/ltx/Bench.swift:479-493``): the
    top 24 bits of each word over 2^24 (exact in fp32), centred and doubled, RNE to bf16.
    """
    top = (splitmix64(count, seed) >> np.uint64(40)).astype(np.float32)
    unit = top / np.float32(1 << 24)
    return f32_to_bf16_bits((unit - np.float32(0.5)) * np.float32(2))


# --------------------------------------------------------------------------------------
# QK-RMSNorm over the inner dim (DiTAttention.swift:190-204)
# --------------------------------------------------------------------------------------

def rms_norm(x: np.ndarray, w: np.ndarray, eps: float = 1e-6, mode: str = "exact") -> np.ndarray:
    """``y = x * rsqrt(mean(x^2 over the LAST axis) + eps) * w``.

    ``x`` is ``[..., inner]`` (inner = H*D, all heads of one token), ``w`` is ``[inner]``.
    The statistic spans every head -- ``q_norm.weight`` is ``[4096]``/``[2048]``, one weight
    per inner channel (``DiTAttention.swift:190-197``).
    """
    if mode == "exact":
        x64 = np.asarray(x, dtype=np.float64)
        ms = np.mean(x64 * x64, axis=-1, keepdims=True)
        return x64 / np.sqrt(ms + eps) * np.asarray(w, dtype=np.float64)
    x32 = np.asarray(x, dtype=np.float32)
    # fp32 statistic (summed exactly), fp32 normalise-and-weight, one bf16 rounding.
    ms = np.mean(x32.astype(np.float64) ** 2, axis=-1, keepdims=True).astype(np.float32)
    rstd = (np.float32(1.0) / np.sqrt(ms + np.float32(eps))).astype(np.float32)
    y = (x32 * rstd) * np.asarray(w, dtype=np.float32)
    return round_bf16(y)


# --------------------------------------------------------------------------------------
# Split-half RoPE (DiTAttention.swift:206-234)
# --------------------------------------------------------------------------------------

def split_rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, mode: str = "exact") -> np.ndarray:
    """``[x1*cos - x2*sin, x2*cos + x1*sin]`` with ``x1 = x[..., :D/2]``, ``x2 = x[..., D/2:]``.

    ``x`` is ``[B, H, L, D]``; ``cos``/``sin`` are ``[H, L, D/2]`` (the reference's
    ``[1, H, L, D/2]`` broadcast over batch). In ``reference`` mode every multiply and
    add is rounded to bf16, as MLX's bf16 elementwise ops do (no upcast,
    ``DiTAttention.swift:222-234``).
    """
    d = x.shape[-1]
    half = d // 2
    if mode == "exact":
        x = np.asarray(x, dtype=np.float64)
        c = np.asarray(cos, dtype=np.float64)[None]
        s = np.asarray(sin, dtype=np.float64)[None]
        x1, x2 = x[..., :half], x[..., half:]
        return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1)
    x = np.asarray(x, dtype=np.float32)
    c = np.asarray(cos, dtype=np.float32)[None]
    s = np.asarray(sin, dtype=np.float32)[None]
    x1, x2 = x[..., :half], x[..., half:]
    r = round_bf16
    o1 = r(r(x1 * c) - r(x2 * s))
    o2 = r(r(x2 * c) + r(x1 * s))
    return np.concatenate([o1, o2], axis=-1)


# --------------------------------------------------------------------------------------
# SDPA (explicit path, DiTAttention.swift:377-381)
# --------------------------------------------------------------------------------------

def sdpa(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float,
         valid_len=None) -> np.ndarray:
    """``softmax(q k^T * scale) v`` per (b, h), float64.

    ``q`` ``[B, H, Lq, D]``, ``k``/``v`` ``[B, H, Lk, D]``. ``valid_len[b]`` keeps the first
    ``n`` keys of batch row ``b`` (key-padding mask); ``None`` keeps all.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B = q.shape[0]
    out = np.empty(q.shape[:-1] + (v.shape[-1],), dtype=np.float64)
    for b in range(B):
        n = k.shape[2] if valid_len is None else int(valid_len[b])
        if n < 1:
            raise ValueError("a key-padding mask with no valid key (emptyMask)")
        logits = np.matmul(q[b], np.swapaxes(k[b, :, :n], -1, -2)) * scale
        logits -= logits.max(axis=-1, keepdims=True)
        p = np.exp(logits)
        p /= p.sum(axis=-1, keepdims=True)
        out[b] = np.matmul(p, v[b, :, :n])
    return out


def head_gate(logit_bits, mode: str = "exact") -> np.ndarray:
    """Per-head output gate ``2 * sigmoid(logits)`` (``DiTAttention.swift:395-399``).

    ``logit_bits``: bf16 bits ``[B, L, H]`` (``to_gate_logits(x)``). ``mode="exact"`` returns
    float64; ``mode="reference"`` rounds to bf16, the dtype of the reference's gate array.
    """
    x = bf16_bits_to_f32(logit_bits).astype(np.float64)
    g = 2.0 / (1.0 + np.exp(-x))
    return g if mode == "exact" else round_bf16(g)


def _split_heads(x_bits: np.ndarray, heads: int) -> np.ndarray:
    """``[B, L, H*D]`` -> ``[B, H, L, D]`` fp32 (``DiTAttention.swift:346-349``)."""
    B, L, inner = x_bits.shape
    x = bf16_bits_to_f32(x_bits)
    return x.reshape(B, L, heads, inner // heads).transpose(0, 2, 1, 3)


def attention(q_bits, k_bits, v_bits, heads: int, *, q_norm_w=None, k_norm_w=None,
              eps: float = 1e-6, q_cos=None, q_sin=None, k_cos=None, k_sin=None,
              valid_len=None, scale=None, mode: str = "exact", gate_bits=None) -> np.ndarray:
    """The replaced unit ``DiTAttention.swift:358-381`` from the pre-norm projections, and with
    ``gate_bits`` (bf16 bits ``[B, Lq, H]``) the per-head gate of ``:395-399``.

    Inputs are bf16 bit patterns: ``q_bits`` ``[B, Lq, H*D]``, ``k_bits``/``v_bits``
    ``[B, Lk, H*D]``; norm weights ``[H*D]`` bits or None (inputs already normed); RoPE
    tables ``[H, L, D/2]`` bits or None (no rotation; ``k_*`` None with ``q_*`` given means
    "use q's", as ``keyRotary ?? rotary`` at ``DiTAttention.swift:366``).
    Returns float64 ``[B, Lq, H*D]`` (merged layout, before the final bf16 cast).
    """
    B, Lq, inner = q_bits.shape
    D = inner // heads
    if scale is None:
        scale = float(np.float32(1.0 / math.sqrt(D)))  # DiTAttention.swift:372
    q = bf16_bits_to_f32(q_bits)
    k = bf16_bits_to_f32(k_bits)
    if q_norm_w is not None:
        q = rms_norm(q, bf16_bits_to_f32(q_norm_w), eps, mode)
    if k_norm_w is not None:
        k = rms_norm(k, bf16_bits_to_f32(k_norm_w), eps, mode)

    def heads4(x):
        Bx, L, _ = x.shape
        return np.asarray(x).reshape(Bx, L, heads, D).transpose(0, 2, 1, 3)

    qh, kh = heads4(q), heads4(k)
    vh = _split_heads(v_bits, heads)
    if q_cos is not None:
        qc, qs = bf16_bits_to_f32(q_cos), bf16_bits_to_f32(q_sin)
        kc = qc if k_cos is None else bf16_bits_to_f32(k_cos)
        ks = qs if k_sin is None else bf16_bits_to_f32(k_sin)
        qh = split_rope(qh, qc, qs, mode)
        kh = split_rope(kh, kc, ks, mode)
    o = sdpa(qh, kh, vh, scale, valid_len)
    o = o.transpose(0, 2, 1, 3)                       # [B, Lq, H, D]
    if gate_bits is not None:
        if mode != "exact":
            o = round_bf16(o)                         # the attention output is bf16 (:381)
        o = o * head_gate(gate_bits, mode)[..., None]
    return o.reshape(B, Lq, inner)


# --------------------------------------------------------------------------------------
# Projections and the whole module (DiTAttention.swift:178-188, :315-405)
# --------------------------------------------------------------------------------------

def linear(x_bits, w_bits, bias_bits=None, mode: str = "exact") -> np.ndarray:
    """``linear(_:_:)`` (``DiTAttention.swift:178-188``): ``y = x . w^T (+ bias)``.

    ``x_bits`` ``[..., K]``, ``w_bits`` ``[N, K]`` (the checkpoint's ``[out, in]``),
    ``bias_bits`` ``[N]`` or None -- bf16 bit patterns. ``mode="exact"``: float64, nothing
    rounded. ``mode="reference"``: the matmul's bf16 output (the exact sum rounded to fp32,
    then to bf16: an fp32 accumulation up to its summation order), then the bias added as
    two bf16 values in fp32 and rounded to bf16 (``:180``, ``:186``). LoRA deltas
    (``:183-185``) are not part of this function.
    """
    x = bf16_bits_to_f32(x_bits).astype(np.float64)
    w = bf16_bits_to_f32(w_bits).astype(np.float64)
    y = x @ w.T
    b = None if bias_bits is None else bf16_bits_to_f32(bias_bits)
    if mode == "exact":
        return y if b is None else y + b
    y = round_bf16(y.astype(np.float32))
    if b is not None:
        y = round_bf16((y + b).astype(np.float32))
    return y


def sumsq_partials(y, cols: int = 256) -> np.ndarray:
    """Sums of squares of ``y`` ``[..., N]`` over the column blocks ``[cols*j, cols*j + cols)``
    (float64, ``[..., ceil(N/cols)]``); their row sum is the ``rms_norm`` statistic times N."""
    y = np.asarray(y, dtype=np.float64)
    N = y.shape[-1]
    nb = -(-N // cols)
    pad = np.zeros(y.shape[:-1] + (nb * cols - N,))
    yp = np.concatenate([y, pad], axis=-1).reshape(y.shape[:-1] + (nb, cols))
    return (yp * yp).sum(axis=-1)


def attention_module(x_bits, weights: dict, heads: int, *, context_bits=None, q_cos=None,
                     q_sin=None, k_cos=None, k_sin=None, valid_len=None,
                     all_perturbed: bool = False, eps: float = 1e-6,
                     mode: str = "reference") -> np.ndarray:
    """``DiTAttention.callAsFunction`` (``DiTAttention.swift:315-405``) for one module.

    ``weights`` maps the module's tensor names (``to_q.weight``, ``to_q.bias``, ``to_k.*``,
    ``to_v.*``, ``q_norm.weight``, ``k_norm.weight``, optional ``to_gate_logits.*``,
    ``to_out.0.*``; biases optional) to bf16 bit arrays. ``context_bits`` None means
    self-attention (``:327``). Between operations the data is bf16 as in the reference: each
    projection output, the attention output (``:381``) and the gated output (``:397-399``) are
    rounded to bf16; ``mode`` is the arithmetic inside each operation. Returns float64
    ``[B, Lq, out]`` (before ``to_out``'s final rounding in ``mode="exact"``, rounded in
    ``"reference"``).
    """
    kv_bits = x_bits if context_bits is None else context_bits

    def lin(t_bits, name):
        return linear(t_bits, weights[name + ".weight"], weights.get(name + ".bias"), mode)

    bits = lambda y: f32_to_bf16_bits(np.asarray(y, dtype=np.float32))   # noqa: E731
    v = bits(lin(kv_bits, "to_v"))
    B, Lq = x_bits.shape[0], x_bits.shape[1]
    inner = v.shape[-1]
    if all_perturbed:
        o = bf16_bits_to_f32(v).astype(np.float64)                # :351-356
    else:
        q = bits(lin(x_bits, "to_q"))
        k = bits(lin(kv_bits, "to_k"))
        o = attention(q, k, v, heads, q_norm_w=weights["q_norm.weight"],
                      k_norm_w=weights["k_norm.weight"], eps=eps, q_cos=q_cos, q_sin=q_sin,
                      k_cos=k_cos, k_sin=k_sin, valid_len=valid_len, mode=mode)
    o = round_bf16(o)                                               # bf16 attention output
    if "to_gate_logits.weight" in weights:
        g = head_gate(bits(lin(x_bits, "to_gate_logits")), "reference")
        o = round_bf16(o.reshape(B, Lq, heads, inner // heads) * g[..., None]).reshape(o.shape)
    return lin(bits(o), "to_out.0")


# --------------------------------------------------------------------------------------
# RoPE tables (DiTForward.swift:440-738)
# --------------------------------------------------------------------------------------

def frequency_grid(theta: float, positional_dimensions: int, inner_dim: int) -> np.ndarray:
    """``f_i = theta^(i * step) * pi/2`` in float64 with the endpoint overwritten, -> fp32.

    ``DiTForward.swift:455-466``: ``step = 1/(n-1)``, exponent ``i*step`` except the last,
    which is exactly 1.
    """
    count = inner_dim // (2 * positional_dimensions)
    if count <= 1:
        raise ValueError("a one-element grid has no linspace step")
    step = 1.0 / float(count - 1)
    vals = np.empty(count, dtype=np.float32)
    for i in range(count):
        e = 1.0 if i == count - 1 else float(i) * step
        vals[i] = np.float32(math.pow(theta, e) * math.pi / 2)
    return vals


def video_positions(latent_frames: int, latent_height: int, latent_width: int,
                    temporal_scale: int = 8, spatial_scale: int = 32,
                    frame_rate: float = 24.0) -> np.ndarray:
    """Patch bounds ``[1, 3, tokens, 2]`` fp32; token order (t, y, x), x fastest.

    ``DiTForward.swift:486-520``: integer pixel bounds, causal time correction
    ``max(v + 1 - temporalScale, 0)``, then time divided by the frame rate in fp32.
    """
    tokens = latent_frames * latent_height * latent_width
    out = np.zeros((1, 3, tokens, 2), dtype=np.float32)
    scales = (temporal_scale, spatial_scale, spatial_scale)
    fr = np.float32(frame_rate)
    tok = 0
    for t in range(latent_frames):
        for y in range(latent_height):
            for x in range(latent_width):
                start = (t, y, x)
                for dim in range(3):
                    lo = start[dim] * scales[dim]
                    hi = (start[dim] + 1) * scales[dim]
                    if dim == 0:
                        lo = max(lo + 1 - temporal_scale, 0)
                        hi = max(hi + 1 - temporal_scale, 0)
                    lo_f, hi_f = np.float32(lo), np.float32(hi)
                    if dim == 0:
                        lo_f = np.float32(lo_f / fr)
                        hi_f = np.float32(hi_f / fr)
                    out[0, dim, tok, 0] = lo_f
                    out[0, dim, tok, 1] = hi_f
                tok += 1
    return out


def reference_positions(latent_frames: int, latent_height: int, latent_width: int, *,
                        frame_rate: float = 24.0, downscale_factor: int = 1,
                        temporal_scale_factor: int = 1, frame_offset: int = 0,
                        target=None, temporal_scale: int = 8,
                        spatial_scale: int = 32) -> np.ndarray:
    """An in-context reference's bounds ``[1, 3, tokens, 2]`` in the target's frame
    (``DiTForward.swift:553-593``): its own grid at frame rate 1 (pixel frames), the offset
    added in pixel frames, then divided by ``float(fps / temporalScaleFactor)``; a temporally
    sparse reference is slid by ``(factor - 1) * target[0, 0, 0, 1]`` and clamped at 0; the
    spatial axes are multiplied by the downscale factor. All in fp32, step by step."""
    if frame_offset != 0 and temporal_scale_factor != 1:
        raise ValueError("a reference cannot carry both a frame offset and a temporal scale")
    grid = video_positions(latent_frames, latent_height, latent_width, temporal_scale,
                           spatial_scale, 1.0)
    time = grid[:, 0:1].copy()
    space = grid[:, 1:3].copy()
    if frame_offset != 0:
        time = (time + np.float32(frame_offset)).astype(np.float32)
    time = (time / np.float32(frame_rate / float(temporal_scale_factor))).astype(np.float32)
    if temporal_scale_factor != 1:
        t_target = np.float32(np.asarray(target, dtype=np.float32)[0, 0, 0, 1])
        shift = np.float32(np.float32(temporal_scale_factor - 1) * t_target)
        time = np.maximum((time - shift).astype(np.float32), np.float32(0.0))
    if downscale_factor != 1:
        space = (space * np.float32(downscale_factor)).astype(np.float32)
    return np.concatenate([time, space], axis=1)


def video_positions_with_references(latent_frames: int, latent_height: int, latent_width: int,
                                    references, frame_rate: float = 24.0) -> np.ndarray:
    """``rotaries``' video grid with references (``DiTForward.swift:698-711``): the target's
    grid, then every reference's (dicts of ``reference_positions`` keywords plus
    ``latent_frames/height/width``), each shifted against the target's own grid."""
    target = video_positions(latent_frames, latent_height, latent_width, 8, 32, frame_rate)
    blocks = [target]
    for ref in references:
        kw = dict(ref)
        dims = (kw.pop("latent_frames"), kw.pop("latent_height"), kw.pop("latent_width"))
        blocks.append(reference_positions(*dims, frame_rate=frame_rate, target=target, **kw))
    return np.concatenate(blocks, axis=2)


def audio_positions(tokens: int, hop_length: int = 160, sample_rate: int = 16000,
                    downsample: int = 4) -> np.ndarray:
    """Audio bounds ``[1, 1, tokens, 2]`` in seconds (``DiTForward.swift:606-619``)."""
    def seconds(i):
        frame = np.float32(i * downsample)
        frame = max(np.float32(frame + np.float32(1) - np.float32(downsample)), np.float32(0))
        return np.float32(np.float32(frame * np.float32(hop_length)) / np.float32(sample_rate))

    out = np.zeros((1, 1, tokens, 2), dtype=np.float32)
    for i in range(tokens):
        out[0, 0, i, 0] = seconds(i)
        out[0, 0, i, 1] = seconds(i + 1)
    return out


def rotary_tables(positions: np.ndarray, inner_dim: int, max_pos, heads: int = 32,
                  theta: float = 10000.0, as_bits: bool = True):
    """cos/sin ``[H, tokens, inner/2/H]`` from patch bounds (``DiTForward.swift:641-678``).

    Centre of each ``[start, end)`` pair over ``maxPos`` -> ``angle = f * (2*frac - 1)``,
    positional dimension fastest, leading identity padding, per-head reshape, bf16 cast.
    Returns bf16 bits (default) or fp32 values.
    """
    n_pos = positions.shape[1]
    tokens = positions.shape[2]
    if len(max_pos) != n_pos:
        raise ValueError("maxPos length must equal the positional dimension count")
    bounds = positions.astype(np.float32)
    middle = ((bounds[0, :, :, 0] + bounds[0, :, :, 1]) / np.float32(2.0)).astype(np.float32)
    frac = np.stack([middle[d] / np.float32(max_pos[d]) for d in range(n_pos)], axis=-1)
    frac = frac.astype(np.float32)                                # [tokens, nPos]
    freqs = frequency_grid(theta, n_pos, inner_dim)               # [count]
    scaled = (frac * np.float32(2.0) - np.float32(1.0)).astype(np.float32)
    angles = (freqs[None, None, :] * scaled[:, :, None]).astype(np.float32)  # [T, nPos, cnt]
    ordered = angles.transpose(0, 2, 1).reshape(tokens, freqs.size * n_pos)
    cos = np.cos(ordered).astype(np.float32)
    sin = np.sin(ordered).astype(np.float32)
    pad = inner_dim // 2 - ordered.shape[-1]
    if pad < 0:
        raise ValueError("inner dim cannot hold the frequencies")
    if pad > 0:
        cos = np.concatenate([np.ones((tokens, pad), np.float32), cos], axis=-1)
        sin = np.concatenate([np.zeros((tokens, pad), np.float32), sin], axis=-1)
    per_head = inner_dim // 2 // heads
    cos = cos.reshape(tokens, heads, per_head).transpose(1, 0, 2)
    sin = sin.reshape(tokens, heads, per_head).transpose(1, 0, 2)
    if as_bits:
        return (np.ascontiguousarray(f32_to_bf16_bits(cos)),
                np.ascontiguousarray(f32_to_bf16_bits(sin)))
    return np.ascontiguousarray(cos), np.ascontiguousarray(sin)


def rotaries(frames: int, height: int, width: int, frame_rate: float = 24.0,
             video_width: int = 4096, audio_width: int = 2048, heads: int = 32,
             theta: float = 10000.0, video_max_pos=(20, 2048, 2048), audio_max_pos=(20,),
             cross_max_pos: int = 20, audio_tokens=None):
    """The four tables a block uses (``DiTForward.swift:698-738``).

    Returns a dict ``videoSelf``/``audioSelf``/``videoCross``/``audioCross`` of
    ``(cos_bits, sin_bits)``. Geometry per ``LatentGeometry`` defaults: spatial scale 32,
    temporal scale 8, audio ``round(frames/fps*25)`` tokens.
    """
    latent_frames = 1 if frames <= 1 else (frames - 1) // 8 + 1
    video = video_positions(latent_frames, height // 32, width // 32, 8, 32, frame_rate)
    if audio_tokens is None:
        audio_tokens = int(round(frames / frame_rate * 25.0))
    audio = audio_positions(audio_tokens)
    time = video[:, 0:1]
    return {
        "videoSelf": rotary_tables(video, video_width, list(video_max_pos), heads, theta),
        "audioSelf": rotary_tables(audio, audio_width, list(audio_max_pos), heads, theta),
        "videoCross": rotary_tables(time, audio_width, [cross_max_pos], heads, theta),
        "audioCross": rotary_tables(audio, audio_width, [cross_max_pos], heads, theta),
    }


# --------------------------------------------------------------------------------------
# Comparison (BenchComparison, Sources/ltx/Bench.swift:508-536)
# --------------------------------------------------------------------------------------

# ---------------------------------------------------------------------------------------
# Gemma-4 text-encoder attention
# ---------------------------------------------------------------------------------------

def gemma_inverse_frequencies(head_dim: int, theta: float, partial_factor: float,
                              rope_type: str) -> np.ndarray:
    """``GemmaAttentionSpec.inverseFrequencies`` (GemmaAttentionSpec.swift:88-121), float64,
    length ``head_dim / 2``."""
    half = head_dim // 2
    out = np.zeros(half, dtype=np.float64)
    if rope_type == "proportional":
        n = int(partial_factor * head_dim / 2.0)
        for i in range(min(n, half)):
            out[i] = 1.0 / theta ** (2.0 * i / head_dim)
        return out
    dim = int(head_dim * partial_factor)
    res = np.zeros(dim // 2, dtype=np.float64)
    for i in range(dim // 2):
        res[i] = 1.0 / theta ** (2.0 * i / dim)
    return res


def gemma_rope_tables(tokens: int, inv_freq: np.ndarray):
    """fp32 ``cos``, ``sin`` ``[tokens, head_dim/2]`` (GemmaTextEncoder.swift:135-145): the
    frequencies narrowed to fp32, fp32 angles ``position * inv``, fp32 cos/sin (the table is
    duplicated over the two halves of a head, which ``rotate_half`` pairs)."""
    inv = np.asarray(inv_freq, dtype=np.float32)
    pos = np.arange(tokens, dtype=np.float32)[:, None]
    ang = (pos * inv[None, :]).astype(np.float32)
    return (np.cos(ang.astype(np.float64)).astype(np.float32),
            np.sin(ang.astype(np.float64)).astype(np.float32))


def gemma_mask(tokens: int, window: int = 0, first_valid: int = 0) -> np.ndarray:
    """Allowed (query, key) pairs (GemmaTextEncoder.swift:288-321): causal, keys within the
    sliding window when one is set, keys before ``first_valid`` (left padding) never; rows
    left with no allowed key are un-masked entirely."""
    rows = np.arange(tokens)[:, None]
    cols = np.arange(tokens)[None, :]
    allowed = cols <= rows
    if window > 0:
        allowed &= (rows - cols) < window
    allowed &= cols >= first_valid
    empty = ~allowed.any(axis=1, keepdims=True)
    return allowed | empty


def gemma_attention(q_bits, k_bits, v_bits, q_heads: int, kv_heads: int, q_norm_w, k_norm_w,
                    cos, sin, *, eps: float = 1e-6, window: int = 0, first_valid=None,
                    scale: float = 1.0, mode: str = "exact") -> np.ndarray:
    """One Gemma-4 attention from its projections to the merged output before ``o_proj``
    (GemmaTextEncoder.swift:158-239). ``q_bits`` ``[B, T, Hq*D]``, ``k_bits``/``v_bits``
    ``[B, T, Hkv*D]`` bf16 bits (``v_bits`` is ``k_bits`` on the K-shares-V layers: V is
    the weightless norm of the PRE-norm K projection); norm weights ``[D]`` bits; ``cos``,
    ``sin`` fp32 ``[T, D/2]``; ``first_valid`` per batch row (left padding). Returns float64
    ``[B, T, Hq*D]``.

    ``mode="exact"``: float64 throughout. ``mode="reference"``: the norms round to bf16 (the
    reference casts back to the input dtype), RoPE in fp32 (bf16 x fp32 tables promote), and
    the explicit path's fp32 logits/softmax/P.V."""
    B, T, _ = q_bits.shape
    D = q_bits.shape[2] // q_heads
    rep = q_heads // kv_heads

    def heads(bits, h):
        return bf16_bits_to_f32(bits).astype(np.float64).reshape(B, T, h, D)

    def norm(x, w):
        ms = (x * x).mean(axis=-1, keepdims=True)
        y = x * (ms + eps) ** -0.5
        if w is not None:
            y = y * bf16_bits_to_f32(w).astype(np.float64)
        return round_bf16(y).astype(np.float64) if mode == "reference" else y

    def rope(x):
        c = np.asarray(cos, dtype=np.float64)[None, :, None, :]
        s_ = np.asarray(sin, dtype=np.float64)[None, :, None, :]
        x1, x2 = x[..., : D // 2], x[..., D // 2:]
        return np.concatenate([x1 * c - x2 * s_, x2 * c + x1 * s_], axis=-1)

    q = rope(norm(heads(q_bits, q_heads), q_norm_w))
    kp = heads(k_bits, kv_heads)
    k = rope(norm(kp, k_norm_w))
    v = norm(heads(v_bits, kv_heads), None)
    if mode == "reference":
        q, k = q.astype(np.float32).astype(np.float64), k.astype(np.float32).astype(np.float64)
    out = np.zeros((B, T, q_heads, D), dtype=np.float64)
    fv = [0] * B if first_valid is None else list(first_valid)
    for b in range(B):
        allowed = gemma_mask(T, window, fv[b])
        for h in range(q_heads):
            kh = h // rep
            logits = (q[b, :, h, :] @ k[b, :, kh, :].T) * scale
            logits = np.where(allowed, logits, -np.inf)
            logits -= logits.max(axis=1, keepdims=True)
            p = np.exp(logits)
            p /= p.sum(axis=1, keepdims=True)
            out[b, :, h, :] = p @ v[b, :, kh, :]
    return out.reshape(B, T, q_heads * D)


def compare(candidate, reference) -> dict:
    """relRMS = sqrt(sum (a-b)^2 / sum b^2), maxAbs, bit-identical fraction (on bf16)."""
    a = np.asarray(candidate, dtype=np.float64).ravel()
    b = np.asarray(reference, dtype=np.float64).ravel()
    diff = a - b
    ssd = float(np.sum(diff * diff))
    ssr = float(np.sum(b * b))
    rel = math.sqrt(ssd / ssr) if ssr > 0 else (math.inf if ssd > 0 else 0.0)
    ident = float(np.mean(f32_to_bf16_bits(a.astype(np.float32))
                          == f32_to_bf16_bits(b.astype(np.float32)))) if a.size else math.nan
    return {"rel_rms": rel, "max_abs": float(np.max(np.abs(diff))) if a.size else 0.0,
            "bit_identical": ident, "elements": int(a.size)}


# --------------------------------------------------------------------------------------
# The C restatement (attn_oracle.c): multithreaded fp32, used for medium and large checks
# and as the timed CPU baseline.
# --------------------------------------------------------------------------------------

import ctypes as _ct
import os as _os

_C_LIB_DIR = _os.path.join(_os.path.dirname(_os.path.abspath(__file__)), "lib")
_C_LIB_PATH = _os.path.join(_C_LIB_DIR, "liboracle.so")
_C_LIB_V4_PATH = _os.path.join(_C_LIB_DIR, "liboracle_v4.so")
_c_lib = None
c_library_isa = None


def _cpu_has_avx512() -> bool:
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("flags"):
                    flags = set(line.split(":", 1)[1].split())
                    return {"avx512f", "avx512bw", "avx512dq", "avx512vl"} <= flags
    except OSError:
        pass
    return False


class _OracleArgs(_ct.Structure):
    _fields_ = [
        ("B", _ct.c_int32), ("H", _ct.c_int32), ("Lq", _ct.c_int32), ("Lk", _ct.c_int32),
        ("D", _ct.c_int32),
        ("q", _ct.c_void_p), ("k", _ct.c_void_p), ("v", _ct.c_void_p),
        ("q_norm_w", _ct.c_void_p), ("k_norm_w", _ct.c_void_p), ("eps", _ct.c_float),
        ("q_cos", _ct.c_void_p), ("q_sin", _ct.c_void_p),
        ("k_cos", _ct.c_void_p), ("k_sin", _ct.c_void_p),
        ("k_valid_len", _ct.c_void_p), ("scale", _ct.c_float), ("mode", _ct.c_int32),
        ("h_begin", _ct.c_int32), ("h_end", _ct.c_int32),
        ("q_begin", _ct.c_int32), ("q_end", _ct.c_int32), ("threads", _ct.c_int32),
        ("out", _ct.c_void_p),
    ]


def c_library():
    """The C restatement: the AVX-512 build where the CPU has AVX-512, else the AVX2 one."""
    global _c_lib, c_library_isa
    if _c_lib is None:
        path, c_library_isa = _C_LIB_PATH, "x86-64-v3 (AVX2)"
        if _cpu_has_avx512() and _os.path.exists(_C_LIB_V4_PATH):
            path, c_library_isa = _C_LIB_V4_PATH, "x86-64-v4 (AVX-512)"
        if not _os.path.exists(path):
            raise RuntimeError(f"{path} missing; run `make -C oracle`")
        lib = _ct.CDLL(path)
        lib.oracle_attention.argtypes = [_ct.POINTER(_OracleArgs)]
        lib.oracle_attention.restype = _ct.c_int
        lib.oracle_max_threads.restype = _ct.c_int
        _c_lib = lib
    return _c_lib


def c_attention(q_bits, k_bits, v_bits, heads: int, *, q_norm_w=None, k_norm_w=None,
                eps: float = 1e-6, q_cos=None, q_sin=None, k_cos=None, k_sin=None,
                valid_len=None, scale=None, mode: str = "reference", heads_range=None,
                q_range=None, threads: int = 0) -> np.ndarray:
    """Same contract as ``attention`` (fp32 instead of float64). Returns float32
    ``[B, nq, nh, D]`` for the requested query and head ranges."""
    lib = c_library()
    B, Lq, inner = q_bits.shape
    Lk = k_bits.shape[1]
    D = inner // heads
    h0, h1 = heads_range if heads_range is not None else (0, heads)
    q0, q1 = q_range if q_range is not None else (0, Lq)
    if scale is None:
        scale = float(np.float32(1.0 / math.sqrt(D)))
    keep = []

    def arr(x, dt):
        if x is None:
            return None
        a = np.ascontiguousarray(x, dtype=dt)
        keep.append(a)
        return a.ctypes.data

    out = np.zeros((B, q1 - q0, h1 - h0, D), dtype=np.float32)
    a = _OracleArgs(B, heads, Lq, Lk, D, arr(q_bits, np.uint16), arr(k_bits, np.uint16),
                    arr(v_bits, np.uint16), arr(q_norm_w, np.uint16), arr(k_norm_w, np.uint16),
                    eps, arr(q_cos, np.uint16), arr(q_sin, np.uint16), arr(k_cos, np.uint16),
                    arr(k_sin, np.uint16), arr(valid_len, np.int32), scale,
                    0 if mode == "exact" else 1, h0, h1, q0, q1, threads, out.ctypes.data)
    rc = lib.oracle_attention(_ct.byref(a))
    if rc != 0:
        raise ValueError(f"oracle_attention failed ({rc})")
    return out
