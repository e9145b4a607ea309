"""Python host binding of libltx_attn.so (MI355X fused DiT attention).

A thin ctypes layer over the C ABI in ``include/ltx_attn.h``. It mirrors the reference's call
surface for the replaced unit:

* ``DiTAttentionModule`` -- the whole ``DiTAttention.callAsFunction`` (``:315-405``):
  projections (``linear``, with the RMS statistic from the q / k projections), the replaced
  unit, the gate and ``to_out``.
* ``DiTAttentionCore``  -- the norm -> split -> RoPE -> SDPA part of
  ``DiTAttention.callAsFunction`` (``Sources/LTXModules/DiTAttention.swift:315-381``), with the
  reference's ``Variant`` / ``Rotary`` / ``Failure`` vocabulary (``:69-122``).
* ``scaled_dot_product_attention`` -- ``MLXFast.scaledDotProductAttention(queries:keys:values:
  scale:mask:)`` on ``[B, H, L, D]`` inputs (``DiTAttention.swift:374-376``), plus an optional
  key-padding length per batch row.
* ``rope_*`` -- the rotary-table builders of ``Sources/LTXModules/DiTForward.swift:455-738``.

PyTorch supplies device memory and the stream only; every arithmetic step runs in the HIP
library. If the library is missing this module raises -- there is no fallback path.
"""

from __future__ import annotations

import ctypes
import enum
import math
import os
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("LTX_ATTN_LIBRARY",
                          os.path.join(os.path.dirname(_HERE), "lib", "libltx_attn.so"))

OK, EINVAL, EUNSUPPORTED, EHIP, EWORKSPACE = 0, 1, 2, 3, 4
KPREP_AUTO, KPREP_FUSED, KPREP_PROLOGUE = 0, 1, 2
MAX_BATCH = 64


class Args(ctypes.Structure):
    """``ltx_attn_args`` (field order and types as in include/ltx_attn.h)."""

    _fields_ = [
        ("B", ctypes.c_int32), ("H", ctypes.c_int32), ("Lq", ctypes.c_int32),
        ("Lk", ctypes.c_int32), ("D", ctypes.c_int32),
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("q_bs", ctypes.c_int64), ("q_rs", ctypes.c_int64), ("q_hs", ctypes.c_int64),
        ("k_bs", ctypes.c_int64), ("k_rs", ctypes.c_int64), ("k_hs", ctypes.c_int64),
        ("v_bs", ctypes.c_int64), ("v_rs", ctypes.c_int64), ("v_hs", ctypes.c_int64),
        ("q_norm_w", ctypes.c_void_p), ("k_norm_w", ctypes.c_void_p),
        ("norm_eps", ctypes.c_float),
        ("q_cos", ctypes.c_void_p), ("q_sin", ctypes.c_void_p),
        ("k_cos", ctypes.c_void_p), ("k_sin", ctypes.c_void_p),
        ("k_valid_len", ctypes.POINTER(ctypes.c_int32)),
        ("scale", ctypes.c_float),
        ("out", ctypes.c_void_p),
        ("o_bs", ctypes.c_int64), ("o_rs", ctypes.c_int64), ("o_hs", ctypes.c_int64),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
        ("kprep", ctypes.c_int32), ("num_splits", ctypes.c_int32),
        ("ev_attn_start", ctypes.c_void_p), ("ev_attn_stop", ctypes.c_void_p),
        ("gate_logits", ctypes.c_void_p),
        ("g_bs", ctypes.c_int64), ("g_rs", ctypes.c_int64), ("g_hs", ctypes.c_int64),
        ("all_perturbed", ctypes.c_int32),
        ("q_sumsq", ctypes.c_void_p), ("k_sumsq", ctypes.c_void_p),
        ("q_sumsq_rs", ctypes.c_int64), ("k_sumsq_rs", ctypes.c_int64),
        ("sumsq_blocks", ctypes.c_int32),
        ("resident_groups", ctypes.c_int32),
    ]


class LinearArgs(ctypes.Structure):
    """``ltx_linear_args`` (field order and types as in include/ltx_attn.h)."""

    _fields_ = [
        ("M", ctypes.c_int32), ("N", ctypes.c_int32), ("K", ctypes.c_int32),
        ("x", ctypes.c_void_p), ("w", ctypes.c_void_p), ("bias", ctypes.c_void_p),
        ("y", ctypes.c_void_p),
        ("x_rs", ctypes.c_int64), ("w_rs", ctypes.c_int64), ("y_rs", ctypes.c_int64),
        ("sumsq", ctypes.c_void_p), ("sumsq_rs", ctypes.c_int64),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
        ("resident_groups", ctypes.c_int32),
    ]


SUMSQ_COLS = 256   # LTX_LINEAR_SUMSQ_COLS: columns of y per partial sum of squares


class GemmaArgs(ctypes.Structure):
    """``ltx_gemma_attn_args`` (field order and types as in include/ltx_attn.h)."""

    _fields_ = [
        ("B", ctypes.c_int32), ("T", ctypes.c_int32),
        ("Hq", ctypes.c_int32), ("Hkv", ctypes.c_int32), ("D", ctypes.c_int32),
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("q_bs", ctypes.c_int64), ("q_rs", ctypes.c_int64),
        ("k_bs", ctypes.c_int64), ("k_rs", ctypes.c_int64),
        ("v_bs", ctypes.c_int64), ("v_rs", ctypes.c_int64),
        ("q_norm_w", ctypes.c_void_p), ("k_norm_w", ctypes.c_void_p),
        ("eps", ctypes.c_float),
        ("cos", ctypes.c_void_p), ("sin", ctypes.c_void_p),
        ("window", ctypes.c_int32),
        ("first_valid", ctypes.POINTER(ctypes.c_int32)),
        ("scale", ctypes.c_float),
        ("out", ctypes.c_void_p),
        ("o_bs", ctypes.c_int64), ("o_rs", ctypes.c_int64),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
    ]


# GemmaAttentionSpec.ltx25 (Sources/LTXFoundation/GemmaAttentionSpec.swift:67-71) and the
# text-encoder topology (Tests/LTXCatalogTests/TextEncoderTopologyTests.swift:53-68)
GEMMA_SLIDING = dict(head_dim=256, q_heads=16, kv_heads=8, theta=10_000.0, partial=1.0,
                     proportional=False, window=1024, shares_kv=False)
GEMMA_FULL = dict(head_dim=512, q_heads=16, kv_heads=1, theta=1_000_000.0, partial=0.25,
                  proportional=True, window=0, shares_kv=True)


EXPORTED_SYMBOLS = (
    "ltx_attn_args_init", "ltx_attn_workspace_bytes", "ltx_attn_validate", "ltx_attn_fwd",
    "ltx_attn_status_string", "ltx_attn_last_error", "ltx_attn_provenance",
    "ltx_attn_abi_version", "ltx_attn_args_size", "ltx_rope_frequency_grid", "ltx_rope_video_positions",
    "ltx_rope_audio_positions", "ltx_rope_tables", "ltx_rope_tables_device",
    "ltx_linear", "ltx_linear_sumsq_blocks", "ltx_linear_workspace_bytes", "ltx_gemma_attn_workspace_bytes",
    "ltx_gemma_attn_fwd", "ltx_gemma_rope_tables", "ltx_device_count", "ltx_device_query",
    "ltx_attn_fwd_static", "ltx_rope_reference_positions",
    "ltx_rope_video_positions_with_references",
)


class Reference(ctypes.Structure):
    """``ltx_rope_reference``: an in-context reference clip appended to the video stream
    (``DiTForward.Geometry.Reference``, DiTForward.swift:220-252)."""
    _fields_ = [("latent_frames", ctypes.c_int32), ("latent_height", ctypes.c_int32),
                ("latent_width", ctypes.c_int32), ("downscale_factor", ctypes.c_int32),
                ("temporal_scale_factor", ctypes.c_int32), ("frame_offset", ctypes.c_int32)]

    def __init__(self, latent_frames, latent_height, latent_width, downscale_factor=1,
                 temporal_scale_factor=1, frame_offset=0):
        super().__init__(latent_frames, latent_height, latent_width, downscale_factor,
                         temporal_scale_factor, frame_offset)

    @property
    def tokens(self) -> int:
        return self.latent_frames * self.latent_height * self.latent_width


def msr_slots(count: int, latent_frames: int, latent_height: int, latent_width: int):
    """Multiple-Subject-Reference slots: slot i of n sits at -(n - i) pixel frames, the first
    furthest back in time (DiTForward.swift:229-242)."""
    return [Reference(latent_frames, latent_height, latent_width, frame_offset=-(count - i))
            for i in range(count)]

# ltx_attn_fwd_static's per-device scratch (LTX_ATTN_STATIC_SCRATCH_BYTES)
STATIC_SCRATCH_BYTES = 128 << 20


class DeviceInfo(ctypes.Structure):
    """``ltx_device_info`` (include/ltx_attn.h)."""
    _fields_ = [
        ("ordinal", ctypes.c_int32), ("compute_units", ctypes.c_int32),
        ("memory_bytes", ctypes.c_int64), ("clock_khz", ctypes.c_int32),
        ("lds_bytes_per_cu", ctypes.c_int32), ("supported", ctypes.c_int32),
        ("name", ctypes.c_char * 128), ("arch", ctypes.c_char * 64),
    ]

_lib = None


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load (once) and type the library. Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    # torch (when installed) ships its own HIP and HSA runtimes under the same sonames as the
    # system's. Loaded first, they are the ones this library binds to: one runtime in the
    # process. Loaded after the library, torch would bring a second HSA runtime, and the two
    # would contend for the device.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    if not os.path.exists(path):
        raise RuntimeError(f"libltx_attn.so not found at {path}; build it with "
                           "`python -c 'import __graft_entry__ as g; g.build()'` or "
                           "`make -C ltx-2.5-swift_amd/csrc`")
    lib = ctypes.CDLL(path)
    P = ctypes.POINTER(Args)
    lib.ltx_attn_args_init.argtypes = [P]
    lib.ltx_attn_args_init.restype = None
    lib.ltx_attn_workspace_bytes.argtypes = [P]
    lib.ltx_attn_workspace_bytes.restype = ctypes.c_size_t
    lib.ltx_attn_validate.argtypes = [P]
    lib.ltx_attn_validate.restype = ctypes.c_int
    lib.ltx_attn_fwd.argtypes = [P, ctypes.c_void_p]
    lib.ltx_attn_fwd.restype = ctypes.c_int
    lib.ltx_attn_status_string.argtypes = [ctypes.c_int]
    lib.ltx_attn_status_string.restype = ctypes.c_char_p
    lib.ltx_attn_last_error.argtypes = []
    lib.ltx_attn_last_error.restype = ctypes.c_char_p
    lib.ltx_attn_provenance.argtypes = []
    lib.ltx_attn_provenance.restype = ctypes.c_char_p
    lib.ltx_attn_abi_version.argtypes = []
    lib.ltx_attn_abi_version.restype = ctypes.c_int32
    lib.ltx_attn_args_size.argtypes = []
    lib.ltx_attn_args_size.restype = ctypes.c_size_t
    if lib.ltx_attn_args_size() != ctypes.sizeof(Args):
        raise RuntimeError(f"ltx_attn_args layout mismatch: library {lib.ltx_attn_args_size()} "
                           f"bytes, binding {ctypes.sizeof(Args)} bytes")
    lib.ltx_rope_frequency_grid.argtypes = [ctypes.c_double, ctypes.c_int32, ctypes.c_int32,
                                            ctypes.c_void_p, ctypes.c_int32]
    lib.ltx_rope_frequency_grid.restype = ctypes.c_int32
    lib.ltx_rope_video_positions.argtypes = [ctypes.c_int32] * 5 + [
        ctypes.c_double, ctypes.c_void_p, ctypes.c_int64]
    lib.ltx_rope_video_positions.restype = ctypes.c_int32
    lib.ltx_rope_audio_positions.argtypes = [ctypes.c_int32] * 4 + [ctypes.c_void_p,
                                                                     ctypes.c_int64]
    lib.ltx_rope_audio_positions.restype = ctypes.c_int32
    lib.ltx_rope_reference_positions.argtypes = [ctypes.POINTER(Reference), ctypes.c_int32,
                                                 ctypes.c_int32, ctypes.c_double,
                                                 ctypes.c_float, ctypes.c_void_p,
                                                 ctypes.c_int64]
    lib.ltx_rope_reference_positions.restype = ctypes.c_int32
    lib.ltx_rope_video_positions_with_references.argtypes = [ctypes.c_int32] * 5 + [
        ctypes.c_double, ctypes.POINTER(Reference), ctypes.c_int32, ctypes.c_void_p,
        ctypes.c_int64]
    lib.ltx_rope_video_positions_with_references.restype = ctypes.c_int32
    lib.ltx_rope_tables.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
                                    ctypes.c_int32, ctypes.c_void_p, ctypes.c_int32,
                                    ctypes.c_double, ctypes.c_void_p, ctypes.c_void_p]
    lib.ltx_rope_tables.restype = ctypes.c_int32
    lib.ltx_rope_tables_device.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
                                           ctypes.c_int32, ctypes.c_void_p, ctypes.c_int32,
                                           ctypes.c_double, ctypes.c_void_p, ctypes.c_void_p,
                                           ctypes.c_void_p]
    lib.ltx_rope_tables_device.restype = ctypes.c_int
    lib.ltx_linear.argtypes = [ctypes.POINTER(LinearArgs), ctypes.c_void_p]
    lib.ltx_linear.restype = ctypes.c_int
    lib.ltx_linear_workspace_bytes.argtypes = [ctypes.POINTER(LinearArgs)]
    lib.ltx_linear_workspace_bytes.restype = ctypes.c_size_t
    lib.ltx_linear_sumsq_blocks.argtypes = [ctypes.c_int32]
    lib.ltx_linear_sumsq_blocks.restype = ctypes.c_int32
    lib.ltx_gemma_attn_workspace_bytes.argtypes = [ctypes.POINTER(GemmaArgs)]
    lib.ltx_gemma_attn_workspace_bytes.restype = ctypes.c_size_t
    lib.ltx_gemma_attn_fwd.argtypes = [ctypes.POINTER(GemmaArgs), ctypes.c_void_p]
    lib.ltx_gemma_attn_fwd.restype = ctypes.c_int
    lib.ltx_gemma_rope_tables.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_double,
                                          ctypes.c_double, ctypes.c_int32, ctypes.c_void_p,
                                          ctypes.c_void_p]
    lib.ltx_gemma_rope_tables.restype = ctypes.c_int32
    lib.ltx_attn_fwd_static.argtypes = [P, ctypes.c_void_p]
    lib.ltx_attn_fwd_static.restype = ctypes.c_int
    lib.ltx_device_count.argtypes = []
    lib.ltx_device_count.restype = ctypes.c_int32
    lib.ltx_device_query.argtypes = [ctypes.c_int32, ctypes.POINTER(DeviceInfo)]
    lib.ltx_device_query.restype = ctypes.c_int
    _lib = lib
    return lib


def device_info(ordinal: int = 0) -> dict:
    """The HIP device as the library sees it (``ltx_device_query``)."""
    info = DeviceInfo()
    _check(load_library().ltx_device_query(ordinal, ctypes.byref(info)))
    return {"ordinal": info.ordinal, "compute_units": info.compute_units,
            "memory_bytes": info.memory_bytes, "clock_khz": info.clock_khz,
            "lds_bytes_per_cu": info.lds_bytes_per_cu, "supported": bool(info.supported),
            "name": info.name.decode(), "arch": info.arch.decode()}


def provenance() -> str:
    return load_library().ltx_attn_provenance().decode()


# --------------------------------------------------------------------------------------
# Errors (DiTAttention.Failure, DiTAttention.swift:107-121)
# --------------------------------------------------------------------------------------

class Failure(Exception):
    """A status other than OK from the library, or a structural misuse caught here."""

    def __init__(self, status: int, detail: str):
        self.status = status
        self.detail = detail
        name = {EINVAL: "invalid argument", EUNSUPPORTED: "unsupported configuration",
                EHIP: "HIP runtime error", EWORKSPACE: "workspace too small"}.get(status, "?")
        super().__init__(f"{name}: {detail}")


class RotaryWithoutPosition(Failure):
    """``Failure.rotaryWithoutPosition`` (DiTAttention.swift:110, :118-119)."""

    def __init__(self, variant: "Variant"):
        super().__init__(EINVAL, f"{variant.value} takes no rotary embedding; supplying one "
                                 "would rotate a stream that has no latent position")
        self.variant = variant


def _check(status: int) -> None:
    if status != OK:
        detail = load_library().ltx_attn_last_error().decode()
        raise Failure(status, detail)


# --------------------------------------------------------------------------------------
# Variants and rotary pairs (DiTAttention.swift:69-105)
# --------------------------------------------------------------------------------------

class Variant(enum.Enum):
    videoSelf = "attn1"
    videoCross = "attn2"
    audioSelf = "audio_attn1"
    audioCross = "audio_attn2"
    audioToVideo = "audio_to_video_attn"   # video queries over audio K/V
    videoToAudio = "video_to_audio_attn"   # audio queries over video K/V

    @property
    def takes_rotary(self) -> bool:
        """``attn2`` / ``audio_attn2`` are never rotated (DiTAttention.swift:84-89)."""
        return self not in (Variant.videoCross, Variant.audioCross)


@dataclass
class Rotary:
    """One ``(cos, sin)`` pair, each bf16 ``[H, L, D/2]`` on the device (the reference's
    ``[1, H, L, D/2]`` with the batch axis dropped)."""

    cos: "object"
    sin: "object"


# --------------------------------------------------------------------------------------
# Core call
# --------------------------------------------------------------------------------------

def _strides_merged(t, heads):
    """Element strides (bs, rs, hs) of a ``[B, L, H*D]`` tensor view."""
    B, L, inner = t.shape
    sb, sr, sc = t.stride()
    if sc != 1:
        raise Failure(EINVAL, "the channel axis must be contiguous")
    return sb, sr, inner // heads


def _strides_split(t):
    """Element strides (bs, rs, hs) of a ``[B, H, L, D]`` tensor view."""
    sb, sh, sr, sd = t.stride()
    if sd != 1:
        raise Failure(EINVAL, "the head-dim axis must be contiguous")
    return sb, sr, sh


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def attention_fwd(q, k, v, *, heads: int, layout: str = "merged", q_norm_w=None,
                  k_norm_w=None, eps: float = 1e-6, rotary: Optional[Rotary] = None,
                  key_rotary: Optional[Rotary] = None,
                  k_valid_len: Optional[Sequence[int]] = None, scale: Optional[float] = None,
                  out=None, kprep: int = KPREP_AUTO, num_splits: int = 0, stream=None,
                  workspace=None, events=None, gate_logits=None, all_perturbed: bool = False,
                  q_sumsq=None, k_sumsq=None, no_alloc: bool = False,
                  resident_groups: int = 0):
    """One call of ``ltx_attn_fwd``. Tensors are torch bf16 on the current HIP device.

    ``layout="merged"``: q ``[B, Lq, H*D]``, k/v ``[B, Lk, H*D]``, out ``[B, Lq, H*D]``.
    ``layout="split"``:  q ``[B, H, Lq, D]``, k/v ``[B, H, Lk, D]``, out ``[B, H, Lq, D]``.
    ``gate_logits``: bf16 ``[B, Lq, H]`` (the output of ``to_gate_logits(x)``); each output row
    of head h is multiplied by ``2*sigmoid(logit)`` (``DiTAttention.swift:395-399``).
    ``all_perturbed``: the STG passthrough (``:351-356``): ``out = v`` per head (times the
    gate), no attention; ``q`` and ``k`` may then be None.
    ``q_sumsq`` / ``k_sumsq``: the projection's statistic partials for q / k (fp32
    ``[B*L, blocks]`` views with a unit column stride, as ``linear(..., sumsq=True)`` returns
    them, column-sliced to the q / k range of a fused projection); the norm then takes its
    statistic from them. Both must have the same number of blocks.
    ``no_alloc``: call ``ltx_attn_fwd_static`` instead, whose scratch is the library's own
    per-device array (no workspace is made or passed; calls needing more than
    ``STATIC_SCRATCH_BYTES`` raise ``Failure``).
    ``resident_groups``: 0 plans the work for the device's CU count; n > 0 plans it as if n
    workgroups were resident at once (a test of another part size's plan).
    Returns ``out``.
    """
    import torch

    lib = load_library()
    if all_perturbed:
        q = v if q is None else q
        k = v if k is None else k
    if layout == "merged":
        B, Lq, inner = q.shape
        Lk = k.shape[1]
        D = inner // heads
        qs, ks, vs = (_strides_merged(t, heads) for t in (q, k, v))
        if out is None:
            out = torch.empty((B, Lq, inner), dtype=q.dtype, device=q.device)
        os_ = _strides_merged(out, heads)
    elif layout == "split":
        B, H, Lq, D = q.shape
        if H != heads:
            raise Failure(EINVAL, f"q has {H} heads, expected {heads}")
        Lk = k.shape[2]
        qs, ks, vs = (_strides_split(t) for t in (q, k, v))
        if out is None:
            out = torch.empty((B, heads, Lq, D), dtype=q.dtype, device=q.device)
        os_ = _strides_split(out)
    else:
        raise ValueError(layout)
    for name, t in (("q", q), ("k", k), ("v", v), ("out", out)):
        if t.dtype != torch.bfloat16 or not t.is_cuda:
            raise Failure(EINVAL, f"{name} must be a bf16 device tensor")

    a = Args()
    lib.ltx_attn_args_init(ctypes.byref(a))
    a.B, a.H, a.Lq, a.Lk, a.D = B, heads, Lq, Lk, D
    a.q, a.k, a.v = _ptr(q), _ptr(k), _ptr(v)
    a.q_bs, a.q_rs, a.q_hs = qs
    a.k_bs, a.k_rs, a.k_hs = ks
    a.v_bs, a.v_rs, a.v_hs = vs
    keep = []
    if q_norm_w is not None:
        a.q_norm_w = _ptr(q_norm_w)
    if k_norm_w is not None:
        a.k_norm_w = _ptr(k_norm_w)
    a.norm_eps = eps
    if rotary is not None:
        a.q_cos, a.q_sin = _ptr(rotary.cos), _ptr(rotary.sin)
    if key_rotary is not None:
        a.k_cos, a.k_sin = _ptr(key_rotary.cos), _ptr(key_rotary.sin)
    if k_valid_len is not None:
        arr = (ctypes.c_int32 * B)(*[int(x) for x in k_valid_len])
        keep.append(arr)
        a.k_valid_len = ctypes.cast(arr, ctypes.POINTER(ctypes.c_int32))
    a.scale = float(np.float32(1.0 / math.sqrt(D))) if scale is None else float(scale)
    a.out = _ptr(out)
    a.o_bs, a.o_rs, a.o_hs = os_
    a.kprep = kprep
    a.num_splits = num_splits
    a.resident_groups = resident_groups
    if events is not None:
        a.ev_attn_start, a.ev_attn_stop = events
    a.all_perturbed = 1 if all_perturbed else 0
    if gate_logits is not None:
        if gate_logits.dtype != torch.bfloat16 or not gate_logits.is_cuda:
            raise Failure(EINVAL, "gate_logits must be a bf16 device tensor")
        if tuple(gate_logits.shape) != (B, Lq, heads):
            raise Failure(EINVAL, f"gate_logits shape {tuple(gate_logits.shape)} is not "
                                  f"{(B, Lq, heads)}")
        a.gate_logits = _ptr(gate_logits)
        a.g_bs, a.g_rs, a.g_hs = gate_logits.stride()
    blocks = None
    for name, t in (("q_sumsq", q_sumsq), ("k_sumsq", k_sumsq)):
        if t is None:
            continue
        if t.dtype != torch.float32 or not t.is_cuda or t.dim() != 2 or t.stride(1) != 1:
            raise Failure(EINVAL, f"{name} must be a 2-D fp32 device tensor, unit column stride")
        if blocks is not None and t.shape[1] != blocks:
            raise Failure(EINVAL, "q_sumsq and k_sumsq have different block counts")
        blocks = t.shape[1]
        setattr(a, name, _ptr(t))
        setattr(a, name + "_rs", t.stride(0))
    if blocks is not None:
        a.sumsq_blocks = blocks
    if stream is None:
        stream = torch.cuda.current_stream(q.device).cuda_stream
    if no_alloc:
        _check(lib.ltx_attn_fwd_static(ctypes.byref(a), ctypes.c_void_p(stream)))
        return out
    need = lib.ltx_attn_workspace_bytes(ctypes.byref(a))
    st = lib.ltx_attn_validate(ctypes.byref(a))
    if st not in (OK, EWORKSPACE):
        _check(st)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need + 256):
        workspace = torch.empty(need + 256, dtype=torch.uint8, device=q.device)
    if workspace is not None:
        # all of it: on a part with another CU count the call may plan for that count when
        # the workspace covers it
        base = workspace.data_ptr()
        aligned = (base + 255) // 256 * 256
        a.workspace = ctypes.c_void_p(aligned)
        a.workspace_bytes = workspace.numel() * workspace.element_size() - (aligned - base)
    _check(lib.ltx_attn_fwd(ctypes.byref(a), ctypes.c_void_p(stream)))
    # keep the workspace alive until the stream has consumed it
    if workspace is not None:
        out._ltx_workspace = workspace  # noqa: SLF001 -- lifetime anchor
    return out


def linear_sumsq_blocks(n: int) -> int:
    """Partial sums of squares per row of a projection with ``n`` output columns."""
    return load_library().ltx_linear_sumsq_blocks(n)


def linear_workspace_bytes(M: int, N: int, K: int) -> int:
    """Device scratch ``ltx_linear`` uses to split the tiles past its last whole round along K
    (0 when it would not split them)."""
    a = LinearArgs()
    a.M, a.N, a.K = M, N, K
    return load_library().ltx_linear_workspace_bytes(ctypes.byref(a))


def linear(x, weight, bias=None, *, out=None, sumsq=False, stream=None, workspace=None,
           resident_groups: int = 0):
    """``linear(_:_:)`` of ``DiTAttention.swift:178-188`` through ``ltx_linear``:
    ``y = x . weight^T (+ bias)``, bf16 in and out, fp32 accumulation.

    ``x``: bf16 ``[..., K]`` with a unit last stride (leading axes are flattened to rows, so
    they must be collapsible); ``weight``: bf16 ``[N, K]`` (the checkpoint's layout);
    ``bias``: bf16 ``[N]`` or None. ``out``: optional bf16 ``[..., N]`` view to write (unit
    last stride; e.g. a column slice of a fused buffer). ``sumsq=True`` also returns the
    statistic partials: fp32 ``[rows, ceil(N/256)]``, partial j of a row being the sum of
    squares of its bf16 outputs over columns ``[256 j, 256 j + 256)``. ``workspace``: a
    device tensor of at least ``linear_workspace_bytes(M, N, K)`` bytes for the split tail;
    None allocates one when the shape splits, ``False`` runs every tile whole.
    ``resident_groups``: as in ``attention_fwd`` (0: the device's CU count).
    Returns ``y`` or ``(y, partials)``.
    """
    import torch

    lib = load_library()
    for name, t in (("x", x), ("weight", weight), ("bias", bias), ("out", out)):
        if t is not None and (t.dtype != torch.bfloat16 or not t.is_cuda):
            raise Failure(EINVAL, f"{name} must be a bf16 device tensor")
    N, K = weight.shape
    if weight.stride(1) != 1 or x.stride(-1) != 1:
        raise Failure(EINVAL, "x and weight need a unit last stride")
    if x.shape[-1] != K:
        raise Failure(EINVAL, f"x has {x.shape[-1]} columns, weight expects {K}")
    lead = tuple(x.shape[:-1])
    x2 = x.reshape(-1, K) if x.dim() != 2 else x
    M = x2.shape[0]
    if out is None:
        out = torch.empty(lead + (N,), dtype=torch.bfloat16, device=x.device)
    if tuple(out.shape) != lead + (N,) or out.stride(-1) != 1:
        raise Failure(EINVAL, f"out must be {lead + (N,)} with a unit last stride")
    y2 = out.view(-1, N) if out.dim() != 2 else out
    if bias is not None and (bias.dim() != 1 or bias.shape[0] != N or not bias.is_contiguous()):
        raise Failure(EINVAL, f"bias must be a contiguous [{N}] tensor")
    a = LinearArgs()
    a.M, a.N, a.K = M, N, K
    a.resident_groups = resident_groups
    a.x, a.w, a.bias, a.y = _ptr(x2), _ptr(weight), _ptr(bias), _ptr(y2)
    a.x_rs = x2.stride(0) if M > 1 else K
    a.w_rs = weight.stride(0) if N > 1 else K
    a.y_rs = y2.stride(0) if M > 1 else N
    parts = None
    if sumsq:
        nb = lib.ltx_linear_sumsq_blocks(N)
        parts = torch.empty((M, nb), dtype=torch.float32, device=x.device)
        a.sumsq, a.sumsq_rs = _ptr(parts), nb
    need = lib.ltx_linear_workspace_bytes(ctypes.byref(a)) if M > 0 else 0
    if workspace is None and need:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    if workspace is not None and workspace is not False:
        nbytes = workspace.numel() * workspace.element_size()
        a.workspace, a.workspace_bytes = _ptr(workspace), nbytes
    if stream is None:
        stream = torch.cuda.current_stream(x.device).cuda_stream
    _check(lib.ltx_linear(ctypes.byref(a), ctypes.c_void_p(stream)))
    return (out, parts) if sumsq else out


def workspace_bytes(**kw) -> int:
    """Workspace the call with these shapes/options needs (host-only query)."""
    lib = load_library()
    a = Args()
    lib.ltx_attn_args_init(ctypes.byref(a))
    for k_, v_ in kw.items():
        setattr(a, k_, v_)
    return lib.ltx_attn_workspace_bytes(ctypes.byref(a))


def scaled_dot_product_attention(queries, keys, values, scale: float, mask=None,
                                 k_valid_len=None, **kw):
    """``MLXFast.scaledDotProductAttention`` on ``[B, H, L, D]`` bf16 tensors.

    ``mask`` must be None (the DiT path passes ``.none``, DiTAttention.swift:374-376); a
    key-padding mask is given as ``k_valid_len`` (first n keys valid per batch row).
    """
    if mask is not None:
        raise Failure(EUNSUPPORTED, "only mask=None or k_valid_len key padding is supported")
    return attention_fwd(queries, keys, values, heads=queries.shape[1], layout="split",
                         scale=scale, k_valid_len=k_valid_len, **kw)


class DiTAttentionCore:
    """The replaced unit of ``DiTAttention`` (``DiTAttention.swift:358-381``).

    Takes the pre-norm projections ``q = to_q(x)``, ``k = to_k(context)``, ``v = to_v(context)``
    in the merged ``[B, L, H*D]`` layout plus the ``q_norm`` / ``k_norm`` weights, and returns
    the attention output in the merged layout (what the gate and ``to_out`` consume).
    """

    heads = 32            # DiTAttention.heads (:64)
    norm_epsilon = 1e-6   # DiTAttention.normEpsilon (:66)

    def __init__(self, q_norm_weight, k_norm_weight, heads: int = 32):
        self.q_norm_weight = q_norm_weight
        self.k_norm_weight = k_norm_weight
        self.heads = heads

    def __call__(self, q, k, v, *, variant: Variant, rotary: Optional[Rotary] = None,
                 key_rotary: Optional[Rotary] = None, k_valid_len=None, **kw):
        if rotary is not None and not variant.takes_rotary:
            raise RotaryWithoutPosition(variant)
        if key_rotary is not None and rotary is None:
            raise Failure(EINVAL, "keyRotary without rotary")
        inner = (v if q is None else q).shape[-1]
        if inner % self.heads:
            raise Failure(EINVAL, f"inner dim {inner} is not a multiple of {self.heads} heads")
        return attention_fwd(q, k, v, heads=self.heads, q_norm_w=self.q_norm_weight,
                             k_norm_w=self.k_norm_weight, eps=self.norm_epsilon,
                             rotary=rotary, key_rotary=key_rotary, k_valid_len=k_valid_len,
                             **kw)


class DiTAttentionModule:
    """The whole attention module, ``DiTAttention.callAsFunction``
    (``Sources/LTXModules/DiTAttention.swift:315-405``): ``to_v`` / ``to_q`` / ``to_k`` through
    ``linear`` (q and k emitting the RMS statistic partials), the replaced unit taking its
    statistic from them, the gate from ``to_gate_logits(x)`` and ``to_out.0``. The Python
    mirror of ``ltx-2.5-swift_amd/host/dit_module.hpp``.

    ``weights`` maps the module's tensor names (``to_q.weight``, ``to_q.bias``, ``to_k.*``,
    ``to_v.*``, ``q_norm.weight``, ``k_norm.weight``, ``to_out.0.*``, optional
    ``to_gate_logits.*``; biases optional) to bf16 device tensors.
    """

    heads = 32
    norm_epsilon = 1e-6

    def __init__(self, weights, heads: int = 32):
        self.w = weights
        self.heads = heads
        q = weights["to_q.weight"]
        if q.shape[0] % heads:
            raise Failure(EINVAL, f"to_q.weight {tuple(q.shape)} is not [k * {heads}, queryDim]")
        self.core = DiTAttentionCore(weights["q_norm.weight"], weights["k_norm.weight"], heads)

    def _lin(self, t, name, sumsq=False, workspace=None):
        w = self.w[name + ".weight"]
        # the call's workspace doubles as the projection's split-tail scratch when it is
        # large enough (the projections and the attention run in stream order)
        need = linear_workspace_bytes(t.numel() // t.shape[-1], w.shape[0], w.shape[1])
        if workspace is not None and workspace.numel() * workspace.element_size() < need:
            workspace = None
        return linear(t, w, self.w.get(name + ".bias"), sumsq=sumsq, workspace=workspace)

    def __call__(self, x, context=None, *, variant: Variant, rotary: Optional[Rotary] = None,
                 key_rotary: Optional[Rotary] = None, k_valid_len=None,
                 all_perturbed: bool = False, workspace=None):
        kv = x if context is None else context                       # :327
        B, Lq, Lk = x.shape[0], x.shape[1], kv.shape[1]
        v = self._lin(kv, "to_v", workspace=workspace)                # :341
        gate = None
        if "to_gate_logits.weight" in self.w:                          # :387-391
            gate = self._lin(x, "to_gate_logits", workspace=workspace)
        if all_perturbed:                                              # :351-356
            o = self.core(None, None, v, variant=variant, gate_logits=gate, all_perturbed=True,
                          workspace=workspace)
        else:
            q, qs = self._lin(x, "to_q", sumsq=True, workspace=workspace)     # :358-359
            k, ks = self._lin(kv, "to_k", sumsq=True, workspace=workspace)
            o = self.core(q, k, v, variant=variant, rotary=rotary, key_rotary=key_rotary,
                          k_valid_len=k_valid_len, gate_logits=gate, workspace=workspace,
                          q_sumsq=qs.view(B * Lq, -1), k_sumsq=ks.view(B * Lk, -1))
        return self._lin(o, "to_out.0", workspace=workspace)          # :402-404


class DiTBlockAttention:
    """The six attention calls of one DiT block in the reference's order
    (``Sources/LTXModules/DiTBlock.swift:343-438``), phase by phase, on one stream with one
    workspace; the Python mirror of ``ltx-2.5-swift_amd/host/dit_block.hpp``.

    ``norms`` maps each variant's raw value (``attn1``, ``audio_attn1``, ``attn2``,
    ``audio_attn2``, ``audio_to_video_attn``, ``video_to_audio_attn``) to its
    ``(q_norm.weight, k_norm.weight)``. Each call takes ``(q, k, v, out)`` merged-layout
    tensors and an optional ``gate`` (``[B, Lq, 32]`` logits). Between phases the caller
    updates the residual streams and projects the next inputs; phase 3's inputs come from the
    streams as they stood before audio-to-video (the snapshot, ``:383-387``).
    """

    def __init__(self, norms):
        self.m = {v: DiTAttentionCore(*norms[v.value]) for v in Variant}

    def _run(self, variant, io, workspace, **kw):
        q, k, v, out = io[:4]
        gate = io[4] if len(io) > 4 else None
        return self.m[variant](q, k, v, variant=variant, out=out, workspace=workspace,
                               gate_logits=gate, **kw)

    def self_attention(self, video, audio, rot, video_perturbed=False, audio_perturbed=False,
                       workspace=None):
        """attn1 and audio_attn1 (:343-368); a perturbed stream takes the STG passthrough."""
        self._run(Variant.videoSelf, video, workspace, rotary=rot["videoSelf"],
                  all_perturbed=video_perturbed)
        self._run(Variant.audioSelf, audio, workspace, rotary=rot["audioSelf"],
                  all_perturbed=audio_perturbed)

    def text_cross(self, video, audio, text_valid_len=None, workspace=None):
        """attn2 and audio_attn2 (:370-381): text K/V, never rotated. ``text_valid_len=None``
        is the reference's arithmetic: every text token is attended, with no mask
        (DiTForward.swift:38-42, DiTAttention.swift:374-376). A list of per-row counts adds key
        padding, an extension whose outputs differ from the reference's."""
        self._run(Variant.videoCross, video, workspace, k_valid_len=text_valid_len)
        self._run(Variant.audioCross, audio, workspace, k_valid_len=text_valid_len)

    def cross_modal(self, a2v, v2a, rot, workspace=None):
        """audio_to_video then video_to_audio (:383-435); pe is the query stream's cross grid,
        k_pe the other stream's."""
        self._run(Variant.audioToVideo, a2v, workspace, rotary=rot["videoCross"],
                  key_rotary=rot["audioCross"])
        self._run(Variant.videoToAudio, v2a, workspace, rotary=rot["audioCross"],
                  key_rotary=rot["videoCross"])


# --------------------------------------------------------------------------------------
# RoPE tables (host, through the C ABI)
# --------------------------------------------------------------------------------------

def rope_frequency_grid(theta: float, n_pos: int, inner: int) -> np.ndarray:
    lib = load_library()
    cap = max(1, inner // (2 * max(1, n_pos)))
    out = np.zeros(cap, dtype=np.float32)
    n = lib.ltx_rope_frequency_grid(theta, n_pos, inner, out.ctypes.data, cap)
    if n < 0:
        raise Failure(EINVAL, "bad frequency-grid arguments")
    return out[:n]


def rope_video_positions(latent_frames, latent_height, latent_width, temporal_scale=8,
                         spatial_scale=32, frame_rate=24.0) -> np.ndarray:
    lib = load_library()
    tokens = latent_frames * latent_height * latent_width
    out = np.zeros((3, tokens, 2), dtype=np.float32)
    n = lib.ltx_rope_video_positions(latent_frames, latent_height, latent_width,
                                     temporal_scale, spatial_scale, frame_rate,
                                     out.ctypes.data, out.size)
    if n < 0:
        raise Failure(EINVAL, "bad video-position arguments")
    return out


def rope_reference_positions(ref: "Reference", target_first_end: float, frame_rate=24.0,
                             temporal_scale=8, spatial_scale=32) -> np.ndarray:
    """referencePositions (DiTForward.swift:553-593): ``[3, tokens, 2]`` bounds of one
    reference in the target's frame; ``target_first_end`` is the target grid's first patch
    end (``positions[0, 0, 1]``)."""
    lib = load_library()
    out = np.zeros((3, ref.tokens, 2), dtype=np.float32)
    n = lib.ltx_rope_reference_positions(ctypes.byref(ref), temporal_scale, spatial_scale,
                                         frame_rate, target_first_end, out.ctypes.data,
                                         ref.tokens)
    if n < 0:
        raise Failure(EINVAL, "bad reference-position arguments")
    return out


def rope_video_positions_with_references(latent_frames, latent_height, latent_width,
                                         references, temporal_scale=8, spatial_scale=32,
                                         frame_rate=24.0) -> np.ndarray:
    """The video grid of a render with references (DiTForward.swift:698-711): ``[3, total,
    2]`` with the target's tokens first, then every reference's in order."""
    lib = load_library()
    refs = (Reference * max(1, len(references)))(*references)
    total = latent_frames * latent_height * latent_width + sum(r.tokens for r in references)
    out = np.zeros((3, total, 2), dtype=np.float32)
    n = lib.ltx_rope_video_positions_with_references(
        latent_frames, latent_height, latent_width, temporal_scale, spatial_scale, frame_rate,
        refs, len(references), out.ctypes.data, out.size)
    if n != total:
        raise Failure(EINVAL, "bad video/reference-position arguments")
    return out


def audio_latent_count(frames: int, frame_rate: float = 24.0,
                       latents_per_second: float = 25.0) -> int:
    """Audio tokens of a clip: ``round(frames / frame_rate * latents_per_second)`` with halves
    rounded away from zero, as Swift's ``rounded()`` does, not to even
    (LatentGeometry.audioLatentCount, Sources/LTXFoundation/LatentGeometry.swift:128-132):
    97 frames at 24 fps are 101 tokens, 121 frames 126, 12 frames 13."""
    if frames <= 0 or not frame_rate > 0:
        raise Failure(EINVAL, "frames and frame_rate must be positive")
    x = float(frames) / float(frame_rate) * float(latents_per_second)
    whole = math.floor(x)
    return int(whole) + (1 if x - whole >= 0.5 else 0)   # x - whole is exact


def rope_audio_positions(tokens, hop_length=160, sample_rate=16000, downsample=4) -> np.ndarray:
    lib = load_library()
    out = np.zeros((1, tokens, 2), dtype=np.float32)
    n = lib.ltx_rope_audio_positions(tokens, hop_length, sample_rate, downsample,
                                     out.ctypes.data, out.size)
    if n < 0:
        raise Failure(EINVAL, "bad audio-position arguments")
    return out


def rope_connector_positions(sequence: int) -> np.ndarray:
    """The embeddings connector's 1-D index grid (EmbeddingsConnector.swift:239-248):
    positions ``0 .. sequence-1`` as ``[1, sequence, 2]`` bounds whose centre is the index,
    for ``rope_tables(..., max_pos=[CONNECTOR_MAX_POS])``."""
    idx = np.arange(sequence, dtype=np.float32)
    return np.stack([idx, idx], axis=-1)[None]


CONNECTOR_MAX_POS = 4096   # EmbeddingsConnector.positionalMaxPosition (:84)


def connector_rotary(sequence: int, width: int, heads: int = 32, device=None):
    """The connector's split-RoPE tables for ``sequence`` tokens of a ``width``-wide stream
    (4096 video, 2048 audio; theta 1e4, maxPos 4096, one positional dimension, no identity
    padding) as a ``Rotary`` of bf16 device tensors."""
    import torch

    cos, sin = rope_tables(rope_connector_positions(sequence), width, [CONNECTOR_MAX_POS], heads)
    dev = device or "cuda"
    to = lambda b: torch.from_numpy(b.view(np.int16)).to(dev).view(torch.bfloat16)  # noqa: E731
    return Rotary(to(cos), to(sin))


def rope_tables(positions: np.ndarray, inner: int, max_pos, heads: int = 32,
                theta: float = 10000.0):
    """bf16 bit patterns ``(cos, sin)``, each ``[heads, tokens, inner/2/heads]`` uint16."""
    lib = load_library()
    positions = np.ascontiguousarray(positions, dtype=np.float32)
    n_pos, tokens = positions.shape[0], positions.shape[1]
    mp = np.ascontiguousarray(max_pos, dtype=np.int32)
    per_head = inner // 2 // heads
    cos = np.zeros((heads, tokens, per_head), dtype=np.uint16)
    sin = np.zeros_like(cos)
    rc = lib.ltx_rope_tables(positions.ctypes.data, n_pos, tokens, inner, mp.ctypes.data,
                             heads, theta, cos.ctypes.data, sin.ctypes.data)
    if rc != 0:
        raise Failure(EINVAL, "bad rotary-table arguments")
    return cos, sin


def rope_tables_device(positions, inner: int, max_pos, heads: int = 32,
                       theta: float = 10000.0, stream=None):
    """``rope_tables`` built on the GPU: ``positions`` is a float32 ``[n_pos, tokens, 2]``
    tensor (moved to the current HIP device if it is not there); returns bf16 device tensors
    ``(cos, sin)``, each ``[heads, tokens, inner/2/heads]``, with the host builder's bits."""
    import torch

    lib = load_library()
    if isinstance(positions, np.ndarray):
        positions = torch.from_numpy(np.ascontiguousarray(positions, dtype=np.float32))
    if not positions.is_cuda:
        positions = positions.to("cuda")
    positions = positions.to(torch.float32).contiguous()
    n_pos, tokens = positions.shape[0], positions.shape[1]
    mp = np.ascontiguousarray(max_pos, dtype=np.int32)
    if mp.size != n_pos:
        raise Failure(EINVAL, "maxPos length must equal the positional dimension count")
    per_head = inner // 2 // heads
    cos = torch.empty((heads, tokens, per_head), dtype=torch.bfloat16, device=positions.device)
    sin = torch.empty_like(cos)
    if stream is None:
        stream = torch.cuda.current_stream(positions.device).cuda_stream
    _check(lib.ltx_rope_tables_device(ctypes.c_void_p(positions.data_ptr()), n_pos, tokens,
                                      inner, mp.ctypes.data, heads, theta,
                                      ctypes.c_void_p(cos.data_ptr()),
                                      ctypes.c_void_p(sin.data_ptr()), ctypes.c_void_p(stream)))
    cos._ltx_positions = positions  # noqa: SLF001 -- keep the input alive until the stream ran
    return cos, sin


def rotaries_device(frames: int, height: int, width: int, frame_rate: float = 24.0,
                    video_width: int = 4096, audio_width: int = 2048, heads: int = 32,
                    theta: float = 10000.0, audio_tokens: Optional[int] = None,
                    references=()):
    """``rotaries`` with the tables built on the GPU: the positions (a few floats per token)
    are built on the host and copied; the tables are written in device memory. Returns
    ``Rotary`` pairs of bf16 device tensors keyed like ``rotaries``."""
    lf = 1 if frames <= 1 else (frames - 1) // 8 + 1
    video = rope_video_positions_with_references(lf, height // 32, width // 32,
                                                 list(references), 8, 32, frame_rate)
    if audio_tokens is None:
        audio_tokens = audio_latent_count(frames, frame_rate)
    audio = rope_audio_positions(audio_tokens)
    out = {
        "videoSelf": rope_tables_device(video, video_width, [20, 2048, 2048], heads, theta),
        "audioSelf": rope_tables_device(audio, audio_width, [20], heads, theta),
        "videoCross": rope_tables_device(video[0:1], audio_width, [20], heads, theta),
        "audioCross": rope_tables_device(audio, audio_width, [20], heads, theta),
    }
    return {k: Rotary(c, s) for k, (c, s) in out.items()}


def rotaries(frames: int, height: int, width: int, frame_rate: float = 24.0,
             video_width: int = 4096, audio_width: int = 2048, heads: int = 32,
             theta: float = 10000.0, audio_tokens: Optional[int] = None, references=()):
    """The four tables of ``DiTForward.rotaries(geometry:dtype:)`` (DiTForward.swift:698-738)
    as numpy bf16 bit patterns, keyed ``videoSelf``, ``audioSelf``, ``videoCross``,
    ``audioCross``. ``references``: ``Reference`` clips appended to the video stream (the
    video tables then cover ``videoTokensWithReference`` tokens, :707-711)."""
    lf = 1 if frames <= 1 else (frames - 1) // 8 + 1
    video = rope_video_positions_with_references(lf, height // 32, width // 32,
                                                 list(references), 8, 32, frame_rate)
    if audio_tokens is None:
        audio_tokens = audio_latent_count(frames, frame_rate)
    audio = rope_audio_positions(audio_tokens)
    return {
        "videoSelf": rope_tables(video, video_width, [20, 2048, 2048], heads, theta),
        "audioSelf": rope_tables(audio, audio_width, [20], heads, theta),
        "videoCross": rope_tables(video[0:1], audio_width, [20], heads, theta),
        "audioCross": rope_tables(audio, audio_width, [20], heads, theta),
    }


# --------------------------------------------------------------------------------------
# Gemma-4 text-encoder attention (GemmaTextEncoder.swift:158-239, mask :288-321)
# --------------------------------------------------------------------------------------

def gemma_rope_tables(tokens: int, head_dim: int, theta: float, partial: float = 1.0,
                      proportional: bool = False):
    """fp32 ``(cos, sin)`` ``[tokens, head_dim/2]`` for positions ``0 .. tokens-1``
    (GemmaTextEncoder.positionEmbeddings, GemmaTextEncoder.swift:135-145)."""
    lib = load_library()
    cos = np.zeros((tokens, head_dim // 2), dtype=np.float32)
    sin = np.zeros_like(cos)
    if lib.ltx_gemma_rope_tables(tokens, head_dim, theta, partial, int(bool(proportional)),
                                 cos.ctypes.data, sin.ctypes.data) != 0:
        raise Failure(EINVAL, "bad Gemma rotary-table arguments")
    return cos, sin


def gemma_attention_fwd(q, k, v, *, q_heads: int, kv_heads: int, q_norm_w, k_norm_w, cos, sin,
                        window: int = 0, first_valid=None, scale: float = 1.0, eps: float = 1e-6,
                        out=None, workspace=None, stream=None):
    """One Gemma-4 attention from the projections: ``q`` ``[B, T, Hq*D]``, ``k``/``v``
    ``[B, T, Hkv*D]`` bf16 (pass ``v = k`` on the K-shares-V layers), norm weights ``[D]``,
    ``cos``/``sin`` fp32 device tensors ``[T, D/2]``; ``first_valid`` per batch row (keys
    before it are left padding). Returns ``out`` ``[B, T, Hq*D]`` fp32 (the dtype of the
    reference's explicit path)."""
    import torch

    lib = load_library()
    B, T, qw = q.shape
    D = qw // q_heads
    for t in (q, k, v):
        if t.stride(-1) != 1:
            raise Failure(EINVAL, "projection rows must be contiguous")
    if out is None:
        out = torch.empty((B, T, q_heads * D), dtype=torch.float32, device=q.device)
    a = GemmaArgs()
    a.B, a.T, a.Hq, a.Hkv, a.D = B, T, q_heads, kv_heads, D
    a.q, a.k, a.v = _ptr(q), _ptr(k), _ptr(v)
    a.q_bs, a.q_rs = q.stride(0), q.stride(1)
    a.k_bs, a.k_rs = k.stride(0), k.stride(1)
    a.v_bs, a.v_rs = v.stride(0), v.stride(1)
    a.q_norm_w, a.k_norm_w = _ptr(q_norm_w), _ptr(k_norm_w)
    a.eps = eps
    a.cos, a.sin = _ptr(cos), _ptr(sin)
    a.window = window
    fv = None
    if first_valid is not None:
        fv = (ctypes.c_int32 * B)(*[int(x) for x in first_valid])
        a.first_valid = ctypes.cast(fv, ctypes.POINTER(ctypes.c_int32))
    a.scale = scale
    a.out = _ptr(out)
    a.o_bs, a.o_rs = out.stride(0), out.stride(1)
    need = lib.ltx_gemma_attn_workspace_bytes(ctypes.byref(a))
    if need == 0:
        _check(lib.ltx_gemma_attn_fwd(ctypes.byref(a), None))
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    a.workspace, a.workspace_bytes = _ptr(workspace), workspace.numel()
    if stream is None:
        stream = torch.cuda.current_stream(q.device).cuda_stream
    _check(lib.ltx_gemma_attn_fwd(ctypes.byref(a), ctypes.c_void_p(stream)))
    out._ltx_keepalive = (workspace, fv)  # noqa: SLF001 -- until the stream has run
    return out
