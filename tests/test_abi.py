"""The C-ABI boundary on the host: the library loads, exports every symbol include/ltx_attn.h
declares, validates arguments before launching anything (so every error path is testable
without a GPU), sizes its workspace, and builds the RoPE tables like the reference."""

import ctypes
import json
import math
import os
import re
import subprocess

import numpy as np
import pytest

import ltx_attn as L
import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ltx_attn.h")
GOLDEN = os.path.join(ROOT, "tests", "golden")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ltx_(?:attn_|rope_|linear|gemma_|device_)\w*)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = L.load_library()
    declared = _declared_functions()
    assert len(declared) >= 12
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(L.EXPORTED_SYMBOLS)
    nm = subprocess.run(["nm", "-D", "--defined-only", L.LIB_PATH], capture_output=True,
                        text=True, check=True).stdout
    for name in declared:
        assert re.search(rf"\bT {name}\b", nm), name


def test_struct_layout_and_version():
    lib = L.load_library()
    assert lib.ltx_attn_args_size() == ctypes.sizeof(L.Args)
    assert lib.ltx_attn_abi_version() == 8
    assert "gfx950" in L.provenance()
    for s in range(5):
        assert lib.ltx_attn_status_string(s)


# ---------------------------------------------------------------------------------------
# Validation: host-only, nothing is dereferenced on the device.
# ---------------------------------------------------------------------------------------

FAKE = 0x7F0000000000   # 256-byte aligned fake device address (never dereferenced)


def _args(B=1, H=32, Lq=3120, Lk=3120, D=128, ws=True, **kw):
    """Arguments of a plausible call; `ws` attaches a (fake) workspace large enough for any
    plan, so that validation reaches the field under test."""
    a = L.Args()
    L.load_library().ltx_attn_args_init(ctypes.byref(a))
    a.B, a.H, a.Lq, a.Lk, a.D = B, H, Lq, Lk, D
    inner = H * D
    a.q, a.k, a.v, a.out = FAKE, FAKE + (1 << 32), FAKE + (2 << 32), FAKE + (3 << 32)
    a.q_bs, a.q_rs, a.q_hs = Lq * inner, inner, D
    a.k_bs, a.k_rs, a.k_hs = Lk * inner, inner, D
    a.v_bs, a.v_rs, a.v_hs = Lk * inner, inner, D
    a.o_bs, a.o_rs, a.o_hs = Lq * inner, inner, D
    a.scale = 1.0 / np.sqrt(D)
    if ws:
        a.workspace, a.workspace_bytes = FAKE + (4 << 32), 1 << 40
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def _validate(a):
    lib = L.load_library()
    st = lib.ltx_attn_validate(ctypes.byref(a))
    return st, lib.ltx_attn_last_error().decode()


def test_valid_arguments_pass():
    # register-staged kernel without K work, whole rounds of items (32 heads x 8 query
    # blocks = 256): no workspace
    st, msg = _validate(_args(Lq=2048, kprep=L.KPREP_FUSED, ws=False))
    assert st == L.OK, msg
    # LDS-DMA kernel over 13 query blocks per head (416 items): the last round of 160 would
    # fill most CUs, so it is not split and needs no workspace
    st, msg = _validate(_args(ws=False))
    assert st == L.OK, msg
    # 9 query blocks over 2 x 32 heads (576 items): the last round's 64 items are split,
    # whose partials must be provided
    st, msg = _validate(_args(B=2, Lq=2100, Lk=3000, ws=False))
    assert st == L.EWORKSPACE, msg
    st, msg = _validate(_args(B=2, Lq=2100, Lk=3000))
    assert st == L.OK, msg


@pytest.mark.parametrize("field,value,status", [
    ("D", 96, L.EUNSUPPORTED),
    ("D", 80, L.EUNSUPPORTED),
    ("B", 0, L.EINVAL),
    ("Lk", 0, L.EINVAL),
    ("q", FAKE + 8, L.EINVAL),          # misaligned
    ("v", 0, L.EINVAL),                 # NULL
    ("k_rs", 4100, L.EINVAL),           # not a multiple of 8
    ("q_hs", 64, L.EINVAL),             # heads overlap
    ("scale", 0.0, L.EINVAL),
    ("scale", float("nan"), L.EINVAL),
    ("kprep", 7, L.EINVAL),
    ("num_splits", 17, L.EINVAL),
    ("resident_groups", -1, L.EINVAL),
    ("resident_groups", 65537, L.EINVAL),
])
def test_invalid_arguments_are_rejected(field, value, status):
    a = _args()
    setattr(a, field, value)
    st, msg = _validate(a)
    assert st == status, msg
    assert msg


def test_gate_rules():
    # [B, Lq, H] logits: any 2-byte aligned pointer, non-negative strides
    a = _args(gate_logits=FAKE + 2, g_bs=3120 * 32, g_rs=32, g_hs=1)
    st, msg = _validate(a)
    assert st == L.OK, msg
    a.gate_logits = FAKE + 1
    st, msg = _validate(a)
    assert st == L.EINVAL and "gate_logits" in msg
    a.gate_logits, a.g_rs = FAKE, -32
    st, msg = _validate(a)
    assert st == L.EINVAL and "gate_logits" in msg
    # the gate costs no workspace
    lib = L.load_library()
    assert (lib.ltx_attn_workspace_bytes(ctypes.byref(_args(ws=False, gate_logits=FAKE)))
            == lib.ltx_attn_workspace_bytes(ctypes.byref(_args(ws=False))))


def test_passthrough_rules():
    """STG passthrough (DiTAttention.swift:351-356): q and k are not needed (NULL is fine),
    nothing is allocated, and it is refused for cross-attention (Lq != Lk)."""
    lib = L.load_library()
    a = _args(ws=False, all_perturbed=1, q=0, k=0, q_norm_w=FAKE, q_cos=FAKE)
    st, msg = _validate(a)
    assert st == L.OK, msg
    assert lib.ltx_attn_workspace_bytes(ctypes.byref(a)) == 0
    st, msg = _validate(_args(ws=False, all_perturbed=1, Lq=3120, Lk=1024))
    assert st == L.EINVAL and "self-attention" in msg
    st, msg = _validate(_args(ws=False, all_perturbed=1, v=0))
    assert st == L.EINVAL
    st, msg = _validate(_args(ws=False, all_perturbed=1, gate_logits=FAKE + 1))
    assert st == L.EINVAL and "gate_logits" in msg


def test_rotary_rules():
    # k tables without q tables: keyRotary without rotary
    st, msg = _validate(_args(k_cos=FAKE, k_sin=FAKE))
    assert st == L.EINVAL and "keyRotary" in msg
    # only one of a pair
    st, _ = _validate(_args(q_cos=FAKE))
    assert st == L.EINVAL
    # K reuses Q's tables but the streams differ in length (cross-modal without k_pe)
    st, msg = _validate(_args(Lq=3120, Lk=126, D=64, H=32, q_cos=FAKE, q_sin=FAKE))
    assert st == L.EINVAL and "Lq" in msg
    st, msg = _validate(_args(Lq=3120, Lk=126, D=64, H=32, q_cos=FAKE, q_sin=FAKE,
                              k_cos=FAKE, k_sin=FAKE, ws=False))
    assert st == L.EWORKSPACE, msg      # arguments fine; the K prologue needs scratch


def test_key_padding_rules():
    lens = (ctypes.c_int32 * 2)(94, 0)
    a = _args(B=2, Lk=1024)
    a.k_valid_len = ctypes.cast(lens, ctypes.POINTER(ctypes.c_int32))
    st, msg = _validate(a)
    assert st == L.EINVAL and "k_valid_len[1]" in msg     # empty mask
    lens[1] = 1025
    st, _ = _validate(a)
    assert st == L.EINVAL
    lens[1] = 1
    st, msg = _validate(a)
    assert st == L.OK, msg
    big = (ctypes.c_int32 * 65)(*([5] * 65))
    a = _args(B=65, Lk=16, Lq=16)
    a.k_valid_len = ctypes.cast(big, ctypes.POINTER(ctypes.c_int32))
    assert _validate(a)[0] == L.EUNSUPPORTED


def test_workspace_sizing_and_check():
    lib = L.load_library()
    # plain attention over 13 query blocks (LDS-DMA kernel, which reads K and V in place):
    # 416 items = one whole round of 256 + 160, a last round more than half full: no split,
    # nothing to hold
    a = _args(ws=False)
    assert lib.ltx_attn_workspace_bytes(ctypes.byref(a)) == 0
    a = _args(kprep=L.KPREP_FUSED, ws=False)
    assert lib.ltx_attn_workspace_bytes(ctypes.byref(a)) == 0
    # 2 x 32 heads x 9 query blocks = 576 items: the last 64 are split (the tail round at a
    # quarter of the CUs) into 4 key ranges of 12 tiles, each partial row 128 fp32 + (max, sum)
    rows = 4 * 64 * 256
    tail = rows * 128 * 4 + rows * 2 * 4
    a = _args(B=2, Lq=2100, Lk=3000, ws=False)
    assert lib.ltx_attn_workspace_bytes(ctypes.byref(a)) == tail
    a = _args(B=2, Lq=2100, Lk=3000, kprep=L.KPREP_FUSED, ws=False)
    assert lib.ltx_attn_workspace_bytes(ctypes.byref(a)) == tail
    # whole rounds only (256 items): nothing
    a = _args(Lq=2048, kprep=L.KPREP_FUSED, ws=False)
    assert lib.ltx_attn_workspace_bytes(ctypes.byref(a)) == 0
    # 12480-token self-attention with norm + RoPE: q statistic + prepared K + the tail
    # split (1568 items = 6 rounds of 256 + 32 items split into 7 ranges of 28 tiles)
    a = _args(Lq=12480, Lk=12480, q_norm_w=FAKE, k_norm_w=FAKE, q_cos=FAKE, q_sin=FAKE,
              ws=False)
    need = lib.ltx_attn_workspace_bytes(ctypes.byref(a))
    rstd = (12480 * 4 + 255) // 256 * 256
    kprep = (12480 * 4096 * 2 + 255) // 256 * 256
    rows = 7 * 32 * 256
    assert need == rstd + kprep + rows * 128 * 4 + rows * 2 * 4
    st, msg = _validate(a)
    assert st == L.EWORKSPACE and str(need) in msg
    a.workspace, a.workspace_bytes = FAKE, need - 1
    assert _validate(a)[0] == L.EWORKSPACE
    a.workspace_bytes = need
    assert _validate(a)[0] == L.OK
    a.workspace = FAKE + 16
    assert _validate(a)[0] == L.EINVAL      # 256-byte alignment
    # fused K strategy: the statistics and the tail split
    a = _args(Lq=12480, Lk=12480, q_norm_w=FAKE, k_norm_w=FAKE, q_cos=FAKE, q_sin=FAKE,
              kprep=L.KPREP_FUSED)
    fused = 2 * rstd + rows * 128 * 4 + rows * 2 * 4
    assert lib.ltx_attn_workspace_bytes(ctypes.byref(a)) == fused
    # V rows too far apart for the LDS-DMA kernel's 32-bit offsets (12480 padded rows of
    # 262144 bytes): the register-staged kernel takes the call, with its fused K work
    a = _args(Lq=12480, Lk=12480, q_norm_w=FAKE, k_norm_w=FAKE, q_cos=FAKE, q_sin=FAKE,
              v_rs=131072, v_bs=12480 * 131072)
    assert lib.ltx_attn_workspace_bytes(ctypes.byref(a)) == fused
    a.v_rs = 65536                          # 12480 * 131072 bytes fit: back to the DMA kernel
    assert lib.ltx_attn_workspace_bytes(ctypes.byref(a)) == need
    # 126 audio queries over 3120 video keys (49 key tiles): split-KV partials for every
    # (head, query block) item, 256 rows each; 8 requested splits become 7 splits of 7 tiles
    # (no split is left empty)
    a = _args(Lq=126, Lk=3120, D=64, num_splits=8, kprep=L.KPREP_FUSED)
    need = lib.ltx_attn_workspace_bytes(ctypes.byref(a))
    rows = 7 * 32 * 256
    assert need == (rows * 64 * 4 + 255) // 256 * 256 + (rows * 2 * 4 + 255) // 256 * 256


def test_projection_statistic_rules():
    """q_sumsq / k_sumsq (the projection's partial sums of squares) replace the statistic pass;
    they need their norm weight, a block count and a row stride that holds the blocks."""
    w = FAKE + (5 << 32)
    a = _args(q_norm_w=w, k_norm_w=w, q_sumsq=FAKE + (6 << 32), q_sumsq_rs=16,
              k_sumsq=FAKE + (7 << 32), k_sumsq_rs=48, sumsq_blocks=16)
    st, msg = _validate(a)
    assert st == L.OK, msg
    for field, value in (("sumsq_blocks", 0), ("q_sumsq_rs", 15), ("k_sumsq", FAKE + 2),
                         ("q_norm_w", None)):
        b = _args(q_norm_w=w, k_norm_w=w, q_sumsq=FAKE + (6 << 32), q_sumsq_rs=16,
                  k_sumsq=FAKE + (7 << 32), k_sumsq_rs=48, sumsq_blocks=16)
        setattr(b, field, value)
        st, msg = _validate(b)
        assert st == L.EINVAL and msg, (field, msg)
    # the statistic still lands in the workspace, so the workspace is unchanged
    lib = L.load_library()
    plain = _args(ws=False, q_norm_w=w, k_norm_w=w)
    given = _args(ws=False, q_norm_w=w, k_norm_w=w, q_sumsq=FAKE, q_sumsq_rs=16,
                  k_sumsq=FAKE, k_sumsq_rs=16, sumsq_blocks=16)
    assert (lib.ltx_attn_workspace_bytes(ctypes.byref(given))
            == lib.ltx_attn_workspace_bytes(ctypes.byref(plain)) > 0)


def _linear_args(M=12480, N=4096, K=4096, **kw):
    a = L.LinearArgs()
    a.M, a.N, a.K = M, N, K
    a.x, a.w, a.y = FAKE, FAKE + (1 << 32), FAKE + (2 << 32)
    a.x_rs, a.w_rs, a.y_rs = K, K, N
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("field,value,status", [
    ("N", 12, L.EINVAL),                # not a multiple of 8
    ("N", 0, L.EINVAL),
    ("K", 96, L.EUNSUPPORTED),          # not a multiple of 64
    ("K", 32, L.EINVAL),
    ("M", -1, L.EINVAL),
    ("x", FAKE + 8, L.EINVAL),          # misaligned
    ("w", None, L.EINVAL),
    ("y", FAKE + (2 << 32) + 4, L.EINVAL),
    ("bias", FAKE + 2, L.EINVAL),
    ("x_rs", 4100, L.EINVAL),           # not a multiple of 8
    ("w_rs", 2048, L.EINVAL),           # below K
    ("y_rs", 4098, L.EINVAL),           # not a multiple of 4
    ("x_rs", 1 << 23, L.EUNSUPPORTED),  # a 256-row tile past 32-bit offsets
    ("sumsq", FAKE + (3 << 32) + 2, L.EINVAL),
    ("y", FAKE + 1024, L.EINVAL),       # y overlaps x
    ("resident_groups", -3, L.EINVAL),
])
def test_linear_rejects_bad_arguments(field, value, status):
    """Every rejection happens on the host before a launch (this host has no GPU)."""
    lib = L.load_library()
    a = _linear_args(sumsq=FAKE + (3 << 32), sumsq_rs=16)
    setattr(a, field, value)
    assert lib.ltx_linear(ctypes.byref(a), None) == status
    assert lib.ltx_attn_last_error().decode()


def test_linear_statistic_layout():
    lib = L.load_library()
    assert [lib.ltx_linear_sumsq_blocks(n) for n in (8, 256, 264, 2048, 4096, 12288 + 32)] == \
        [1, 1, 2, 8, 16, 49]
    # a row stride below the block count is rejected; M = 0 launches nothing
    a = _linear_args(sumsq=FAKE + (3 << 32), sumsq_rs=15)
    assert lib.ltx_linear(ctypes.byref(a), None) == L.EINVAL
    assert lib.ltx_linear(ctypes.byref(_linear_args(M=0)), None) == L.OK


@pytest.mark.parametrize("M,N,K,tail_tiles,ranges", [
    (12480, 4096, 4096, 16, 8),    # 784 tiles: 3 rounds + 16 tiles, 8 ranges of 8 steps
    (12480, 12288, 4096, 48, 4),   # fused q/k/v: 2352 = 9 rounds + 48 tiles, 4 ranges of 16
    (12480, 32, 4096, 49, 4),      # gate logits: 49 tiles in one round
    (1000, 4096, 2048, 64, 2),     # 64 tiles, 2 ranges of 16 steps
    (77, 32, 4096, 1, 32),         # one tile: 32 ranges of 2 steps
    (3120, 4096, 4096, 0, 0),      # 208 tiles: a tail of more than half a round runs whole
    (4096, 4096, 4096, 0, 0),      # 256 tiles: one whole round
    (300, 520, 192, 0, 0),         # 3 k steps: too few to split
])
def test_linear_tail_split_workspace(M, N, K, tail_tiles, ranges):
    """ltx_linear_workspace_bytes: 256 KiB of fp32 partials per k range of each tile past the
    last whole round of 256, the range count minimising ceil(steps / ranges) x 1.3 us plus
    tiles x ranges x 0.116 us (a range's k steps against its partials' round trip); a
    host-only query."""
    assert L.linear_workspace_bytes(M, N, K) == tail_tiles * ranges * 256 * 256 * 4
    lib = L.load_library()
    bad = _linear_args(K=96)
    assert lib.ltx_linear_workspace_bytes(ctypes.byref(bad)) == 0
    assert lib.ltx_attn_last_error().decode()


def test_linear_workspace_is_checked():
    """A workspace large enough to split is checked for alignment and overlap before a
    launch; a smaller one (or none) means whole tiles, not an error."""
    lib = L.load_library()
    need = L.linear_workspace_bytes(12480, 4096, 4096)
    assert need > 0                       # 784 tiles: the 16 past three rounds split along K
    base = FAKE + (8 << 32)
    a = _linear_args(M=12480, N=4096, K=4096, x=base, w=base + (1 << 30),
                     y=base + (2 << 30), x_rs=4096, w_rs=4096, y_rs=4096)
    # the plan the workspace was sized for, whatever device (or none) this host has: the
    # checks below run before any launch on the fake pointers
    a.resident_groups = 256
    a.workspace, a.workspace_bytes = base + (3 << 30) + 128, need
    assert lib.ltx_linear(ctypes.byref(a), None) == L.EINVAL          # not 256-byte aligned
    a.workspace = base + (2 << 30)                                    # on top of y
    assert lib.ltx_linear(ctypes.byref(a), None) == L.EINVAL
    assert "overlaps" in lib.ltx_attn_last_error().decode()


def test_zero_work_needs_no_gpu():
    """Validation failures return before any HIP call: this runs on a GPU-less host."""
    lib = L.load_library()
    a = _args(D=96)
    assert lib.ltx_attn_fwd(ctypes.byref(a), None) == L.EUNSUPPORTED


# ---------------------------------------------------------------------------------------
# RoPE tables built by the library (host code) vs the oracle and the reference digests
# ---------------------------------------------------------------------------------------

def test_frequency_grid_and_positions_bit_exact():
    for n_pos, inner in ((3, 4096), (1, 2048), (1, 4096)):
        np.testing.assert_array_equal(L.rope_frequency_grid(10000.0, n_pos, inner),
                                      O.frequency_grid(10000.0, n_pos, inner))
    np.testing.assert_array_equal(L.rope_video_positions(4, 6, 10)[None],
                                  O.video_positions(4, 6, 10))
    np.testing.assert_array_equal(L.rope_video_positions(13, 24, 40)[None],
                                  O.video_positions(13, 24, 40))
    np.testing.assert_array_equal(L.rope_audio_positions(126)[None], O.audio_positions(126))


def test_rope_tables_match_oracle():
    lib_t = L.rotaries(25, 192, 320)
    ora_t = O.rotaries(25, 192, 320)
    for name in lib_t:
        for a, b in zip(lib_t[name], ora_t[name]):
            assert a.shape == b.shape
            same = np.mean(a == b)
            diff = np.max(np.abs(a.astype(np.int32) - b.astype(np.int32)))
            assert same > 0.999 and diff <= 1, (name, same, diff)


def test_rope_tables_match_reference_digests():
    with open(os.path.join(GOLDEN, "tiny_v5_rope_digests.json")) as fh:
        dig = json.load(fh)
    tabs = L.rotaries(25, 192, 320)
    for table, tap, tol in (("videoSelf", "block_00.attn1.in.kw_pe", 1e-9),
                            ("videoCross", "block_00.audio_to_video_attn.in.kw_pe", 1e-9),
                            ("audioSelf", "block_00.audio_attn1.in.kw_pe", 2e-6),
                            ("audioCross", "block_00.video_to_audio_attn.in.kw_pe", 2e-6)):
        for bits, key in zip(tabs[table], (tap, tap + ".el1")):
            x = O.bf16_bits_to_f32(bits).astype(np.float64)
            assert abs(x.mean() - dig[key]["mean"]) < tol, key
            assert abs(x.std(ddof=1) - dig[key]["std"]) < tol, key


def test_rope_builders_reject_bad_arguments():
    with pytest.raises(L.Failure):
        L.rope_frequency_grid(10000.0, 3, 4)      # one-element grid
    with pytest.raises(L.Failure):
        L.rope_tables(np.zeros((1, 4, 2), np.float32), 2048, [0], 32)   # maxPos 0


def test_device_rope_builder_rejects_bad_arguments():
    """ltx_rope_tables_device checks everything before a launch: these return EINVAL on a
    host without a GPU (the pointers are never dereferenced)."""
    lib = L.load_library()
    mp3 = (ctypes.c_int32 * 3)(20, 2048, 2048)
    mp0 = (ctypes.c_int32 * 1)(0)
    good = dict(positions=FAKE, n_pos=3, tokens=240, inner=4096, max_pos=mp3, heads=32,
                theta=10000.0, cos=FAKE + 256, sin=FAKE + 512)

    def call(**kw):
        a = dict(good, **kw)
        return lib.ltx_rope_tables_device(a["positions"], a["n_pos"], a["tokens"], a["inner"],
                                          ctypes.cast(a["max_pos"], ctypes.c_void_p),
                                          a["heads"], a["theta"], a["cos"], a["sin"], None)

    assert call(n_pos=0) == L.EINVAL
    assert call(n_pos=9) == L.EINVAL                 # more positional dims than supported
    assert call(inner=4096, heads=3) == L.EINVAL     # 2048 columns do not split into 3 heads
    assert call(n_pos=1, max_pos=mp0) == L.EINVAL    # maxPos 0
    assert call(positions=FAKE + 2) == L.EINVAL      # float positions misaligned
    assert call(cos=FAKE + 1) == L.EINVAL            # bf16 output misaligned
    assert call(sin=None) == L.EINVAL
    assert call(theta=0.0) == L.EINVAL
    assert call(inner=6, n_pos=3) == L.EINVAL        # a one-element frequency grid


def test_cpp_block_driver_host_behaviour(tmp_path):
    """The C++ block driver (ltx-2.5-swift_amd/host/dit_block.hpp): one workspace sized for the
    largest of the six calls, none for an STG passthrough, failures thrown before a launch."""
    src = os.path.join(ROOT, "tests", "cpp", "test_dit_block.cpp")
    exe = str(tmp_path / "test_dit_block")
    libdir = os.path.dirname(L.LIB_PATH)
    subprocess.run(["g++", "-std=c++17", "-O1", src, "-o", exe, f"-L{libdir}", "-lltx_attn",
                    f"-Wl,-rpath,{libdir}", "-L/opt/rocm/lib", "-Wl,-rpath-link,/opt/rocm/lib"],
                   check=True, capture_output=True)
    run = subprocess.run([exe], capture_output=True, text=True)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "0 failure(s)" in run.stdout


def test_cpp_module_driver_host_behaviour(tmp_path):
    """The C++ module driver (ltx-2.5-swift_amd/host/dit_module.hpp): weight shapes checked at
    construction, the workspace layout, and failures thrown before any launch."""
    src = os.path.join(ROOT, "tests", "cpp", "test_dit_module.cpp")
    exe = str(tmp_path / "test_dit_module")
    libdir = os.path.dirname(L.LIB_PATH)
    subprocess.run(["g++", "-std=c++17", "-O1", src, "-o", exe, f"-L{libdir}", "-lltx_attn",
                    f"-Wl,-rpath,{libdir}", "-L/opt/rocm/lib", "-Wl,-rpath-link,/opt/rocm/lib"],
                   check=True, capture_output=True)
    run = subprocess.run([exe], capture_output=True, text=True)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "0 failure(s)" in run.stdout


def test_cpp_host_mirror_error_behaviour(tmp_path):
    """The C++ DiTAttention mirror (ltx-2.5-swift_amd/host/dit_attention.hpp) throws the
    reference's structural failures before anything reaches a device."""
    src = os.path.join(ROOT, "tests", "cpp", "test_dit_attention.cpp")
    exe = str(tmp_path / "test_dit_attention")
    libdir = os.path.dirname(L.LIB_PATH)
    subprocess.run(["g++", "-std=c++17", "-O1", src, "-o", exe, f"-L{libdir}", "-lltx_attn",
                    f"-Wl,-rpath,{libdir}", "-L/opt/rocm/lib", "-Wl,-rpath-link,/opt/rocm/lib"],
                   check=True, capture_output=True)
    run = subprocess.run([exe], capture_output=True, text=True)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "0 failure(s)" in run.stdout


def test_connector_rope_tables():
    """The embeddings connector's tables (EmbeddingsConnector.swift:218-248): positions
    arange(seq) over maxPos 4096, one positional dimension filling width/2 frequencies (no
    identity padding), per-head reshape. Checked against the oracle's table recipe (the two
    evaluate cos/sin of the same float32 angle with different float32 libraries, which may
    land on either side of a bf16 rounding boundary: at most one step, in at most 1e-5 of the
    entries), and against the closed form angle_i = f_i * (2p/4096 - 1),
    f_i = 1e4^(i/(n-1)) * pi/2, with cos/sin of the float32 angle in float64 (within one bf16
    step, plus the float32 evaluation's absolute error)."""
    import oracle as O

    seq, heads = 1024, 32
    for width in (4096, 2048):
        cos, sin = L.rope_tables(L.rope_connector_positions(seq), width, [L.CONNECTOR_MAX_POS],
                                 heads)
        pos = np.zeros((1, 1, seq, 2), dtype=np.float32)
        pos[0, 0, :, 0] = pos[0, 0, :, 1] = np.arange(seq)
        oc, os_ = O.rotary_tables(pos, width, [L.CONNECTOR_MAX_POS], heads)
        for got, ref in ((cos, oc), (sin, os_)):
            diff = got != ref
            assert diff.mean() <= 1e-5
            step = np.abs(got.astype(np.int32) - ref.astype(np.int32))
            assert step.max() <= 1
        n = width // 2
        t = np.array([1.0 if i == n - 1 else i * (1.0 / (n - 1)) for i in range(n)])
        f = (10000.0 ** t * math.pi / 2).astype(np.float32)
        frac = (np.arange(seq, dtype=np.float32) / np.float32(4096.0)).astype(np.float32)
        ang = (f[None, :] * (frac * np.float32(2.0) - np.float32(1.0))[:, None]).astype(np.float32)
        want_c = np.cos(ang.astype(np.float64)).reshape(seq, heads, n // heads).transpose(1, 0, 2)
        want_s = np.sin(ang.astype(np.float64)).reshape(seq, heads, n // heads).transpose(1, 0, 2)
        for got, want in ((cos, want_c), (sin, want_s)):
            g = O.bf16_bits_to_f32(got).astype(np.float64)
            assert np.all(np.abs(g - want) <= 2.0 ** -7 * np.abs(want) + 1e-7)


def test_gemma_rope_tables_match_oracle():
    """ltx_gemma_rope_tables against the oracle (GemmaTextEncoder.swift:135-145): both the
    sliding (default, theta 1e4, D 256) and full (proportional 0.25, theta 1e6, D 512) kinds;
    float cos/sin of the same float angle, within one float step of the correctly rounded
    value; the zero-frequency tail is exactly cos 1, sin 0."""
    for D, theta, part, prop, kind in ((256, 1e4, 1.0, False, "default"),
                                       (512, 1e6, 0.25, True, "proportional")):
        cos, sin = L.gemma_rope_tables(1024, D, theta, part, prop)
        oc, os_ = O.gemma_rope_tables(1024, O.gemma_inverse_frequencies(D, theta, part, kind))
        assert np.all(np.abs(cos - oc) <= 2.0 ** -23 * np.abs(oc) + 2.0 ** -30)
        assert np.all(np.abs(sin - os_) <= 2.0 ** -23 * np.abs(os_) + 2.0 ** -30)
        if prop:
            assert np.all(cos[:, 64:] == 1.0) and np.all(sin[:, 64:] == 0.0)


def test_gemma_partials_at_a_long_prompt():
    """Split partials only for the query blocks that split, per batch row: a full layer (D 512,
    64-query workgroups, one KV head) at 8192 tokens runs its 256 key blocks in ranges of 32;
    query block j walks 2j + 2 key blocks, so blocks 0-15 run one range and 16-127 run 2..8
    (16 blocks each): 16 * (2 + ... + 8) = 560 ranges per head, 16 heads, 64 rows each, fp32 O
    (512) and (max, sum) per row: 1.18 GB (every block sized for 8 ranges would be 2.16 GB).
    A second batch row padded on the left by 4000 tokens walks every key in its first 63 blocks
    (8 ranges each) and the causal range after that."""
    lib = L.load_library()
    T, D, Hq = 8192, 512, 16
    a = L.GemmaArgs()
    a.B, a.T, a.Hq, a.Hkv, a.D = 1, T, Hq, 1, D
    a.q = a.k = a.v = FAKE
    a.q_bs, a.q_rs = T * Hq * D, Hq * D
    a.k_bs = a.v_bs = T * D
    a.k_rs = a.v_rs = D
    a.q_norm_w = a.k_norm_w = FAKE
    a.eps, a.scale = 1e-6, 1.0
    a.cos = a.sin = FAKE
    a.out = FAKE
    a.o_bs, a.o_rs = T * Hq * D, Hq * D
    prep = 2 * T * D * (Hq + 1 + 1)                    # q', k', v'^T (fp16)
    rows = Hq * 16 * sum(range(2, 9)) * 64
    need = lib.ltx_gemma_attn_workspace_bytes(ctypes.byref(a))
    assert need == prep + rows * D * 4 + rows * 2 * 4
    assert 1.17e9 < need - prep < 1.19e9
    # B = 2, the second row left-padded by 4000 tokens: its blocks 0-62 (rows below 4032)
    # hold padding rows and walk all 256 key blocks (8 ranges); block 63 onward starts at key
    # block 4000 // 32 = 125 and ends at 2j + 1
    fv = (ctypes.c_int32 * 2)(0, 4000)
    a.B = 2
    a.q_bs, a.k_bs, a.v_bs, a.o_bs = T * Hq * D, T * D, T * D, T * Hq * D
    a.first_valid = ctypes.cast(fv, ctypes.POINTER(ctypes.c_int32))
    second = 63 * 8 + sum(n for n in ((2 * j + 1 - 125 + 32) // 32 for j in range(63, 128))
                          if n > 1)
    rows2 = rows + Hq * second * 64
    assert lib.ltx_gemma_attn_workspace_bytes(ctypes.byref(a)) == \
        2 * prep + rows2 * D * 4 + rows2 * 2 * 4


def test_gemma_attention_rejects_bad_arguments():
    lib = L.load_library()

    def args(**kw):
        a = L.GemmaArgs()
        a.B, a.T, a.Hq, a.Hkv, a.D = 1, 1024, 16, 8, 256
        a.q = a.k = a.v = FAKE
        a.q_bs = 1024 * 4096
        a.q_rs = 4096
        a.k_bs = a.v_bs = 1024 * 2048
        a.k_rs = a.v_rs = 2048
        a.q_norm_w = a.k_norm_w = FAKE
        a.eps, a.scale = 1e-6, 1.0
        a.cos = a.sin = FAKE
        a.window = 1024
        a.out = FAKE
        a.o_bs, a.o_rs = 1024 * 4096, 4096
        for n, val in kw.items():
            setattr(a, n, val)
        return a

    def status(a):
        st = lib.ltx_gemma_attn_fwd(ctypes.byref(a), None)
        return st, lib.ltx_attn_last_error().decode()

    a = args()
    need = lib.ltx_gemma_attn_workspace_bytes(ctypes.byref(a))
    # q', k', v'^T (fp16), then the key split's partials: 128-query workgroups, whose 4..32
    # key blocks run in ranges of at most 16; query blocks 4-7 (20..32 blocks) have two ranges,
    # 0-3 one (no partials): 16 heads x 4 blocks x 2 ranges x 128 rows of fp32 O and (max, sum)
    rows = 16 * 4 * 2 * 128
    assert need == 2 * 1024 * 256 * (16 + 8 + 8) + rows * 256 * 4 + rows * 2 * 4
    assert status(a)[0] == L.EWORKSPACE
    assert status(args(D=128))[0] == L.EUNSUPPORTED
    assert status(args(Hkv=3))[0] == L.EINVAL
    assert status(args(T=1022))[0] == L.EUNSUPPORTED
    assert status(args(window=-1))[0] == L.EINVAL
    assert status(args(cos=None))[0] == L.EINVAL
    assert status(args(q_rs=2048))[0] == L.EINVAL        # row narrower than Hq*D
    fv = (ctypes.c_int32 * 1)(1025)
    st, msg = status(args(first_valid=ctypes.cast(fv, ctypes.POINTER(ctypes.c_int32))))
    assert st == L.EINVAL and "first_valid" in msg
