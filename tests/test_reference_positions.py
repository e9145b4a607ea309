"""Reference-clip positions (DiTForward.referencePositions, DiTForward.swift:553-593) and the
reference-appended video grid of rotaries(geometry:dtype:) (:698-711), in the library's host
builder and in the oracle.

The four expectations of the reference's own suite (Tests/LTXModulesTests/
ReferencePositionTests.swift:38-150), at its geometry (25 frames of 128x192 at 24 fps,
references of 5 latent frames of 4x6): zero offset is bit-identical to the plain grid; an
offset moves time by exactly offset/fps; MSR slots are negative, ordered and separated; the
grid appends every reference in order. Then closed forms for the spatial downscale and the
temporally sparse shift, the refused offset + sparse combination, and the library against the
oracle bit for bit.
"""

import numpy as np
import pytest

import ltx_attn as L
import oracle as O

FPS = 24.0


def _times(grid):
    """Time starts of a [3, tokens, 2] grid (the [0, 0, :, 0] column of the reference's
    [1, 3, tokens, 2])."""
    return grid[0, :, 0]


def test_zero_offset_is_bit_identical_to_the_plain_grid():
    """ReferencePositionTests.swift:55-77."""
    target = L.rope_video_positions(4, 4, 6, 8, 32, FPS)
    got = L.rope_reference_positions(L.Reference(1, 4, 6), float(target[0, 0, 1]), FPS)
    want = L.rope_video_positions(1, 4, 6, 8, 32, FPS)
    assert got.shape == want.shape
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_offset_shifts_time_by_exactly_offset_over_fps():
    """ReferencePositionTests.swift:84-104: pixel frames, applied before the fps divide."""
    plain = L.Reference(5, 4, 6)
    shifted = L.Reference(5, 4, 6, frame_offset=-3)
    base = _times(L.rope_reference_positions(plain, 0.0, FPS))
    moved = _times(L.rope_reference_positions(shifted, 0.0, FPS))
    assert base.size == moved.size == 5 * 4 * 6
    assert np.all(np.abs((base - moved) - np.float32(3.0 / FPS)) < 1e-7)
    assert moved[0] < 0
    # not 3 seconds, not 3 latent frames
    assert abs(float(base[0] - moved[0]) - 3.0) > 1.0


def test_slots_are_ordered_and_separated():
    """ReferencePositionTests.swift:111-133: slot i of n at -(n - i) frames, pic1 earliest."""
    count = 4
    starts = [float(_times(L.rope_reference_positions(r, 0.0, FPS))[0])
              for r in L.msr_slots(count, 5, 4, 6)]
    assert all(s < 0 for s in starts)
    assert all(b > a for a, b in zip(starts, starts[1:]))
    assert abs(starts[0] + count / FPS) < 1e-7
    assert abs(starts[-1] + 1.0 / FPS) < 1e-7


def test_grid_appends_every_reference_in_order():
    """ReferencePositionTests.swift:140-169: [target, ref 0, ref 1, ref 2] along the tokens,
    each block's first time at its offset / fps, total = videoTokensWithReference."""
    count = 3
    refs = L.msr_slots(count, 5, 4, 6)
    # 25 frames of 128x192: 4 latent frames of 4x6
    grid = L.rope_video_positions_with_references(4, 4, 6, refs, frame_rate=FPS)
    target = L.rope_video_positions(4, 4, 6, 8, 32, FPS)
    video_tokens = 4 * 4 * 6
    assert grid.shape[1] == video_tokens + count * 5 * 4 * 6
    assert np.array_equal(grid[:, :video_tokens], target)
    at = video_tokens
    for r in refs:
        first = float(grid[0, at, 0])
        assert abs(first - r.frame_offset / FPS) < 1e-7
        block = L.rope_reference_positions(r, float(target[0, 0, 1]), FPS)
        assert np.array_equal(grid[:, at:at + r.tokens], block)
        at += r.tokens


def test_spatial_downscale_multiplies_space_only():
    """Step 5 (:583-585): a half-resolution reference covers the target's pixel range."""
    plain = L.rope_reference_positions(L.Reference(3, 6, 10), 1.0 / 24, FPS)
    half = L.rope_reference_positions(L.Reference(3, 6, 10, downscale_factor=2), 1.0 / 24, FPS)
    assert np.array_equal(half[0], plain[0])
    assert np.array_equal(half[1:], plain[1:] * 2)
    assert half[2, :, 1].max() == 10 * 32 * 2


def test_temporally_sparse_reference_slides_to_the_target_end():
    """Step 4 (:578-582), against its closed form: factor f spaces the reference at fps/f and
    slides it by (f - 1) * the target's first patch end, clamped at 0."""
    f, first_end = 2, np.float32(1.0 / 24)
    got = L.rope_reference_positions(L.Reference(4, 2, 2, temporal_scale_factor=f),
                                     float(first_end), FPS)
    pix = L.rope_video_positions(4, 2, 2, 8, 32, 1.0)[0]          # time in pixel frames
    want = np.maximum(pix.astype(np.float64) / (FPS / f) - (f - 1) * float(first_end), 0.0)
    assert np.all(np.abs(got[0] - want) < 1e-6)
    assert got[0].min() == 0.0 and np.array_equal(got[1:], L.rope_video_positions(4, 2, 2)[1:])


def test_offset_and_sparse_shift_do_not_compose():
    """:564-567: the clamp of step 4 would erase the negative times of step 3."""
    with pytest.raises(L.Failure):
        L.rope_reference_positions(L.Reference(2, 2, 2, temporal_scale_factor=2,
                                               frame_offset=-1), 0.0, FPS)
    with pytest.raises(ValueError):
        O.reference_positions(2, 2, 2, temporal_scale_factor=2, frame_offset=-1,
                              target=np.zeros((1, 3, 1, 2), np.float32))


@pytest.mark.parametrize("kw", [
    dict(), dict(frame_offset=-2), dict(downscale_factor=2), dict(temporal_scale_factor=3),
    dict(frame_offset=5, downscale_factor=2),
])
def test_library_matches_oracle_bit_for_bit(kw):
    target = O.video_positions(13, 12, 20, 8, 32, 25.0)
    lib = L.rope_reference_positions(L.Reference(7, 6, 10, **kw), float(target[0, 0, 0, 1]),
                                     25.0)
    ora = O.reference_positions(7, 6, 10, frame_rate=25.0, target=target, **kw)[0]
    assert np.array_equal(lib.view(np.uint32), ora.view(np.uint32))


def test_rotaries_with_references_extend_the_video_tables():
    """The video self and video cross tables cover target + reference tokens; the target's
    rows are the no-reference tables' rows; audio tables are untouched (:698-738)."""
    refs = [L.Reference(2, 4, 6, downscale_factor=2)] + L.msr_slots(2, 1, 4, 6)
    plain = L.rotaries(25, 128, 192)
    withr = L.rotaries(25, 128, 192, references=refs)
    T = 4 * 4 * 6
    extra = sum(r.tokens for r in refs)
    for key in ("videoSelf", "videoCross"):
        for a, b in zip(plain[key], withr[key]):
            assert b.shape[1] == T + extra
            assert np.array_equal(b[:, :T], a)
    for key in ("audioSelf", "audioCross"):
        for a, b in zip(plain[key], withr[key]):
            assert np.array_equal(a, b)
    # the appended rows are the tables of the appended positions
    grid = L.rope_video_positions_with_references(4, 4, 6, refs, frame_rate=FPS)
    cos, sin = L.rope_tables(grid[:, T:], 4096, [20, 2048, 2048], 32)
    assert np.array_equal(withr["videoSelf"][0][:, T:], cos)
    assert np.array_equal(withr["videoSelf"][1][:, T:], sin)


@pytest.mark.parametrize("frames,fps,tokens", [
    (97, 24.0, 101), (121, 24.0, 126), (25, 24.0, 26), (12, 24.0, 13), (1, 24.0, 1),
    (121, 30.0, 101), (36, 24.0, 38),
])
def test_audio_latent_count_rounds_half_away_from_zero(frames, fps, tokens):
    """LatentGeometry.audioLatentCount (LatentGeometry.swift:128-132): round, not ceil, and
    Swift's rounded() takes 12.5 (12 frames at 24 fps) to 13 where Python's round gives 12;
    36 frames are 37.5 -> 38 (even would also give 38), 121 at 30 fps 100.83 -> 101."""
    assert L.audio_latent_count(frames, fps) == tokens
    assert L.rotaries(frames, 64, 64)["audioSelf"][0].shape[1] == \
        L.audio_latent_count(frames, 24.0)


def test_audio_latent_count_refuses_empty_clips():
    with pytest.raises(L.Failure):
        L.audio_latent_count(0, 24.0)
    with pytest.raises(L.Failure):
        L.audio_latent_count(97, 0.0)
