"""The windowed pipeline's host logic: the seam stitcher restated from
src/engines/asr-parakeet/stitcher.js:7-41, pinned by hand-worked cases of the
reference's rules (frame-estimated overlap skip, refined by the longest exact
token match of 2 .. frameSkip + 8 tokens, Math.round half-up)."""
import pytest

SR, WIN, OVL = 16000, 240000, 32000
HOP = WIN - OVL


@pytest.fixture(scope="module")
def pl(fa):
    import importlib
    return importlib.import_module(fa.__name__ + ".pipeline")


def test_first_window_kept_whole(pl):
    ids, times, stitch = pl.createStitcher(HOP, SR, OVL)
    stitch(0, WIN, 188, [1, 2, 3], [0, 5, 10])
    assert ids == [1, 2, 3] and times == pytest.approx([0.0, 0.4, 0.8])


def test_frame_skip_then_token_match(pl):
    ids, times, stitch = pl.createStitcher(HOP, SR, OVL)
    stitch(0, WIN, 188, [1, 2, 3], [0, 5, 10])
    # overlapEnc = round(188 * 32000 / 240000) = 25: frames 3, 20 lie in the
    # overlap (frameSkip 2); the tail [2, 3] matches the head (matched 2)
    stitch(1, WIN, 188, [2, 3, 7, 8], [3, 20, 30, 40])
    assert ids == [1, 2, 3, 7, 8]
    assert times[3:] == pytest.approx([13 + 30 * 0.08, 13 + 40 * 0.08])


def test_token_match_longer_than_frame_skip(pl):
    ids, _, stitch = pl.createStitcher(HOP, SR, OVL)
    stitch(0, WIN, 188, [5, 6, 7, 8], [100, 110, 120, 130])
    stitch(1, WIN, 188, [6, 7, 8, 9], [30, 31, 32, 33])  # no frame in the overlap; [6, 7, 8] matches
    assert ids == [5, 6, 7, 8, 9]


def test_single_token_match_ignored_and_empty_window(pl):
    ids, _, stitch = pl.createStitcher(HOP, SR, OVL)
    stitch(0, WIN, 188, [4, 9], [0, 1])
    stitch(1, WIN, 188, [9, 4], [40, 50])  # a 1-token match does not count (L >= 2)
    stitch(2, WIN, 188, [], [])
    assert ids == [4, 9, 9, 4]


def test_overlap_estimate_rounds_half_up(pl):
    ids, _, stitch = pl.createStitcher(HOP, SR, 1)
    stitch(0, 2, 5, [1], [0])
    # Tenc * overlap / sliceLen = 5 * 1 / 2 = 2.5 -> Math.round 3: frames 0..2 skipped
    stitch(1, 2, 5, [7, 8, 9, 10], [0, 1, 2, 3])
    assert ids == [1, 10]


def test_longer_than_tested_transcription_is_refused(pl):
    """Inputs past the longest transcription that has run on the GPU are refused
    before any device work (no context is touched), unless the caller opts in."""
    import numpy as np
    audio = np.zeros(int((pl.MAX_TESTED_SECONDS + 1) * 16000), np.float32)
    with pytest.raises(ValueError, match="faulted the GPU"):
        pl.transcribeWindowed(None, None, None, None, None, audio)
