"""Window planning for long-form audio.

planWindows / groupWindows restate src/engines/asr-parakeet/windowing.js:5-34
(fixed windows, equal-length groups of up to wb, short tail alone).  The
ragged planner is new: it cuts variable-length windows and packs them into
batches of up to `max_batch` windows that the GPU encodes in one call
(packed back to back, so no padding frames are computed).
"""
from __future__ import annotations

import numpy as np


def planWindows(totalSamples: int, winSamples: int, hop: int) -> list:
    """windowing.js:5-13: window starts at a fixed hop; short input -> one window."""
    starts = []
    single = totalSamples <= winSamples
    s = 0
    while s < totalSamples:
        starts.append(s)
        if single:
            break
        s += hop
    return starts


def groupWindows(starts: list, totalSamples: int, winSamples: int, wb: int) -> list:
    """windowing.js:17-34: groups of up to wb equal-length windows; a short tail alone."""
    groups, cur = [], []
    for i, st in enumerate(starts):
        ln = min(st + winSamples, totalSamples) - st
        if cur and (ln != winSamples or len(cur) >= wb):
            groups.append(cur)
            cur = []
        cur.append(i)
        if ln != winSamples:
            groups.append(cur)
            cur = []
    if cur:
        groups.append(cur)
    return groups


def planRaggedWindows(total_frames: int, min_len: int, max_len: int, overlap: int, seed: int = 1) -> tuple:
    """Cut [0, total_frames) into consecutive windows with lengths drawn
    uniformly from [min_len, max_len] (frames) and `overlap` frames shared
    with the previous window.  Returns (starts, lens) int32 arrays."""
    rng = np.random.default_rng(seed)
    starts, lens = [], []
    s = 0
    while s < total_frames:
        ln = int(rng.integers(min_len, max_len + 1))
        ln = min(ln, total_frames - s)
        starts.append(s)
        lens.append(ln)
        if s + ln >= total_frames:
            break
        s += ln - overlap
    return np.asarray(starts, np.int32), np.asarray(lens, np.int32)


def packBatches(lens, max_batch: int = 32, sort: bool = True) -> list:
    """Group window indices into batches of <= max_batch.  Sorting by length
    keeps similar lengths together (it matters only for the padded layout)."""
    idx = np.argsort(-np.asarray(lens), kind="stable") if sort else np.arange(len(lens))
    return [idx[i:i + max_batch].tolist() for i in range(0, len(idx), max_batch)]
