"""Windowed transcription on the GPU: PCM in, stitched token ids out.

Mirrors src/engines/asr-parakeet/pipeline.js transcribeWindowed (:31-143):
windows are planned and grouped as windowing.js does (:5-34), every group is
featurised, encoded, projected and decoded on the GPU, and the per-window
tokens are merged by the reference's seam stitcher (stitcher.js:7-41).

The reference overlaps three stages across CPU and GPU (mel and the WASM
decode on the CPU, the encoder on the GPU).  Here every stage runs on the GPU,
so the host only plans windows and stitches tokens:
  PCM (uploaded once) -> fa_mel_windows (all windows of a group)
    -> fa_encoder_forward_stream (ragged batch read in place from the stream)
    -> matmul(projW, projB) -> fa_tdt_decode (all windows in lock-step)
    -> tokens back to the host -> stitch.
pipelined=True: the whole group loop is one native call,
fa_transcribe_groups, which queues group g+1's mel, encoder and projection on
an encoder lane before group g decodes on the context stream (the tokens equal
the stage-by-stage calls'); its first run at full size (24 layers, one hour)
faulted the GPU with no cause shown, so the default stays stage by stage.  Projected frames never leave the
device.  A group holds up to `wb` windows
(at most 32, the largest encoder batch validated on the GPU; one run with
64-window groups over an hour of audio faulted the GPU and its cause has not
been found): the encoder's GEMMs and the decoder's steps both get cheaper per
window as the batch grows.
"""
from __future__ import annotations

import time

import numpy as np

from .windowing import groupWindows, planWindows

HOP = 160  # mel hop in samples
MAX_WINDOWS = 32  # windows per encoder / decoder batch (largest validated encoder batch)
# The longest input a windowed transcription has run on the GPU.  Every
# transcription of one hour (64- and 32-window groups, stage by stage and
# pipelined) made an illegal memory access on the GPU with no cause shown, so
# longer inputs are refused unless the caller opts in (untested=True).
MAX_TESTED_SECONDS = 470.0


def createStitcher(hop: int, sampleRate: int, overlapSamples: int):
    """stitcher.js:7-41.  Returns (ids, idTimes, stitch); ids / idTimes grow
    across stitch() calls, which must come in window order.  A window's tokens
    that fall in the overlap with the previous window are dropped: the frame
    estimate skips tokens before the overlap's last encoder frame, refined by
    the longest exact match (2 .. frameSkip + 8 tokens) between the running
    transcript's tail and the window's head."""
    ids: list = []
    idTimes: list = []

    def stitch(windowIdx: int, sliceLen: int, Tenc: int, wids, idFrames):
        winStartSec = windowIdx * hop / sampleRate
        skip = 0
        if windowIdx > 0 and len(wids):
            overlapEnc = _js_round(Tenc * overlapSamples / sliceLen)
            frameSkip = 0
            while frameSkip < len(idFrames) and idFrames[frameSkip] < overlapEnc:
                frameSkip += 1
            maxL = min(len(ids), len(wids), frameSkip + 8)
            matched = 0
            for L in range(maxL, 1, -1):
                if all(ids[len(ids) - L + i] == wids[i] for i in range(L)):
                    matched = L
                    break
            skip = max(matched, frameSkip)
        for k in range(skip, len(wids)):
            ids.append(int(wids[k]))
            idTimes.append(winStartSec + idFrames[k] * 0.08)

    return ids, idTimes, stitch


def _js_round(x: float) -> int:
    """Math.round: halves round up (towards +infinity)."""
    return int(np.floor(x + 0.5))


def transcribeWindowed(ctx, enc, dec, projW, projB, samples, sampleRate: int = 16000, windowSec: float = 15, overlapSec: float = 2,
                       wb: int = MAX_WINDOWS, keepFrames: bool = False, pipelined: bool = False, untested: bool = False) -> dict:
    """pipeline.js:31 transcribeWindowed(ctx, enc, dec, mel, projW, projB,
    samples, opts) with the GPU stages: enc a FusedEncoder, dec a TdtDecoder,
    projW / projB device tensors [D, 640] / [1, 640] (the decoder manifest's
    encW / encB).  Returns {"ids", "idTimes", "stats"} like the reference;
    keepFrames=True adds "frames" (each window's projected frames, host copies)
    for checks (stage by stage).  pipelined=True runs the group loop as one
    native call (fa_transcribe_groups) with group g+1's encoder overlapping
    group g's decode.  Inputs longer than MAX_TESTED_SECONDS are refused unless
    untested=True."""
    if not 1 <= wb <= MAX_WINDOWS:
        raise ValueError(f"wb={wb}: 1..{MAX_WINDOWS} windows per group")
    t_start = time.perf_counter()
    x = np.ascontiguousarray(samples, np.float32).reshape(-1)
    total = len(x)
    if not untested and total > MAX_TESTED_SECONDS * sampleRate:
        raise ValueError(f"{total / sampleRate:.1f} s of audio: transcriptions longer than {MAX_TESTED_SECONDS:.0f} s have faulted the GPU "
                         "with no cause shown (untested=True runs them anyway)")
    winSamples = int(round(windowSec * sampleRate))
    overlapSamples = int(round(overlapSec * sampleRate))
    hop = winSamples - overlapSamples
    starts = planWindows(total, winSamples, hop)
    groups = groupWindows(starts, total, winSamples, wb)
    ids, idTimes, stitch = createStitcher(hop, sampleRate, overlapSamples)
    stats = {"windows": 0, "groups": 0, "tokens": 0, "wallMs": 0.0}
    frames_out = [] if keepFrames else None
    if not groups:
        stats["wallMs"] = (time.perf_counter() - t_start) * 1e3
        return {"ids": ids, "idTimes": idTimes, "stats": stats, **({"frames": frames_out} if keepFrames else {})}
    from .encoder import tsub

    pcm = ctx.upload(x.reshape(1, -1), 1, total)
    if pipelined and not keepFrames:
        try:
            _run_pipelined(ctx, enc, dec, projW, projB, pcm, starts, groups, winSamples, total, stitch, stats)
        finally:
            ctx.freeTensor(pcm)
        stats["tokens"] = len(ids)
        stats["wallMs"] = (time.perf_counter() - t_start) * 1e3
        return {"ids": ids, "idTimes": idTimes, "stats": stats}
    try:
        for grp in groups:
            st = [starts[i] for i in grp]
            ln = [min(s + winSamples, total) - s for s in st]
            keep = [j for j, l in enumerate(ln) if l // HOP > 0]  # the mel scheduler drops zero-length mels
            if not keep:
                continue
            st, ln = [st[j] for j in keep], [ln[j] for j in keep]
            T = [l // HOP for l in ln]
            offs = np.concatenate([[0], np.cumsum(T)[:-1]]).astype(np.int32)
            arena = ctx.pushArena()
            try:
                feats = ctx.melWindows(pcm, st, ln)
                y = enc.forwardStream(feats, offs, T)
                proj = ctx.matmul(y, projW, bias=projB)
                ts = [tsub(t) for t in T]
                res = dec.decodeBatch(proj, ts)
                if keepFrames:
                    h = ctx.download(proj).reshape(proj.rows, proj.cols)
                    o = 0
                    for t in ts:
                        frames_out.append(h[o:o + t].copy())
                        o += t
            finally:
                ctx.popArena(arena)
            for j, r in enumerate(res):
                w = grp[keep[j]]
                stitch(w, ln[j], ts[j], r["ids"], r["idFrames"])
            stats["windows"] += len(res)
            stats["groups"] += 1
    finally:
        ctx.freeTensor(pcm)
    stats["tokens"] = len(ids)
    stats["wallMs"] = (time.perf_counter() - t_start) * 1e3
    out = {"ids": ids, "idTimes": idTimes, "stats": stats}
    if keepFrames:
        out["frames"] = frames_out
    return out


def _run_pipelined(ctx, enc, dec, projW, projB, pcm, starts, groups, winSamples, total, stitch, stats):
    """The group loop as one fa_transcribe_groups call, then the seam
    stitcher over the windows in order (zero-length mels are dropped, as the
    reference's mel scheduler drops them)."""
    import ctypes as C

    from . import _lib as L
    from .decoder import MAX_OUT_PER_WINDOW

    win, lns, counts = [], [], []
    for grp in groups:
        kept = [(w, min(starts[w] + winSamples, total) - starts[w]) for w in grp]
        kept = [(w, l) for w, l in kept if l // HOP > 0]
        if kept:
            counts.append(len(kept))
            win += [w for w, _ in kept]
            lns += [l for _, l in kept]
    if not win:
        return
    nw, cap = len(win), MAX_OUT_PER_WINDOW
    st = np.asarray([starts[w] for w in win], np.int32)
    ln = np.asarray(lns, np.int32)
    cn = np.asarray(counts, np.int32)
    ids = np.empty((nw, cap), np.int32)
    frs = np.empty((nw, cap), np.int32)
    nout = np.empty(nw, np.int32)
    ts = np.empty(nw, np.int32)
    I = L.I32P
    L.check(ctx._p, L.lib().fa_transcribe_groups(ctx._p, enc._p, dec._p, pcm.h, len(cn), cn.ctypes.data_as(I), st.ctypes.data_as(I),
                                                 ln.ctypes.data_as(I), projW.h, projB.h if projB is not None else 0, int(enc.cfg["melBins"]), C.c_double(2.0 ** -24),
                                                 1, cap, ids.ctypes.data_as(I), frs.ctypes.data_as(I), nout.ctypes.data_as(I), ts.ctypes.data_as(I)))
    for i, w in enumerate(win):
        k = min(int(nout[i]), cap)
        stitch(w, int(ln[i]), int(ts[i]), ids[i, :k].tolist(), frs[i, :k].tolist())
    stats["windows"] += nw
    stats["groups"] += len(cn)
