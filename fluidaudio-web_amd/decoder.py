"""Greedy TDT decoding on the GPU (fa_tdt_*), mirroring the reference's batch
decoder API.

    dec = TdtDecoder(ctx, decoderWeights)       # loadGpuDecoder (gpu-decoder.js:220-246)
    out = dec.decodeBatch(frames, lens)         # gpuDecodeBatch (:248-273): [{"ids", "idFrames"}, ...]

`frames` is a device tensor [Σ lens, 640] of pre-projected encoder frames (the
joint's encoder projection applied, src/engines/asr-parakeet/pipeline.js:57-61)
or a list of [T_i, 640] arrays; window i owns lens[i] consecutive rows.  The
arithmetic is rust/parakeet-decoder/src/lib.rs decode_proj's, so the token ids
and frames equal the reference's.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib as L
from ._lib import check, lib

KEYS = ["embed", "l0_W", "l0_R", "l0_B", "l1_W", "l1_R", "l1_B", "predW", "predB", "outW", "outB"]
HID = 640
MAX_OUT_PER_WINDOW = 4096  # gpu-decoder.js:16


class TdtDecoder:
    def __init__(self, ctx, weights: dict):
        self.ctx = ctx
        arrs = [np.ascontiguousarray(weights[k], np.float32).reshape(-1) for k in KEYS]
        ptrs = (C.POINTER(C.c_float) * len(arrs))(*[a.ctypes.data_as(C.POINTER(C.c_float)) for a in arrs])
        p = L.P()
        check(ctx._p, lib().fa_tdt_load(ctx._p, ptrs, C.byref(p)))
        self._h = ctx._own(p, lib().fa_tdt_destroy)

    @property
    def _p(self):
        h = getattr(self, "_h", None)
        return h.p if h is not None else None

    def close(self):
        h = getattr(self, "_h", None)
        if h is not None:
            h.release()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def decodeBatch(self, frames, lens=None, cap: int = MAX_OUT_PER_WINDOW):
        """Per window {"ids": [...], "idFrames": [...]} (gpu-decoder.js:265-272)."""
        up = None
        if isinstance(frames, (list, tuple)):
            lens = [len(f) for f in frames]
            host = np.concatenate([np.ascontiguousarray(f, np.float32).reshape(-1, HID) for f in frames]) if frames else np.zeros((0, HID), np.float32)
            up = self.ctx.upload(host, host.shape[0], HID)
            frames = up
        l = np.ascontiguousarray(lens, np.int32)
        n = len(l)
        ids = np.empty((n, cap), np.int32)
        frs = np.empty((n, cap), np.int32)
        cnt = np.empty(n, np.int32)
        try:
            check(self.ctx._p, lib().fa_tdt_decode(self._p, frames.h, l.ctypes.data_as(L.I32P), n, cap, ids.ctypes.data_as(L.I32P),
                                                   frs.ctypes.data_as(L.I32P), cnt.ctypes.data_as(L.I32P)))
        finally:
            if up is not None:
                self.ctx.freeTensor(up)
        return [{"ids": ids[i, :min(cnt[i], cap)].tolist(), "idFrames": frs[i, :min(cnt[i], cap)].tolist(), "count": int(cnt[i])} for i in range(n)]
