"""Streaming encode: the reference's stream API (src/engines/asr-parakeet/
streaming-encoder.js: createEncodeStream, encodeStreamPush, encodeStreamFlush,
disposeEncodeStream) over the native stream (fa_stream_*, csrc/stream.hip).

The stream runs chunk passes of the fused encoder on the GPU with the K / V
and depthwise-conv caches kept on the device; frames equal the offline
chunked-causal encoder's (FusedEncoder.encode on the same model).  The
encoder must be a FusedEncoder loaded with a streaming config (attChunk,
convCausal, subPad t = 2).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib as L
from ._lib import check, lib


class EncodeStream:
    """Handle of one native stream (fa_stream)."""

    def __init__(self, ctx, enc, lookaheadChunks: int, maxChunk: int, proj):
        self.ctx, self.enc, self.proj = ctx, enc, proj
        p = L.P()
        check(ctx._p, lib().fa_stream_create(ctx._p, enc._p, int(lookaheadChunks), int(maxChunk), C.byref(p)))
        self._h = ctx._own(p, lib().fa_stream_destroy)

    def _frames(self, h: int):
        if not h:
            return None
        t = self.ctx._t(h)
        if self.proj is not None:  # the joint projection rides the stream (streaming-encoder.js:69-71)
            y = self.ctx.matmul(t, self.proj["w"], bias=self.proj.get("b"))
            self.ctx.freeTensor(t)
            t = y
        out = self.ctx.download(t).reshape(t.rows, t.cols)
        self.ctx.freeTensor(t)
        return out

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


def createEncodeStream(ctx, enc, proj=None, lookaheadChunks: int = 0, maxChunk: int = 64) -> EncodeStream:
    """enc: FusedEncoder with a streaming config; proj: optional {"w", "b"}
    device tensors applied to emitted frames; lookaheadChunks: provisional
    right-context chunks (needed when attRight > 0)."""
    return EncodeStream(ctx, enc, lookaheadChunks, maxChunk, proj)


def encodeStreamPush(ctx, st: EncodeStream, mel):
    """mel: [melBins, count] (mel-major).  Returns [nNew, D] new frames or None."""
    m = np.ascontiguousarray(mel, np.float32)
    o = L.T()
    check(ctx._p, lib().fa_stream_push(st._p, m.ctypes.data_as(L.F32P), int(m.shape[1]) if m.ndim == 2 else 0, C.byref(o)))
    return st._frames(o.value)


def encodeStreamsPush(ctx, streams: list, mels: list) -> list:
    """encodeStreamPush for several distinct streams at once (fa_stream_push_many):
    each stream's chunk passes run on a HIP stream of its own, so the streams'
    passes are in flight together.  Returns each stream's new frames (or None)."""
    if len(streams) != len(mels):
        raise ValueError("encodeStreamsPush: %d streams, %d mel blocks" % (len(streams), len(mels)))
    n = len(streams)
    if n == 0:
        return []
    ms = [np.ascontiguousarray(m, np.float32) for m in mels]
    hs = (L.P * n)(*[s._p for s in streams])
    ps = (L.F32P * n)(*[m.ctypes.data_as(L.F32P) for m in ms])
    cn = (C.c_int * n)(*[int(m.shape[1]) if m.ndim == 2 else 0 for m in ms])
    outs = (L.T * n)()
    check(ctx._p, lib().fa_stream_push_many(n, hs, ps, cn, outs))
    return [s._frames(o) for s, o in zip(streams, outs)]


def encodeStreamFlush(ctx, st: EncodeStream):
    """Encode the final partial chunk (bottom-padded); the stream accepts no
    push afterwards."""
    o = L.T()
    check(ctx._p, lib().fa_stream_flush(st._p, C.byref(o)))
    return st._frames(o.value)


def disposeEncodeStream(ctx, st: EncodeStream) -> None:
    st.close()
