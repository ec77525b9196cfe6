"""Streaming FastConformer encode on the GPU: per-chunk continuation with
device-resident K/V and depthwise-conv caches.

Restates src/engines/asr-parakeet/streaming-encoder.js (createEncodeStream,
encodeStreamPush, encodeStreamFlush, disposeEncodeStream, runChunk) on the
HipContext op path.  It computes the same function as the offline
chunked-causal encoder (encoder.parakeetEncodeBatch with a streaming config:
attChunk + convCausal): queries of a chunk see keys [chunkStart - left,
chunkStart + chunk - 1 + right], so carrying exactly those activations from
chunk to chunk reproduces the offline frames.

State per stream: per-layer K/V caches [<= left, D] (what attention reads),
the depthwise conv's input tail [D, dwK - 1], a mel FIFO holding the
subsampling look-back (14 frames), and subT, the absolute count of emitted
frames, which keeps the chunk grid aligned with the offline one.
"""
from __future__ import annotations

import math

import numpy as np

from .encoder import SUB_CONVS

SUB_LOOKBACK = 14  # subsampled frame s reads mel rows [8s - 14, 8s] (three stride-2 k=3 convs, padTop 2)


def streamPosEncoding(dMax: int, dMin: int, D: int) -> np.ndarray:
    """streaming-encoder.js:14-26: sinusoidal rows for relative distances dMax .. dMin."""
    pos = (dMax - np.arange(dMax - dMin + 1, dtype=np.float64))[:, None]
    dv = np.exp(np.arange(0, D, 2, dtype=np.float64) * -(math.log(10000.0) / D))
    pe = np.empty((dMax - dMin + 1, D), np.float32)
    pe[:, 0::2] = np.sin(pos * dv)
    pe[:, 1::2] = np.cos(pos * dv)
    return pe


class EncodeStream:
    pass


def createEncodeStream(ctx, enc, proj=None, lookaheadChunks: int = 0) -> EncodeStream:
    """streaming-encoder.js:33-78.  enc: loadParakeetEncoder(..., cfg=streaming
    config).  proj: optional {"w", "b"} joint projection applied to emitted
    frames.  lookaheadChunks: provisional right-context chunks recomputed each
    pass (needed when attRight > 0)."""
    cfg = enc["cfg"]
    C = cfg.get("attChunk")
    if not C or not cfg.get("convCausal"):
        raise ValueError("createEncodeStream: needs a streaming config (attChunk + convCausal)")
    sp = cfg.get("subPad") or {}
    if sp.get("t") != 2:
        raise ValueError("createEncodeStream: subsampling continuation assumes subPad.t == 2")
    LEFT, RIGHT = cfg.get("attLeft", 70), cfg.get("attRight", 0)
    if RIGHT != 0 and lookaheadChunks < 1:
        raise ValueError("createEncodeStream: attRight > 0 needs lookaheadChunks >= 1")
    D, L, K = cfg["D"], cfg["layers"], cfg["dwK"]
    st = EncodeStream()
    st.enc, st.C, st.LEFT, st.RIGHT = enc, C, LEFT, RIGHT
    st.dMax = LEFT + C - 1
    dMin = -(C - 1 + RIGHT)
    st.subT = 0
    st.fifo = np.zeros((0, cfg["melBins"]), np.float32)  # frame-major
    st.fifoStart = 0
    st.k, st.v, st.cc = [None] * L, [None] * L, [None] * L
    st.pe = ctx.upload(streamPosEncoding(st.dMax, dMin, D), st.dMax - dMin + 1, D)
    st.posP = [ctx.pin(ctx.matmul(st.pe, w["pos"])) for w in enc["layers"]]
    st.zeroCC = ctx.upload(np.zeros((D, K - 1), np.float32), D, K - 1)
    st.proj = proj
    st.B = lookaheadChunks * C if RIGHT > 0 else 0
    st.flushed = st.disposed = False
    return st


def encodeStreamPush(ctx, st: EncodeStream, mel, maxChunk: int = 64):
    """streaming-encoder.js:82-115.  mel: [melBins, count] (mel-major).  Runs as
    many chunk passes as the FIFO allows; returns [nNew, D] new frames or None."""
    if st.flushed:
        raise RuntimeError("encodeStreamPush: stream already flushed; create a new stream")
    mel = np.asarray(mel, np.float32)
    if mel.size:
        st.fifo = np.concatenate([st.fifo, mel.T], 0)
    outs = []
    while True:
        M = st.fifo.shape[0]
        n = (M + 7) // 8 - st.B if st.subT == 0 else (M - 7) // 8 - st.B  # first pass consumes 8 nComp - 7 frames, later ones 8 nComp + 7
        n = min(n, maxChunk)
        n -= n % st.C
        if n < st.C:
            break
        nComp = n + st.B
        m = 8 * nComp - 7 if st.subT == 0 else 8 * nComp + 7
        outs.append(_runChunk(ctx, st, st.fifo[:m], m, n, False, nComp))
        _advanceFifo(st, n)
    return _concat(outs)


def encodeStreamFlush(ctx, st: EncodeStream):
    """streaming-encoder.js:119-140: the final partial chunk with the offline
    bottom pad (signal end).  Call once."""
    if st.flushed:
        raise RuntimeError("encodeStreamFlush: stream already flushed")
    st.flushed = True
    M = st.fifo.shape[0]
    if M == 0 and st.subT == 0:
        return None
    sp = st.enc["cfg"]["subPad"]
    pt = sp["t"] if st.subT == 0 else 0
    T = M
    for _ in range(3):
        T = (T + pt + sp["b"] - 3) // 2 + 1
    if T <= 0:
        return None
    out = _runChunk(ctx, st, st.fifo, M, T, True, T)
    st.fifo = st.fifo[:0]
    return out


def disposeEncodeStream(ctx, st: EncodeStream):
    """streaming-encoder.js:142-149."""
    if st.disposed:
        return
    st.disposed = True
    for t in [*st.posP, *st.k, *st.v, *st.cc]:
        if t is not None:
            ctx.freeTensor(t)
    ctx.freeTensor(st.pe)
    ctx.freeTensor(st.zeroCC)


def _advanceFifo(st, n):
    st.subT += n
    keepFrom = 8 * st.subT - SUB_LOOKBACK  # global mel frame
    st.fifo = st.fifo[keepFrom - st.fifoStart:]
    st.fifoStart = keepFrom


def _concat(outs):
    kept = [o for o in outs if o is not None]
    if not kept:
        return None
    return kept[0] if len(kept) == 1 else np.concatenate(kept, 0)


def _runChunk(ctx, st, melSlice, m, n, isFlush, nComp):
    """streaming-encoder.js:182-297: mel slice (frame-major, m frames) ->
    nComp computed frames, the first n emitted; the provisional tail is
    attention right context only (never cached, recomputed next pass)."""
    enc = st.enc
    cfg = enc["cfg"]
    D, H, HD, K, Csub, mb = cfg["D"], cfg["H"], cfg["HD"], cfg["dwK"], cfg["Csub"], cfg["melBins"]
    sp = cfg["subPad"]
    isFirst = st.subT == 0
    ln = lambda t, lp: ctx.layernorm(t, lp[0], lp[1])  # noqa: E731
    ff = lambda t, lp, w1, w2, b1, b2: ctx.matmul(ctx.matmul(ln(t, lp), w1, bias=b1, act="silu"), w2, bias=b2, add=t)  # noqa: E731
    swaps = []
    arena = ctx.pushArena()
    melUp = None
    try:
        def run():
            nonlocal melUp
            # subsampling with continuation pads: time pads only at the stream's
            # edges (top on the first chunk, bottom at flush), frequency pads always
            s = melUp = ctx.upload(np.ascontiguousarray(melSlice[:m]).reshape(1, -1), 1, m * mb)
            Hh, Wd = m, mb
            for i, (cout, cin, k, stride, gr, act, s2) in enumerate(SUB_CONVS(Csub)):
                pt = sp["t"] if (s2 and isFirst) else 0
                pb = sp["b"] if (s2 and isFlush) else 0
                pl, pr = (sp["l"], sp["r"]) if s2 else (0, 0)
                s = ctx.conv2d(s, enc["sub"]["conv"][i]["w"], cout, cin, Hh, Wd, k, k, bias=enc["sub"]["conv"][i]["b"], strideH=stride,
                               strideW=stride, padTop=pt, padBottom=pb, padLeft=pl, padRight=pr, groups=gr, act=act)
                Hh = (Hh + pt + pb - k) // stride + 1
                Wd = (Wd + pl + pr - k) // stride + 1
            if Hh != nComp:
                raise RuntimeError(f"streaming subsample: expected {nComp} frames, got {Hh}")
            x = ctx.matmul(ctx.subReshape(s, Csub, Hh, Wd), enc["sub"]["linw"], bias=enc["sub"]["linb"])
            for Li, w in enumerate(enc["layers"]):
                x = ff(x, w["lnff1"], w["ff1w1"], w["ff1w2"], w["ff1b1"], w["ff1b2"])
                xln = ln(x, w["lnatt"])
                q = ctx.matmul(xln, w["q"], bias=w["qb"])
                kN = ctx.matmul(xln, w["k"], bias=w["kb"])
                vN = ctx.matmul(xln, w["v"], bias=w["vb"])
                Lc = st.k[Li].rows if st.k[Li] is not None else 0
                Kt = ctx.concatRows([st.k[Li], kN]) if Lc else kN
                Vt = ctx.concatRows([st.v[Li], vN]) if Lc else vN
                Lk = Lc + nComp
                ac = ctx.bmmQK(q, Kt, w["pbuAll"], H, HD, 1)  # [H*nComp, Lk]
                bdRaw = ctx.bmmQK(q, st.posP[Li], w["pbvAll"], H, HD, 1, True)  # [H*nComp, P]
                bd = ctx.relShiftStream(bdRaw, H=H, n=nComp, Lk=Lk, dMax=st.dMax, Lc=Lc, subT=st.subT, C=st.C, left=st.LEFT, right=st.RIGHT)
                probs = ctx.softmax(ctx.add(ac, bd))
                x = ctx.matmul(ctx.bmmPV(probs, Vt, H, HD, 1), w["out"], bias=w["outb"], add=x)
                # cache K/V of emitted frames only: the provisional tail is not final
                keep = min(st.LEFT, Lc + n)
                swaps.append(("k", Li, ctx.pin(ctx.sliceRows(Kt, Lc + n - keep, keep))))
                swaps.append(("v", Li, ctx.pin(ctx.sliceRows(Vt, Lc + n - keep, keep))))
                # conv module: depthwise input = [conv cache | GLU output], causal k,
                # so exactly nComp outputs; the cache is the K - 1 columns before the emit boundary
                pre1 = ctx.matmul(ln(x, w["lnconv"]), w["pw1T"], bias=w["pw1b"])  # [nComp, 2D]
                glu = ctx.glu(ctx.transpose(pre1))  # [D, nComp]
                gfull = ctx.alloc(D, K - 1 + nComp)
                ctx.setCols(gfull, st.cc[Li] if st.cc[Li] is not None else st.zeroCC, 0)
                ctx.setCols(gfull, glu, K - 1)
                swaps.append(("cc", Li, ctx.pin(ctx.sliceCols(gfull, n, K - 1))))
                if w["bn"] is not None:
                    d = ctx.conv1d(gfull, w["dw"], D, K, bias=w["dwb"], padLeft=0, padRight=0, groups=D)
                    dwo = ctx.transpose(ctx.silu(ln(ctx.transpose(d), w["bn"])))
                else:
                    dwo = ctx.conv1d(gfull, w["dw"], D, K, bias=w["dwb"], padLeft=0, padRight=0, groups=D, act="silu")
                x = ctx.matmul(ctx.transpose(dwo), w["pw2T"], bias=w["pw2b"], add=x)
                x = ff(x, w["lnff2"], w["ff2w1"], w["ff2w2"], w["ff2b1"], w["ff2b2"])
                x = ln(x, w["lnout"])
            if nComp != n:
                x = ctx.sliceRows(x, 0, n)  # drop the provisional tail
            if st.proj is not None:
                x = ctx.matmul(x, st.proj["w"], bias=st.proj["b"])
            return ctx.pin(x)

        frames = ctx.withBatchSync(run)
    finally:
        ctx.popArena(arena)
    if melUp is not None:
        ctx.freeTensor(melUp)
    for slot, Li, t in swaps:
        old = getattr(st, slot)[Li]
        if old is not None:
            ctx.freeTensor(old)
        getattr(st, slot)[Li] = t
    data = ctx.download(frames).reshape(frames.rows, frames.cols)
    ctx.freeTensor(frames)
    return data
