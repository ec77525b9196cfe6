"""Parakeet FastConformer encoder on a HipContext.

Two forms with the same result contract:

* ``loadParakeetEncoder`` / ``parakeetEncodeBatch`` restate the reference's
  op-by-op encoder (src/engines/asr-parakeet/raw-encoder.js:39-161, 177-222,
  235-386) against the ComputeContext methods, so the sequence of backend
  calls is the reference's.  With ``weights="f32"`` every matmul runs the
  fp32 MFMA kernels: this is the GPU fp32 path used as the reference for the
  fused f16 encoder at full size.
* ``FusedEncoder`` is the production path: one native call per batch
  (fa_encoder_forward) over packed or padded variable-length windows, with
  f16 / int8 / int4 weight storage.
"""
from __future__ import annotations

import ctypes as C
import math

import numpy as np

from . import _lib as L
from ._lib import check, lib
from .compute import HipContext, HipTensor


def inferConfig(man: dict) -> dict:
    """raw-encoder.js:28-35 on a {name: array} manifest."""
    layers = sum(1 for k in man if k.startswith("L") and k.endswith("_lnff1_w"))
    D, DFF = man["L0_ff1w1"].shape
    H, HD = man["L0_pbu"].shape
    Csub = man["c0w"].shape[0]
    Fsub = man["linw"].shape[0] // Csub
    return dict(D=D, DFF=DFF, H=H, HD=HD, layers=layers, dwK=man["L0_dw"].shape[2], Csub=Csub, Fsub=Fsub, melBins=Fsub * 8)


def _f32(a):
    return np.ascontiguousarray(np.asarray(a, np.float32))


# ── op-by-op restatement ────────────────────────────────────────────────────
def loadParakeetEncoder(ctx: HipContext, man: dict, weights: str = "f16", layers: int | None = None, cfg: dict | None = None) -> dict:
    """Upload weights with the reference's load-time folds (raw-encoder.js:
    124-156): q·1/√HD, pos_bias·1/√HD, FF linear2·0.5; pointwise convs as
    transposed [cin, cout] matrices.  weights: "f16" (uploadF16) or "f32".
    cfg adds the streaming-model fields the manifest does not carry
    (eou-parakeet/config.js: melBins, subPad {t, b, l, r}, convCausal,
    attChunk, attLeft, attRight); layers with bnw / bnb get the conv-module
    LayerNorm (raw-encoder.js:151,361-364)."""
    cfg = dict(inferConfig(man), **(cfg or {}))
    if layers is not None:
        cfg["layers"] = layers
    INV = 1.0 / math.sqrt(cfg["HD"])
    up_mat = ctx.uploadF16 if weights == "f16" else ctx.upload

    def mat(k, s=1.0):
        a = _f32(man[k]).astype(np.float64) * s if s != 1.0 else _f32(man[k])
        a = _f32(a)
        return up_mat(a, a.shape[0], a.shape[1])

    def vec(k, s=1.0):
        a = _f32(_f32(man[k]).astype(np.float64) * s) if s != 1.0 else _f32(man[k])
        return ctx.upload(a.reshape(-1), 1, a.size)

    def vec_opt(k, s=1.0):
        return vec(k, s) if k in man else None

    def pwT(k, cout, cin):
        w = _f32(man[k]).reshape(cout, cin)
        t = np.ascontiguousarray(w.T)
        return up_mat(t, cin, cout)

    D = cfg["D"]
    sub = {"conv": [{"w": vec(f"c{i}w"), "b": vec(f"c{i}b")} for i in range(5)], "linw": mat("linw"), "linb": vec("linb")}
    Ls = []
    for Li in range(cfg["layers"]):
        g = lambda s: f"L{Li}_{s}"
        Ls.append({
            "lnff1": [vec(g("lnff1_w")), vec(g("lnff1_b"))],
            "ff1w1": mat(g("ff1w1")), "ff1w2": mat(g("ff1w2"), 0.5),
            "ff1b1": vec_opt(g("ff1b1")), "ff1b2": vec_opt(g("ff1b2"), 0.5),
            "lnatt": [vec(g("lnatt_w")), vec(g("lnatt_b"))],
            "q": mat(g("q"), INV), "k": mat(g("k")), "v": mat(g("v")), "pos": mat(g("pos")), "out": mat(g("out")),
            "qb": vec_opt(g("qb"), INV), "kb": vec_opt(g("kb")), "vb": vec_opt(g("vb")), "outb": vec_opt(g("outb")),
            "pbuAll": vec(g("pbu"), INV), "pbvAll": vec(g("pbv"), INV),
            "lnconv": [vec(g("lnconv_w")), vec(g("lnconv_b"))],
            "pw1T": pwT(g("pw1"), 2 * D, D), "dw": vec(g("dw")), "dwb": vec(g("dwb")), "pw2T": pwT(g("pw2"), D, D),
            "pw1b": vec_opt(g("pw1b")), "pw2b": vec_opt(g("pw2b")),
            "lnff2": [vec(g("lnff2_w")), vec(g("lnff2_b"))],
            "ff2w1": mat(g("ff2w1")), "ff2w2": mat(g("ff2w2"), 0.5),
            "ff2b1": vec_opt(g("ff2b1")), "ff2b2": vec_opt(g("ff2b2"), 0.5),
            "lnout": [vec(g("lnout_w")), vec(g("lnout_b"))],
            "bn": [vec(g("bnw")), vec(g("bnb"))] if g("bnw") in man else None,
        })
    return {"sub": sub, "layers": Ls, "cfg": cfg}


def posEncoding(Tsub: int, D: int) -> np.ndarray:
    """raw-encoder.js:163-174."""
    pos = (Tsub - 1 - np.arange(2 * Tsub - 1, dtype=np.float64))[:, None]
    dv = np.exp(np.arange(0, D, 2, dtype=np.float64) * -(math.log(10000.0) / D))
    pe = np.empty((2 * Tsub - 1, D), np.float32)
    pe[:, 0::2] = np.sin(pos * dv)
    pe[:, 1::2] = np.cos(pos * dv)
    return pe


def SUB_CONVS(Csub):
    """The dw-striding stack (raw-encoder.js:187-193): (cout, cin, k, stride, groups, act, stride-2)."""
    return [(Csub, 1, 3, 2, 1, "relu", True), (Csub, Csub, 3, 2, Csub, "none", True), (Csub, Csub, 1, 1, 1, "relu", False),
            (Csub, Csub, 3, 2, Csub, "none", True), (Csub, Csub, 1, 1, 1, "relu", False)]


def chunkMask(cfg: dict, T: int) -> np.ndarray:
    """raw-encoder.js:256-276: 0 where query i may see key j (j in
    [cs - left, cs + C - 1 + right], cs = C*floor(i/C)), -10000 elsewhere."""
    Cc, left, right = cfg["attChunk"], cfg.get("attLeft", 70), cfg.get("attRight", 0)
    i = np.arange(T)[:, None]
    j = np.arange(T)[None, :]
    cs = Cc * (i // Cc)
    lo, hi = np.maximum(0, cs - left), np.minimum(T - 1, cs + Cc - 1 + right)
    return np.where((j >= lo) & (j <= hi), 0.0, -10000.0).astype(np.float32)


def _pre_encode(ctx, enc, mel):
    """raw-encoder.js:177-222 for one window; mel [melBins, T] channel-major."""
    cfg = enc["cfg"]
    Csub, mb = cfg["Csub"], cfg["melBins"]
    T = mel.shape[1]
    s = ctx.upload(np.ascontiguousarray(_f32(mel).T), 1, T * mb)
    Hh, Wd = T, mb
    sp = cfg.get("subPad") or {"t": 1, "b": 1, "l": 1, "r": 1}
    for i, (cout, cin, k, st, gr, act, s2) in enumerate(SUB_CONVS(Csub)):
        pt, pb, pl, pr = (sp["t"], sp["b"], sp["l"], sp["r"]) if s2 else (0, 0, 0, 0)
        s = ctx.conv2d(s, enc["sub"]["conv"][i]["w"], cout, cin, Hh, Wd, k, k, bias=enc["sub"]["conv"][i]["b"], strideH=st, strideW=st,
                       padTop=pt, padBottom=pb, padLeft=pl, padRight=pr, groups=gr, act=act)
        Hh = (Hh + pt + pb - k) // st + 1
        Wd = (Wd + pl + pr - k) // st + 1
    flat = ctx.subReshape(s, Csub, Hh, Wd)
    return ctx.matmul(flat, enc["sub"]["linw"], bias=enc["sub"]["linb"]), Hh


def parakeetEncodeBatch(ctx: HipContext, enc: dict, mels: list, attnFused: bool = False) -> tuple:
    """raw-encoder.js:235-386, including the streaming models' options
    (chunk-limited attention mask, causal depthwise conv, conv-module
    LayerNorm).  Returns (frames [W*Tsub, D] tensor, Tsub).  As in the
    reference, the positional projection of a batched (W > 1) Tsub is cached
    per layer (raw-encoder.js:304-321), and attnFused=True (the reference's
    opt-in globalThis.__attnFused, raw-encoder.js:334) sends unmasked
    attention through the context's attnFused member instead of the
    bmmQK / relShiftB / softmax / bmmPV chain."""
    cfg = enc["cfg"]
    D, H, HD, K = cfg["D"], cfg["H"], cfg["HD"], cfg["dwK"]
    W = len(mels)
    pre = [_pre_encode(ctx, enc, m) for m in mels]
    Tsub = pre[0][1]
    if any(p[1] != Tsub for p in pre):
        raise ValueError("parakeetEncodeBatch: windows must have equal Tsub")
    x = pre[0][0] if W == 1 else ctx.concatRows([p[0] for p in pre])
    peT = ctx.upload(posEncoding(Tsub, D), 2 * Tsub - 1, D)
    ln = lambda t, lp: ctx.layernorm(t, lp[0], lp[1])
    ff = lambda t, lp, w1, w2, b1, b2: ctx.matmul(ctx.matmul(ln(t, lp), w1, bias=b1, act="silu"), w2, bias=b2, add=t)
    padL, padR = (K - 1, 0) if cfg.get("convCausal") else ((K - 1) >> 1, (K - 1) >> 1)
    maskT = None
    if cfg.get("attChunk"):
        m = np.tile(chunkMask(cfg, Tsub), (W * H, 1))
        maskT = ctx.upload(m, W * H * Tsub, Tsub)

    def run():
        nonlocal x
        for w in enc["layers"]:
            arena = ctx.pushArena()
            x = ff(x, w["lnff1"], w["ff1w1"], w["ff1w2"], w["ff1b1"], w["ff1b2"])
            xln = ln(x, w["lnatt"])
            q = ctx.matmul(xln, w["q"], bias=w["qb"])
            k = ctx.matmul(xln, w["k"], bias=w["kb"])
            v = ctx.matmul(xln, w["v"], bias=w["vb"])
            if W > 1:
                cache = enc.setdefault("_posProj", {})
                key = (id(w), Tsub)
                p = cache.get(key)
                if p is None:
                    p = ctx.matmul(peT, w["pos"])
                    ctx.pin(p)  # cached across groups: exempt from the arena
                    cache[key] = p
            else:
                p = ctx.matmul(peT, w["pos"])
            outc = None
            if maskT is None and attnFused and hasattr(ctx, "attnFused"):
                outc = ctx.attnFused(q, k, v, p, w["pbuAll"], w["pbvAll"], H, HD, W)
            if outc is None:
                ac = ctx.bmmQK(q, k, w["pbuAll"], H, HD, W)
                bd = ctx.relShiftB(ctx.bmmQK(q, p, w["pbvAll"], H, HD, W, True), W * H)
                sc = ctx.add(ac, bd)
                if maskT is not None:
                    sc = ctx.add(sc, maskT)
                probs = ctx.softmax(sc)
                outc = ctx.bmmPV(probs, v, H, HD, W)
            x = ctx.matmul(outc, w["out"], bias=w["outb"], add=x)
            pre1 = ctx.matmul(ln(x, w["lnconv"]), w["pw1T"], bias=w["pw1b"])
            glu = ctx.glu(ctx.transpose(pre1))
            act = "none" if w["bn"] is not None else "silu"
            if W == 1:
                dwo = ctx.conv1d(glu, w["dw"], D, K, groups=D, padLeft=padL, padRight=padR, bias=w["dwb"], act=act)
            else:
                dwo = ctx.alloc(D, W * Tsub)
                for wi in range(W):
                    ctx.setCols(dwo, ctx.conv1d(ctx.sliceCols(glu, wi * Tsub, Tsub), w["dw"], D, K, groups=D, padLeft=padL, padRight=padR,
                                                bias=w["dwb"], act=act), wi * Tsub)
            if w["bn"] is not None:  # EOU: depthwise -> LayerNorm over channels -> SiLU
                dwo = ctx.transpose(ctx.silu(ln(ctx.transpose(dwo), w["bn"])))
            x = ctx.matmul(ctx.transpose(dwo), w["pw2T"], bias=w["pw2b"], add=x)
            x = ff(x, w["lnff2"], w["ff2w1"], w["ff2w2"], w["ff2b1"], w["ff2b2"])
            x = ln(x, w["lnout"])
            ctx.pin(x, True)
            ctx.popArena(arena)
        return x

    out = ctx.withBatchSync(run)
    return out, Tsub


# ── fused production path ───────────────────────────────────────────────────
FORMATS = {"f16": L.W_F16, "int8": L.W_INT8, "int4": L.W_INT4}


def tsub(T: int) -> int:
    """Subsampled length of T mel frames (raw-encoder.js:217-218)."""
    return int(lib().fa_encoder_tsub(int(T)))


class FusedEncoder:
    """Native whole-encoder forward (fa_encoder_load / fa_encoder_forward)."""

    def __init__(self, ctx: HipContext, man: dict, fmt: str = "f16", max_T: int = 512, layers: int | None = None, cfg: dict | None = None):
        """cfg: the streaming models' fields the manifest does not carry
        (melBins, subPad {t, b, l, r}, convCausal, attChunk, attLeft,
        attRight; eou-parakeet/config.js), as loadParakeetEncoder takes them."""
        cfg = dict(inferConfig(man), **(cfg or {}))
        if layers is not None:
            cfg["layers"] = min(layers, cfg["layers"])
        self.ctx, self.cfg, self.fmt, self.max_T = ctx, cfg, fmt, max_T
        keep = {k: _f32(v).reshape(-1) for k, v in man.items()
                if not (k.startswith("L") and int(k[1:k.index("_")]) >= cfg["layers"])}
        names = list(keep)
        arr_names = (C.c_char_p * len(names))(*[n.encode() for n in names])
        arr_data = (L.F32P * len(names))(*[keep[n].ctypes.data_as(L.F32P) for n in names])
        arr_cnt = (C.c_int64 * len(names))(*[keep[n].size for n in names])
        c = L.EncoderCfg(*(cfg[k] for k in ("D", "DFF", "H", "HD", "layers", "dwK", "Csub", "Fsub", "melBins")))
        sp = cfg.get("subPad") or {"t": 1, "b": 1, "l": 1, "r": 1}
        o = L.EncoderOpts(sp["t"], sp["b"], sp["l"], sp["r"], int(bool(cfg.get("convCausal"))), int(cfg.get("attChunk") or 0),
                          int(cfg.get("attLeft", 70)) if cfg.get("attChunk") else 0, int(cfg.get("attRight", 0)) if cfg.get("attChunk") else 0)
        p = L.P()
        check(ctx._p, lib().fa_encoder_load_opts(ctx._p, C.byref(c), C.byref(o), len(names), arr_names, arr_data, arr_cnt, FORMATS[fmt], max_T,
                                                 C.byref(p)))
        self._h = ctx._own(p, lib().fa_encoder_destroy)

    # operand-precision bits (fa_encoder_set_exact)
    EXACT = dict(ln_out=1, ff_hidden=2, attn_out=4, glu=8, dw_out=16)

    def setExact(self, mask: int, first: int = 0, last: int | None = None):
        """Carry the masked operands of layers [first, last] as exact f16 pairs
        (0 = plain f16 operands everywhere)."""
        last = self.cfg["layers"] - 1 if last is None else last
        check(self.ctx._p, lib().fa_encoder_set_exact(self._p, first, last, int(mask)))

    def exact(self, layer: int) -> int:
        return int(lib().fa_encoder_get_exact(self._p, layer))

    def tsub(self, T: int) -> int:
        """Encoder frames of a window of T mel frames (this model's subsampling pads)."""
        return int(lib().fa_encoder_tsub_of(self._p, int(T)))

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

    def forward(self, mel: HipTensor, lens, layout: str = "packed", layers: int = -1) -> HipTensor:
        """mel: packed/padded time-major [rows, melBins] tensor (packWindows);
        returns [Σ Tsub, D] (packed) or [n*TsubMax, D] (padded) frames."""
        l = np.ascontiguousarray(lens, np.int32)
        o = L.T()
        check(self.ctx._p, lib().fa_encoder_forward(self.ctx._p, self._p, mel.h, l.ctypes.data_as(L.I32P), len(l),
                                                    0 if layout == "packed" else 1, layers, C.byref(o)))
        return self.ctx._t(o.value)

    def forwardStream(self, feats: HipTensor, starts, lens, layout: str = "packed", layers: int = -1) -> HipTensor:
        """Windows [starts[i], starts[i]+lens[i]) of the channel-major feature
        stream feats [melBins, T] (melWindows' output), encoded without a
        packed copy (fa_encoder_forward_stream); frames as forward() returns
        them for packWindows(feats, starts, lens, layout)."""
        s = np.ascontiguousarray(starts, np.int32)
        l = np.ascontiguousarray(lens, np.int32)
        if len(s) != len(l):
            raise ValueError("forwardStream: %d starts for %d windows" % (len(s), len(l)))
        o = L.T()
        check(self.ctx._p, lib().fa_encoder_forward_stream(self.ctx._p, self._p, feats.h, s.ctypes.data_as(L.I32P), l.ctypes.data_as(L.I32P),
                                                           len(l), 0 if layout == "packed" else 1, layers, C.byref(o)))
        return self.ctx._t(o.value)

    def forwardStreamBatches(self, feats: HipTensor, batches, layout: str = "packed", layers: int = -1) -> list:
        """Several batches [(starts, lens), ...] of one feature stream; outputs
        equal forwardStream of each batch, bit for bit.  Consecutive batches
        run on two workspace lanes with streams of their own, so they overlap
        on the GPU (fa_encoder_forward_stream_batches); the windowed
        transcription's loop over groups (pipeline.js:66-80) in one call."""
        if not batches:
            return []
        st = [np.ascontiguousarray(b[0], np.int32) for b in batches]
        ln = [np.ascontiguousarray(b[1], np.int32) for b in batches]
        for s_, l_ in zip(st, ln):
            if len(s_) != len(l_) or len(l_) == 0:
                raise ValueError("forwardStreamBatches: %d starts for %d windows" % (len(s_), len(l_)))
        s = np.ascontiguousarray(np.concatenate(st), np.int32)
        l = np.ascontiguousarray(np.concatenate(ln), np.int32)
        cnt = np.array([len(x) for x in ln], np.int32)
        outs = (L.T * len(batches))()
        check(self.ctx._p, lib().fa_encoder_forward_stream_batches(self.ctx._p, self._p, feats.h, len(batches), s.ctypes.data_as(L.I32P),
                                                                   l.ctypes.data_as(L.I32P), cnt.ctypes.data_as(L.I32P),
                                                                   0 if layout == "packed" else 1, layers, outs))
        return [self.ctx._t(o) for o in outs]

    def encode(self, mels: list, layout: str = "packed", layers: int = -1) -> np.ndarray:
        """Convenience: list of [melBins, T_i] windows -> list of [Tsub_i, D] arrays."""
        lens = [m.shape[1] for m in mels]
        stream = np.concatenate([_f32(m) for m in mels], axis=1)
        starts = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int32)
        feats = self.ctx.upload(stream, stream.shape[0], stream.shape[1])
        arena = self.ctx.pushArena()
        try:
            y = self.forwardStream(feats, starts, lens, layout, layers)
            out = self.ctx.download(y).reshape(y.rows, y.cols)
        finally:
            self.ctx.popArena(arena)
            self.ctx.freeTensor(feats)
        ts = [self.tsub(t) for t in lens]
        res, off = [], 0
        tmax = max(ts)
        for i, t in enumerate(ts):
            base = off if layout == "packed" else i * tmax
            res.append(out[base:base + t].copy())
            off += t
        return res
