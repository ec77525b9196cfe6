"""Independent float64 restatement of the Parakeet FastConformer encoder, written
the way NeMo's modules compute it (unfolded scalings, pad->reshape->slice
rel_shift, library conv/layernorm/softmax), to cross-check the C oracle.

TEST INFRASTRUCTURE ONLY (used by tests/ and tests/golden/make_golden.py).

It shares no code with fa_oracle.c: the C oracle restates the reference's
WASM-backend op sequence (src/engines/asr-parakeet/raw-encoder.js with the
src/gpu/wasm-context.js ops, weights pre-folded); this module restates the
architecture from its textbook definition:
  - dw-striding subsampling: three 3x3 stride-2 convs (pad 1) with 1x1 convs
    between the depthwise ones, ReLU after c0/c2/c4, flatten (C, F) per time
    step, linear  (raw-encoder.js:187-221);
  - RelPositionalEncoding over positions T-1 .. -(T-1)  (raw-encoder.js:163-174);
  - rel-pos MHSA: scores = ((q+u)kᵀ + rel_shift((q+v)pᵀ)) / sqrt(d_k), with
    rel_shift = NeMo's left-pad, reshape, drop-first-row, reshape, crop;
  - conv module: pw1 -> GLU -> depthwise k -> (BN folded) -> SiLU -> pw2;
  - macaron FF with the 0.5 residual factor.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

f64 = torch.float64


def _t(a):
    return torch.as_tensor(np.asarray(a, dtype=np.float64))


def rel_shift_nemo(x: torch.Tensor) -> torch.Tensor:
    """NeMo RelPositionMultiHeadAttention.rel_shift for x [..., t, 2t-1]:
    pad one zero column on the left, view as [..., 2t, t] ... then keep the
    first t columns of the shifted view."""
    *lead, t, p = x.shape
    x = F.pad(x, (1, 0))  # [..., t, 2t]
    x = x.reshape(*lead, p + 1, t)  # [..., 2t, t]
    x = x[..., 1:, :].reshape(*lead, t, p)  # drop first row
    return x[..., :t]


def pos_encoding(T: int, D: int) -> torch.Tensor:
    pos = torch.arange(T - 1, -T, -1, dtype=f64).unsqueeze(1)
    div = torch.exp(torch.arange(0, D, 2, dtype=f64) * -(math.log(10000.0) / D))
    pe = torch.zeros(2 * T - 1, D, dtype=f64)
    pe[:, 0::2] = torch.sin(pos * div)
    pe[:, 1::2] = torch.cos(pos * div)
    return pe


def subsample(cfg, man, mel):
    """mel [melBins, T] -> [Tsub, D].  cfg["subPad"] {t, b, l, r} pads the three
    stride-2 convs asymmetrically (streaming models); default 1 on every side."""
    C = cfg["Csub"]
    sp = cfg.get("subPad") or {"t": 1, "b": 1, "l": 1, "r": 1}
    pad = lambda x: F.pad(x, (sp["l"], sp["r"], sp["t"], sp["b"]))  # noqa: E731
    x = _t(mel).T.unsqueeze(0).unsqueeze(0)  # [1, 1, T, melBins] (time = H, freq = W)
    x = F.relu(F.conv2d(pad(x), _t(man["c0w"]).reshape(C, 1, 3, 3), _t(man["c0b"]), stride=2))
    x = F.conv2d(pad(x), _t(man["c1w"]).reshape(C, 1, 3, 3), _t(man["c1b"]), stride=2, groups=C)
    x = F.relu(F.conv2d(x, _t(man["c2w"]).reshape(C, C, 1, 1), _t(man["c2b"])))
    x = F.conv2d(pad(x), _t(man["c3w"]).reshape(C, 1, 3, 3), _t(man["c3b"]), stride=2, groups=C)
    x = F.relu(F.conv2d(x, _t(man["c4w"]).reshape(C, C, 1, 1), _t(man["c4b"])))
    b, c, t, f = x.shape
    x = x.transpose(1, 2).reshape(t, c * f)
    return x @ _t(man["linw"]) + _t(man["linb"])


def _lin(x, man, w, b=None):
    y = x @ _t(man[w])
    return y + _t(man[b]) if b is not None and man.get(b) is not None else y


def _ln(x, man, pfx):
    return F.layer_norm(x, (x.shape[-1],), _t(man[pfx + "_w"]), _t(man[pfx + "_b"]), eps=1e-5)


def layer(cfg, man, L, x, W, T):
    D, H, HD, K = cfg["D"], cfg["H"], cfg["HD"], cfg["dwK"]
    g = lambda s: f"L{L}_{s}"
    # FF1 (macaron, 0.5 residual)
    h = _ln(x, man, g("lnff1"))
    h = F.silu(_lin(h, man, g("ff1w1"), g("ff1b1")))
    x = x + 0.5 * _lin(h, man, g("ff1w2"), g("ff1b2"))
    # rel-pos MHSA
    h = _ln(x, man, g("lnatt"))
    q = _lin(h, man, g("q"), g("qb")).reshape(W, T, H, HD).transpose(1, 2)  # [W,H,T,HD]
    k = _lin(h, man, g("k"), g("kb")).reshape(W, T, H, HD).transpose(1, 2)
    v = _lin(h, man, g("v"), g("vb")).reshape(W, T, H, HD).transpose(1, 2)
    p = (pos_encoding(T, D) @ _t(man[g("pos")])).reshape(2 * T - 1, H, HD).transpose(0, 1)  # [H,2T-1,HD]
    u = _t(man[g("pbu")]).reshape(1, H, 1, HD)
    vb = _t(man[g("pbv")]).reshape(1, H, 1, HD)
    ac = (q + u) @ k.transpose(-1, -2)
    bd = rel_shift_nemo((q + vb) @ p.unsqueeze(0).transpose(-1, -2))
    sc = (ac + bd) / math.sqrt(HD)
    if cfg.get("attChunk"):  # chunk-limited attention: query i sees keys [cs - left, cs + C - 1 + right]
        Cc, left, right = cfg["attChunk"], cfg.get("attLeft", 70), cfg.get("attRight", 0)
        i = torch.arange(T).unsqueeze(1)
        j = torch.arange(T).unsqueeze(0)
        cs = Cc * torch.div(i, Cc, rounding_mode="floor")
        sc = sc + torch.where((j >= cs - left) & (j <= cs + Cc - 1 + right), 0.0, -10000.0).to(sc.dtype)
    att = torch.softmax(sc, dim=-1)
    o = (att @ v).transpose(1, 2).reshape(W * T, D)
    x = x + _lin(o, man, g("out"), g("outb"))
    # conv module
    h = _ln(x, man, g("lnconv"))
    pw1 = _t(man[g("pw1")]).reshape(2 * D, D)
    h = h @ pw1.T
    if man.get(g("pw1b")) is not None:
        h = h + _t(man[g("pw1b")])
    h = F.glu(h, dim=-1)  # [W*T, D]
    h = h.reshape(W, T, D).transpose(1, 2)  # [W, D, T]
    h = F.pad(h, (K - 1, 0) if cfg.get("convCausal") else ((K - 1) // 2, (K - 1) // 2))
    h = F.conv1d(h, _t(man[g("dw")]).reshape(D, 1, K), _t(man[g("dwb")]), groups=D)
    if man.get(g("bnw")) is not None:  # streaming conv module: LayerNorm over channels before SiLU
        h = F.layer_norm(h.transpose(1, 2), (D,), _t(man[g("bnw")]), _t(man[g("bnb")]), eps=1e-5).transpose(1, 2)
    h = F.silu(h).transpose(1, 2).reshape(W * T, D)
    h = h @ _t(man[g("pw2")]).reshape(D, D).T
    if man.get(g("pw2b")) is not None:
        h = h + _t(man[g("pw2b")])
    x = x + h
    # FF2 + norm_out
    h = _ln(x, man, g("lnff2"))
    h = F.silu(_lin(h, man, g("ff2w1"), g("ff2b1")))
    x = x + 0.5 * _lin(h, man, g("ff2w2"), g("ff2b2"))
    return _ln(x, man, g("lnout"))


def encode(cfg, man, mels, layers=None):
    """mels: list of [melBins, T] windows of one length -> np.float64 [W*Tsub, D]."""
    layers = cfg["layers"] if layers is None else layers
    with torch.no_grad():
        xs = [subsample(cfg, man, m) for m in mels]
        T = xs[0].shape[0]
        x = torch.cat(xs, 0)
        for L in range(layers):
            x = layer(cfg, man, L, x, len(mels), T)
    return x.numpy()
