"""CPU restatements of the reference CPU backend's TTS / decoder-side ops.

TEST INFRASTRUCTURE ONLY (the checker for the HIP kernels of the same ops;
only tests/ import it).

The reference's WasmContext runs these in plain JS (src/gpu/wasm-context.js):
arithmetic in JS doubles, results stored into Float32Arrays.  Each function
below computes in float64 and rounds to float32 at the same points; inputs
are float32 numpy arrays shaped as the tensors ([rows, cols]).
"""
from __future__ import annotations

import numpy as np

F64 = np.float64


def _act(v, act):
    """actf.js:5-22 applyAct on float64 values."""
    if act == "none":
        return v
    if act == "relu":
        return np.maximum(v, 0.0)
    if act == "silu":
        return v / (1.0 + np.exp(-np.clip(v, -30.0, 30.0)))
    if act == "tanh":
        return np.tanh(np.clip(v, -20.0, 20.0))
    if act == "gelu":
        t = np.clip(0.7978845608028654 * (v + 0.044715 * v * v * v), -20.0, 20.0)
        return 0.5 * v * (1.0 + np.tanh(t))
    raise ValueError(act)


def leaky_relu(x, slope=0.2):
    """wasm-context.js:406-413."""
    v = x.astype(F64)
    return np.where(v > 0, v, slope * v).astype(np.float32)


def snake(x, alpha):
    """wasm-context.js:414-427: x + (1 / (a + 1e-9)) sin(a x)^2, a per row."""
    a = alpha.reshape(-1)[: x.shape[0]].astype(F64)[:, None]
    v = x.astype(F64)
    s = np.sin(a * v)
    return (v + (1.0 / (a + 1e-9)) * s * s).astype(np.float32)


def adain(x, scale, shift, eps=1e-5):
    """wasm-context.js:344-362: per-row mean, biased variance, affine per row."""
    v = x.astype(F64)
    m = v.sum(1, keepdims=True) / v.shape[1]
    var = ((v - m) ** 2).sum(1, keepdims=True) / v.shape[1]
    inv = 1.0 / np.sqrt(var + eps)
    sc = scale.reshape(-1)[: x.shape[0]].astype(F64)[:, None]
    sh = shift.reshape(-1)[: x.shape[0]].astype(F64)[:, None]
    return ((v - m) * inv * sc + sh).astype(np.float32)


def im2col(x, k, stride=1, pad=0, dilation=1):
    """wasm-context.js:271-285: [Cin, L] -> [Cin*k, Lout], zeros outside."""
    Cin, L = x.shape
    Lout = (L + 2 * pad - dilation * (k - 1) - 1) // stride + 1
    out = np.zeros((Cin * k, Lout), np.float32)
    for ci in range(Cin):
        for kk in range(k):
            for lo in range(Lout):
                li = lo * stride + kk * dilation - pad
                if 0 <= li < L:
                    out[ci * k + kk, lo] = x[ci, li]
    return out


def conv_transpose1d(x, w, cout, k, bias=None, stride=1, pad=0, dilation=1, groups=1, output_padding=0, act="none"):
    """wasm-context.js:686-741 (the direct form; the GEMM + col2im route for
    groups = 1, dilation = 1 sums the same products): x [Cin, L],
    w flat [Cin][Cout/groups][k]."""
    Cin, L = x.shape
    Lout = (L - 1) * stride - 2 * pad + dilation * (k - 1) + output_padding + 1
    cinG, coutG = Cin // groups, cout // groups
    wv = w.reshape(-1).astype(F64)
    out = np.zeros((cout, Lout), F64)
    for co in range(cout):
        g, coInG = co // coutG, co % coutG
        for lo in range(Lout):
            acc = float(bias.reshape(-1)[co]) if bias is not None else 0.0
            for ci in range(cinG):
                rc = g * cinG + ci
                for kk in range(k):
                    num = lo + pad - kk * dilation
                    if num >= 0 and num % stride == 0 and num // stride < L:
                        acc += float(x[rc, num // stride]) * wv[rc * (coutG * k) + coInG * k + kk]
            out[co, lo] = acc
    return _act(out, act).astype(np.float32)


def gather_cols(x, idx):
    """wasm-context.js:453-460."""
    return x[:, np.asarray(idx, np.int64)].astype(np.float32)


def lstm(x, w, r, b, hid):
    """wasm-context.js:742-776: bidirectional, batch 1, gates i, o, f, c;
    w [2*4H, inp], r [2*4H, H], b [2, 8H] (W bias then R bias); c and h kept
    as float32 between steps.  -> [seq, 2H]."""
    seq, inp = x.shape
    W = w.reshape(2, 4 * hid, inp).astype(F64)
    R = r.reshape(2, 4 * hid, hid).astype(F64)
    B = b.reshape(2, 8 * hid).astype(F64)
    out = np.zeros((seq, 2 * hid), np.float32)
    sig = lambda v: 1.0 / (1.0 + np.exp(-v))
    for d in range(2):
        h = np.zeros(hid, np.float32)
        c = np.zeros(hid, np.float32)
        for s in range(seq):
            t = seq - 1 - s if d else s
            g = B[d, : 4 * hid] + B[d, 4 * hid:] + W[d] @ x[t].astype(F64) + R[d] @ h.astype(F64)
            it, ot, ft, ct = sig(g[:hid]), sig(g[hid:2 * hid]), sig(g[2 * hid:3 * hid]), np.tanh(g[3 * hid:])
            c = (ft * c.astype(F64) + it * ct).astype(np.float32)
            h = (ot * np.tanh(c.astype(F64))).astype(np.float32)
            out[t, d * hid:(d + 1) * hid] = h
    return out


def jbatch(enc, base, B, pred, hid):
    """wasm-context.js:564-572."""
    v = enc.reshape(-1, hid)[base:base + B].astype(F64) + pred.reshape(-1)[:hid].astype(F64)
    return np.maximum(v, 0.0).astype(np.float32)


def _argmax_row(s, vocab):
    """The reference's scan: strict > from (0, -1e30) for tokens [0, vocab)
    and durations [vocab, logits)."""
    bt, bv, bd, bdv = 0, -1e30, 0, -1e30
    for n, v in enumerate(s):
        if n < vocab:
            if v > bv:
                bv, bt = v, n
        elif v > bdv:
            bdv, bd = v, n - vocab
    return [bt, bv, bd, bdv]


def argmax_rows(x, B, vocab, logits):
    """wasm-context.js:573-598 -> [B, 4] float32."""
    xr = x.reshape(-1)[: B * logits].reshape(B, logits).astype(F64)
    return np.array([_argmax_row(xr[i], vocab) for i in range(B)], np.float64).astype(np.float32)


def joint_argmax(enc, frame, count, pred, outW, outB, hidden, vocab, logits):
    """wasm-context.js:599-633: j = relu(enc + pred) (float32), logits summed
    in float64 over hidden units in order, then the row argmax."""
    Wt = outW.reshape(hidden, logits).astype(F64)
    res = []
    for w in range(count):
        j = jbatch(enc, frame + w, 1, pred, hidden)[0].astype(F64)
        s = outB.reshape(-1)[:logits].astype(F64).copy()
        for k in range(hidden):  # sequential, as the reference's inner loop
            s = s + j[k] * Wt[k]
        res.append(_argmax_row(s, vocab))
    return np.array(res, np.float64).astype(np.float32)

