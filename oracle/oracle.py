"""ctypes binding to the CPU oracle (liboracle.so, built from oracle/fa_oracle.c).

TEST INFRASTRUCTURE ONLY: the parity checker and the reported CPU baseline.
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module; the product library never does.

Each wrapper calls one C restatement of a reference routine; the C file cites
the reference file:line for each.  Arrays are numpy, C-contiguous.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

ACT = {"none": 0, "gelu": 1, "tanh": 2, "relu": 3, "silu": 4, "gelu_erf": 5}

# Flat weight-table order; must match the enum in fa_oracle.c.
GLOBAL_KEYS = ["c0w", "c0b", "c1w", "c1b", "c2w", "c2b", "c3w", "c3b", "c4w", "c4b", "linw", "linb"]
LAYER_KEYS = [
    "lnff1_w", "lnff1_b", "ff1w1", "ff1w2", "ff1b1", "ff1b2", "lnatt_w", "lnatt_b", "q", "k", "v", "pos", "out",
    "qb", "kb", "vb", "outb", "pbu", "pbv", "lnconv_w", "lnconv_b", "pw1", "pw1b", "dw", "dwb", "pw2", "pw2b",
    "lnff2_w", "lnff2_b", "ff2w1", "ff2w2", "ff2b1", "ff2b2", "lnout_w", "lnout_b",
]


class OrCfg(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("D", "DFF", "H", "HD", "layers", "dwK", "Csub", "Fsub", "melBins")]


def build() -> None:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(L):
    f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
    i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
    u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
    u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
    i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
    vp = C.c_void_p
    I = C.c_int
    L.or_set_threads.argtypes = [I]
    L.or_matmul_f32.argtypes = [f32p, f32p, f32p, I, I, I]
    L.or_matmul.argtypes = [f32p, f32p, f32p, I, I, I, vp, I, vp]
    L.or_matmul_int8.argtypes = [f32p, i8p, f32p, f32p, I, I, I, vp, I]
    L.or_matmul_nbits.argtypes = [f32p, u8p, f32p, u8p, f32p, I, I, I, I, I, I]
    L.or_layernorm.argtypes = [f32p, f32p, f32p, f32p, I, I, C.c_double]
    L.or_softmax.argtypes = [f32p, f32p, I, I]
    L.or_glu.argtypes = [f32p, f32p, I, I]
    L.or_silu.argtypes = [f32p, f32p, C.c_size_t]
    L.or_transpose.argtypes = [f32p, f32p, I, I]
    L.or_conv2d.argtypes = [f32p, f32p, vp, f32p] + [I] * 14
    L.or_conv1d_grouped.argtypes = [f32p, f32p, vp, f32p] + [I] * 10
    L.or_subreshape.argtypes = [f32p, f32p, I, I, I]
    L.or_bmm_qk.argtypes = [f32p, I, f32p, I, vp, f32p, I, I, I, I]
    L.or_bmm_pv.argtypes = [f32p, I, f32p, I, f32p, I, I, I]
    L.or_relshift_b.argtypes = [f32p, f32p, I, I]
    L.or_relshift_stream.argtypes = [f32p, f32p] + [I] * 10
    L.or_pos_encoding.argtypes = [I, I, f32p]
    L.or_quantize_int8_cols.argtypes = [f32p, I, I, i8p, f32p]
    L.or_dequant_int8_cols.argtypes = [i8p, f32p, I, I, f32p]
    L.or_quantize_int4_g32.argtypes = [f32p, I, I, u8p, u16p, vp, vp]
    L.or_dequant_int4_g32.argtypes = [u8p, u16p, I, I, f32p]
    L.or_pre_encode.argtypes = [C.POINTER(OrCfg), f32p, i64p, f32p, I, f32p]
    L.or_pre_encode.restype = I
    L.or_encode_batch.argtypes = [C.POINTER(OrCfg), f32p, i64p, f32p, I, I, I, f32p]
    L.or_encode_batch.restype = I
    L.or_tsub.argtypes = [I]
    L.or_tsub.restype = I
    L.or_f32_to_f16.argtypes = [C.c_float]
    L.or_f32_to_f16.restype = C.c_uint16

    f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
    L.or_mel_filterbank.argtypes = [C.c_int, f32p]
    L.or_mel_hann.argtypes = [f64p]
    L.or_mel_twiddles.argtypes = [C.c_int, f64p, f64p]
    L.or_mel_power.argtypes = [f64p, f32p]
    L.or_mel.argtypes = [f32p, C.c_long, C.c_int, C.c_double, C.c_int, f32p]
    L.or_mel.restype = C.c_int
    i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
    L.or_tdt_expf.argtypes = [C.c_float]
    L.or_tdt_expf.restype = C.c_float
    L.or_tdt_decode_proj.argtypes = [f32p] * 12 + [C.c_int, i32p, i32p, C.c_int]
    L.or_tdt_decode_proj.restype = C.c_int
    L.or_tdt_lstm.argtypes = [f32p] * 8
    L.or_tdt_joint.argtypes = [f32p] * 5


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def set_threads(n: int) -> None:
    lib().or_set_threads(int(n))


def matmul_f32(a, b):
    a, b = _f32(a), _f32(b)
    M, K = a.shape
    N = b.shape[1]
    c = np.empty((M, N), np.float32)
    lib().or_matmul_f32(a, b, c, M, K, N)
    return c


def matmul(a, b, bias=None, act="none", add=None):
    a, b = _f32(a), _f32(b)
    M, K = a.shape
    N = b.shape[1]
    bias = None if bias is None else _f32(bias).reshape(-1)
    add = None if add is None else _f32(add)
    c = np.empty((M, N), np.float32)
    lib().or_matmul(a, b, c, M, K, N, _ptr(bias), ACT[act], _ptr(add))
    return c


def matmul_int8(a, wq, scale, N, K, bias=None, act="none"):
    a = _f32(a)
    M = a.shape[0]
    wq = np.ascontiguousarray(wq, np.int8).reshape(-1)
    bias = None if bias is None else _f32(bias).reshape(-1)
    y = np.empty((M, N), np.float32)
    lib().or_matmul_int8(a, wq, _f32(scale).reshape(-1), y, M, N, K, _ptr(bias), ACT[act])
    return y


def matmul_nbits(a, bq, scales, zp, N, block_size=32):
    a = _f32(a)
    M, K = a.shape
    nblk = -(-K // block_size)
    zpb = -(-nblk // 2)
    y = np.empty((M, N), np.float32)
    lib().or_matmul_nbits(a, np.ascontiguousarray(bq, np.uint8).reshape(-1), _f32(scales).reshape(-1),
                          np.ascontiguousarray(zp, np.uint8).reshape(-1), y, M, N, K, nblk, zpb, block_size)
    return y


def layernorm(x, g, b, eps=1e-5):
    x = _f32(x)
    out = np.empty_like(x)
    lib().or_layernorm(x, _f32(g).reshape(-1), _f32(b).reshape(-1), out, x.shape[0], x.shape[1], eps)
    return out


def softmax(x):
    x = _f32(x)
    out = np.empty_like(x)
    lib().or_softmax(x, out, x.shape[0], x.shape[1])
    return out


def glu(x):
    x = _f32(x)
    out = np.empty((x.shape[0] // 2, x.shape[1]), np.float32)
    lib().or_glu(x, out, x.shape[0], x.shape[1])
    return out


def silu(x):
    x = _f32(x)
    out = np.empty_like(x)
    lib().or_silu(x, out, x.size)
    return out


def transpose(x):
    x = _f32(x)
    out = np.empty((x.shape[1], x.shape[0]), np.float32)
    lib().or_transpose(x, out, x.shape[0], x.shape[1])
    return out


def conv2d(x, w, cout, cin, h, wd, kh, kw, bias=None, sh=1, sw=1, pt=0, pb=0, pl=0, pr=0, groups=1, act="none"):
    x, w = _f32(x), _f32(w)
    Ho, Wo = (h + pt + pb - kh) // sh + 1, (wd + pl + pr - kw) // sw + 1
    out = np.empty((cout, Ho * Wo), np.float32)
    bias = None if bias is None else _f32(bias).reshape(-1)
    lib().or_conv2d(x, w, _ptr(bias), out, cout, cin, h, wd, kh, kw, sh, sw, pt, pb, pl, pr, groups, ACT[act])
    return out


def conv1d_grouped(x, w, cout, k, bias=None, stride=1, pad_left=0, pad_right=0, dilation=1, groups=1, act="none"):
    x, w = _f32(x), _f32(w)
    cin, L = x.shape
    lout = (L + pad_left + pad_right - dilation * (k - 1) - 1) // stride + 1
    y = np.empty((cout, lout), np.float32)
    bias = None if bias is None else _f32(bias).reshape(-1)
    lib().or_conv1d_grouped(x, w, _ptr(bias), y, cout, cin, L, k, stride, pad_left, pad_right, dilation, groups, ACT[act])
    return y


def subreshape(x, C_, Tsub, F):
    x = _f32(x)
    out = np.empty((Tsub, C_ * F), np.float32)
    lib().or_subreshape(x, out, C_, Tsub, F)
    return out


def bmm_qk(q, b, qb, H, HD, W=1, b_shared=False):
    q, b = _f32(q), _f32(b)
    T = q.shape[0] // W
    Tb = b.shape[0] if b_shared else b.shape[0] // W
    out = np.empty((W * H * T, Tb), np.float32)
    qb = None if qb is None else _f32(qb).reshape(-1)
    lib().or_bmm_qk(q, q.shape[0], b, b.shape[0], _ptr(qb), out, H, HD, W, int(b_shared))
    return out


def bmm_pv(p, v, H, HD, W=1):
    p, v = _f32(p), _f32(v)
    Tq = p.shape[0] // (W * H)
    out = np.empty((W * Tq, H * HD), np.float32)
    lib().or_bmm_pv(p, p.shape[0], v, v.shape[0], out, H, HD, W)
    return out


def relshift_stream(x, H, n, Lk, dMax, Lc, subT, C, left, right):
    """wasm-context.js:509-524: streaming rel_shift + chunked-causal mask."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty((H * n, Lk), np.float32)
    lib().or_relshift_stream(x, out, H, n, Lk, x.shape[1], dMax, Lc, subT, C, left, right)
    return out


def relshift_b(x, H):
    x = _f32(x)
    t = x.shape[0] // H
    out = np.empty((H * t, t), np.float32)
    lib().or_relshift_b(x, out, x.shape[0], H)
    return out


def pos_encoding(T, D):
    pe = np.empty((2 * T - 1, D), np.float32)
    lib().or_pos_encoding(T, D, pe)
    return pe


def quantize_int8_cols(w):
    w = _f32(w)
    K, N = w.shape
    q = np.empty((K, N), np.int8)
    s = np.empty(N, np.float32)
    lib().or_quantize_int8_cols(w, K, N, q, s)
    return q, s


def dequant_int8_cols(q, s):
    K, N = q.shape
    w = np.empty((K, N), np.float32)
    lib().or_dequant_int8_cols(np.ascontiguousarray(q, np.int8), _f32(s), K, N, w)
    return w


def quantize_int4_g32(w):
    """Returns (bq [N, nblk, 16] u8, scales_f16 [N, nblk] u16, scales_f32, zp [N, zpb] u8)."""
    w = _f32(w)
    K, N = w.shape
    nblk = -(-K // 32)
    zpb = -(-nblk // 2)
    bq = np.empty((N, nblk, 16), np.uint8)
    sh = np.empty((N, nblk), np.uint16)
    sf = np.empty((N, nblk), np.float32)
    zp = np.empty((N, zpb), np.uint8)
    lib().or_quantize_int4_g32(w, K, N, bq, sh, _ptr(sf), _ptr(zp))
    return bq, sh, sf, zp


def dequant_int4_g32(bq, sh, K, N):
    w = np.empty((K, N), np.float32)
    lib().or_dequant_int4_g32(np.ascontiguousarray(bq, np.uint8), np.ascontiguousarray(sh, np.uint16), K, N, w)
    return w


def f32_to_f16_bits(x: float) -> int:
    return int(lib().or_f32_to_f16(float(x)))


def tsub(T: int) -> int:
    return int(lib().or_tsub(int(T)))


# ── encoder ─────────────────────────────────────────────────────────────────
def cfg_struct(cfg: dict) -> OrCfg:
    return OrCfg(cfg["D"], cfg["DFF"], cfg["H"], cfg["HD"], cfg["layers"], cfg["dwK"], cfg["Csub"], cfg["Fsub"], cfg["melBins"])


def flatten_weights(man: dict, layers: int):
    """man: manifest-style dict {"c0w": arr, ..., "L0_q": arr, ...} (reference
    manifest key names).  Returns (flat f32, offsets int64) in the C table order."""
    keys = list(GLOBAL_KEYS) + [f"L{L}_{k}" for L in range(layers) for k in LAYER_KEYS]
    parts, offs, pos = [], [], 0
    for k in keys:
        a = man.get(k)
        if a is None:
            offs.append(-1)
            continue
        a = _f32(a).reshape(-1)
        offs.append(pos)
        parts.append(a)
        pos += a.size
    return np.concatenate(parts).astype(np.float32), np.asarray(offs, np.int64)


def pre_encode(cfg, man, mel):
    """mel [melBins, T] channel-major -> x [Tsub, D] (enc:177-222)."""
    flat, off = flatten_weights(man, 0)
    T = mel.shape[1]
    out = np.empty((tsub(T), cfg["D"]), np.float32)
    ts = lib().or_pre_encode(C.byref(cfg_struct(cfg)), flat, off, _f32(mel), T, out)
    assert ts == out.shape[0]
    return out


def encode_batch(cfg, man, mels, layers=None):
    """mels: list of W [melBins, T] arrays of one length.  Returns [W*Tsub, D]
    (enc:235-386, WASM-backend arithmetic)."""
    layers = cfg["layers"] if layers is None else layers
    flat, off = flatten_weights(man, layers)
    W = len(mels)
    T = mels[0].shape[1]
    m = np.ascontiguousarray(np.stack([_f32(x) for x in mels]), np.float32)
    out = np.empty((W * tsub(T), cfg["D"]), np.float32)
    ts = lib().or_encode_batch(C.byref(cfg_struct(cfg)), flat, off, m, W, T, layers, out)
    if ts < 0:
        raise ValueError("encode_batch: windows must have equal Tsub")
    return out


# ── log-mel front end (nemotron-mel.js JsPreprocessor, Parakeet settings) ──
MEL_LOG_GUARD = 2.0 ** -24


def mel_filterbank(nmels=128):
    fb = np.empty((nmels, 257), np.float32)
    lib().or_mel_filterbank(nmels, fb)
    return fb


def mel_hann():
    w = np.empty(512, np.float64)
    lib().or_mel_hann(w)
    return w


def mel_twiddles(n):
    c, s = np.empty(n // 2, np.float64), np.empty(n // 2, np.float64)
    lib().or_mel_twiddles(n, c, s)
    return c, s


def mel_power(frame):
    """257-bin f32 power spectrum of one windowed 512-sample f64 frame."""
    p = np.empty(257, np.float32)
    lib().or_mel_power(np.ascontiguousarray(frame, np.float64), p)
    return p


def mel(audio, nmels=128, log_guard=MEL_LOG_GUARD, normalize=True):
    """[nmels, floor(len/160)] f32 log-mel features of one mono 16 kHz window."""
    a = _f32(audio).reshape(-1)
    T = len(a) // 160
    out = np.empty((nmels, max(T, 0)), np.float32)
    got = lib().or_mel(a, len(a), nmels, float(log_guard), int(bool(normalize)), out) if T > 0 else 0
    assert got == T
    return out


# ── greedy TDT decoder (rust/parakeet-decoder/src/lib.rs decode_proj) ──────
TDT_HID, TDT_VOCAB, TDT_LOGITS, TDT_BLANK = 640, 8193, 8198, 8192
DEC_KEYS = ["embed", "l0_W", "l0_R", "l0_B", "l1_W", "l1_R", "l1_B", "predW", "predB", "outW", "outB"]


def tdt_expf(x: float) -> float:
    return float(lib().or_tdt_expf(float(x)))


def tdt_lstm(w, r, b, x, h, c):
    nh, nc = np.empty(TDT_HID, np.float32), np.empty(TDT_HID, np.float32)
    lib().or_tdt_lstm(_f32(w), _f32(r), _f32(b), _f32(x), _f32(h), _f32(c), nh, nc)
    return nh, nc


def tdt_joint(out_w, out_b, frame, predproj):
    o = np.empty(TDT_LOGITS, np.float32)
    lib().or_tdt_joint(_f32(out_w), _f32(out_b), _f32(frame), _f32(predproj), o)
    return o


def tdt_decode(dec: dict, frames, cap: int = 1 << 16):
    """Greedy TDT decode of pre-projected frames [T, 640] -> (ids, frame indices)."""
    f = _f32(frames).reshape(-1, TDT_HID)
    ids, fr = np.empty(cap, np.int32), np.empty(cap, np.int32)
    n = lib().or_tdt_decode_proj(*[_f32(dec[k]) for k in DEC_KEYS], f, f.shape[0], ids, fr, cap)
    n = min(n, cap)
    return ids[:n].copy(), fr[:n].copy()
