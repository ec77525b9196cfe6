"""Pins for the CPU oracle (oracle/fa_oracle.c), CPU only.

Each check compares the oracle with something it does not share code with:
the float64 NeMo-style restatement and its committed fixtures, torch library
routines (conv2d/conv1d/layer_norm/softmax/gelu), closed forms and hand-made
known answers, or bit-level emulation of the reference's operation order.
"""
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
rng = np.random.default_rng(1234)


def r(*shape, s=1.0):
    return (rng.standard_normal(shape) * s).astype(np.float32)


def f64(a):
    return torch.as_tensor(np.asarray(a, np.float64))


def err(a, b):
    """max |a-b| relative to max(1, |b|): f32 rounding of an exact result is <= 6e-8."""
    return float(np.max(np.abs(np.asarray(a, np.float64) - b) / np.maximum(1.0, np.abs(b))))


@pytest.fixture(scope="module")
def npref():
    import sys

    sys.path.insert(0, os.path.join(os.path.dirname(HERE), "oracle"))
    import np_ref

    return np_ref


# ── GEMM (lib.rs:59-94) ────────────────────────────────────────────────────
def test_matmul_f32_is_ikj_without_fma_bitexact(orc):
    a, b = r(7, 33), r(33, 21)
    got = orc.matmul_f32(a, b)
    c = np.zeros((7, 21), np.float32)
    for k in range(33):  # c = c + a_ik * b_k, f32 multiply then f32 add
        c = (c + (a[:, k:k + 1] * b[k:k + 1, :]).astype(np.float32)).astype(np.float32)
    assert np.array_equal(got, c)


def test_matmul_close_to_f64(orc):
    a, b = r(50, 300), r(300, 70)
    assert np.abs(orc.matmul_f32(a, b) - a.astype(np.float64) @ b).max() < 1e-3


@pytest.mark.parametrize("act", ["none", "relu", "silu", "gelu", "gelu_erf", "tanh"])
def test_bias_act_against_library(orc, act):
    a, b, bias = r(9, 40), r(40, 17), r(1, 17)
    got = orc.matmul(a, b, bias, act).astype(np.float64)
    z = f64(orc.matmul_f32(a, b)) + f64(bias)
    ref = {"none": lambda t: t, "relu": F.relu, "silu": F.silu, "tanh": torch.tanh,
           "gelu": lambda t: F.gelu(t, approximate="tanh"), "gelu_erf": F.gelu}[act](z).numpy()
    # gelu_erf uses the reference's 5-term erf polynomial (|err| < 1.5e-7)
    assert np.abs(got - ref).max() < (2e-6 if act == "gelu_erf" else 1e-6)


def test_matmul_residual_add(orc):
    a, b, d = r(5, 8), r(8, 6), r(5, 6)
    assert np.array_equal(orc.matmul(a, b, add=d), (orc.matmul_f32(a, b) + d).astype(np.float32))


# ── row ops (wasm-context.js:308-343, 428-434) ─────────────────────────────
def test_layernorm_softmax_glu(orc):
    x, g, b = r(11, 96, s=3) + 2, r(96) + 1, r(96)
    ln = F.layer_norm(f64(x), (96,), f64(g), f64(b), eps=1e-5).numpy()
    assert np.abs(orc.layernorm(x, g, b) - ln).max() < 2e-6
    s = r(13, 50, s=5)
    assert np.abs(orc.softmax(s) - torch.softmax(f64(s), -1).numpy()).max() < 1e-7
    y = r(8, 10, s=3)
    gl = F.glu(f64(y), dim=0).numpy()
    assert np.max(np.abs(orc.glu(y) - gl) / np.maximum(1.0, np.abs(gl))) < 2e-7  # f32 rounding of a double result


# ── convolutions ────────────────────────────────────────────────────────────
def test_conv2d_matches_torch_for_the_subsampling_convs(orc):
    C, T, Fq = 6, 17, 12
    x = r(1, T * Fq)
    w0, b0 = r(C, 1, 3, 3), r(C)
    y0 = orc.conv2d(x, w0, C, 1, T, Fq, 3, 3, b0, 2, 2, 1, 1, 1, 1, 1, "relu")
    t0 = F.relu(F.conv2d(f64(x).reshape(1, 1, T, Fq), f64(w0), f64(b0), stride=2, padding=1)).numpy().reshape(C, -1)
    assert err(y0, t0) < 1e-6
    T1, F1 = (T - 1) // 2 + 1, (Fq - 1) // 2 + 1
    w1, b1 = r(C, 1, 3, 3), r(C)
    y1 = orc.conv2d(y0, w1, C, C, T1, F1, 3, 3, b1, 2, 2, 1, 1, 1, 1, C, "none")
    t1 = F.conv2d(f64(y0).reshape(1, C, T1, F1), f64(w1), f64(b1), stride=2, padding=1, groups=C).numpy().reshape(C, -1)
    assert err(y1, t1) < 1e-6
    w2, b2 = r(C, C, 1, 1), r(C)
    y2 = orc.conv2d(y1, w2, C, C, (T1 - 1) // 2 + 1, (F1 - 1) // 2 + 1, 1, 1, b2, act="relu")
    t2 = F.relu(F.conv2d(f64(y1).reshape(1, C, (T1 - 1) // 2 + 1, -1), f64(w2), f64(b2))).numpy().reshape(C, -1)
    assert err(y2, t2) < 1e-6


def test_depthwise_conv1d_matches_torch(orc):
    D, T = 12, 40
    x, w, b = r(D, T), r(D, 1, 9), r(D)
    got = orc.conv1d_grouped(x, w, D, 9, b, 1, 4, 4, 1, D, "silu")
    ref = F.silu(F.conv1d(f64(x)[None], f64(w), f64(b), padding=4, groups=D))[0].numpy()
    assert err(got, ref) < 1e-5


def test_subreshape_is_channel_time_freq_to_time_channel_freq(orc):
    C, Ts, Fq = 3, 4, 5
    x = np.arange(C * Ts * Fq, dtype=np.float32).reshape(C, Ts * Fq)
    ref = x.reshape(C, Ts, Fq).transpose(1, 0, 2).reshape(Ts, C * Fq)
    assert np.array_equal(orc.subreshape(x, C, Ts, Fq), ref)


# ── relative positions ─────────────────────────────────────────────────────
def test_relshift_fixture_and_closed_form(orc):
    g = np.load(os.path.join(HERE, "golden", "relpos.npz"))
    got = orc.relshift_b(g["x"], 3)
    assert np.array_equal(got, g["relshift"].astype(np.float32))
    t = 5
    x = g["x"].reshape(3, t, 2 * t - 1)
    closed = np.stack([[x[h, i, t - 1 - i:2 * t - 1 - i] for i in range(t)] for h in range(3)]).reshape(15, t)
    assert np.array_equal(got, closed)


def test_pos_encoding_fixture(orc):
    g = np.load(os.path.join(HERE, "golden", "relpos.npz"))
    pe = orc.pos_encoding(7, 16)
    assert np.abs(pe - g["pe_T7_D16"]).max() < 1e-7
    assert np.allclose(pe[6, 0::2], 0) and np.allclose(pe[6, 1::2], 1)  # relative position 0


def test_bmm_qk_pv_against_einsum(orc):
    H, HD, W, T = 2, 8, 3, 5
    q, k, v, qb = r(W * T, H * HD), r(W * T, H * HD), r(W * T, H * HD), r(H * HD)
    got = orc.bmm_qk(q, k, qb, H, HD, W)
    Q = (q + qb).astype(np.float64).reshape(W, T, H, HD)
    ref = np.einsum("wihd,wjhd->whij", Q, k.astype(np.float64).reshape(W, T, H, HD)).reshape(W * H * T, T)
    assert np.abs(got - ref).max() < 1e-5
    p = orc.softmax(got)
    o = orc.bmm_pv(p, v, H, HD, W)
    ref2 = np.einsum("whij,wjhd->wihd", p.astype(np.float64).reshape(W, H, T, T), v.astype(np.float64).reshape(W, T, H, HD)).reshape(W * T, H * HD)
    assert np.abs(o - ref2).max() < 1e-5


# ── int8 GEMM, SiLU, transpose (lib.rs:143-162, wasm-context.js:22,396-441) ─
def test_matmul_int8_known_answer_layout_and_scale(orc):
    # wq is [K, N] row-major (index k*N + n): a transposed read, a scale taken
    # per row instead of per column or a signed/unsigned mix-up all change this
    a = np.array([[1.0, 10.0]], np.float32)
    wq = np.array([[1, 2, -3], [4, -128, 6]], np.int8)
    s = np.array([1.0, 0.5, 2.0], np.float32)
    y = orc.matmul_int8(a, wq, s, 3, 2)
    assert y.tolist() == [[41.0, (2 - 1280) * 0.5, (-3 + 60) * 2.0]]
    # bias then activation after the column scale (JS applies them, wasm-context.js:290-297)
    y = orc.matmul_int8(a, wq, s, 3, 2, bias=np.array([0.0, 1000.0, -200.0], np.float32), act="relu")
    assert y.tolist() == [[41.0, 361.0, 0.0]]


def test_matmul_int8_against_f64_dequant(orc):
    K, N = 200, 37
    a = r(5, K)
    wq = rng.integers(-127, 128, size=(K, N)).astype(np.int8)
    s = (rng.random(N) * 0.01 + 1e-3).astype(np.float32)
    bias = r(1, N)
    ref = a.astype(np.float64) @ (wq.astype(np.float64) * s.astype(np.float64)) + bias.astype(np.float64)
    got = orc.matmul_int8(a, wq, s, N, K, bias=bias)
    assert np.abs(got - ref).max() < 2e-5 * max(1.0, np.abs(ref).max())
    # f32 accumulate in k order, then one multiply by the scale (lib.rs:153-158)
    acc = np.zeros((5, N), np.float32)
    for k in range(K):
        acc = (acc + (a[:, k:k + 1] * wq[k:k + 1, :].astype(np.float32)).astype(np.float32)).astype(np.float32)
    assert np.array_equal(orc.matmul_int8(a, wq, s, N, K), (acc * s).astype(np.float32))


def test_silu_against_torch(orc):
    x = np.concatenate([r(1000, s=6.0).reshape(-1), np.array([0.0, 29.0, 31.0, -31.0, -100.0, 1e-30], np.float32)])
    got = orc.silu(x)
    ref = F.silu(f64(x)).numpy()
    assert err(got, ref) < 2e-7
    assert got[x.size - 6] == 0.0 and got[x.size - 1] == np.float32(5e-31)  # silu(0) = 0, silu(tiny) = tiny/2
    # the reference clamps the exponent at +-30 (actf.js:19): -100 -> -100/(1+e^30)
    assert np.isclose(got[x.size - 2], -100.0 / (1.0 + math.exp(30.0)), rtol=1e-6)


def test_transpose_against_numpy(orc):
    x = r(13, 7)
    assert np.array_equal(orc.transpose(x), x.T)
    assert np.array_equal(orc.transpose(orc.transpose(x)), x)
    assert orc.transpose(r(1, 5)).shape == (5, 1)


# ── quantisation formats ───────────────────────────────────────────────────
def test_int8_quantizer_known_answers(orc):
    # column 0: max 127 -> s = 1: 63.5 rounds half-even to 64, -0.5 to -0;
    # column 1: all zero -> s = 1 (quantize-parakeet-encoder.py:33);
    # column 2: max 2.54 -> s = 0.02: values land on exact multiples
    w = np.array([[127.0, 0.0, 2.54], [63.5, 0.0, -2.54], [-0.5, 0.0, 0.02], [62.5, 0.0, 0.0]], np.float32)
    q, s = orc.quantize_int8_cols(w)
    assert s[0] == 1.0 and s[1] == 1.0 and s[2] == np.float32(np.float32(2.54) / np.float32(127.0))
    assert q[:, 0].tolist() == [127, 64, 0, 62] and q[:, 1].tolist() == [0, 0, 0, 0]
    assert q[:, 2].tolist() == [127, -127, 1, 0]
    assert np.array_equal(orc.dequant_int8_cols(q, s), q.astype(np.float32) * s)


def test_int4_nibble_order_known_answer(orc):
    K, N = 32, 1
    w = np.zeros((K, N), np.float32)
    w[:, 0] = np.arange(K) % 16 - 8  # q = k%16 - 8, max |w| = 8 -> s = f16(8/7)
    bq, sh, sf, zp = orc.quantize_int4_g32(w)
    s = np.float16(8 / 7)
    assert sh[0, 0] == s.view(np.uint16) and sf[0, 0] == np.float32(s)
    q = np.clip(np.rint(w[:, 0] / np.float32(s)), -8, 7).astype(int)
    nib = q + 8
    expect = np.array([nib[2 * i] | (nib[2 * i + 1] << 4) for i in range(16)], np.uint8)  # low nibble = even k
    assert np.array_equal(bq[0, 0], expect)
    assert np.all(zp == 0x88)


def test_int4_format_is_matmulnbits_with_zero_point_8(orc):
    K, N = 96, 5
    w, a = r(K, N, s=0.02), r(3, K)
    bq, sh, sf, zp = orc.quantize_int4_g32(w)
    deq = orc.dequant_int4_g32(bq, sh, K, N)
    y = orc.matmul_nbits(a, bq, sf, zp, N)  # the reference kernel (lib.rs:169-203)
    assert np.abs(y - a.astype(np.float64) @ deq).max() < 1e-5
    assert np.abs(deq - w).max() <= np.max(sf) / 2 + 1e-7  # rounding error <= s/2


def test_matmul_nbits_zero_point_nibbles_known_answer(orc):
    """Asymmetric MatMulNBits with a different zero point in every block:
    block b of a row reads the low nibble of zero-point byte b // 2 when b is
    even and the high nibble when b is odd (lib.rs:185-186).  The expected
    product is built from the zero points as chosen, not from their packing,
    so a swapped nibble order, a zero point read from the wrong byte or a
    flipped (q - zp) sign each fail."""
    K, N, bs = 96, 2, 32                       # three blocks, two zero-point bytes per row
    zps = [[3, 11, 5], [14, 0, 9]]             # per row, per block
    sc = np.array([[0.5, 0.25, 2.0], [1.5, 0.125, 0.75]], np.float32)
    q = (np.arange(K)[None, :] * np.array([[5], [7]]) + np.array([[1], [4]])) % 16  # 4-bit codes, [N][K]
    bq = np.zeros((N, 3, 16), np.uint8)
    for n in range(N):
        for k in range(K):
            b, t = divmod(k, bs)
            bq[n, b, t // 2] |= np.uint8(q[n, k] << (4 * (t & 1)))  # low nibble = even index
    zp = np.array([[zps[n][0] | (zps[n][1] << 4), zps[n][2]] for n in range(N)], np.uint8)
    assert zp.tolist() == [[0xB3, 0x05], [0x0E, 0x09]]
    a = np.zeros((2, K), np.float32)
    a[0, :] = 1.0                                # row 0: column sums
    a[1, 5], a[1, 40], a[1, 77] = 1.0, 2.0, -1.0  # row 1: one k in each block
    w = np.array([[(q[n, k] - zps[n][k // bs]) * sc[n, k // bs] for n in range(N)] for k in range(K)], np.float64)  # [K][N]
    y = orc.matmul_nbits(a, bq, sc, zp, N)
    assert np.abs(y - a.astype(np.float64) @ w).max() < 1e-4
    # row 1, column 0 by hand: k = 5 (block 0), 40 (block 1), 77 (block 2)
    hand = (q[0, 5] - 3) * 0.5 + 2.0 * (q[0, 40] - 11) * 0.25 - (q[0, 77] - 5) * 2.0
    assert y[1, 0] == np.float32(hand)


def test_library_quantizer_is_bitexact_with_oracle(fa, orc):
    import ctypes as C

    L = fa.lib()
    for K, N in ((64, 9), (70, 3)):
        w = r(K, N, s=0.05)
        w[:, 1] = 0.0
        q, s = orc.quantize_int8_cols(w)
        q8 = np.empty((N, K), np.int8)
        s8 = np.empty(N, np.float32)
        assert L.fa_quantize_weights(1, w.ctypes.data_as(C.POINTER(C.c_float)), K, N, q8.ctypes.data_as(C.c_void_p), s8.ctypes.data_as(C.c_void_p)) == 0
        assert np.array_equal(q8, q.T) and np.array_equal(s8, s)
        bq, sh, _, _ = orc.quantize_int4_g32(w)
        nblk = -(-K // 32)
        q4 = np.empty((N, nblk, 16), np.uint8)
        s4 = np.empty((N, nblk), np.uint16)
        assert L.fa_quantize_weights(2, w.ctypes.data_as(C.POINTER(C.c_float)), K, N, q4.ctypes.data_as(C.c_void_p), s4.ctypes.data_as(C.c_void_p)) == 0
        assert np.array_equal(q4, bq) and np.array_equal(s4, sh)


# ── whole encoder ──────────────────────────────────────────────────────────
def test_encoder_matches_golden_fixture(orc):
    g = np.load(os.path.join(HERE, "golden", "encoder_tiny.npz"))
    cfg = dict(zip(("D", "DFF", "H", "HD", "layers", "dwK", "Csub", "Fsub", "melBins"), g["cfg"].tolist()))
    man = {k[2:]: g[k] for k in g.files if k.startswith("w_")}
    got = orc.encode_batch(cfg, man, [g["mel0"], g["mel1"]])
    exp = g["expected"]
    assert got.shape == exp.shape
    assert np.linalg.norm(got - exp) / np.linalg.norm(exp) < 1e-5


@pytest.mark.parametrize("biases", [False, True])
def test_encoder_matches_independent_f64(fa, orc, npref, biases):
    cfg = fa.synth.tiny_cfg(2)
    man = fa.synth.make_weights(cfg, seed=5, biases=biases)
    mels = fa.synth.make_features(cfg["melBins"], 77, seed=6, W=3)
    a = orc.encode_batch(cfg, man, mels)
    b = npref.encode(cfg, man, mels)
    assert np.linalg.norm(a - b) / np.linalg.norm(b) < 1e-5


def test_encoder_batch_equals_single_and_is_permutation_equivariant(fa, orc):
    cfg = fa.synth.tiny_cfg(1)
    man = fa.synth.make_weights(cfg, seed=8)
    mels = fa.synth.make_features(cfg["melBins"], 50, seed=9, W=3)
    batch = orc.encode_batch(cfg, man, mels)
    T = orc.tsub(50)
    for i, m in enumerate(mels):
        assert np.array_equal(batch[i * T:(i + 1) * T], orc.encode_batch(cfg, man, [m]))
    perm = orc.encode_batch(cfg, man, [mels[2], mels[0], mels[1]])
    assert np.array_equal(perm, np.concatenate([batch[2 * T:], batch[:2 * T]]))


def test_tsub_formula(fa, orc):
    for T in (1, 2, 3, 7, 8, 9, 100, 1500, 3000):
        t = T
        for _ in range(3):
            t = math.floor((t + 2 - 3) / 2) + 1
        assert orc.tsub(T) == t == fa.tsub(T)
    assert orc.tsub(1500) == 188
