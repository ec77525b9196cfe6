"""The TTS / decoder-side ComputeContext members on the GPU against the
oracle's restatement of the reference CPU backend (oracle/js_ops.py, pinned
on the CPU by test_oracle_js_ops.py).  Shapes and tolerances follow the
reference's numeric conformance gate (scripts/backend-conformance.mjs), plus
Parakeet-size decoder shapes where the indices must match exactly."""
import os
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle"))
import js_ops as J  # noqa: E402

pytestmark = pytest.mark.gpu
rng = np.random.default_rng(2024)


def r(*shape, s=1.0):
    return ((rng.random(shape) - 0.5) * s).astype(np.float32)


def up(ctx, a):
    a = np.asarray(a, np.float32)
    a2 = a.reshape(a.shape[0], -1) if a.ndim > 1 else a.reshape(1, -1)
    return ctx.upload(a2, a2.shape[0], a2.shape[1])


def down(ctx, t):
    return ctx.download(t).reshape(t.rows, t.cols)


def maxd(a, b):
    return float(np.abs(np.asarray(a, np.float64) - b).max())


def test_leaky_relu_snake_adain(ctx):
    x = r(6, 11)
    assert maxd(down(ctx, ctx.leakyRelu(up(ctx, x), 0.3)), J.leaky_relu(x, 0.3)) <= 1e-6
    assert maxd(down(ctx, ctx.leakyRelu(up(ctx, x))), J.leaky_relu(x)) <= 1e-6
    x, a = r(4, 17, s=8), r(1, 4)
    assert maxd(down(ctx, ctx.snake(up(ctx, x), up(ctx, a))), J.snake(x, a)) <= 1e-5
    x, sc, sh = r(5, 20, s=4), r(1, 5), r(1, 5)
    assert maxd(down(ctx, ctx.adain(up(ctx, x), up(ctx, sc), up(ctx, sh))), J.adain(x, sc, sh)) <= 1e-4
    x, sc, sh = r(64, 3000, s=4), r(1, 64), r(1, 64)  # rows longer than the block
    assert maxd(down(ctx, ctx.adain(up(ctx, x), up(ctx, sc), up(ctx, sh), 1e-3)), J.adain(x, sc, sh, 1e-3)) <= 1e-4


@pytest.mark.parametrize("k,stride,pad,dil", [(3, 2, 1, 1), (5, 1, 2, 1), (3, 1, 0, 2)])
def test_im2col_and_conv1d_compositions(ctx, k, stride, pad, dil):
    x = r(4, 15)
    assert np.array_equal(down(ctx, ctx.im2col(up(ctx, x), k, stride=stride, pad=pad, dilation=dil)), J.im2col(x, k, stride, pad, dil))
    w = r(6, 4 * k)
    ref = J.im2col(x, k, stride, pad, dil).astype(np.float64)
    ref = np.maximum(w.astype(np.float64) @ ref, 0)
    got = down(ctx, ctx.conv1dGemm(up(ctx, x), up(ctx, w), 6, k, stride=stride, pad=pad, dilation=dil, act="relu"))
    assert maxd(got, ref) <= 1e-3
    b = r(1, 6)
    fast = down(ctx, ctx.conv1dFast(up(ctx, x), up(ctx, w), 6, k, bias=up(ctx, b), stride=stride, pad=pad, dilation=dil, act="relu"))
    direct = down(ctx, ctx.conv1d(up(ctx, x), up(ctx, w), 6, k, bias=up(ctx, b), stride=stride, pad=pad, dilation=dil, act="relu"))
    assert np.array_equal(fast, direct)
    assert np.array_equal(down(ctx, ctx.conv1dFastF16(up(ctx, x), up(ctx, w), 6, k, stride=stride, pad=pad, dilation=dil)),
                          down(ctx, ctx.conv1d(up(ctx, x), up(ctx, w), 6, k, stride=stride, pad=pad, dilation=dil)))


@pytest.mark.parametrize("groups,stride,pad,dil,op,act", [(2, 2, 1, 1, 0, "none"), (1, 2, 1, 1, 1, "relu"), (1, 1, 0, 2, 0, "silu"),
                                                          (3, 3, 2, 1, 2, "none")])
def test_conv_transpose1d(ctx, groups, stride, pad, dil, op, act):
    Cin, cout, k, L = 6, 12, 4, 12
    x, w, b = r(Cin, L), r(1, Cin * (cout // groups) * k), r(1, cout)
    got = down(ctx, ctx.convTranspose1d(up(ctx, x), up(ctx, w), cout, k, bias=up(ctx, b), stride=stride, pad=pad, dilation=dil, groups=groups,
                                        outputPadding=op, act=act))
    assert maxd(got, J.conv_transpose1d(x, w, cout, k, b, stride, pad, dil, groups, op, act)) <= 1e-5


def test_gather_cols(ctx, fa):
    x = r(5, 12)
    idx = rng.integers(0, 12, 20).astype(np.uint32)
    assert np.array_equal(down(ctx, ctx.gatherCols(up(ctx, x), idx)), J.gather_cols(x, idx))
    with pytest.raises(fa.FaError):
        ctx.gatherCols(up(ctx, x), np.array([3, 12], np.uint32))


@pytest.mark.parametrize("seq,inp,hid", [(6, 8, 16), (40, 80, 256)])
def test_lstm(ctx, seq, inp, hid):
    x, w, rr, b = r(seq, inp), r(8 * hid, inp), r(8 * hid, hid), r(2, 8 * hid)
    got = down(ctx, ctx.lstm(up(ctx, x), up(ctx, w), up(ctx, rr), up(ctx, b), hid))
    assert maxd(got, J.lstm(x, w, rr, b, hid)) <= 1e-5


def test_decoder_fusions_conformance_shapes(ctx):
    e, p = r(10, 32), r(1, 32)
    assert np.array_equal(down(ctx, ctx.jbatch(up(ctx, e), 2, 5, up(ctx, p), 32)), J.jbatch(e, 2, 5, p, 32))
    x = r(6, 40)
    assert np.array_equal(down(ctx, ctx.argmaxRows(up(ctx, x), 6, 32, 40)), J.argmax_rows(x, 6, 32, 40))
    W, b = r(32, 44), r(1, 44)
    got = down(ctx, ctx.jointArgmax(up(ctx, e), 1, 4, up(ctx, p), up(ctx, W), up(ctx, b), 32, 36, 44))
    assert np.array_equal(got, J.joint_argmax(e, 1, 4, p, W, b, 32, 36, 44))


def test_decoder_fusions_parakeet_shapes_and_ties(ctx):
    """Parakeet TDT joint: hidden 640, 8193 tokens + 5 durations; indices and
    maxima bit-identical (f64 sums in the reference's order); rows with ties."""
    hid, vocab, logits, T = 640, 8193, 8198, 24
    e, p = r(T, hid), r(1, hid)
    W, b = (rng.standard_normal((hid, logits)) * 0.05).astype(np.float32), r(1, logits)
    got = down(ctx, ctx.jointArgmax(up(ctx, e), 3, 16, up(ctx, p), up(ctx, W), up(ctx, b), hid, vocab, logits))
    assert np.array_equal(got, J.joint_argmax(e, 3, 16, p, W, b, hid, vocab, logits))
    x = np.round(r(9, logits, s=4), 1)  # coarse values: many ties
    x[4] = -3e30
    got = down(ctx, ctx.argmaxRows(up(ctx, x), 9, vocab, logits))
    assert np.array_equal(got, J.argmax_rows(x, 9, vocab, logits))
