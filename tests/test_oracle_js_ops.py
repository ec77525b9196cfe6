"""Pins for oracle/js_ops.py (the checker of the TTS / decoder-side HIP ops),
CPU only: torch library routines (leaky_relu, instance_norm, unfold,
conv_transpose1d, nn.LSTM), numpy indexing, closed forms and known answers
with ties."""
import math
import os
import sys

import numpy as np
import pytest
import torch
import torch.nn.functional as F

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle"))
import js_ops as J  # noqa: E402

rng = np.random.default_rng(99)


def r(*shape, s=1.0):
    return (rng.standard_normal(shape) * s).astype(np.float32)


def t64(a):
    return torch.as_tensor(np.asarray(a, np.float64))


def test_leaky_relu_matches_torch():
    x = r(7, 13)
    for slope in (0.2, 0.3, 0.01):
        assert np.array_equal(J.leaky_relu(x, slope), F.leaky_relu(t64(x), slope).numpy().astype(np.float32))


def test_snake_known_answers():
    a = np.array([[0.5], [2.0], [1.0]], np.float32)
    x = np.array([[math.pi / (2 * 0.5), 0.0], [math.pi / (2 * 2.0), math.pi / 2.0], [math.pi, -math.pi / 2]], np.float32)
    got = J.snake(x, a)
    # sin(a x) = +-1 -> x + 1/(a + 1e-9); sin(a x) = 0 -> x
    assert abs(got[0, 0] - (x[0, 0] + 1 / (0.5 + 1e-9))) < 1e-6 and got[0, 1] == 0.0
    assert abs(got[1, 0] - (x[1, 0] + 1 / (2 + 1e-9))) < 1e-6 and abs(got[1, 1] - x[1, 1]) < 1e-6
    assert abs(got[2, 0] - x[2, 0]) < 1e-6 and abs(got[2, 1] - (x[2, 1] + 1.0)) < 1e-6
    # the added term is non-negative and periodic in x with period pi / a
    x2, a2 = r(4, 50), (np.abs(r(4, 1)) + 0.1)
    d1 = J.snake(x2, a2).astype(np.float64) - x2
    d2 = J.snake((x2 + np.pi / a2).astype(np.float32), a2).astype(np.float64) - (x2 + np.pi / a2).astype(np.float32)
    assert d1.min() >= -1e-6 and np.abs(d1 - d2).max() < 1e-4 * np.abs(d1).max() + 1e-5


def test_adain_matches_instance_norm():
    x, sc, sh = r(5, 20, s=3.0), r(1, 5), r(1, 5)
    ref = F.instance_norm(t64(x)[None], eps=1e-5)[0] * t64(sc).reshape(-1, 1) + t64(sh).reshape(-1, 1)
    assert np.abs(J.adain(x, sc, sh) - ref.numpy()).max() < 1e-5


@pytest.mark.parametrize("k,stride,pad,dil", [(3, 2, 1, 1), (5, 1, 2, 1), (3, 1, 0, 2), (4, 3, 3, 1)])
def test_im2col_matches_unfold(k, stride, pad, dil):
    x = r(4, 15)
    ref = F.unfold(t64(x)[None, :, None, :], (1, k), dilation=(1, dil), padding=(0, pad), stride=(1, stride))[0]
    assert np.array_equal(J.im2col(x, k, stride, pad, dil), ref.numpy().astype(np.float32))


@pytest.mark.parametrize("groups,stride,pad,dil,op", [(2, 2, 1, 1, 0), (1, 2, 1, 1, 1), (1, 1, 0, 2, 0), (3, 3, 2, 1, 2)])
def test_conv_transpose1d_matches_torch(groups, stride, pad, dil, op):
    Cin, cout, k, L = 6, 12, 4, 12
    x, w, b = r(Cin, L), r(Cin * (cout // groups) * k), r(1, cout)
    ref = F.conv_transpose1d(t64(x)[None], t64(w).reshape(Cin, cout // groups, k), t64(b).reshape(-1), stride=stride, padding=pad,
                             output_padding=op, groups=groups, dilation=dil)[0]
    got = J.conv_transpose1d(x, w, cout, k, b, stride, pad, dil, groups, op)
    assert got.shape == tuple(ref.shape) and np.abs(got - ref.numpy()).max() < 1e-5
    got_r = J.conv_transpose1d(x, w, cout, k, b, stride, pad, dil, groups, op, act="relu")
    assert np.array_equal(got_r, np.maximum(got, 0))


def test_gather_cols():
    x = r(5, 12)
    idx = rng.integers(0, 12, 20)
    assert np.array_equal(J.gather_cols(x, idx), np.take(x, idx, axis=1))


def test_lstm_matches_torch_bidirectional():
    """ONNX gate order (i, o, f, c) mapped onto torch's (i, f, g, o)."""
    seq, inp, hid = 6, 8, 16
    x, w, rr, b = r(seq, inp), r(8 * hid, inp), r(8 * hid, hid), r(2, 8 * hid)
    perm = np.concatenate([np.arange(0, hid), np.arange(2 * hid, 3 * hid), np.arange(3 * hid, 4 * hid), np.arange(hid, 2 * hid)])
    m = torch.nn.LSTM(inp, hid, bidirectional=True).double()
    W, R = w.reshape(2, 4 * hid, inp), rr.reshape(2, 4 * hid, hid)
    with torch.no_grad():
        for d, sfx in ((0, ""), (1, "_reverse")):
            getattr(m, "weight_ih_l0" + sfx).copy_(t64(W[d][perm]))
            getattr(m, "weight_hh_l0" + sfx).copy_(t64(R[d][perm]))
            getattr(m, "bias_ih_l0" + sfx).copy_(t64(b[d, :4 * hid][perm]))
            getattr(m, "bias_hh_l0" + sfx).copy_(t64(b[d, 4 * hid:][perm]))
        ref = m(t64(x)[:, None, :])[0][:, 0, :].numpy()
    assert np.abs(J.lstm(x, w, rr, b, hid) - ref).max() < 1e-5


def test_jbatch_and_argmax_known_answers():
    enc = np.array([[1, -2, 3], [0, 0, 0], [-1, 5, -5], [2, 2, 2]], np.float32)
    pred = np.array([[0.5, 1.0, -4.0]], np.float32)
    assert J.jbatch(enc, 1, 2, pred, 3).tolist() == [[0.5, 1.0, 0.0], [0.0, 6.0, 0.0]]
    # tokens [0, 4), durations [4, 7): first maximum wins on ties; an all
    # -inf-like row keeps the start values (index 0, -1e30)
    x = np.array([[1, 3, 3, 2, 0, 7, 7], [-2e30, -2e30, -2e30, -2e30, -3, -1, -1], [5, 5, 5, 5, 9, 8, 9]], np.float32)
    got = J.argmax_rows(x, 3, 4, 7)
    assert got[:, 0].tolist() == [1, 0, 0] and got[:, 2].tolist() == [1, 1, 0]
    assert got[0, 1] == 3 and got[1, 1] == np.float32(-1e30) and got[2, 3] == 9


def test_joint_argmax_is_jbatch_matmul_argmax():
    hid, vocab, logits = 32, 36, 44
    enc, pred, W, b = r(10, hid), r(1, hid), r(hid, logits), r(1, logits)
    got = J.joint_argmax(enc, 1, 4, pred, W, b, hid, vocab, logits)
    j = J.jbatch(enc, 1, 4, pred, hid).astype(np.float64)
    s = j @ W.astype(np.float64) + b.astype(np.float64)
    want = J.argmax_rows(s.astype(np.float32), 4, vocab, logits)
    assert np.array_equal(got[:, [0, 2]], want[:, [0, 2]])
    assert np.allclose(got[:, 1], s[:, :vocab].max(1), rtol=1e-6) and np.allclose(got[:, 3], s[:, vocab:].max(1), rtol=1e-6)
