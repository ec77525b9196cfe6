"""Pins of the CPU greedy-TDT oracle (oracle/fa_oracle.c `or_tdt_*`, restating
rust/parakeet-decoder/src/lib.rs decode_proj) against independent float64
numpy computations and closed-form known answers.  The reference holds no
decoder fixture (its gate compares GPU and wasm outputs on downloaded model
weights, scripts/gpu-decoder-check.mjs); these pins stand in for it."""
import math

import numpy as np
import pytest

H, V, L, BLANK = 640, 8193, 8198, 8192
rng = np.random.default_rng(41)


def poly_exp(x):
    """The decoder's expf (lib.rs:47-54): clamp to +-30, 2^floor(t) times a
    degree-4 polynomial in frac(t), t = x / ln 2 (vectorised, float64)."""
    t = np.clip(x, -30, 30) * 1.4426950408889634
    fl = np.floor(t)
    fr = t - fl
    return (1 + fr * (0.6931472 + fr * (0.2402265 + fr * (0.0555041 + fr * 0.0096181)))) * np.exp2(fl)


def np_lstm(w, r, b, x, h, c, exp=np.exp):
    """ONNX LSTM cell, gate rows i, o, f, c; W bias then R bias."""
    sig = lambda v: 1 / (1 + exp(-v))  # noqa: E731
    tanh = lambda v: (exp(2 * v) - 1) / (exp(2 * v) + 1)  # noqa: E731
    z = w.astype(np.float64) @ x + r.astype(np.float64) @ h + b[:4 * H] + b[4 * H:]
    i, o, f, g = z[:H], z[H:2 * H], z[2 * H:3 * H], z[3 * H:]
    cc = sig(f) * c + sig(i) * tanh(g)
    return sig(o) * tanh(cc), cc


def np_decode(dec, frames):
    """Greedy TDT (durations 0..4, at most 10 symbols per frame) in float64."""
    d = {k: v.astype(np.float64) for k, v in dec.items()}
    h = [np.zeros(H), np.zeros(H)]
    c = [np.zeros(H), np.zeros(H)]

    def predict(tok):
        nh0, nc0 = np_lstm(d["l0_W"], d["l0_R"], d["l0_B"], d["embed"][tok], h[0], c[0], poly_exp)
        nh1, nc1 = np_lstm(d["l1_W"], d["l1_R"], d["l1_B"], nh0, h[1], c[1], poly_exp)
        return (nh0, nc0, nh1, nc1), d["predB"] + nh1 @ d["predW"]

    cand, pp = predict(BLANK)
    ids, fr, t, emitted = [], [], 0, 0
    while t < len(frames):
        j = np.maximum(frames[t] + pp, 0)
        out = d["outB"] + j @ d["outW"]
        mx, step = int(np.argmax(out[:V])), int(np.argmax(out[V:]))
        if mx != BLANK:
            h[0], c[0], h[1], c[1] = cand
            ids.append(mx)
            fr.append(t)
            emitted += 1
            cand, pp = predict(mx)
        if step > 0:
            t += step
            emitted = 0
        elif mx == BLANK or emitted >= 10:
            t += 1
            emitted = 0
    return np.array(ids), np.array(fr)


def test_expf_polynomial(orc):
    xs = np.linspace(-30, 30, 2001)
    got = np.array([orc.tdt_expf(x) for x in xs])
    assert np.max(np.abs(got / poly_exp(xs) - 1)) < 5e-6  # f32 vs f64 evaluation of t = x / ln 2
    assert np.max(np.abs(got / np.exp(xs) - 1)) < 1e-3  # the decoder's degree-4 polynomial: 7.5e-4 worst case
    assert orc.tdt_expf(0.0) == 1.0
    assert orc.tdt_expf(50.0) == orc.tdt_expf(30.0) and orc.tdt_expf(-80.0) == orc.tdt_expf(-30.0)


def test_lstm_step_matches_numpy(orc, fa):
    dec = fa.synth.make_decoder_weights(3)
    x, h, c = rng.standard_normal(H), rng.standard_normal(H) * 0.5, rng.standard_normal(H)
    nh, nc = orc.tdt_lstm(dec["l0_W"], dec["l0_R"], dec["l0_B"], x, h, c)
    rh, rc = np_lstm(dec["l0_W"], dec["l0_R"], dec["l0_B"], x.astype(np.float32), h.astype(np.float32), c.astype(np.float32))
    # against exact exp: the decoder's expf is good to 7.5e-4 (a gate-order or
    # bias mistake is off by O(0.1))
    assert np.abs(nh - rh).max() < 1e-3 and np.abs(nc - rc).max() < 1e-3
    ph, pc = np_lstm(dec["l0_W"], dec["l0_R"], dec["l0_B"], x.astype(np.float32), h.astype(np.float32), c.astype(np.float32), poly_exp)
    assert np.abs(nh - ph).max() < 2e-6 and np.abs(nc - pc).max() < 1e-5


def test_joint_matches_numpy(orc, fa):
    dec = fa.synth.make_decoder_weights(4)
    frame, pp = rng.standard_normal(H).astype(np.float32), rng.standard_normal(H).astype(np.float32)
    got = orc.tdt_joint(dec["outW"], dec["outB"], frame, pp)
    ref = dec["outB"] + np.maximum(frame.astype(np.float64) + pp, 0) @ dec["outW"].astype(np.float64)
    assert np.abs(got - ref).max() < 1e-4


def constant_logits(fa, token, dur):
    """Weights whose joint logits do not depend on the frame: outW = 0."""
    dec = fa.synth.make_decoder_weights(5)
    dec["outW"] = np.zeros_like(dec["outW"])
    ob = np.zeros(L, np.float32)
    ob[token] = 1.0
    ob[V + dur] = 1.0
    dec["outB"] = ob
    return dec


@pytest.mark.parametrize("token,dur", [(BLANK, 2), (BLANK, 0), (5, 0), (7, 3), (9, 1)])
def test_decode_loop_known_answers(orc, fa, token, dur):
    T = 23
    ids, fr = orc.tdt_decode(constant_logits(fa, token, dur), np.zeros((T, H), np.float32))
    if token == BLANK:  # never emits; advances max(dur, 1) frames per step
        assert len(ids) == 0
    elif dur == 0:  # MAX_SYMBOLS tokens per frame, then one frame
        assert np.array_equal(ids, np.full(10 * T, token)) and np.array_equal(fr, np.repeat(np.arange(T), 10))
    else:  # one token per step, advancing dur frames
        assert np.array_equal(fr, np.arange(0, T, dur)) and np.all(ids == token)


@pytest.mark.parametrize("seed", [1, 2])
def test_decode_matches_numpy_decoder(orc, fa, seed):
    dec = fa.synth.make_decoder_weights(seed)
    frames = fa.synth.make_projected_frames(120, seed + 10)
    ids, fr = orc.tdt_decode(dec, frames)
    rid, rfr = np_decode(dec, frames.astype(np.float64))
    assert 10 < len(ids) < 120
    assert np.array_equal(ids, rid) and np.array_equal(fr, rfr)
