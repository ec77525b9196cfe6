"""Streaming encoder (streaming.py, restating streaming-encoder.js) on the
HIP op path, for a small streaming (EOU-style) model: chunk-limited attention,
causal depthwise conv with a LayerNorm, top-padded subsampling.

* the offline chunked-causal encoder (encoder.parakeetEncodeBatch with the
  streaming config, f32 weights) against the float64 NeMo-formulation
  restatement (oracle/np_ref.py, whose mask / causal conv / pads are pinned by
  causality and identity checks on the CPU);
* the reference's own gate (scripts/streaming-encode-check.mjs): mel pushed in
  arbitrary pieces + flush reproduces the offline frames;
* with right context (Nemotron-style), the provisional-tail error shrinks as
  the lookahead grows (streaming-encoder.js:38-46)."""
import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def npref():
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle"))
    import np_ref

    return np_ref


def _model(ctx, fa, right=0, chunk=2):
    cfg = fa.synth.tiny_stream_cfg(layers=2, right=right, chunk=chunk)
    man = fa.synth.make_weights(cfg, seed=11)
    return cfg, man, fa.loadParakeetEncoder(ctx, man, weights="f32", cfg=cfg)


def _offline(ctx, fa, enc, mel):
    a = ctx.pushArena()
    y, T = fa.parakeetEncodeBatch(ctx, enc, [mel])
    out = ctx.download(y).reshape(T, -1)
    ctx.popArena(a)
    return out


def _stream(ctx, fa, enc, mel, pieces, lookahead=0):
    st = fa.createEncodeStream(ctx, enc, lookaheadChunks=lookahead)
    outs, t = [], 0
    for p in pieces:
        o = fa.encodeStreamPush(ctx, st, mel[:, t:t + p])
        t += p
        if o is not None:
            outs.append(o)
    o = fa.encodeStreamFlush(ctx, st)
    if o is not None:
        outs.append(o)
    fa.disposeEncodeStream(ctx, st)
    return np.concatenate(outs, 0)


def test_offline_chunked_causal_matches_np_ref(ctx, fa, npref):
    cfg, man, enc = _model(ctx, fa)
    mel = fa.synth.make_features(cfg["melBins"], 301, seed=5)[0]
    got = _offline(ctx, fa, enc, mel)
    ref = npref.encode(cfg, man, [mel])
    assert got.shape == ref.shape
    err = np.abs(got - ref).max() / np.abs(ref).max()
    assert err < 1e-4, err


@pytest.mark.parametrize("pieces", [[301], [37, 100, 5, 64, 95], [8] * 38])
def test_stream_reproduces_offline_frames(ctx, fa, pieces):
    cfg, man, enc = _model(ctx, fa)
    mel = fa.synth.make_features(cfg["melBins"], 301, seed=6)[0]
    off = _offline(ctx, fa, enc, mel)
    got = _stream(ctx, fa, enc, mel, pieces)
    assert got.shape == off.shape, (got.shape, off.shape)
    err = np.abs(got - off).max() / np.abs(off).max()
    assert err < 1e-5, err


def test_right_context_error_shrinks_with_lookahead(ctx, fa):
    cfg, man, enc = _model(ctx, fa, right=3, chunk=4)
    mel = fa.synth.make_features(cfg["melBins"], 400, seed=7)[0]
    off = _offline(ctx, fa, enc, mel)
    errs = []
    for B in (1, 2, 4):
        got = _stream(ctx, fa, enc, mel, [50] * 8, lookahead=B)
        assert got.shape == off.shape
        errs.append(np.abs(got - off).max() / np.abs(off).max())
    assert errs[2] < errs[0], errs


def test_stream_errors(ctx, fa):
    cfg, man, enc = _model(ctx, fa)
    with pytest.raises(ValueError):
        fa.createEncodeStream(ctx, dict(enc, cfg={k: v for k, v in cfg.items() if k != "attChunk"}))
    st = fa.createEncodeStream(ctx, enc)
    fa.encodeStreamFlush(ctx, st)
    with pytest.raises(RuntimeError):
        fa.encodeStreamPush(ctx, st, np.zeros((cfg["melBins"], 8), np.float32))
    fa.disposeEncodeStream(ctx, st)
    with pytest.raises(ValueError):
        _model_r = _model(ctx, fa, right=3, chunk=4)
        fa.createEncodeStream(ctx, _model_r[2], lookaheadChunks=0)
