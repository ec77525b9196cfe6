"""Pins of the oracle's streaming rel_shift (oracle/fa_oracle.c
or_relshift_stream, restating src/gpu/wasm-context.js:509-524): reduction to
the offline rel_shift (itself pinned against NeMo's pad-reshape), a hand-worked
known answer with mask and clamp, and the per-row count of unmasked keys."""
import os
import sys

import numpy as np
import pytest


@pytest.fixture(scope="module")
def npref():
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle"))
    import np_ref

    return np_ref


def test_full_context_equals_offline_rel_shift(orc):
    rng = np.random.default_rng(1)
    for H, t in [(1, 5), (4, 13), (2, 64)]:
        x = rng.standard_normal((H * t, 2 * t - 1)).astype(np.float32)
        # one chunk over every query, unlimited left/right context, keys from 0
        got = orc.relshift_stream(x, H, t, t, t - 1, 0, 0, t, t, t)
        assert np.array_equal(got, orc.relshift_b(x, H)), (H, t)


def test_known_answer_mask_and_clamp(orc):
    x = np.arange(10, dtype=np.float32).reshape(2, 5)
    # queries q = 2, 3 (chunk 2..3, left 1 -> keys 1..3 allowed), keys k = 0..3
    got = orc.relshift_stream(x, 1, 2, 4, 3, 2, 2, 2, 1, 0)
    assert np.array_equal(got, np.array([[-1e4, 2, 3, 4], [-1e4, 6, 7, 8]], np.float32))
    # dMax beyond the table: distances clamp to the last column
    got = orc.relshift_stream(x, 1, 2, 4, 9, 2, 2, 2, 2, 0)
    assert np.array_equal(got, np.array([[4, 4, 4, 4], [9, 9, 9, 9]], np.float32))


def test_unmasked_key_count(orc):
    rng = np.random.default_rng(2)
    for _ in range(50):
        H, n, Lk, C = int(rng.integers(1, 4)), int(rng.integers(1, 9)), int(rng.integers(1, 40)), int(rng.integers(1, 6))
        subT, Lc, left, right = int(rng.integers(0, 30)), int(rng.integers(0, 20)), int(rng.integers(0, 12)), int(rng.integers(0, 4))
        x = rng.standard_normal((H * n, 11)).astype(np.float32)
        y = orc.relshift_stream(x, H, n, Lk, 5, Lc, subT, C, left, right)
        for r in range(H * n):
            q = subT + r % n
            cs = C * (q // C)
            lo, hi = max(cs - left, subT - Lc), min(cs + C - 1 + right, subT - Lc + Lk - 1)
            assert int((y[r] != -1e4).sum()) == max(0, hi - lo + 1)


def _stream_model(fa, layers=2, right=0, chunk=2):
    cfg = fa.synth.tiny_stream_cfg(layers=layers, right=right, chunk=chunk)
    return cfg, fa.synth.make_weights(cfg, seed=11)


def test_np_ref_mask_wider_than_sequence_is_identity(fa, npref):
    np_ref = npref
    cfg, man = _stream_model(fa)
    mel = fa.synth.make_features(cfg["melBins"], 160, seed=3)[0]
    wide = dict(cfg, attChunk=64, attLeft=64)  # one chunk covers all 20 frames
    free = {k: v for k, v in cfg.items() if k not in ("attChunk", "attLeft", "attRight")}
    assert np.array_equal(np_ref.encode(wide, man, [mel]), np_ref.encode(free, man, [mel]))


def test_np_ref_streaming_model_is_causal_up_to_its_chunk(fa, npref):
    """With right context 0 (causal depthwise conv, top-padded subsampling,
    chunk-limited attention) output frame s depends on mel frames up to 8 e
    only, e = the last frame of s's chunk: later mel frames change nothing
    before e + 1, and do change later frames."""
    np_ref = npref
    cfg, man = _stream_model(fa, chunk=2)
    T = 240
    mel = fa.synth.make_features(cfg["melBins"], T, seed=4)[0]
    base = np_ref.encode(cfg, man, [mel])
    for e in (5, 13):  # ends of chunks (chunk 2: frames 4..5 and 12..13)
        pert = mel.copy()
        pert[:, 8 * e + 1:] += np.random.default_rng(e).standard_normal(pert[:, 8 * e + 1:].shape).astype(np.float32)
        out = np_ref.encode(cfg, man, [pert])
        assert np.array_equal(out[:e + 1], base[:e + 1]), e
        assert np.abs(out[e + 1:] - base[e + 1:]).max() > 1e-3, e
