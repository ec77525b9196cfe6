"""Streaming models on the fused encoder (csrc/encoder.hip options +
csrc/stream.hip), for a small EOU-style model: chunk-limited attention,
causal depthwise conv with the conv-module LayerNorm, subsampling pads
t2 b1 l2 r1.

* offline chunked-causal encode (FusedEncoder with the streaming config)
  against the float64 NeMo-formulation restatement (oracle/np_ref.py, whose
  mask / causal conv / pads are pinned on the CPU by causality and identity
  checks): rel-L2 <= 1e-2 and projected argmax, and tighter with every
  operand exact;
* the reference's own gate (scripts/streaming-encode-check.mjs): mel pushed in
  arbitrary pieces + flush reproduces the offline frames, here the native
  stream (device-resident K/V and conv caches) against the fused offline
  encoder and against np_ref;
* steady-state passes replayed from captured graphs give the eager passes' bits;
* with right context, the provisional-tail error shrinks as the lookahead
  grows (streaming-encoder.js:38-46)."""
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


def _model(ctx, fa, right=0, chunk=2, left=8, layers=2):
    cfg = fa.synth.small_stream_cfg(layers=layers, right=right, chunk=chunk, left=left)
    man = fa.synth.make_weights(cfg, seed=11)
    return cfg, man, fa.FusedEncoder(ctx, man, "f16", max_T=128, cfg=cfg)


def _stream(ctx, fa, enc, mel, pieces, lookahead=0, maxChunk=64):
    st = fa.createEncodeStream(ctx, enc, lookaheadChunks=lookahead, maxChunk=maxChunk)
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


def rel_l2(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))


def flips(a, b):
    R = np.random.default_rng(2).standard_normal((a.shape[1], 64)).astype(np.float32)
    return int(np.sum(np.argmax(a @ R, 1) != np.argmax(b @ R, 1)))


def test_offline_chunked_causal_matches_np_ref(ctx, fa, npref):
    cfg, man, enc = _model(ctx, fa)
    mel = fa.synth.make_features(cfg["melBins"], 601, seed=5)[0]
    got = enc.encode([mel])[0]
    ref = npref.encode(cfg, man, [mel])
    assert got.shape == ref.shape == (enc.tsub(601), cfg["D"])
    r, f = rel_l2(got, ref), flips(got, ref)
    enc.setExact(31)
    r_exact = rel_l2(enc.encode([mel])[0], ref)
    enc.setExact(0)
    r_plain = rel_l2(enc.encode([mel])[0], ref)
    enc.close()
    print(f"offline chunked-causal vs np_ref: rel-L2 {r:.2e} (default), {r_exact:.2e} (all exact), {r_plain:.2e} (plain f16); flips {f}/{len(ref)}")
    assert r <= 1e-2 and f <= max(1, 0.001 * len(ref))
    assert r_exact < 1e-4 and r_plain > 2 * r_exact


@pytest.mark.parametrize("chunk,pieces", [(2, [601]), (2, [37, 100, 5, 64, 95, 300]), (2, [16] * 38), (2, [8] * 76), (1, [8] * 76), (1, [3, 9, 8, 200, 381])])
def test_stream_reproduces_offline_frames(ctx, fa, npref, chunk, pieces):
    """chunk 1 with 8-frame pieces: a first pass could finish one frame, and the
    next pass reads 14 mel rows back; the stream waits for two."""
    cfg, man, enc = _model(ctx, fa, chunk=chunk)
    mel = fa.synth.make_features(cfg["melBins"], sum(pieces), seed=6)[0]
    off = enc.encode([mel])[0]
    got = _stream(ctx, fa, enc, mel, pieces)
    enc.close()
    assert got.shape == off.shape, (got.shape, off.shape)
    ref = npref.encode(cfg, man, [mel])
    d = float(np.abs(got - off).max() / np.abs(off).max())
    print(f"pieces {pieces[:4]}...: stream vs fused offline max rel {d:.2e}; stream vs np_ref rel-L2 {rel_l2(got, ref):.2e}")
    assert d < 2e-3
    assert rel_l2(got, ref) <= 1e-2


def test_stream_graph_replay_equals_eager(ctx, fa, monkeypatch):
    """Steady-state passes (full key cache) run from two captured graphs
    (the caches are double-buffered); bits equal the eager passes'."""
    cfg, man, enc = _model(ctx, fa)
    mel = fa.synth.make_features(cfg["melBins"], 1200, seed=8)[0]
    graphed = _stream(ctx, fa, enc, mel, [16] * 75)
    monkeypatch.setenv("FA_GRAPH", "0")
    eager = _stream(ctx, fa, enc, mel, [16] * 75)
    enc.close()
    assert np.array_equal(graphed, eager)


def test_right_context_error_shrinks_with_lookahead(ctx, fa):
    cfg, man, enc = _model(ctx, fa, right=3, chunk=4)
    mel = fa.synth.make_features(cfg["melBins"], 400, seed=7)[0]
    off = enc.encode([mel])[0]
    errs = []
    for B in (1, 2, 4):
        got = _stream(ctx, fa, enc, mel, [50] * 8, lookahead=B)
        assert got.shape == off.shape
        errs.append(float(np.abs(got - off).max() / np.abs(off).max()))
    enc.close()
    print("right context 3: provisional-tail error by lookahead 1/2/4:", errs)
    assert errs[2] < errs[0], errs


def test_stream_errors(ctx, fa):
    cfg, man, enc = _model(ctx, fa)
    pcfg = fa.synth.small_stream_cfg(layers=1)
    plain = fa.FusedEncoder(ctx, fa.synth.make_weights(pcfg, seed=1), "f16", max_T=64,
                            cfg={k: v for k, v in pcfg.items() if k not in ("attChunk", "convCausal")})
    with pytest.raises(fa.FaError):
        fa.createEncodeStream(ctx, plain)
    plain.close()
    st = fa.createEncodeStream(ctx, enc)
    fa.encodeStreamFlush(ctx, st)
    with pytest.raises(fa.FaError, match="flushed"):
        fa.encodeStreamPush(ctx, st, np.zeros((cfg["melBins"], 8), np.float32))
    fa.disposeEncodeStream(ctx, st)
    cfg_r, _, enc_r = _model(ctx, fa, right=3, chunk=4)
    with pytest.raises(fa.FaError):
        fa.createEncodeStream(ctx, enc_r, lookaheadChunks=0)
    enc_r.close()
    enc.close()


@pytest.mark.parametrize("graph", ["1", "0"])
@pytest.mark.parametrize("aligned", [False, True])
def test_streams_pushed_together_equal_streams_pushed_alone(ctx, fa, monkeypatch, graph, aligned):
    """fa_stream_push_many: four streams of one encoder, each with its own mel,
    pushed together give every stream the bits of pushing it alone.  Aligned:
    every stream gets the same piece pattern, so each push runs one batched
    pass of all four (window w = stream w, caches from the device table);
    otherwise each has its own pattern (different pass counts and shapes per
    call, one ends long before the others), so passes group only when their
    shapes and cached-key counts meet and the rest run as separate passes on
    the lanes.  A repeated stream and a flushed stream in one call are
    refused."""
    monkeypatch.setenv("FA_GRAPH", graph)
    cfg, man, enc = _model(ctx, fa)
    if aligned:
        mels = [fa.synth.make_features(cfg["melBins"], 608, seed=40 + i)[0] for i in range(4)]
        patterns = [[16] * 38] * 4
    else:
        mels = [fa.synth.make_features(cfg["melBins"], n, seed=30 + i)[0] for i, n in enumerate((600, 480, 200, 640))]
        patterns = [[16] * 38, [37, 100, 5, 64, 95, 179], [8] * 25, [24] * 27]
    alone = [_stream(ctx, fa, enc, m, p) for m, p in zip(mels, patterns)]
    sts = [fa.createEncodeStream(ctx, enc) for _ in mels]
    got = [[] for _ in mels]
    pos = [0] * len(mels)
    for step in range(max(len(p) for p in patterns)):
        live = [i for i, p in enumerate(patterns) if step < len(p)]
        blocks = []
        for i in live:
            n = patterns[i][step]
            blocks.append(mels[i][:, pos[i]:pos[i] + n])
            pos[i] += n
        for i, o in zip(live, fa.encodeStreamsPush(ctx, [sts[i] for i in live], blocks)):
            if o is not None:
                got[i].append(o)
        for i in range(len(mels)):
            if step == len(patterns[i]) - 1:
                o = fa.encodeStreamFlush(ctx, sts[i])
                if o is not None:
                    got[i].append(o)
    for i, (g, a) in enumerate(zip(got, alone)):
        g = np.concatenate(g, 0)
        assert g.shape == a.shape, (i, g.shape, a.shape)
        assert np.array_equal(g, a), f"stream {i}: max diff {np.abs(g - a).max()}"
    fresh = fa.createEncodeStream(ctx, enc)
    with pytest.raises(fa.FaError, match="repeats"):
        fa.encodeStreamsPush(ctx, [fresh, fresh], [mels[0][:, :8]] * 2)
    with pytest.raises(fa.FaError, match="flushed"):
        fa.encodeStreamsPush(ctx, [fresh, sts[1]], [mels[0][:, :8], mels[1][:, :8]])
    fa.disposeEncodeStream(ctx, fresh)
    for st in sts:
        fa.disposeEncodeStream(ctx, st)
    enc.close()


def test_sixteen_streams_pushed_together_track_streams_pushed_alone(ctx, fa, monkeypatch):
    """Sixteen aligned streams: every push is one batched pass of 32 rows, whose
    GEMMs with N <= 2048 split K over four workgroups per 16 columns (a
    second launch adds the partial tiles), so the sums are ordered unlike the
    solo passes': each stream stays within the stream-vs-offline bar of its
    solo frames, and the batched run is deterministic (a second run gives
    the same bits, and eager passes give the captured passes' bits)."""
    cfg, man, enc = _model(ctx, fa)
    mels = [fa.synth.make_features(cfg["melBins"], 304, seed=60 + i)[0] for i in range(16)]
    alone = [_stream(ctx, fa, enc, m, [16] * 19) for m in mels]

    def together():
        sts = [fa.createEncodeStream(ctx, enc) for _ in mels]
        got = [[] for _ in mels]
        for t in range(0, 304, 16):
            for i, o in enumerate(fa.encodeStreamsPush(ctx, sts, [m[:, t:t + 16] for m in mels])):
                if o is not None:
                    got[i].append(o)
        for i, st in enumerate(sts):
            o = fa.encodeStreamFlush(ctx, st)
            if o is not None:
                got[i].append(o)
            fa.disposeEncodeStream(ctx, st)
        return [np.concatenate(g, 0) for g in got]

    g1, g2 = together(), together()
    monkeypatch.setenv("FA_GRAPH", "0")
    g3 = together()
    for i, (a, b, c, e) in enumerate(zip(alone, g1, g2, g3)):
        assert a.shape == b.shape
        assert np.array_equal(b, c), f"stream {i}: batched runs differ"
        assert np.array_equal(b, e), f"stream {i}: eager passes differ from captured ones"
        d = float(np.abs(b - a).max() / np.abs(a).max())
        assert d < 2e-3, f"stream {i}: max rel {d:.2e}"
    enc.close()


def test_sixteen_streams_at_full_width_track_streams_pushed_alone(ctx, fa):
    """The split-K skinny GEMMs at this path's widths (d_model 1024, FF 4096,
    8 heads; two layers): in 32-row batched passes the out-projection, pw2
    (K 1024, N 1024), pw1 (N 2048) and FF W2 (K 4096) all split K; every
    stream stays within the stream-vs-offline bar of its solo frames."""
    cfg = dict(fa.synth.small_stream_cfg(layers=2), D=1024, DFF=4096, H=8)
    man = fa.synth.make_weights(cfg, seed=12)
    enc = fa.FusedEncoder(ctx, man, "f16", max_T=128, cfg=cfg)
    mels = [fa.synth.make_features(cfg["melBins"], 160, seed=80 + i)[0] for i in range(16)]
    alone = [_stream(ctx, fa, enc, m, [16] * 10) for m in mels]
    sts = [fa.createEncodeStream(ctx, enc) for _ in mels]
    got = [[] for _ in mels]
    for t in range(0, 160, 16):
        for i, o in enumerate(fa.encodeStreamsPush(ctx, sts, [m[:, t:t + 16] for m in mels])):
            if o is not None:
                got[i].append(o)
    for i, st in enumerate(sts):
        o = fa.encodeStreamFlush(ctx, st)
        if o is not None:
            got[i].append(o)
        fa.disposeEncodeStream(ctx, st)
    for i, (a, g) in enumerate(zip(alone, got)):
        g = np.concatenate(g, 0)
        assert g.shape == a.shape
        d = float(np.abs(g - a).max() / np.abs(a).max())
        assert d < 2e-3, f"stream {i}: max rel {d:.2e}"
    enc.close()


@pytest.mark.parametrize("exact", [False, True])
def test_layernorm_folded_into_skinny_gemms_matches_separate_launches(ctx, fa, monkeypatch, exact):
    """Stream passes fold norm_att / norm_conv / norm_ff2 into the skinny GEMMs
    that consume them (the A rows normalised in the kernel with the
    LayerNorm kernel's own sums and expression): the streamed frames match
    the separate LayerNorm launches (FA_LN_FOLD=0) to f16-rounding noise --
    the compiler rounds the LayerNorm kernel's outputs to f16 partly with a
    single-rounding mixed fma, so the two differ in a few last f16 bits --
    also with every operand exact (the folded GEMM then builds the lo plane
    too)."""
    cfg = fa.synth.small_stream_cfg(layers=2, right=0, chunk=2, left=8)
    cfg = dict(cfg, D=1024, DFF=4096, H=8, HD=128)  # the fold needs K = D = 1024
    man = fa.synth.make_weights(cfg, seed=13)
    enc = fa.FusedEncoder(ctx, man, "f16", max_T=128, cfg=cfg)
    if exact:
        enc.setExact(31)
    mel = fa.synth.make_features(cfg["melBins"], 320, seed=14)[0]
    outs = []
    for fold in ("1", "0"):
        monkeypatch.setenv("FA_LN_FOLD", fold)
        outs.append(_stream(ctx, fa, enc, mel, [16] * 20))
    enc.close()
    assert outs[0].shape == outs[1].shape
    r = rel_l2(outs[0], outs[1])
    print(f"folded vs separate LayerNorm: rel-L2 {r:.2e}, max |diff| {np.abs(outs[0] - outs[1]).max():.2e}")
    assert r < 2e-5, r


def test_split_k_skinny_gemms_match_single_workgroup_route(ctx, fa, monkeypatch):
    """The split-K skinny route (32-row batched passes, K of every GEMM with
    N <= 2048 split over four workgroups and summed in split order) against
    the single-workgroup route at the same rows (FA_SKINNY_SPLIT=0), at this
    path's widths: the two differ only in the f32 summation order, so the
    frames agree to rel-L2 1e-4 (an f32 difference can move an f16 rounding
    of a later operand by one ulp; the stream-vs-offline bar is 2e-3)."""
    cfg = dict(fa.synth.small_stream_cfg(layers=2), D=1024, DFF=4096, H=8)
    man = fa.synth.make_weights(cfg, seed=13)
    enc = fa.FusedEncoder(ctx, man, "f16", max_T=128, cfg=cfg)
    mels = [fa.synth.make_features(cfg["melBins"], 96, seed=120 + i)[0] for i in range(16)]

    def run():
        sts = [fa.createEncodeStream(ctx, enc) for _ in mels]
        got = [[] for _ in mels]
        for t in range(0, 96, 16):
            for i, o in enumerate(fa.encodeStreamsPush(ctx, sts, [m[:, t:t + 16] for m in mels])):
                if o is not None:
                    got[i].append(o)
        for st in sts:
            fa.disposeEncodeStream(ctx, st)
        return [np.concatenate(g, 0) for g in got]

    split = run()
    monkeypatch.setenv("FA_SKINNY_SPLIT", "0")
    single = run()
    monkeypatch.delenv("FA_SKINNY_SPLIT")
    for i, (a, b) in enumerate(zip(single, split)):
        assert a.shape == b.shape and a.shape[0] > 0
        assert rel_l2(b, a) < 1e-4, f"stream {i}: rel-L2 {rel_l2(b, a):.2e}"
    assert any(not np.array_equal(a, b) for a, b in zip(single, split)), "the split route did not run"
    enc.close()
