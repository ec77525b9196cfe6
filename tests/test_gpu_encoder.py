"""Fused encoder (fa_encoder_forward) parity against the CPU oracle's
restatement of parakeetEncodeBatch, on reduced dims the oracle finishes in
seconds.  Bar: rel-L2 <= 1e-2 vs the fp32 path, and
frame-wise argmax of a fixed random projection R [D, 64] ~ N(0,1) (seed 2)
identical on >= 99.9% of frames."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SMALL = dict(D=256, DFF=1024, H=2, HD=128, layers=2, dwK=9, Csub=64, Fsub=16, melBins=128)


def rel_l2(a, b):
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def argmax_agree(a, b, D, seed=2):
    R = np.random.default_rng(seed).standard_normal((D, 64)).astype(np.float32)
    return float(np.mean(np.argmax(a @ R, 1) == np.argmax(b @ R, 1)))


@pytest.fixture(scope="module")
def small(fa):
    return fa.synth.make_weights(SMALL, seed=1)


def test_fused_single_window(ctx, fa, orc, small):
    mel = fa.synth.make_features(128, 300, seed=4)
    enc = fa.FusedEncoder(ctx, small, "f16", max_T=128)
    got = enc.encode(mel)[0]
    ref = orc.encode_batch(SMALL, small, mel)
    assert got.shape == ref.shape
    assert rel_l2(got, ref) <= 1e-2
    enc.close()


def test_fused_batch_equals_oracle_batch(ctx, fa, orc, small):
    mels = fa.synth.make_features(128, 200, seed=5, W=3)
    enc = fa.FusedEncoder(ctx, small, "f16", max_T=128)
    got = np.concatenate(enc.encode(mels))
    ref = orc.encode_batch(SMALL, small, mels)
    assert rel_l2(got, ref) <= 1e-2
    assert argmax_agree(got, ref, SMALL["D"]) >= 0.999
    enc.close()


@pytest.mark.parametrize("layout", ["packed", "padded"])
def test_ragged_windows_equal_standalone(ctx, fa, small, layout):
    """Each window of a ragged batch equals its standalone encode (the
    W-vs-1 equivalence of scripts/parakeet-profile.mjs:67-79, maxΔ < 1e-4 there)."""
    lens = [333, 80, 257, 401, 9]
    mels = [fa.synth.make_features(128, t, seed=10 + i)[0] for i, t in enumerate(lens)]
    enc = fa.FusedEncoder(ctx, small, "f16", max_T=128)
    batch = enc.encode(mels, layout=layout)
    for m, g in zip(mels, batch):
        alone = enc.encode([m])[0]
        assert g.shape == alone.shape == (fa.tsub(m.shape[1]), SMALL["D"])
        assert np.abs(g - alone).max() < 1e-4
    enc.close()


@pytest.mark.parametrize("fmt,tol", [("int8", 2e-2), ("int4", 1e-1)])
def test_quantized_encoder_tracks_f16(ctx, fa, small, fmt, tol):
    mels = fa.synth.make_features(128, 240, seed=6, W=2)
    e16 = fa.FusedEncoder(ctx, small, "f16", max_T=128)
    eq = fa.FusedEncoder(ctx, small, fmt, max_T=128)
    a = np.concatenate(e16.encode(mels))
    b = np.concatenate(eq.encode(mels))
    assert rel_l2(b, a) <= tol
    e16.close()
    eq.close()


def test_graph_replay_equals_eager(ctx, fa, small, monkeypatch):
    """The captured forward (hipGraph, replayed per signature) must give the
    eager forward's bits on every replay, with eager library work and
    synchronisations between replays, for two signatures in turn."""
    enc = fa.FusedEncoder(ctx, small, "f16", max_T=128)
    sets = [fa.synth.make_features(128, 300, seed=7, W=3), fa.synth.make_features(128, 177, seed=8, W=2)]
    monkeypatch.setenv("FA_GRAPH", "0")
    eager = [enc.encode(m) for m in sets]
    monkeypatch.setenv("FA_GRAPH", "1")
    feats = []
    for m in sets:  # resident inputs so the signature (tensor addresses) repeats
        lens = [x.shape[1] for x in m]
        stream = np.concatenate(m, axis=1)
        f = ctx.upload(stream, stream.shape[0], stream.shape[1])
        starts = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int32)
        feats.append((f, starts, np.asarray(lens, np.int32), ctx.packWindows(f, starts, lens, "packed")))
    a = np.ones((64, 64), np.float32)
    for rep in range(3):
        for (f, starts, lens, packed), ref in zip(feats, eager):
            y = enc.forward(packed, lens, "packed")
            got = ctx.download(y).reshape(y.rows, y.cols)
            ctx.freeTensor(y)
            want = np.concatenate(ref)
            assert np.array_equal(got, want), f"replay {rep}: max diff {np.abs(got - want).max()}"
            ctx.download(ctx.matmul(ctx.upload(a, 64, 64), ctx.upload(a, 64, 64)))  # eager work in between
            ctx.sync()
    enc.close()


@pytest.mark.parametrize("cfg", ["auto", "1", "2", "3", "4", "5"])
@pytest.mark.parametrize("fmt", ["int8", "int4"])
def test_quantized_direct_to_lds_route_matches_staged_route(ctx, fa, small, monkeypatch, fmt, cfg):
    """Quantised weights through the direct-to-LDS GEMM (each tile
    configuration pinned in turn; a pin whose tile width does not divide N
    falls back to the automatic choice) give the register-staged dequant
    route's bits.  int8: raw int8 tiles widened exactly to f16 after the LDS
    read, column scale in the epilogue.  int4 group-32: raw nibble tiles,
    block scales loaded a K tile ahead, (q - 8) * s rounded once to f16.  Both
    routes accumulate the same f16 products over the same K order in f32."""
    mels = fa.synth.make_features(128, 300, seed=9 if fmt == "int8" else 10, W=2)
    eq = fa.FusedEncoder(ctx, small, fmt, max_T=128)
    eq.setExact(0)  # single-plane operands: the register-staged route has no lo plane
    monkeypatch.setenv("FA_GRAPH", "0")
    if cfg != "auto":
        monkeypatch.setenv("FA_GEMM_DMA", cfg)
    fast = np.concatenate(eq.encode(mels))
    monkeypatch.setenv("FA_GEMM_DMA", "0")
    staged = np.concatenate(eq.encode(mels))
    eq.close()
    assert np.array_equal(fast, staged), float(np.abs(fast - staged).max())


def test_front_end_lds_mel_rows_match_global_taps(ctx, fa, small, monkeypatch):
    """The front end's c0/c1 kernel reading its 7 mel rows per output row from
    LDS (zero-padded in time and by one bin each side) gives the bits of the
    per-tap global loads with explicit bounds checks: ragged windows whose
    lengths leave partial first and last c0 rows, and a 1-frame window."""
    mels = [fa.synth.make_features(128, t, seed=80 + i)[0] for i, t in enumerate((1500, 777, 1001, 9, 1))]
    monkeypatch.setenv("FA_C01_LDS", "0")
    ref_enc = fa.FusedEncoder(ctx, small, "f16", max_T=188)
    monkeypatch.delenv("FA_C01_LDS")
    enc = fa.FusedEncoder(ctx, small, "f16", max_T=188)
    want, got = ref_enc.encode(mels), enc.encode(mels)
    enc.close()
    ref_enc.close()
    assert all(np.array_equal(g, w) for g, w in zip(got, want))


@pytest.mark.parametrize("layout", ["packed", "padded"])
def test_transposed_v_epilogue_matches_v_transpose(ctx, fa, small, monkeypatch, layout):
    """The q|k|v GEMM writing V straight into the attention's transposed
    [window][head][d][key] buffer (through the row map the front end's last
    kernel writes) gives the bits of the separate v_transpose pass: same f16
    values, same attention.  Ragged windows ending mid-tile, graph replay and
    eager runs, every operand plane (the two-plane q|k|v route included), and
    a second, smaller batch over the same buffers (keys past a window's end
    then hold the first batch's values, which the attention weights by 0)."""
    big = [fa.synth.make_features(128, t, seed=60 + i)[0] for i, t in enumerate((1500, 777, 1001))]
    little = [fa.synth.make_features(128, t, seed=70 + i)[0] for i, t in enumerate((403, 911))]
    monkeypatch.setenv("FA_VT_FUSE", "0")
    ref_enc = fa.FusedEncoder(ctx, small, "f16", max_T=188)
    monkeypatch.delenv("FA_VT_FUSE")
    enc = fa.FusedEncoder(ctx, small, "f16", max_T=188)
    for mask in (None, 31):
        if mask is not None:
            ref_enc.setExact(mask)
            enc.setExact(mask)
        for mels in (big, little, big):
            want = ref_enc.encode(mels, layout)
            for graph in ("1", "0"):
                monkeypatch.setenv("FA_GRAPH", graph)
                got = enc.encode(mels, layout)
                assert all(np.array_equal(g, w) for g, w in zip(got, want)), (mask, graph, [t.shape for t in got])
            monkeypatch.delenv("FA_GRAPH")
    enc.close()
    ref_enc.close()


def test_attention_workgroup_shapes_agree(ctx, fa, small, monkeypatch):
    """The two rel-pos attention workgroup shapes (default: 96 queries as 6
    waves x 1 row tile; FA_ATTN=1: 128 queries as 4 waves x 2 row tiles) give
    the same encoder output up to f16 rounding (their lazy softmax rescaling
    points differ), on ragged windows that end mid-tile in both shapes."""
    mels = [fa.synth.make_features(128, t, seed=40 + i)[0] for i, t in enumerate((1500, 777, 1001))]
    monkeypatch.setenv("FA_GRAPH", "0")
    enc = fa.FusedEncoder(ctx, small, "f16", max_T=188)
    a = np.concatenate(enc.encode(mels))
    monkeypatch.setenv("FA_ATTN", "1")
    b = np.concatenate(enc.encode(mels))
    enc.close()
    assert rel_l2(a, b) < 2e-3, rel_l2(a, b)


@pytest.mark.parametrize("lds", ["1", "0"])
@pytest.mark.parametrize("layout", ["packed", "padded"])
def test_forward_stream_equals_pack_then_forward(ctx, fa, small, monkeypatch, layout, lds):
    """Windows read in place from the channel-major feature stream
    (fa_encoder_forward_stream) give the bits of fa_pack_windows followed by
    fa_encoder_forward: overlapping windows, one ending on the stream's last
    frame, a 1-frame window, ragged first / last c0 rows; the front end's LDS
    mel staging and its per-tap global loads; eager and graph replays, the
    replays moving the same window lengths to other starts (the captured
    forward reads the starts from device memory refreshed per call)."""
    monkeypatch.setenv("FA_C01_LDS", lds)
    enc = fa.FusedEncoder(ctx, small, "f16", max_T=188)
    T = 4000
    stream = fa.synth.make_features(128, T, seed=90)[0]
    f = ctx.upload(stream, 128, T)
    lens = np.array([1500, 777, 1, 1001, 9], np.int32)
    for rep, starts in enumerate(([0, 700, 3999, T - 1001, 13], [5, 0, 17, 2999, 3991], [2500, 1200, 0, 1, 3000])):
        starts = np.asarray(starts, np.int32)
        for graph in ("0", "1"):
            monkeypatch.setenv("FA_GRAPH", graph)
            y0 = enc.forward(ctx.packWindows(f, starts, lens, layout), lens, layout)
            y1 = enc.forwardStream(f, starts, lens, layout)
            a = ctx.download(y0).reshape(y0.rows, y0.cols)
            b = ctx.download(y1).reshape(y1.rows, y1.cols)
            assert a.shape == b.shape
            assert np.array_equal(a, b), f"starts set {rep}, graph {graph}: max diff {np.abs(a - b).max()}"
    ctx.freeTensor(f)
    enc.close()


def test_forward_stream_rejects_windows_outside_the_stream(ctx, fa, small):
    enc = fa.FusedEncoder(ctx, small, "f16", max_T=64)
    f = ctx.upload(np.zeros((128, 100), np.float32), 128, 100)
    for starts, lens in (([0, 90], [50, 11]), ([-1], [10]), ([0], [101])):
        with pytest.raises(Exception, match="outside the 100-frame stream"):
            enc.forwardStream(f, starts, lens)
    with pytest.raises(Exception, match="features must be f32"):
        enc.forwardStream(ctx.upload(np.zeros((64, 100), np.float32), 64, 100), [0], [50])
    ctx.freeTensor(f)
    enc.close()


@pytest.mark.parametrize("graph", ["1", "0"])
def test_forward_stream_batches_equal_one_batch_at_a_time(ctx, fa, small, monkeypatch, graph):
    """fa_encoder_forward_stream_batches (consecutive batches on two workspace
    lanes with streams of their own) gives every batch the bits of
    fa_encoder_forward_stream: five ragged batches of different window counts
    (so the two lanes hold different workspace sizes and captured forwards),
    called twice in a row (graph replays on the lanes), then a single-batch
    call and a plain forward on the context stream reading the same buffers'
    lane 0 afterwards."""
    monkeypatch.setenv("FA_GRAPH", graph)
    enc = fa.FusedEncoder(ctx, small, "f16", max_T=188)
    T = 6000
    stream = fa.synth.make_features(128, T, seed=91)[0]
    f = ctx.upload(stream, 128, T)
    rng = np.random.default_rng(5)
    batches = []
    for n in (3, 1, 5, 2, 4):
        lens = rng.integers(1, 1501, n).astype(np.int32)
        starts = np.array([rng.integers(0, T - l + 1) for l in lens], np.int32)
        batches.append((starts, lens))
    want = []
    for st, ln in batches:
        y = enc.forwardStream(f, st, ln)
        want.append(ctx.download(y).reshape(y.rows, y.cols))
    for call in range(2):
        outs = enc.forwardStreamBatches(f, batches)
        assert len(outs) == len(batches)
        for b, (y, w) in enumerate(zip(outs, want)):
            got = ctx.download(y).reshape(y.rows, y.cols)
            assert got.shape == w.shape
            assert np.array_equal(got, w), f"call {call}, batch {b}: max diff {np.abs(got - w).max()}"
    one = enc.forwardStreamBatches(f, batches[2:3])[0]
    assert np.array_equal(ctx.download(one).reshape(one.rows, one.cols), want[2])
    y = enc.forwardStream(f, *batches[4])
    assert np.array_equal(ctx.download(y).reshape(y.rows, y.cols), want[4])
    with pytest.raises(Exception, match="no batches|windows"):
        enc.forwardStreamBatches(f, [(np.array([], np.int32), np.array([], np.int32))])
    # a failing later batch releases the batches already encoded: repeated
    # failing calls create no new buffers
    # (inside an arena, where outputs come from the buffer pool)
    bad = [batches[0], (np.array([T - 5], np.int32), np.array([10], np.int32))]
    arena = ctx.pushArena()
    with pytest.raises(Exception, match="outside"):
        enc.forwardStreamBatches(f, bad)
    ctx.memStatsStart()
    for _ in range(3):
        with pytest.raises(Exception, match="outside"):
            enc.forwardStreamBatches(f, bad)
    assert ctx.memStats()["created"] == 0
    ctx.popArena(arena)
    ctx.freeTensor(f)
    enc.close()


def test_op_path_attn_fused_member_matches_op_chain(ctx, fa):
    """parakeetEncodeBatch with the reference's opt-in attnFused member
    (raw-encoder.js:334) against the bmmQK / relShiftB / softmax / bmmPV
    chain, fp32 weights, two layers, two windows (the positional projection
    cached per layer across the two calls)."""
    cfg = dict(D=256, DFF=1024, H=2, HD=128, layers=2, dwK=9, Csub=64, Fsub=16, melBins=128)
    man = fa.synth.make_weights(cfg, seed=4)
    enc = fa.loadParakeetEncoder(ctx, man, weights="f32")
    mels = fa.synth.make_features(128, 400, seed=5, W=2)
    outs = []
    for fused in (False, True):
        a = ctx.pushArena()
        y, T = fa.parakeetEncodeBatch(ctx, enc, mels, attnFused=fused)
        outs.append(ctx.download(y).reshape(-1, 256))
        ctx.popArena(a)
    d = float(np.linalg.norm(outs[1] - outs[0]) / np.linalg.norm(outs[0]))
    print(f"op path: attnFused vs op chain rel-L2 {d:.2e}")
    assert d < 1e-4
