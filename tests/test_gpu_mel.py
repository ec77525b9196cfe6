"""Log-mel front end on the GPU (fa_mel_windows, the features in front of the
encoder) vs the CPU oracle's restatement of the reference's JsPreprocessor
(nemotron-mel.js:451-603, Parakeet settings parakeet-mel.js:8-22).  Both run
the same f64 operation sequence with host-computed constants, so outputs agree
bit for bit except where the device log rounds differently from the host's in
the last f64 bit and that flips the f32 rounding of a raw log-mel value (then
that one row's mean and std move).  Bar: raw log-mel >= 99.9 % bit-identical
and within 1 f32 ulp; normalised features bit-identical in every row whose raw
row is, and within 1e-5 everywhere."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
rng = np.random.default_rng(31)


def signals():
    t = np.arange(16000 * 4) / 16000
    speechy = 0.3 * np.sin(2 * np.pi * 180 * t + 3 * np.sin(2 * np.pi * 2 * t)) * (1 + np.sin(2 * np.pi * 3 * t)) + 0.02 * rng.standard_normal(t.size)
    return {
        "speechy": speechy.astype(np.float32),
        "noise": (rng.standard_normal(16000 * 2 + 77) * 0.1).astype(np.float32),
        "tone": np.sin(2 * np.pi * 1000 * t[:16000]).astype(np.float32),
        "quiet": (rng.standard_normal(8000) * 1e-4).astype(np.float32),
        "silence": np.zeros(4800, np.float32),
    }


def agree(got, ref, atol):
    assert got.shape == ref.shape
    same = np.mean(got.view(np.uint32) == ref.view(np.uint32)) if got.size else 1.0
    err = float(np.abs(got.astype(np.float64) - ref).max()) if got.size else 0.0
    return same, err


@pytest.mark.parametrize("name", ["speechy", "noise", "tone", "quiet", "silence"])
def test_single_window_matches_oracle(ctx, fa, orc, name):
    a = signals()[name]
    pcm = ctx.upload(a.reshape(1, -1), 1, len(a))
    got = ctx.download(ctx.melWindows(pcm, [0], [len(a)])).reshape(128, -1)
    ref = orc.mel(a)
    same, err = agree(got, ref, 1e-5)
    raw = ctx.download(ctx.melWindows(pcm, [0], [len(a)], normalize=False)).reshape(128, -1)
    rref = orc.mel(a, normalize=False)
    rsame, _ = agree(raw, rref, 0)
    ulp = np.abs(raw.view(np.int32).astype(np.int64) - rref.view(np.int32).astype(np.int64)).max()
    print(f"{name}: features {same:.5f} bit-identical, max |diff| {err:.2e}; raw log-mel {rsame:.5f} bit-identical, max {ulp} ulp")
    assert rsame >= 0.999 and ulp <= 1
    assert err <= 1e-5
    # a row's normalised features are bit-identical wherever its raw log-mel
    # row is (a 1-ulp raw difference moves only its own row's mean / std)
    rows_same = np.all(raw.view(np.uint32) == rref.view(np.uint32), axis=1)
    assert np.array_equal(got[rows_same].view(np.uint32), ref[rows_same].view(np.uint32))


def test_stream_windows_match_per_window_oracle(ctx, fa, orc):
    """Overlapping ragged windows of one resident stream (the pipeline's
    15 s / 13 s-hop cut, plus short tails): each window's columns equal its
    standalone oracle features; windows under 160 samples add no column."""
    stream = (rng.standard_normal(16000 * 40) * 0.1).astype(np.float32)
    starts = [0, 16000 * 13, 16000 * 26, 16000 * 39, 100, 16000 * 30]
    lens = [16000 * 15, 16000 * 14 - 5, 16000 * 14, 159, 333, 16000 * 2 + 1]
    pcm = ctx.upload(stream.reshape(1, -1), 1, len(stream))
    out = ctx.download(ctx.melWindows(pcm, starts, lens)).reshape(128, -1)
    assert out.shape[1] == sum(l // 160 for l in lens)
    col = 0
    for s, l in zip(starts, lens):
        ref = orc.mel(stream[s:s + l])
        got = out[:, col:col + l // 160]
        same, err = agree(got, ref, 1e-5)
        assert same >= 0.99 and err <= 1e-5, (s, l, same, err)
        col += l // 160


def test_process_matches_reference_contract(ctx, fa, orc):
    a = signals()["speechy"][:16000 * 2 + 50]
    r = fa.ParakeetMel(ctx).process(a)
    assert r["length"] == len(a) // 160 and r["features"].shape == (128 * r["length"],)
    assert np.abs(r["features"].reshape(128, -1) - orc.mel(a)).max() <= 1e-5
    assert fa.ParakeetMel(ctx).process(np.zeros(100, np.float32))["length"] == 0
    one = fa.ParakeetMel(ctx).process(rng.standard_normal(250).astype(np.float32))
    assert one["length"] == 1 and np.all(one["features"] == 0)
    nem = fa.JsPreprocessor(ctx, nMels=80).process(a)  # Nemotron: raw log-mel, guard 1e-10
    ref = orc.mel(a, nmels=80, log_guard=1e-10, normalize=False)
    assert np.abs(nem["features"].reshape(80, -1) - ref).max() <= 1e-5 * np.abs(ref).max()


def test_mel_validation(ctx, fa):
    pcm = ctx.upload(np.zeros((1, 1000), np.float32), 1, 1000)
    with pytest.raises(fa.FaError):
        ctx.melWindows(pcm, [0], [2000])
    with pytest.raises(fa.FaError):
        ctx.melWindows(pcm, [0], [1000], nMels=129)
    with pytest.raises(fa.FaError):
        ctx.melWindows(pcm, [-1], [10])


def test_pcm_to_encoder_equals_oracle_features(ctx, fa, orc):
    """PCM -> GPU mel -> packWindows -> fused encoder gives the encoder's
    output on the oracle's features (same windows) to within the encoder's
    own run-to-run bits."""
    cfg = dict(D=256, DFF=1024, H=2, HD=128, layers=2, dwK=9, Csub=64, Fsub=16, melBins=128)
    man = fa.synth.make_weights(cfg, seed=1)
    stream = (rng.standard_normal(16000 * 9) * 0.1).astype(np.float32)
    starts, lens = [0, 16000 * 4], [16000 * 5, 16000 * 5 - 37]
    pcm = ctx.upload(stream.reshape(1, -1), 1, len(stream))
    feats = ctx.melWindows(pcm, starts, lens)
    T = [l // 160 for l in lens]
    enc = fa.FusedEncoder(ctx, man, "f16", max_T=64)
    a = ctx.pushArena()
    y = ctx.download(enc.forward(ctx.packWindows(feats, [0, T[0]], T), T))
    ctx.popArena(a)
    ref = np.concatenate(enc.encode([orc.mel(stream[s:s + l]) for s, l in zip(starts, lens)]))
    enc.close()
    assert y.reshape(ref.shape).shape == ref.shape
    assert np.abs(y.reshape(ref.shape) - ref).max() < 1e-3
