"""Greedy TDT decoding on the GPU (fa_tdt_decode, the step after the encoder)
vs the CPU oracle's restatement of rust/parakeet-decoder decode_proj.
Both compute the reference's f32 operation sequence (its polynomial expf,
lane-ordered dots, in-order joint sums; no fused multiply-add), so the bar is
identical token ids and frame indices for every window."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
H, L, V, BLANK = 640, 8198, 8193, 8192


@pytest.fixture(scope="module")
def dec_w(fa):
    return fa.synth.make_decoder_weights(1)


@pytest.fixture(scope="module")
def tdt(ctx, fa, dec_w):
    d = fa.TdtDecoder(ctx, dec_w)
    yield d
    d.close()


def test_batch_matches_oracle(ctx, fa, orc, dec_w, tdt):
    lens = [188, 120, 0, 97, 1]
    frames = [fa.synth.make_projected_frames(T, seed=50 + i) for i, T in enumerate(lens)]
    got = tdt.decodeBatch(frames)
    total = 0
    for i, f in enumerate(frames):
        ids, fr = orc.tdt_decode(dec_w, f) if len(f) else (np.zeros(0, np.int32), np.zeros(0, np.int32))
        assert got[i]["ids"] == ids.tolist() and got[i]["idFrames"] == fr.tolist(), i
        assert got[i]["count"] == len(ids)
        total += len(ids)
    print(f"{total} tokens over {sum(lens)} frames")
    assert total > 50


def test_device_frames_and_window_order(ctx, fa, orc, dec_w, tdt):
    """Frames already on the device (the encoder's projected output): window
    results do not depend on batch composition or order."""
    frames = [fa.synth.make_projected_frames(T, seed=70 + i) for i, T in enumerate((64, 150, 33))]
    host = np.concatenate(frames)
    t = ctx.upload(host, host.shape[0], H)
    a = tdt.decodeBatch(t, [64, 150, 33])
    b = tdt.decodeBatch([frames[2], frames[0]])
    assert a[2]["ids"] == b[0]["ids"] and a[0]["ids"] == b[1]["ids"]
    ids, fr = orc.tdt_decode(dec_w, frames[1])
    assert a[1]["ids"] == ids.tolist() and a[1]["idFrames"] == fr.tolist()


@pytest.mark.parametrize("token,dur", [(5, 0), (BLANK, 2), (7, 3)])
def test_known_answer_loops(ctx, fa, token, dur):
    w = fa.synth.make_decoder_weights(5)
    w["outW"] = np.zeros_like(w["outW"])
    ob = np.zeros(L, np.float32)
    ob[token] = 1.0
    ob[V + dur] = 1.0
    w["outB"] = ob
    d = fa.TdtDecoder(ctx, w)
    T = 23
    r = d.decodeBatch([np.zeros((T, H), np.float32)], cap=512)[0]
    d.close()
    if token == BLANK:
        assert r["ids"] == []
    elif dur == 0:
        assert r["ids"] == [token] * (10 * T) and r["idFrames"] == [t for t in range(T) for _ in range(10)]
    else:
        assert r["idFrames"] == list(range(0, T, dur)) and set(r["ids"]) == {token}


def test_capacity_and_validation(ctx, fa, orc, dec_w, tdt):
    f = fa.synth.make_projected_frames(100, seed=90)
    full = tdt.decodeBatch([f])[0]
    cut = tdt.decodeBatch([f], cap=5)[0]
    assert cut["count"] == full["count"] > 5 and cut["ids"] == full["ids"][:5]
    bad = ctx.upload(np.zeros((10, 100), np.float32), 10, 100)
    with pytest.raises(fa.FaError):
        tdt.decodeBatch(bad, [10])
    with pytest.raises(fa.FaError):
        tdt.decodeBatch(ctx.upload(np.zeros((10, H), np.float32), 10, H), [11])


def test_many_windows_match_oracle(ctx, fa, orc, dec_w, tdt):
    """More windows than one block's 16 window slots (several window groups per
    kernel, ragged lengths, empty windows): every window equals the oracle."""
    rng = np.random.default_rng(7)
    lens = [int(x) for x in rng.integers(1, 120, 40)]
    lens[3] = 0
    lens[17] = 188
    frames = [fa.synth.make_projected_frames(T, seed=300 + i) for i, T in enumerate(lens)]
    got = tdt.decodeBatch(frames)
    for i, f in enumerate(frames):
        ids, fr = orc.tdt_decode(dec_w, f) if len(f) else (np.zeros(0, np.int32), np.zeros(0, np.int32))
        assert got[i]["ids"] == ids.tolist() and got[i]["idFrames"] == fr.tolist(), (i, lens[i])


def test_full_batch_equals_small_batches(ctx, fa, tdt):
    """64 windows in one call (the maximum) = the same windows 8 at a time."""
    frames = [fa.synth.make_projected_frames(96, seed=500 + i) for i in range(64)]
    big = tdt.decodeBatch(frames)
    small = []
    for b in range(0, 64, 8):
        small += tdt.decodeBatch(frames[b:b + 8])
    for i in range(64):
        assert big[i]["ids"] == small[i]["ids"] and big[i]["idFrames"] == small[i]["idFrames"], i
