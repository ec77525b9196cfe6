"""End-to-end windowed transcription on the GPU (pipeline.transcribeWindowed:
PCM -> mel -> encoder -> joint projection -> greedy TDT decode -> stitch).
The decode and stitch are exact restatements, so the bar is: the pipeline's
tokens equal the CPU oracle's decode of the pipeline's own projected frames,
stitched by the reference's rules; plus the reference gate's checks
(scripts/parakeet-pipeline-check.mjs: token times ordered within the overlap
and inside the clip)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def parts(ctx, fa):
    import importlib
    pl = importlib.import_module(fa.__name__ + ".pipeline")
    man = fa.synth.make_weights(fa.synth.PARAKEET_CFG, seed=3, layers=2)
    enc = fa.FusedEncoder(ctx, man, "f16", max_T=188)
    dec_w = fa.synth.make_decoder_weights(1)
    dec = fa.TdtDecoder(ctx, dec_w)
    W, b = fa.synth.make_joint_projection(2)
    projW, projB = ctx.upload(W, W.shape[0], W.shape[1]), ctx.upload(b.reshape(1, -1), 1, b.size)
    yield pl, enc, dec, dec_w, projW, projB
    dec.close()
    enc.close()


def test_pipeline_equals_oracle_decode_and_stitch(ctx, fa, orc, parts):
    pl, enc, dec, dec_w, projW, projB = parts
    audio = fa.synth.make_pcm(50.0, seed=4)  # windows 0, 13, 26, 39 s: 15, 15, 15, 11 s
    r = pl.transcribeWindowed(ctx, enc, dec, projW, projB, audio, keepFrames=True)
    assert r["stats"]["windows"] == 4 and r["stats"]["groups"] == 2
    ids, times, stitch = pl.createStitcher(208000, 16000, 32000)
    for w, f in enumerate(r["frames"]):
        wid, fr = orc.tdt_decode(dec_w, f)
        stitch(w, min(w * 208000 + 240000, len(audio)) - w * 208000, len(f), wid.tolist(), fr.tolist())
    assert r["ids"] == ids and r["idTimes"] == times
    assert len(ids) > 20
    t = r["idTimes"]
    assert all(t[i] >= t[i - 1] - 2.05 for i in range(1, len(t)))  # ordered within the 2 s overlap
    assert all(0 <= v <= 50.0 + 1 for v in t)


def test_group_size_does_not_change_tokens(ctx, fa, parts):
    """One window per group (wb=1) vs full groups: same tokens.  40 s gives
    windows at 0, 13, 26, 39 s (15, 15, 14, 1 s); the two short ones go alone."""
    pl, enc, dec, _, projW, projB = parts
    audio = fa.synth.make_pcm(40.0, seed=5)
    a = pl.transcribeWindowed(ctx, enc, dec, projW, projB, audio, wb=1)
    b = pl.transcribeWindowed(ctx, enc, dec, projW, projB, audio)
    assert a["stats"]["groups"] == 4 and b["stats"]["groups"] == 3
    assert a["ids"] == b["ids"]


def test_short_empty_and_tail_inputs(ctx, fa, orc, parts):
    pl, enc, dec, dec_w, projW, projB = parts
    short = fa.synth.make_pcm(6.0, seed=6)  # one window, the whole clip
    r = pl.transcribeWindowed(ctx, enc, dec, projW, projB, short, keepFrames=True)
    wid, _ = orc.tdt_decode(dec_w, r["frames"][0])
    assert r["stats"]["windows"] == 1 and r["ids"] == wid.tolist()
    assert pl.transcribeWindowed(ctx, enc, dec, projW, projB, np.zeros(0, np.float32))["ids"] == []
    assert pl.transcribeWindowed(ctx, enc, dec, projW, projB, short[:100])["ids"] == []  # no mel frame
    # a last window shorter than one hop contributes nothing
    tail = fa.synth.make_pcm(416080 / 16000, seed=7)  # windows of 240000, 208080 and 80 samples
    r = pl.transcribeWindowed(ctx, enc, dec, projW, projB, tail)
    assert r["stats"]["windows"] == 2


@pytest.mark.parametrize("wb,seconds", [(2, 120.0), (3, 100.0), (32, 470.0)])
def test_pipelined_equals_stage_by_stage(ctx, fa, parts, wb, seconds):
    """fa_transcribe_groups (group g+1's mel / encoder / projection on an
    encoder lane while group g decodes, two groups' buffers reused in turn)
    gives the tokens and times of the stage-by-stage calls, for odd and even
    group counts and a full 32-window group."""
    pl, enc, dec, _, projW, projB = parts
    audio = fa.synth.make_pcm(seconds, seed=8)
    a = pl.transcribeWindowed(ctx, enc, dec, projW, projB, audio, wb=wb, pipelined=False)
    b = pl.transcribeWindowed(ctx, enc, dec, projW, projB, audio, wb=wb, pipelined=True)
    assert a["stats"]["groups"] == b["stats"]["groups"] >= 2
    assert a["stats"]["windows"] == b["stats"]["windows"]
    assert a["ids"] == b["ids"] and a["idTimes"] == b["idTimes"]
    assert len(a["ids"]) > 10


def test_pipelined_rejects_bad_plans(ctx, fa, parts):
    import ctypes as C
    from importlib import import_module
    L = import_module(fa.__name__ + "._lib")
    pl, enc, dec, _, projW, projB = parts
    pcm = ctx.upload(np.zeros((1, 16000 * 20), np.float32), 1, 16000 * 20)
    I = L.I32P
    out = [np.zeros(64 * 16, np.int32) for _ in range(2)] + [np.zeros(64, np.int32) for _ in range(2)]

    def call(counts, starts, lens):
        c, s, l = (np.asarray(v, np.int32) for v in (counts, starts, lens))
        return L.lib().fa_transcribe_groups(ctx._p, enc._p, dec._p, pcm.h, len(c), c.ctypes.data_as(I), s.ctypes.data_as(I), l.ctypes.data_as(I),
                                            projW.h, projB.h, 128, C.c_double(2.0 ** -24), 1, 16, *[o.ctypes.data_as(I) for o in out])
    assert call([1], [0], [100]) == L.FA_E_INVALID            # no mel frame
    assert call([1], [0], [16000 * 21]) == L.FA_E_INVALID     # past the stream
    assert call([33], [0] * 33, [16000] * 33) == L.FA_E_INVALID  # more than 32 windows in a group
    assert call([1], [0], [16000]) == L.FA_OK
    ctx.freeTensor(pcm)
