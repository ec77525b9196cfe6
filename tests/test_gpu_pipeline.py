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
