"""Pins of the CPU log-mel oracle (oracle/fa_oracle.c `or_mel*`, restating
src/engines/asr-nemotron/nemotron-mel.js with Parakeet's settings from
src/engines/asr-parakeet/parakeet-mel.js:8-22) against independent
computations: numpy's FFT (a different algorithm from the reference's radix-2
transform), numpy's Hann window, torchaudio's melscale_fbanks definition
(slaney scale and norm) written vectorised, and closed-form properties.  The
reference holds no mel fixture; the reference's own mel tests need model
files that are absent here."""
import numpy as np
import pytest

rng = np.random.default_rng(21)


def np_slaney_fbanks(nmels):
    """torchaudio.functional.melscale_fbanks(257, 0, 8000, nmels, 16000,
    norm="slaney", mel_scale="slaney"), transposed to [nmels, 257]."""
    def hz2mel(f):
        f = np.asarray(f, np.float64)
        lin = f / (200.0 / 3)
        return np.where(f >= 1000.0, 15.0 + np.log(np.maximum(f, 1e-30) / 1000.0) / (np.log(6.4) / 27.0), lin)

    def mel2hz(m):
        m = np.asarray(m, np.float64)
        return np.where(m >= 15.0, 1000.0 * np.exp(np.log(6.4) / 27.0 * (m - 15.0)), m * (200.0 / 3))

    freqs = np.linspace(0, 8000, 257)
    fpts = mel2hz(np.linspace(hz2mel(0.0), hz2mel(8000.0), nmels + 2))
    fdiff = np.diff(fpts)
    slopes = fpts[None, :] - freqs[:, None]
    down = -slopes[:, :-2] / fdiff[:-1]
    up = slopes[:, 2:] / fdiff[1:]
    fb = np.maximum(0, np.minimum(down, up)) * (2.0 / (fpts[2:] - fpts[:-2]))
    return fb.T


def np_mel(audio, nmels=128, guard=2.0 ** -24, normalize=True):
    """The NeMo preprocessor pipeline with numpy's real FFT."""
    a = audio.astype(np.float64)
    x = np.empty_like(a)
    x[0] = a[0]
    x[1:] = (a[1:] - 0.97 * a[:-1]).astype(np.float32)
    T = len(a) // 160
    p = np.concatenate([np.zeros(256), x, np.zeros(256)])
    win = np.zeros(512)
    win[56:456] = np.hanning(400)
    frames = np.stack([p[t * 160:t * 160 + 512] * win for t in range(T)])
    power = (np.abs(np.fft.rfft(frames, axis=1)) ** 2).astype(np.float32).astype(np.float64)
    fb = np_slaney_fbanks(nmels).astype(np.float32).astype(np.float64)
    raw = np.log(power @ fb.T + guard).T.astype(np.float32).astype(np.float64)
    if not normalize:
        return raw
    mean = raw.mean(1, keepdims=True)
    std = raw.std(1, ddof=1, keepdims=True) if T > 1 else np.full_like(mean, np.inf)
    return (raw - mean) / (std + 1e-5)


def test_hann_and_twiddles(orc):
    w = orc.mel_hann()
    ref = np.zeros(512)
    ref[56:456] = np.hanning(400)
    assert np.abs(w - ref).max() < 1e-15
    c, s = orc.mel_twiddles(256)
    ang = -2 * np.pi * np.arange(128) / 256
    assert np.abs(c - np.cos(ang)).max() < 1e-15 and np.abs(s - np.sin(ang)).max() < 1e-15


def test_power_spectrum_matches_numpy_fft(orc):
    for _ in range(4):
        x = rng.standard_normal(512) * rng.uniform(0.01, 3)
        got = orc.mel_power(x).astype(np.float64)
        ref = np.abs(np.fft.rfft(x)) ** 2
        assert np.abs(got - ref).max() <= 1e-6 * ref.max()
    # a pure tone lands in its own bin; DC and Nyquist are real
    n = np.arange(512)
    for b in (0, 7, 128, 200, 256):
        p = orc.mel_power(np.cos(2 * np.pi * b * n / 512))
        assert int(np.argmax(p)) == b


@pytest.mark.parametrize("nmels", [128, 80])
def test_filterbank_is_torchaudio_slaney(orc, nmels):
    fb = orc.mel_filterbank(nmels)
    ref = np_slaney_fbanks(nmels)
    assert np.abs(fb - ref).max() < 1e-6 * ref.max()
    # slaney normalisation: each triangle has unit area in Hz (wide filters
    # integrate accurately on the 31.25 Hz bin grid)
    area = fb.sum(1) * (8000 / 256)
    assert np.all(np.abs(area[-(nmels // 4):] - 1) < 0.03)


def test_features_match_numpy_pipeline(orc):
    t = np.arange(16000 * 3) / 16000
    speechy = (0.3 * np.sin(2 * np.pi * 220 * t) * (1 + np.sin(2 * np.pi * 3 * t)) + 0.05 * rng.standard_normal(t.size)).astype(np.float32)
    for audio in (speechy, (rng.standard_normal(16000 * 2 + 77) * 0.2).astype(np.float32)):
        got = orc.mel(audio)
        ref = np_mel(audio)
        assert got.shape == ref.shape == (128, len(audio) // 160)
        assert np.abs(got - ref).max() < 2e-4
        raw = orc.mel(audio, normalize=False)
        assert np.abs(raw - np_mel(audio, normalize=False)).max() < 1e-4


def test_tone_peaks_in_its_mel_band(orc):
    fb = orc.mel_filterbank(128)
    centers = np.argmax(fb, axis=1) * 8000 / 256
    t = np.arange(16000) / 16000
    for f in (300.0, 1000.0, 4000.0):
        raw = orc.mel(np.sin(2 * np.pi * f * t).astype(np.float32), normalize=False)
        m = int(np.argmax(raw[:, 10:-10].mean(1)))
        assert abs(centers[m] - f) <= 2 * 8000 / 256 + 0.15 * f


def test_edge_lengths_and_silence(orc):
    assert orc.mel(np.zeros(159, np.float32)).shape == (128, 0)
    one = orc.mel(rng.standard_normal(200).astype(np.float32))
    assert one.shape == (128, 1) and np.all(one == 0)  # featuresLen 1: invStd 0
    z = orc.mel(np.zeros(4800, np.float32))
    assert np.all(z == 0)  # constant log-guard rows normalise to 0
    raw = orc.mel(np.zeros(4800, np.float32), normalize=False)
    assert np.all(raw == np.float32(np.log(2.0 ** -24)))
