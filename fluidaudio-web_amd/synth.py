"""Synthetic encoder weights and features in the reference's manifest naming.

There is no network and no checkpoint, so every benchmark and parity test
runs on random-init weights of the real architecture.  Key names and shapes
are the manifest's (src/engines/asr-parakeet/raw-encoder.js:28-35,101-158):
  c{0..4}w / c{0..4}b      subsampling convs, [Cout, Cin/groups, kh, kw] flat
  linw [Csub*Fsub, D], linb [D]
  L{L}_{name}              per conformer layer; matrices are [in, out],
                           pw1 [2D, D, 1], pw2 [D, D, 1], dw [D, 1, K]
Parakeet has no linear biases (the optional *b keys are absent) and its
BatchNorm is folded into dw/dwb.

Distribution choices (documented build choices, seeded):
  - layer matrices ~ N(0, 0.02) rounded to f16-representable values, so the
    fp32 reference path and the f16-storage GPU path see identical weights;
  - LayerNorm gamma = 1 + N(0, 0.02), beta = N(0, 0.02); pos_bias_u/v, dw bias
    ~ N(0, 0.02);
  - depthwise k=9 weights ~ N(0, 1/3) (a unit-gain conv, like a folded BN);
  - subsampling convs use He-style std sqrt(2 / fan_in) so activations stay
    O(1) through the front end instead of decaying into f16 subnormals.
"""
from __future__ import annotations

import numpy as np

PARAKEET_CFG = dict(D=1024, DFF=4096, H=8, HD=128, layers=24, dwK=9, Csub=256, Fsub=16, melBins=128)


def tiny_stream_cfg(layers=2, right=0, chunk=2):
    """Small streaming (EOU-style) model: eou-parakeet/config.js's subsampling
    pads and options at reduced dims.  With subPad l=2, r=1 the frequency axis
    32 -> 17 -> 9 -> 5 gives Fsub 5 (not melBins / 8)."""
    return dict(D=64, DFF=256, H=2, HD=32, layers=layers, dwK=9, Csub=8, Fsub=5, melBins=32, subPad={"t": 2, "b": 1, "l": 2, "r": 1},
                convCausal=True, attChunk=chunk, attLeft=8, attRight=right)


def small_stream_cfg(layers=2, right=0, chunk=2, left=8):
    """Streaming (EOU-style) model at dims the fused encoder takes (HD 128):
    subPad t2 b1 l2 r1 takes 128 mel bins 128 -> 65 -> 33 -> 17 (Fsub 17)."""
    return dict(D=256, DFF=1024, H=2, HD=128, layers=layers, dwK=9, Csub=64, Fsub=17, melBins=128, subPad={"t": 2, "b": 1, "l": 2, "r": 1},
                convCausal=True, attChunk=chunk, attLeft=left, attRight=right)


def tiny_cfg(layers=2):
    """Small config for CPU cross-checks (same structure, reduced dims)."""
    return dict(D=64, DFF=256, H=2, HD=32, layers=layers, dwK=9, Csub=8, Fsub=4, melBins=32)


def _f16r(a: np.ndarray) -> np.ndarray:
    return a.astype(np.float16).astype(np.float32)


def make_weights(cfg: dict, seed: int = 1, layers: int | None = None, biases: bool = False) -> dict:
    """Random weights for `layers` layers (default cfg['layers']).  biases=True
    adds the optional linear biases (Sortformer-style), exercising those
    epilogue paths."""
    rng = np.random.default_rng(seed)
    D, DFF, H, HD, K, C, Fs = cfg["D"], cfg["DFF"], cfg["H"], cfg["HD"], cfg["dwK"], cfg["Csub"], cfg["Fsub"]
    layers = cfg["layers"] if layers is None else layers
    n = lambda shape, std: (rng.standard_normal(shape) * std).astype(np.float32)
    m = {}
    m["c0w"], m["c0b"] = _f16r(n((C, 1, 3, 3), np.sqrt(2 / 9))), n(C, 0.02)
    m["c1w"], m["c1b"] = _f16r(n((C, 1, 3, 3), np.sqrt(2 / 9))), n(C, 0.02)
    m["c2w"], m["c2b"] = _f16r(n((C, C, 1, 1), np.sqrt(2 / C))), n(C, 0.02)
    m["c3w"], m["c3b"] = _f16r(n((C, 1, 3, 3), np.sqrt(2 / 9))), n(C, 0.02)
    m["c4w"], m["c4b"] = _f16r(n((C, C, 1, 1), np.sqrt(2 / C))), n(C, 0.02)
    m["linw"], m["linb"] = _f16r(n((C * Fs, D), 0.02)), n(D, 0.02)
    for L in range(layers):
        g = lambda s: f"L{L}_{s}"
        for ln in ("lnff1", "lnatt", "lnconv", "lnff2", "lnout"):
            m[g(ln + "_w")] = (1 + n(D, 0.02)).astype(np.float32)
            m[g(ln + "_b")] = n(D, 0.02)
        m[g("ff1w1")], m[g("ff1w2")] = _f16r(n((D, DFF), 0.02)), _f16r(n((DFF, D), 0.02))
        m[g("ff2w1")], m[g("ff2w2")] = _f16r(n((D, DFF), 0.02)), _f16r(n((DFF, D), 0.02))
        for k in ("q", "k", "v", "pos", "out"):
            m[g(k)] = _f16r(n((D, D), 0.02))
        m[g("pbu")], m[g("pbv")] = n((H, HD), 0.02), n((H, HD), 0.02)
        m[g("pw1")] = _f16r(n((2 * D, D, 1), 0.02))
        m[g("pw2")] = _f16r(n((D, D, 1), 0.02))
        m[g("dw")] = _f16r(n((D, 1, K), np.sqrt(1 / 3)))
        m[g("dwb")] = n(D, 0.02)
        if cfg.get("convCausal"):  # streaming models normalise the depthwise output with a LayerNorm
            m[g("bnw")], m[g("bnb")] = (1 + n(D, 0.02)).astype(np.float32), n(D, 0.02)
        if biases:
            for k in ("ff1b1", "ff2b1", "pw1b"):
                m[g(k)] = n(DFF if k != "pw1b" else 2 * D, 0.02)
            for k in ("ff1b2", "ff2b2", "qb", "kb", "vb", "outb", "pw2b"):
                m[g(k)] = n(D, 0.02)
    return m


def make_features(melBins: int, T: int, seed: int = 1, W: int = 1) -> list:
    """W synthetic log-mel windows [melBins, T] ~ N(0, 1), channel-major like the
    reference's mel output (raw-encoder.js:224)."""
    rng = np.random.default_rng(seed)
    return [rng.standard_normal((melBins, T)).astype(np.float32) for _ in range(W)]


def make_decoder_weights(seed: int = 1, blank_bias: float = 4.5, hid: int = 640, vocab: int = 8193, ndur: int = 5) -> dict:
    """Synthetic Parakeet TDT decoder + joint weights in the reference's decoder
    manifest naming (src/engines/asr-parakeet/gpu-decoder.js:232-242;
    rust/parakeet-decoder/src/lib.rs:4-7): embed [vocab, hid], l{0,1}_W / _R
    [4*hid, hid] (gate rows i, o, f, c), l{0,1}_B [8*hid] (W bias, R bias),
    predW [hid, hid] (k-major), predB, outW [hid, vocab + ndur] (row n = hidden
    unit), outB.  Random-init weights emit a non-blank token on nearly every
    step; the blank logit is biased (and the duration logits favour one or two
    frames) so emission looks like speech: about one token per three frames."""
    rng = np.random.default_rng(seed)
    f = lambda *s, sc=1.0: (rng.standard_normal(s) * sc).astype(np.float32)  # noqa: E731
    w = {"embed": f(vocab, hid, sc=0.5)}
    for l in (0, 1):
        w[f"l{l}_W"] = f(4 * hid, hid, sc=1 / np.sqrt(hid))
        w[f"l{l}_R"] = f(4 * hid, hid, sc=1 / np.sqrt(hid))
        w[f"l{l}_B"] = f(8 * hid, sc=0.1)
    w["predW"] = f(hid, hid, sc=1 / np.sqrt(hid))
    w["predB"] = f(hid, sc=0.1)
    w["outW"] = f(hid, vocab + ndur, sc=0.06)
    ob = f(vocab + ndur, sc=0.1)
    ob[vocab - 1] += blank_bias
    ob[vocab:vocab + ndur] += np.array([0.0, 1.2, 0.9, 0.3, -0.5], np.float32)[:ndur]
    w["outB"] = ob
    return w


def make_projected_frames(T: int, seed: int = 1, hid: int = 640) -> np.ndarray:
    """Encoder frames after the joint's encoder projection, [T, hid] ~ N(0, 1)."""
    return np.random.default_rng(seed).standard_normal((T, hid)).astype(np.float32)


def make_pcm(seconds: float, seed: int = 1, sr: int = 16000) -> np.ndarray:
    """Speech-like synthetic mono audio: a gliding harmonic tone with syllable-
    rate amplitude modulation plus noise, f32 in [-1, 1]."""
    rng = np.random.default_rng(seed)
    n = int(round(seconds * sr))
    t = np.arange(n, dtype=np.float64) / sr
    f0 = 140 + 40 * np.sin(2 * np.pi * 0.3 * t)
    ph = 2 * np.pi * np.cumsum(f0) / sr
    env = 0.5 + 0.5 * np.sin(2 * np.pi * 3.7 * t) ** 2
    x = env * (0.25 * np.sin(ph) + 0.12 * np.sin(2 * ph) + 0.06 * np.sin(3 * ph)) + 0.02 * rng.standard_normal(n)
    return x.astype(np.float32)


def make_joint_projection(seed: int = 1, D: int = 1024, hid: int = 640) -> tuple:
    """The joint network's encoder projection (decoder manifest encW [D, hid],
    encB [hid]; pipeline.js:57-61), scaled so projected frames are O(1)."""
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((D, hid)) * (2.0 / np.sqrt(D))).astype(np.float32), (rng.standard_normal(hid) * 0.1).astype(np.float32)
