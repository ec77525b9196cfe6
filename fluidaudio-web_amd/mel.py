"""Log-mel front end on the GPU, mirroring the reference's preprocessor API.

    mel = ParakeetMel(ctx)                       # parakeet-mel.js:8-22
    r = mel.process(audio)                       # {"features": [128*T] f32, "length": T}
    feats = mel.processWindows(pcm, starts, lens)  # resident stream -> [128, Σ T_i] on the GPU

`process` has the reference's contract (src/engines/asr-parakeet/parakeet-mel.js:14-22:
mono 16 kHz PCM in, mel-major features of floor(len/160) frames out, length 0
for shorter input); the work runs in fa_mel_windows.  `processWindows` is the
batched form the encoder path uses: every window of a resident sample stream
in one call, output in the channel-major stream layout that
HipContext.packWindows cuts batches from.
"""
from __future__ import annotations

import numpy as np

PARAKEET_LOG_GUARD = 2.0 ** -24  # parakeet-mel.js:12
NEMOTRON_LOG_GUARD = 1e-10       # nemotron-mel.js:45 (raw log-mel, no normalisation)
HOP = 160


class JsPreprocessor:
    """nemotron-mel.js JsPreprocessor options: nMels, logGuard, and whether the
    per-feature normalisation runs (Parakeet) or the raw log-mel is returned
    (Nemotron)."""

    def __init__(self, ctx, nMels: int = 128, logGuard: float = NEMOTRON_LOG_GUARD, normalize: bool = False):
        self.ctx, self.nMels, self.logGuard, self.normalize = ctx, int(nMels), float(logGuard), bool(normalize)

    def processWindows(self, pcm, starts, lens):
        return self.ctx.melWindows(pcm, starts, lens, self.nMels, self.logGuard, self.normalize)

    def process(self, audio):
        a = np.ascontiguousarray(audio, np.float32).reshape(-1)
        T = len(a) // HOP
        if T == 0:
            return {"features": np.zeros(0, np.float32), "length": 0}
        pcm = self.ctx.upload(a.reshape(1, -1), 1, len(a))
        arena = self.ctx.pushArena()
        try:
            f = self.ctx.download(self.processWindows(pcm, [0], [len(a)]))
        finally:
            self.ctx.popArena(arena)
            self.ctx.freeTensor(pcm)
        return {"features": f.reshape(-1), "length": T}


class ParakeetMel(JsPreprocessor):
    """Parakeet's nemo128 front end: log guard 2^-24 and per-feature normalisation."""

    def __init__(self, ctx, nMels: int = 128):
        super().__init__(ctx, nMels, PARAKEET_LOG_GUARD, True)
