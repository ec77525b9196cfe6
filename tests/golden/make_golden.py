"""Write the committed golden fixtures from the independent float64
restatement (oracle/np_ref.py: NeMo-style modules, torch library convs/LN,
pad-reshape rel_shift).  The C oracle (oracle/fa_oracle.c) is checked against
these in tests/test_oracle.py.

    python tests/golden/make_golden.py

Inputs are seeded synthetic data (no reference files are read or run).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, ROOT)
import np_ref  # noqa: E402
import __graft_entry__ as ge  # noqa: E402

synth = ge.load_package().synth


def main():
    cfg = dict(D=64, DFF=128, H=2, HD=32, layers=1, dwK=9, Csub=8, Fsub=4, melBins=32)
    man = synth.make_weights(cfg, seed=3, biases=True)
    mels = synth.make_features(cfg["melBins"], 61, seed=4, W=2)
    out = np_ref.encode(cfg, man, mels)
    arrays = {f"w_{k}": v for k, v in man.items()}
    arrays.update({"mel0": mels[0], "mel1": mels[1], "expected": out, "cfg": np.array([cfg[k] for k in
                   ("D", "DFF", "H", "HD", "layers", "dwK", "Csub", "Fsub", "melBins")], np.int64)})
    np.savez_compressed(os.path.join(HERE, "encoder_tiny.npz"), **arrays)
    # rel_shift known answer (NeMo pad -> reshape -> drop row -> crop)
    import torch
    rng = np.random.default_rng(7)
    x = rng.standard_normal((3 * 5, 9)).astype(np.float32)
    y = np_ref.rel_shift_nemo(torch.as_tensor(x, dtype=torch.float64).reshape(3, 5, 9)).reshape(15, 5).numpy()
    pe = np_ref.pos_encoding(7, 16).numpy()
    np.savez_compressed(os.path.join(HERE, "relpos.npz"), x=x, relshift=y, pe_T7_D16=pe)
    print("wrote", os.listdir(HERE))


if __name__ == "__main__":
    main()
