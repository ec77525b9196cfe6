"""Greedy TDT decode with the decoder's kernel sources executed on the CPU
(tests/emu), through the package's own TdtDecoder, against the CPU oracle.
Run in a process of its own with the emulated library and the ASan runtime:

    LD_PRELOAD=<asan runtime> FA_LIB_PATH=tests/emu/_build/libfa_emu.so \\
        python tests/emu/run_tdt.py <case>

cases: "batch" (5 windows of 0-12 frames), "ragged40" (40 windows of 1-6
frames: five joint workgroups of 8 window slots), "known" (a known-answer
loop: one token ten times per frame).  Prints one JSON line: per window
whether ids and frame indices equal the oracle's, token counts, and the
stand-in's findings.
"""
from __future__ import annotations

import ctypes as C
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))


def main():
    import __graft_entry__ as ge
    fa = ge.load_package()
    import oracle as orc
    case = sys.argv[1]
    ctx = fa.createContext("hip")
    w = fa.synth.make_decoder_weights(1)
    if case == "known":
        w["outW"] = np.zeros_like(w["outW"])
        ob = np.zeros(8198, np.float32)
        ob[5] = 1.0
        ob[8193] = 1.0
        w["outB"] = ob
        lens = [3]
    elif case == "batch":
        lens = [12, 7, 0, 9, 1]
    elif case == "ragged40":
        lens = [1 + (i * 7) % 6 for i in range(40)]
    else:
        raise SystemExit(f"unknown case {case}")
    frames = [np.zeros((T, 640), np.float32) if case == "known" else fa.synth.make_projected_frames(T, seed=50 + i) for i, T in enumerate(lens)]
    d = fa.TdtDecoder(ctx, w)
    got = d.decodeBatch(frames, cap=256)
    d.close()
    ctx.destroy()
    out = {"windows": len(lens), "equal": [], "tokens": 0}
    for i, f in enumerate(frames):
        ids, fr = orc.tdt_decode(w, f) if len(f) else (np.zeros(0, np.int32), np.zeros(0, np.int32))
        out["equal"].append(got[i]["ids"] == ids.tolist() and got[i]["idFrames"] == fr.tolist())
        out["tokens"] += len(ids)
    buf = C.create_string_buffer(1 << 14)
    lib = C.CDLL(os.environ["FA_LIB_PATH"])
    lib.emu_findings(buf, len(buf))
    out["findings"] = [x for x in buf.value.decode().splitlines() if x]
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
