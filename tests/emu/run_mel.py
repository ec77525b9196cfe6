"""Log-mel features with the kernel sources of mel.hip executed on the CPU
(tests/emu), through the package's HipContext, against the CPU oracle.  Run in
a process of its own with the emulated library and the ASan runtime:

    LD_PRELOAD=<asan runtime> FA_LIB_PATH=tests/emu/_build/libfa_emu.so \\
        python tests/emu/run_mel.py <case>

cases: "signals" (speech-like, noise, tone, quiet, silence; normalised and
raw), "stream" (overlapping ragged windows of one resident stream, short tails
included), "static" (fa_mel_windows_static on caller buffers against
fa_mel_windows: two calls in a row, another bin count, and back).  Prints one
JSON line: how many raw log-mel values are bit-identical to the oracle's and
the largest difference in ulps, the largest difference of the normalised
features, and whether the allocation-free entry equals the allocating one bit
for bit.
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
    rng = np.random.default_rng(31)
    case = sys.argv[1]
    ctx = fa.createContext("hip")
    out = {"case": case, "checks": 0, "bit_identical": True}

    out["raw_max_ulp"] = 0
    out["raw_same_frac"] = 1.0
    out["feat_max_abs"] = 0.0

    def check(got, ref, raw=False):
        out["checks"] += 1
        ref = np.asarray(ref, np.float32)
        if got.shape != ref.shape:
            out["bit_identical"] = False
            return
        if not np.array_equal(got.view(np.uint32), ref.view(np.uint32)):
            out["bit_identical"] = False
        if not got.size:
            return
        if raw:
            ulp = np.abs(got.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
            out["raw_max_ulp"] = max(out["raw_max_ulp"], int(ulp.max()))
            out["raw_same_frac"] = min(out["raw_same_frac"], float(np.mean(ulp == 0)))
        else:
            out["feat_max_abs"] = max(out["feat_max_abs"], float(np.abs(got.astype(np.float64) - ref).max()))

    if case == "signals":
        t = np.arange(16000 * 2) / 16000
        sig = {
            "speechy": (0.3 * np.sin(2 * np.pi * 180 * t + 3 * np.sin(2 * np.pi * 2 * t)) * (1 + np.sin(2 * np.pi * 3 * t))
                        + 0.02 * rng.standard_normal(t.size)).astype(np.float32),
            "noise": (rng.standard_normal(16000 + 77) * 0.1).astype(np.float32),
            "tone": np.sin(2 * np.pi * 1000 * t[:8000]).astype(np.float32),
            "quiet": (rng.standard_normal(4000) * 1e-4).astype(np.float32),
            "silence": np.zeros(4800, np.float32),
        }
        for a in sig.values():
            pcm = ctx.upload(a.reshape(1, -1), 1, len(a))
            for norm in (True, False):
                got = ctx.download(ctx.melWindows(pcm, [0], [len(a)], normalize=norm)).reshape(128, -1)
                check(got, orc.mel(a, normalize=norm), raw=not norm)
    elif case == "stream":
        stream = (rng.standard_normal(16000 * 12) * 0.1).astype(np.float32)
        starts = [0, 16000 * 5, 16000 * 9, 16000 * 11, 100, 16000 * 8]
        lens = [16000 * 6, 16000 * 4 - 5, 16000 * 3, 159, 333, 16000 * 2 + 1]
        pcm = ctx.upload(stream.reshape(1, -1), 1, len(stream))
        got = ctx.download(ctx.melWindows(pcm, starts, lens)).reshape(128, -1)
        out["columns"] = got.shape[1]
        col = 0
        for s, l in zip(starts, lens):
            check(got[:, col:col + l // 160], orc.mel(stream[s:s + l]))
            col += l // 160
    elif case == "static":
        L = fa._lib.lib()
        L.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        L.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        L.hipFree.argtypes = [C.c_void_p]
        nsamp = 16000 * 12
        pcm_h = (0.3 * np.sin(2 * np.pi * 220 * np.arange(nsamp) / 16000) + 0.05 * rng.standard_normal(nsamp)).astype(np.float32)
        pcm_d = C.c_void_p()
        L.hipMalloc(C.byref(pcm_d), pcm_h.nbytes)
        L.hipMemcpy(pcm_d, pcm_h.ctypes.data, pcm_h.nbytes, 1)
        pcm_t = ctx.upload(pcm_h.reshape(1, -1), 1, nsamp)
        cases = [([0, 40000, 80000, 5000], [48000, 48000, 48000, 20000], 128, 2.0 ** -24, 1),
                 ([1000, 30000], [16000, 7777], 128, 2.0 ** -24, 1),
                 ([0, 50000, 90000], [32000, 12345, 160], 80, 1e-10, 0),
                 ([300], [24000], 128, 2.0 ** -24, 1)]
        for starts, lens, nm, guard, norm in cases:
            cols = sum(l // 160 for l in lens)
            want = ctx.download(ctx.melWindows(pcm_t, starts, lens, nm, guard, bool(norm))).reshape(nm, cols)
            o = C.c_void_p()
            L.hipMalloc(C.byref(o), nm * cols * 4)
            st = np.ascontiguousarray(starts, np.int32)
            ln = np.ascontiguousarray(lens, np.int32)
            rc = L.fa_mel_windows_static(ctx._p, pcm_d, nsamp, st.ctypes.data_as(C.POINTER(C.c_int32)), ln.ctypes.data_as(C.POINTER(C.c_int32)),
                                         len(st), nm, C.c_double(guard), norm, o, cols)
            if rc != 0:
                raise SystemExit(f"static entry: {rc} {L.fa_last_error(ctx._p)}")
            got = np.empty((nm, cols), np.float32)
            L.hipMemcpy(got.ctypes.data, o, got.nbytes, 2)
            L.hipFree(o)
            check(got, want)
        L.hipFree(pcm_d)
    else:
        raise SystemExit(f"unknown case {case}")
    ctx.destroy()
    buf = C.create_string_buffer(1 << 14)
    C.CDLL(os.environ["FA_LIB_PATH"]).emu_findings(buf, len(buf))
    out["findings"] = [x for x in buf.value.decode().splitlines() if x]
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
