"""Host-side logic and the C ABI's shape, CPU only (no kernel launches)."""
import ctypes as C
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fa_hip.h")


def header_functions():
    src = open(HEADER).read()
    return sorted(set(re.findall(r"^(?:int|void|const char \*)\s*\*?(fa_[a-z0-9_]+)\(", src, re.M)))


def test_library_exports_every_header_symbol(fa):
    L = fa.lib()
    names = header_functions()
    assert len(names) >= 60
    for n in names:
        assert hasattr(L, n), n


def test_binding_table_covers_header_exactly(fa):
    from importlib import import_module

    lib_mod = import_module("fluidaudio_web_amd._lib")
    assert sorted(n for n, _, _ in lib_mod.SIGNATURES) == header_functions()


def test_version_and_pure_functions(fa, orc):
    assert fa.lib().fa_version().startswith(b"fa_hip")
    for T in (1, 5, 188, 1500, 2999):
        assert fa.tsub(T) == orc.tsub(T)


def test_no_gpu_fails_loudly(fa):
    n = C.c_int(0)
    try:
        import torch

        have = torch.cuda.device_count() > 0
    except Exception:
        have = False
    if have:
        pytest.skip("a GPU is visible")
    with pytest.raises(fa.FaError):
        fa.createContext("hip")
    with pytest.raises(ValueError):
        fa.createContext("wasm")


# ── windowing (src/engines/asr-parakeet/windowing.js:5-34) ────────────────
def test_plan_windows_known_answers(fa):
    W = fa.windowing
    sr = 16000
    win, hop = 15 * sr, 13 * sr
    assert W.planWindows(10 * sr, win, hop) == [0]                    # short input: one window
    assert W.planWindows(40 * sr, win, hop) == [0, 13 * sr, 26 * sr, 39 * sr]
    assert W.planWindows(0, win, hop) == []


def test_group_windows_known_answers(fa):
    W = fa.windowing
    sr = 16000
    win, hop = 15 * sr, 13 * sr
    total = 40 * sr  # windows: 15 s, 15 s, 14 s (tail), 1 s (tail)
    starts = W.planWindows(total, win, hop)
    assert W.groupWindows(starts, total, win, 6) == [[0, 1], [2], [3]]
    total = 13 * 9 * sr + 2 * sr  # ten windows, the last nine full... (hop 13 s)
    starts = W.planWindows(total, win, hop)
    g = W.groupWindows(starts, total, win, 6)
    assert sum(len(x) for x in g) == len(starts) and all(len(x) <= 6 for x in g)
    full = [i for i, s in enumerate(starts) if s + win <= total]
    assert g[0] == full[:6]


def test_ragged_plan_invariants(fa):
    starts, lens = fa.windowing.planRaggedWindows(360000, 200, 3000, 100, seed=1)
    assert starts[0] == 0 and starts[-1] + lens[-1] == 360000
    assert np.all(lens[:-1] >= 200) and np.all(lens <= 3000)
    assert np.all(starts[1:] == starts[:-1] + lens[:-1] - 100)  # 1 s overlap at a 10 ms hop
    batches = fa.windowing.packBatches(lens, 32)
    assert sorted(i for b in batches for i in b) == list(range(len(lens)))
    assert all(len(b) <= 32 for b in batches)


# ── synthetic weights / config inference (raw-encoder.js:28-35) ───────────
def test_infer_config_and_determinism(fa):
    cfg = fa.synth.tiny_cfg(2)
    m1 = fa.synth.make_weights(cfg, seed=11)
    m2 = fa.synth.make_weights(cfg, seed=11)
    assert all(np.array_equal(m1[k], m2[k]) for k in m1)
    assert fa.inferConfig(m1) == cfg
    assert all(np.array_equal(m1[k].astype(np.float16).astype(np.float32), m1[k]) for k in ("L0_q", "L1_ff2w1", "linw"))


def test_python_host_implements_every_required_member(fa):
    """The Python HipContext carries every required ComputeContext method
    (the list node/conformance.js checks the Node class against)."""
    import re

    src = open(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "fluidaudio-web_amd", "node", "conformance.js")).read()
    req = re.findall(r'"(\w+)"', src[src.index("const REQUIRED"):src.index("const OPTIONAL")])
    assert len(req) == 63
    missing = [m for m in req if not callable(getattr(fa.HipContext, m, None))]
    assert not missing, missing
