"""The decoder's and the log-mel front end's kernel sources executed on the CPU
(tests/emu): runtime.hip, tdt.hip and mel.hip compiled as host C++ against a
HIP stand-in whose launches run every workgroup's threads as fibers (barriers and wave operations wait for the
threads that take part), device memory malloc'd at its exact size, the whole
build under AddressSanitizer and UBSan.  The package's own TdtDecoder drives it
through FA_LIB_PATH, and each window's token ids and frame indices must equal
the CPU oracle's (the GPU tests' bar), with no sanitizer report and no finding
of the stand-in (buffer loads past their resource, readfirstlane of values
that differ between lanes).  The log-mel features are held to the GPU
tests' bar: raw log-mel >= 99.9 % bit-identical and within 1 ulp of the
oracle (its libm may round a log differently in the last bit), normalised
features within 1e-5, and the allocation-free entry point bit-identical to
the allocating one.

The same run covers the removed two-windows-per-wave joint kernel, which made
an illegal memory access on the GPU at 40 windows: executed from source at 40
windows it stays inside every buffer and matches the oracle, so that fault was
not an indexing error in its source.  CPU only."""
from __future__ import annotations

import json
import os
import shutil
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
EMU = os.path.join(HERE, "emu")
sys.path.insert(0, EMU)


@pytest.fixture(scope="module")
def emu():
    import build_emu
    rt = build_emu.asan_runtime()
    if not os.path.exists(rt) or not shutil.which("gcc"):
        pytest.skip("clang ASan runtime or gcc not available")
    if not os.path.exists(os.path.join(os.path.dirname(HERE), "oracle", "liboracle.so")):
        pytest.skip("oracle not built (run __graft_entry__.build())")
    import joint_two_windows
    os.makedirs(build_emu.OUT, exist_ok=True)
    variant = os.path.join(build_emu.OUT, "tdt_joint_two_windows.hip")
    with open(variant, "w") as f:
        f.write(joint_two_windows.variant_source())
    srcs = ["runtime.hip", "tdt.hip", "mel.hip"]
    return {"shipped": build_emu.build(tag="_dec", sources=srcs), "two_windows": build_emu.build(variant, "_alt", srcs), "rt": rt}


def run(emu, lib, case, script="run_tdt.py"):
    env = dict(os.environ, FA_LIB_PATH=emu[lib], LD_PRELOAD=emu["rt"], ASAN_OPTIONS="detect_leaks=0:detect_stack_use_after_return=0")
    r = subprocess.run([sys.executable, os.path.join(EMU, script), case], env=env, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-4000:]
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-4000:]
    return json.loads(r.stdout.strip().splitlines()[-1])


@pytest.mark.parametrize("case", ["known", "batch", "ragged40"])
def test_decoder_kernel_sources_match_the_oracle_on_the_cpu(emu, case):
    r = run(emu, "shipped", case)
    assert all(r["equal"]) and r["findings"] == [], r
    assert r["tokens"] > 10


def test_two_windows_per_wave_joint_stays_in_bounds_at_40_windows(emu):
    r = run(emu, "two_windows", "ragged40")
    assert r["windows"] == 40 and all(r["equal"]) and r["findings"] == [], r


@pytest.mark.parametrize("case", ["signals", "stream"])
def test_log_mel_kernel_sources_match_the_oracle_on_the_cpu(emu, case):
    r = run(emu, "shipped", case, "run_mel.py")
    assert r["findings"] == [], r
    assert r["raw_same_frac"] >= 0.999 and r["raw_max_ulp"] <= 1 and r["feat_max_abs"] <= 1e-5, r


def test_allocation_free_log_mel_equals_the_allocating_entry_on_the_cpu(emu):
    r = run(emu, "shipped", "static", "run_mel.py")
    assert r["checks"] == 4 and r["bit_identical"] and r["findings"] == [], r

