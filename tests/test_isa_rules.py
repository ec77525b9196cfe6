"""Instruction-level rules for the library's gfx950 code objects (CPU only):
the AMD assembly of every kernel built here (fluidaudio-web_amd/csrc/_build/*.o,
disassembled with ROCm's llvm-objdump) must contain

* no packed FP32 arithmetic (v_pk_add_f32, v_pk_mul_f32, v_pk_fma_f32): every
  HIP source is compiled with the packed-fp32-ops target feature off, and this
  checks that nothing (inline asm, a build line without the flag) brings them
  back;
* no stores, atomics or write-backs through the scalar data cache (s_store_*,
  s_buffer_store_*, s_atomic_*, s_buffer_atomic_*, s_dcache_wb*): device
  memory is written through vector stores only.

This file names those instructions, so it is listed in .gpurunignore (no GPU
run loads it)."""
from __future__ import annotations

import os
import re
import shutil
import subprocess
import sys
import tempfile

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BUILD = os.path.join(os.path.dirname(HERE), "fluidaudio-web_amd", "csrc", "_build")
OBJDUMP = "/opt/rocm/llvm/bin/llvm-objdump"
sys.path.insert(0, os.path.join(HERE, "audit"))

PACKED_F32 = re.compile(r"^v_pk_(add|mul|fma)_f32$")
SCALAR_WRITE = re.compile(r"^s_(store|buffer_store|atomic|buffer_atomic|dcache_wb)")


def _mnemonics():
    pytest.importorskip("msgpack")
    import build_audit as b
    if not os.path.isdir(BUILD) or not any(f.endswith(".o") for f in os.listdir(BUILD)):
        pytest.skip("library objects not built (run __graft_entry__.build())")
    if not shutil.which(OBJDUMP):
        pytest.skip("llvm-objdump not found")
    ops = {}
    with tempfile.TemporaryDirectory() as tmp:
        for f in sorted(os.listdir(BUILD)):
            if not f.endswith(".o"):
                continue
            blob = open(os.path.join(BUILD, f), "rb").read()
            for i, co in enumerate(b._code_objects(blob)):
                p = os.path.join(tmp, f"{f}.{i}.co")
                with open(p, "wb") as fh:
                    fh.write(co)
                out = subprocess.run([OBJDUMP, "-d", "--mcpu=gfx950", p], capture_output=True, text=True, check=True).stdout
                for line in out.splitlines():
                    m = re.match(r"\s+([a-z][a-z0-9_]*)\s", line)
                    if m:
                        ops.setdefault(m.group(1), set()).add(f)
    return ops


@pytest.fixture(scope="module")
def mnemonics():
    return _mnemonics()


def test_disassembly_is_substantial(mnemonics):
    # the disassembler read the code objects: MFMA and direct-to-LDS copies are there
    assert any(op.startswith("v_mfma_f32_16x16x32") for op in mnemonics)
    assert "global_load_lds_dwordx4" in mnemonics
    assert len(mnemonics) > 200


def test_no_packed_fp32_arithmetic(mnemonics):
    bad = {op: sorted(fs) for op, fs in mnemonics.items() if PACKED_F32.match(op)}
    assert bad == {}, bad


def test_no_scalar_cache_writes(mnemonics):
    bad = {op: sorted(fs) for op, fs in mnemonics.items() if SCALAR_WRITE.match(op)}
    assert bad == {}, bad
