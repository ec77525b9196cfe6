"""Build libfa_hip.so (gfx950) in-tree with hipcc.

    python fluidaudio-web_amd/csrc/build.py

Every source is compiled for gfx950 only, with packed-fp32 instruction
selection disabled, and linked into one shared library next to the package
(fluidaudio-web_amd/libfa_hip.so) so it travels with the source tree.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
OUT = os.path.join(PKG, "libfa_hip.so")
SOURCES = ["runtime.hip", "gemm.hip", "gemm_q8.hip", "gemm_q4.hip", "attention.hip", "ops.hip", "quant.hip", "encoder.hip", "pack.hip", "mel.hip", "tdt.hip", "ops_aux.hip", "stream.hip", "transcribe.hip"]
# per-source flags: the log-mel and TDT-decoder kernels restate the
# reference's JS / wasm arithmetic, so no multiply-add may be fused there
EXTRA = {"mel.hip": ["-ffp-contract=off"], "tdt.hip": ["-ffp-contract=off"], "ops_aux.hip": ["-ffp-contract=off"]}
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-result",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _compile(src: str) -> str:
    obj = os.path.join(HERE, "_build", src.replace(".hip", ".o"))
    cmd = [HIPCC, *FLAGS, *EXTRA.get(src, []), "-c", os.path.join(HERE, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    msgs = [l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l]
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n" + "\n".join(msgs))
    if msgs:
        print("\n".join(msgs), file=sys.stderr)
    return obj


def build(jobs: int = 8) -> str:
    os.makedirs(os.path.join(HERE, "_build"), exist_ok=True)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = OUT + ".tmp"
    r = subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, OUT)
    build_node_addon()
    return OUT


NODE_INC = "/usr/include/node"


def build_node_addon() -> str | None:
    """The N-API addon (fluidaudio-web_amd/node/fa_hip.node) over libfa_hip.so,
    when Node's headers are installed (gcc only: N-API is a C interface)."""
    if not os.path.exists(os.path.join(NODE_INC, "node_api.h")):
        return None
    ndir = os.path.join(PKG, "node")
    out = os.path.join(ndir, "fa_hip.node")
    cmd = ["gcc", "-O2", "-Wall", "-shared", "-fPIC", f"-I{NODE_INC}", os.path.join(ndir, "fa_napi.c"), "-o", out,
           f"-L{PKG}", "-l:libfa_hip.so", "-Wl,-rpath,$ORIGIN/.."]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("N-API addon build failed:\n" + r.stdout + r.stderr)
    return out


if __name__ == "__main__":
    print(build())
