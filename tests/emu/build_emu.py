"""Build the CPU execution of the library's kernel sources (test
infrastructure): the sources of fluidaudio-web_amd/csrc compiled as host C++
against the HIP stand-in in tests/emu/include (kernels run as fibers,
emu_rt.cpp), with AddressSanitizer and UBSan, into
tests/emu/_build/libfa_emu<tag>.so, which the package's Python bindings load
through FA_LIB_PATH (C ABI entry points of sources left out are stubs
returning FA_E_UNSUPPORTED).

The sources and headers are used as they are, rewritten into
_build/tree<tag> in four places only: the inline-asm direct-to-LDS copies
(s_mov_b32 m0 + global_load_lds_dwordx4, from a vector address or a scalar
base plus a vector offset) become calls to the stand-in's emu::dma16, which
performs the same copy; an empty asm that pins registers is dropped;
`extern __shared__` arrays become the launch's dynamic LDS buffer; AMDGPU
occupancy attributes are dropped.  Any other inline asm stops the build.

    python tests/emu/build_emu.py [--tdt PATH]   # another decoder source

Every library source is compiled by default (about six minutes under the
sanitizers; an unchanged tree is reused); `sources` limits the build to some
of them, the entry points and internal functions of the others becoming
stubs.
"""
from __future__ import annotations

import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
CSRC = os.path.join(ROOT, "fluidaudio-web_amd", "csrc")
OUT = os.path.join(HERE, "_build")
CLANGXX = "/opt/rocm/llvm/bin/clang++"
FLAGS = ["-std=c++17", "-O1", "-g", "-fPIC", "-fno-omit-frame-pointer", "-ffp-contract=off", "-fsanitize=address,undefined",
         "-Wno-unused-command-line-argument", f"-I{os.path.join(HERE, 'include')}"]

ASM = re.compile(r'asm\s+volatile\s*\((?P<body>(?:[^;])*?)\)\s*;', re.S)


DYN_LDS = re.compile(r'extern\s+__shared__\s+(?:__attribute__\(\((?:[^()]|\([^()]*\))*\)\)\s+)?([A-Za-z_0-9:]+)\s+(\w+)\[\];')


def rewrite(src: str) -> str:
    """The three inline-asm forms the sources use, and dynamic LDS:
    direct-to-LDS copy from a vector address or from a scalar base plus a
    vector offset -> emu::dma16; an empty asm that pins registers -> nothing;
    `extern __shared__ T name[];` -> the launch's dynamic LDS buffer."""
    def sub(m):
        body = m.group("body")
        if "global_load_lds_dwordx4" in body and "s_mov_b32 m0" in body:
            v = re.findall(r'"v"\((.+?)\)', body)
            ss = re.findall(r'"s"\((.+?)\)', body)
            if len(v) == 1 and len(ss) == 1 and ", off" in body:
                return f"::emu::dma16({v[0]}, {ss[0]});"
            if len(v) == 1 and len(ss) == 2:
                return f"::emu::dma16((const char *)({ss[0]}) + (uint32_t)({v[0]}), {ss[1]});"
        if body.lstrip().startswith('""'):
            return ";"
        raise RuntimeError("inline asm the CPU build does not know: " + body[:120])
    src = ASM.sub(sub, src)
    # AMDGPU-only kernel attributes (occupancy hints)
    src = re.sub(r'__attribute__\(\(amdgpu_\w+\((?:[^()]|\([^()]*\))*\)\)\)', '', src)
    return DYN_LDS.sub(lambda m: f"{m.group(1)} *{m.group(2)} = ({m.group(1)} *)::emu::dyn_lds();", src)


def asan_runtime() -> str:
    r = subprocess.run([CLANGXX, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    return r.stdout.strip()


def _entry_points() -> list[str]:
    src = open(os.path.join(ROOT, "fluidaudio-web_amd", "_lib.py")).read()
    return re.findall(r'\("(fa_[a-z0-9_]+)",', src)


def _sources() -> list[str]:
    src = open(os.path.join(CSRC, "build.py")).read()
    return re.findall(r'"(\w+\.hip)"', src[src.index("SOURCES"):src.index("]", src.index("SOURCES"))])


def build(tdt_src: str | None = None, tag: str = "", sources: list[str] | None = None) -> str:
    """Rewrite the library's sources and headers into _build/tree<tag> (the
    include paths stay as they are), compile each source in `sources`
    (default: every library source) with tdt.hip replaced by `tdt_src` if
    given, and link libfa_emu<tag>.so."""
    from concurrent.futures import ThreadPoolExecutor
    tree = os.path.join(OUT, f"tree{tag}")
    tcsrc = os.path.join(tree, "fluidaudio-web_amd", "csrc")
    os.makedirs(tcsrc, exist_ok=True)
    os.makedirs(os.path.join(tree, "include"), exist_ok=True)
    for h in os.listdir(os.path.join(ROOT, "include")):
        with open(os.path.join(tree, "include", h), "w") as f:
            f.write(open(os.path.join(ROOT, "include", h)).read())
    for name in os.listdir(CSRC):
        if name.endswith((".hip", ".h")):
            path = tdt_src if (name == "tdt.hip" and tdt_src) else os.path.join(CSRC, name)
            with open(os.path.join(tcsrc, name), "w") as f:
                f.write(rewrite(open(path).read()))
    srcs = sources or _sources()
    lib = os.path.join(OUT, f"libfa_emu{tag}.so")
    # unchanged inputs (rewritten tree, stand-in, flags, source list): reuse
    import hashlib
    h = hashlib.sha256(repr((FLAGS, srcs)).encode())
    for d in (tcsrc, os.path.join(tree, "include"), os.path.join(HERE, "include", "hip")):
        for name in sorted(os.listdir(d)):
            if name.endswith((".hip", ".h")):
                h.update(name.encode() + open(os.path.join(d, name), "rb").read())
    h.update(open(os.path.join(HERE, "emu_rt.cpp"), "rb").read())
    stamp = lib + ".sha256"
    if os.path.exists(lib) and os.path.exists(stamp) and open(stamp).read() == h.hexdigest():
        return lib

    def one(name):
        obj = os.path.join(tree, name.replace(".hip", ".o"))
        r = subprocess.run([CLANGXX, *FLAGS, "-x", "c++", "-c", os.path.join(tcsrc, name), "-o", obj], capture_output=True, text=True)
        if r.returncode:
            raise RuntimeError(f"{name}:\n{r.stderr[-4000:]}")
        return obj

    with ThreadPoolExecutor(max_workers=8) as ex:
        objs = list(ex.map(one, srcs))
    rt = os.path.join(tree, "emu_rt.o")
    r = subprocess.run([CLANGXX, *FLAGS, "-c", os.path.join(HERE, "emu_rt.cpp"), "-o", rt], capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(r.stderr[-4000:])
    objs.append(rt)
    defined = set()
    for o in objs:
        nm = subprocess.run(["nm", "--defined-only", "-g", o], capture_output=True, text=True).stdout
        defined |= {ln.split()[-1] for ln in nm.splitlines() if ln.strip()}
    undefined = set()
    for o in objs:
        nm = subprocess.run(["nm", "--undefined-only", o], capture_output=True, text=True).stdout
        undefined |= {ln.split()[-1] for ln in nm.splitlines() if ln.strip()}
    stubs = os.path.join(tree, "stubs.c")
    with open(stubs, "w") as f:
        f.write("/* entry points outside the compiled sources: FA_E_UNSUPPORTED */\n")
        for n in _entry_points():
            if n not in defined:
                f.write(f"int {n}(void) {{ return 5; }}\n")
        # internal functions of sources left out that these call: no-ops
        # returning 0
        for i, n in enumerate(sorted(x for x in undefined - defined if x.startswith("_ZN2fa"))):
            f.write(f'int emu_stub_{i}(void) __asm__("{n}");\nint emu_stub_{i}(void) {{ return 0; }}\n')
    so = stubs.replace(".c", ".o")
    r = subprocess.run(["gcc", "-O1", "-fPIC", "-c", stubs, "-o", so], capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(r.stderr)
    r = subprocess.run([CLANGXX, "-shared", "-fPIC", "-shared-libsan", "-fsanitize=address,undefined", "-o", lib, *objs, so],
                       capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(r.stderr[-4000:])
    with open(stamp, "w") as f:
        f.write(h.hexdigest())
    return lib


if __name__ == "__main__":
    path = sys.argv[sys.argv.index("--tdt") + 1] if "--tdt" in sys.argv else None
    print(build(path, "_alt" if path else ""))
