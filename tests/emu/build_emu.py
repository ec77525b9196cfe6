"""Build the CPU execution of the decoder and log-mel kernel sources (test
infrastructure): fluidaudio-web_amd/csrc/runtime.hip, tdt.hip and mel.hip compiled as
host C++ against the HIP stand-in in tests/emu/include (kernels run as fibers,
emu_rt.cpp), with AddressSanitizer and UBSan, into
tests/emu/_build/libfa_emu.so.  The library's C ABI entry points that these
sources do not define are stubs returning FA_E_UNSUPPORTED, so the
package's Python bindings load it through FA_LIB_PATH.

The sources are used as they are, with one rewrite: the inline-asm
direct-to-LDS copy (s_mov_b32 m0 + global_load_lds_dwordx4) becomes a call to
the stand-in's emu::dma16, which performs the same copy.  Any other inline asm
stops the build.

    python tests/emu/build_emu.py [--tdt PATH]   # another decoder source
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
         "-Wno-unused-command-line-argument", f"-I{os.path.join(HERE, 'include')}", f"-I{CSRC}"]

ASM = re.compile(r'asm\s+volatile\s*\((?P<body>(?:[^;])*?)\)\s*;', re.S)


def rewrite(src: str) -> str:
    def sub(m):
        body = m.group("body")
        if "global_load_lds_dwordx4" in body and "s_mov_b32 m0" in body:
            v = re.search(r'"v"\((.+?)\)', body)
            s = re.search(r'"s"\((.+?)\)', body)
            if v and s:
                return f"::emu::dma16({v.group(1)}, {s.group(1)});"
        raise RuntimeError("inline asm the CPU build does not know: " + body[:120])
    return ASM.sub(sub, src)


def asan_runtime() -> str:
    r = subprocess.run([CLANGXX, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    return r.stdout.strip()


def _entry_points() -> list[str]:
    src = open(os.path.join(ROOT, "fluidaudio-web_amd", "_lib.py")).read()
    return re.findall(r'\("(fa_[a-z0-9_]+)",', src)


def build(tdt_src: str | None = None, tag: str = "") -> str:
    os.makedirs(OUT, exist_ok=True)
    objs = []
    srcs = [("runtime.hip", os.path.join(CSRC, "runtime.hip")), ("tdt.hip", tdt_src or os.path.join(CSRC, "tdt.hip")),
            ("mel.hip", os.path.join(CSRC, "mel.hip"))]
    for name, path in srcs:
        cpp = os.path.join(OUT, name.replace(".hip", f"{tag}.cpp"))
        with open(cpp, "w") as f:
            f.write(rewrite(open(path).read()))
        obj = cpp.replace(".cpp", ".o")
        r = subprocess.run([CLANGXX, *FLAGS, "-c", cpp, "-o", obj], capture_output=True, text=True)
        if r.returncode:
            raise RuntimeError(f"{name}:\n{r.stderr[-4000:]}")
        objs.append(obj)
    rt = os.path.join(OUT, "emu_rt.o")
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
    stubs = os.path.join(OUT, f"stubs{tag}.c")
    with open(stubs, "w") as f:
        f.write("/* entry points outside the compiled sources: FA_E_UNSUPPORTED */\n")
        for n in _entry_points():
            if n not in defined:
                f.write(f"int {n}(void) {{ return 5; }}\n")
        # internal functions of the other sources that these call: no-ops
        # returning 0
        for i, n in enumerate(sorted(x for x in undefined - defined if x.startswith("_ZN2fa"))):
            f.write(f'int emu_stub_{i}(void) __asm__("{n}");\nint emu_stub_{i}(void) {{ return 0; }}\n')
    so = stubs.replace(".c", ".o")
    r = subprocess.run(["gcc", "-O1", "-fPIC", "-c", stubs, "-o", so], capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(r.stderr)
    lib = os.path.join(OUT, f"libfa_emu{tag}.so")
    r = subprocess.run([CLANGXX, "-shared", "-fPIC", "-shared-libsan", "-fsanitize=address,undefined", "-o", lib, *objs, so],
                       capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(r.stderr[-4000:])
    return lib


if __name__ == "__main__":
    path = sys.argv[sys.argv.index("--tdt") + 1] if "--tdt" in sys.argv else None
    print(build(path, "_alt" if path else ""))
