"""Builds the launch-audit library: the product's own objects
(fluidaudio-web_amd/csrc/_build/*.o, written by build()) linked with the
host-only HIP stand-in in launch_audit.cpp instead of the HIP runtime, and the
table of every kernel's argument layout read from the gfx950 code objects
inside those objects (the AMDGPU metadata note: argument offsets, sizes and
kinds, maximum workgroup size, static LDS and scratch).

    python tests/audit/build_audit.py [--max-windows N] [--asan]

--max-windows recompiles encoder.hip with FA_ENC_MAX_WINDOWS=N for the audit
build only (the shipped library keeps its limit).  --asan compiles every
library source again with host-side AddressSanitizer and UBSan
(libfa_hip_audit_asan.so; the Python process preloads asan_runtime()).
Outputs go to tests/audit/_build/ (libfa_hip_audit.so, kernargs.txt).
"""
from __future__ import annotations

import os
import struct
import shutil
import subprocess
import sys

import msgpack

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
CSRC = os.path.join(ROOT, "fluidaudio-web_amd", "csrc")
OUT = os.path.join(HERE, "_build")
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def _code_objects(blob: bytes):
    """gfx950 code objects of every offload bundle in an object file."""
    pos = blob.find(MAGIC)
    while pos >= 0:
        n = struct.unpack_from("<Q", blob, pos + 24)[0]
        p = pos + 32
        for _ in range(n):
            off, size, tlen = struct.unpack_from("<QQQ", blob, p)
            triple = blob[p + 24:p + 24 + tlen].decode()
            p += 24 + tlen
            if "gfx950" in triple and size:
                yield blob[pos + off:pos + off + size]
        pos = blob.find(MAGIC, pos + 1)


def _metadata(elf: bytes) -> dict:
    """The NT_AMDGPU_METADATA note (msgpack) of an ELF64 code object."""
    shoff = struct.unpack_from("<Q", elf, 0x28)[0]
    shentsize, shnum = struct.unpack_from("<HH", elf, 0x3A)
    for i in range(shnum):
        sh = shoff + i * shentsize
        stype = struct.unpack_from("<I", elf, sh + 4)[0]
        if stype != 7:  # SHT_NOTE
            continue
        off, size = struct.unpack_from("<QQ", elf, sh + 0x18)
        p = off
        while p < off + size:
            namesz, descsz, ntype = struct.unpack_from("<III", elf, p)
            name = elf[p + 12:p + 12 + namesz]
            dpos = p + 12 + ((namesz + 3) & ~3)
            if ntype == 32 and name.startswith(b"AMDGPU"):
                return msgpack.unpackb(elf[dpos:dpos + descsz], raw=False, strict_map_key=False)
            p = dpos + ((descsz + 3) & ~3)
    return {}


def kernarg_table(objs) -> list[str]:
    lines = {}
    for o in objs:
        blob = open(o, "rb").read()
        for co in _code_objects(blob):
            for k in _metadata(co).get("amdhsa.kernels", []):
                args = k.get(".args", [])
                fields = [k[".name"], str(k.get(".max_flat_workgroup_size", 1024)), str(k.get(".group_segment_fixed_size", 0)),
                          str(k.get(".private_segment_fixed_size", 0)), str(len(args))]
                for a in args:
                    fields += [str(a[".offset"]), str(a[".size"]), a[".value_kind"]]
                lines[k[".name"]] = " ".join(fields)
    return list(lines.values())


# host-side sanitizers (the device code is compiled as for the library)
SAN = ["-fsanitize=address", "-fsanitize=undefined", "-fno-omit-frame-pointer"]
CLANGXX = "/opt/rocm/llvm/bin/clang++"


def asan_runtime() -> str:
    """The clang AddressSanitizer runtime to preload into the Python process
    that loads the sanitized audit library."""
    r = subprocess.run([CLANGXX, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    return r.stdout.strip()


def _asan_objects() -> list[str]:
    """Every library source compiled again with host-side ASan + UBSan
    (`-Xarch_host` before each flag: the gfx950 code is unchanged)."""
    from concurrent.futures import ThreadPoolExecutor
    spec = __import__("importlib.util").util.spec_from_file_location("fa_build", os.path.join(CSRC, "build.py"))
    b = __import__("importlib.util").util.module_from_spec(spec)
    spec.loader.exec_module(b)
    out = os.path.join(OUT, "asan")
    os.makedirs(out, exist_ok=True)
    host = [x for f in SAN for x in ("-Xarch_host", f)]

    def one(src):
        obj = os.path.join(out, src.replace(".hip", ".o"))
        r = subprocess.run([b.HIPCC, *b.FLAGS, *b.EXTRA.get(src, []), *host, "-c", os.path.join(CSRC, src), "-o", obj], capture_output=True, text=True)
        if r.returncode:
            raise RuntimeError(r.stderr[-3000:])
        return obj

    with ThreadPoolExecutor(max_workers=8) as ex:
        return list(ex.map(one, b.SOURCES))


def build(max_windows: int | None = None, asan: bool = False) -> str:
    os.makedirs(OUT, exist_ok=True)
    if asan:
        objs = _asan_objects()
        parts = []
        for src in ("launch_audit.cpp", "extents.cpp"):
            o = os.path.join(OUT, "asan", src.replace(".cpp", ".o"))
            r = subprocess.run([CLANGXX, "-std=c++17", "-O1", "-fPIC", *SAN, "-I/opt/rocm/include", "-c", os.path.join(HERE, src), "-o", o],
                               capture_output=True, text=True)
            if r.returncode:
                raise RuntimeError(r.stderr)
            parts.append(o)
        lib = os.path.join(OUT, "libfa_hip_audit_asan.so")
        r = subprocess.run([CLANGXX, "-shared", "-fPIC", "-shared-libsan", *SAN, "-Wl,-Bsymbolic", "-o", lib, *objs, *parts], capture_output=True, text=True)
        if r.returncode:
            raise RuntimeError(r.stderr)
        with open(os.path.join(OUT, "kernargs_asan.txt"), "w") as f:
            f.write("\n".join(kernarg_table(objs)) + "\n")
        return lib
    objs = [os.path.join(CSRC, "_build", f) for f in sorted(os.listdir(os.path.join(CSRC, "_build"))) if f.endswith(".o")]
    if not objs:
        raise RuntimeError("no objects in fluidaudio-web_amd/csrc/_build: run __graft_entry__.build() first")
    if max_windows:
        spec = __import__("importlib.util").util.spec_from_file_location("fa_build", os.path.join(CSRC, "build.py"))
        b = __import__("importlib.util").util.module_from_spec(spec)
        spec.loader.exec_module(b)
        enc = os.path.join(OUT, f"encoder_w{max_windows}.o")
        cmd = [b.HIPCC, *b.FLAGS, f"-DFA_ENC_MAX_WINDOWS={max_windows}", "-c", os.path.join(CSRC, "encoder.hip"), "-o", enc]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode:
            raise RuntimeError(r.stderr)
        objs = [enc if os.path.basename(o) == "encoder.o" else o for o in objs]
    fake = os.path.join(OUT, "launch_audit.o")
    r = subprocess.run(["g++", "-std=c++17", "-O1", "-fPIC", "-I/opt/rocm/include", "-c", os.path.join(HERE, "launch_audit.cpp"), "-o", fake],
                       capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(r.stderr)
    # the extent models include the product's own argument structs (_Float16
    # members): ROCm's clang++ as a host compiler
    ext = os.path.join(OUT, "extents.o")
    r = subprocess.run(["/opt/rocm/llvm/bin/clang++", "-std=c++17", "-O1", "-fPIC", "-c", os.path.join(HERE, "extents.cpp"), "-o", ext],
                       capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(r.stderr)
    tag = f"_w{max_windows}" if max_windows else ""
    lib = os.path.join(OUT, f"libfa_hip_audit{tag}.so")
    r = subprocess.run(["g++", "-shared", "-fPIC", "-Wl,-Bsymbolic", "-o", lib, *objs, fake, ext], capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(r.stderr)
    tab = kernarg_table(objs)
    with open(os.path.join(OUT, f"kernargs{tag}.txt"), "w") as f:
        f.write("\n".join(tab) + "\n")
    return lib


NODE_INC = "/usr/include/node"
NODE_SRC = os.path.join(os.path.dirname(CSRC), "node")


def build_node(lib: str) -> str | None:
    """The N-API addon (node/fa_napi.c) linked against the audit library
    `lib` instead of libfa_hip.so, beside copies of the package's JS host
    files (they load fa_hip.node from their own folder), in
    tests/audit/_build/node.  None when Node's headers are absent."""
    if not os.path.exists(os.path.join(NODE_INC, "node_api.h")):
        return None
    out = os.path.join(OUT, "node")
    os.makedirs(out, exist_ok=True)
    addon = os.path.join(out, "fa_hip.node")
    r = subprocess.run(["gcc", "-O1", "-g", "-Wall", "-shared", "-fPIC", f"-I{NODE_INC}", os.path.join(NODE_SRC, "fa_napi.c"), "-o", addon,
                        f"-L{os.path.dirname(lib)}", f"-l:{os.path.basename(lib)}", f"-Wl,-rpath,{os.path.dirname(lib)}"], capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(r.stderr)
    for js in ("hip-context.js", "conformance.js", "selftest.js"):
        shutil.copyfile(os.path.join(NODE_SRC, js), os.path.join(out, js))
    return out


if __name__ == "__main__":
    mw = int(sys.argv[sys.argv.index("--max-windows") + 1]) if "--max-windows" in sys.argv else None
    print(build(mw, asan="--asan" in sys.argv))
