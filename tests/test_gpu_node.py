"""The N-API addon + Node HipContext (the TypeScript host's drop-in) on the GPU.

selftest.js: ops against inline references, staged-read semantics, the fused
encoder's packed-vs-standalone equality, mel and TDT through the binding.
conformance.js: the reference's two gates -- interface conformance (every
required ComputeContext member present, no undeclared public member) and the
numeric case list of scripts/backend-conformance.mjs run on seeded inputs --
whose recorded inputs / outputs are checked here case by case against the CPU
oracle with that gate's tolerances (max |HIP - oracle|)."""
import json
import os
import shutil
import subprocess
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NODE_DIR = os.path.join(ROOT, "fluidaudio-web_amd", "node")
sys.path.insert(0, os.path.join(ROOT, "oracle"))

needs_node = pytest.mark.skipif(shutil.which("node") is None or not os.path.exists(os.path.join(NODE_DIR, "fa_hip.node")),
                                reason="node or the N-API addon is not available")


@needs_node
def test_node_selftest():
    r = subprocess.run(["node", os.path.join(NODE_DIR, "selftest.js")], capture_output=True, text=True, timeout=110)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr


def _arr(d):
    return np.asarray(d["data"], np.float32).reshape(d["rows"], d["cols"])


def _f16(a):
    return a.astype(np.float16).astype(np.float32)


def _expected(orc, J, c):
    """The oracle's result for one recorded case (the reference CPU backend's
    arithmetic for the same method and options)."""
    I = {k: (_arr(v) if "data" in v else v) for k, v in c["inputs"].items()}
    lab = c["label"]
    if lab.startswith("matmul bias+"):
        return orc.matmul(I["a"], I["b"], bias=I["bias"], act=lab.split("+")[1])
    if lab == "matmul vec4 + add":
        return orc.matmul(I["a"], I["b"], act="relu", add=I["add"])
    if lab == "matmulV2":
        return orc.matmul(I["a"], I["b"], act="gelu")
    if lab == "matmulV3":
        return orc.matmul(I["a"], I["b"])
    if lab == "matmulV4":
        return orc.matmul(I["a"], I["b"], bias=I["bias"], act="silu")
    if lab == "matmulF16 (f16 a/b)":
        return orc.matmul(_f16(I["a"]), _f16(I["b"]))
    if lab == "matmul f16-B route":
        return orc.matmul(I["a"], _f16(I["b"]), bias=I["bias"], act="silu")
    if lab == "matmulInt8 bias+relu":
        wq = np.asarray(I["wq"]["bytes"], np.uint8).view(np.int8).reshape(20, 16)
        return orc.matmul_int8(I["a"], wq, I["scale"], 16, 20, bias=I["bias"], act="relu")
    if lab == "matmulNBits":
        bq = np.asarray(I["bq"]["bytes"], np.uint8).reshape(8, 2, 16)
        zp = np.asarray(I["zp"]["bytes"], np.uint8)[:8].reshape(8, 1)
        return orc.matmul_nbits(I["a"], bq, I["scales"], zp, 8)
    if lab == "layernorm":
        return orc.layernorm(I["x"], I["g"], I["b"])
    if lab == "softmax":
        return orc.softmax(I["x"])
    if lab == "adain":
        return J.adain(I["x"], I["scale"], I["shift"])
    if lab == "conv1d stride2 pad3 silu":
        return orc.conv1d_grouped(I["x"], I["w"], 8, 5, bias=I["bias"], stride=2, pad_left=3, pad_right=3, act="silu")
    if lab == "conv1d depthwise asym-pad":
        return orc.conv1d_grouped(I["x"], I["w"], 6, 3, pad_left=2, pad_right=0, groups=6)
    if lab == "im2col":
        return J.im2col(I["x"], 3, 2, 1)
    if lab == "conv1dGemm":
        return orc.matmul(I["w"], J.im2col(I["x"], 3, 2, 1), act="relu")
    if lab == "conv1dFast bias+gelu":
        return orc.conv1d_grouped(I["x"], I["w"], 6, 3, bias=I["bias"], pad_left=1, pad_right=1, act="gelu")
    if lab == "conv1dFastF16":
        return orc.conv1d_grouped(_f16(I["x"]), _f16(I["w"]), 6, 3, pad_left=1, pad_right=1, act="silu")
    if lab == "conv2d 3x3 s2 relu":
        return orc.conv2d(I["x"], I["w"], 4, 3, 9, 11, 3, 3, bias=I["bias"], sh=2, sw=2, pt=1, pb=1, pl=1, pr=1, act="relu")
    if lab == "conv2d depthwise 3x3 s2":
        return orc.conv2d(I["x"], I["w"], 6, 6, 9, 11, 3, 3, sh=2, sw=2, pt=1, pb=1, pl=1, pr=1, groups=6, act="silu")
    if lab == "conv2d cin=1 asym pad":
        return orc.conv2d(I["x"], I["w"], 8, 1, 12, 10, 3, 3, sh=2, sw=2, pt=1, pb=0, pl=1, pr=0)
    if lab == "convTranspose1d s2 groups2":
        return J.conv_transpose1d(I["x"], I["w"], 6, 4, I["bias"], 2, 1, 1, 2)
    if lab == "bidirectional lstm":
        return J.lstm(I["x"], I["w"], I["r"], I["b"], 16)
    if lab == "bmmQK W=2 +qb":
        return orc.bmm_qk(I["q"], I["k"], I["qb"], 3, 16, 2)
    if lab == "bmmQK bShared":
        return orc.bmm_qk(I["q"], I["p"], None, 3, 16, 2, True)
    if lab == "bmmPV W=2":
        return orc.bmm_pv(I["p"], I["v"], 3, 16, 2)
    if lab == "relShift":
        return orc.relshift_b(I["x"], 1)
    if lab == "relShiftB":
        return orc.relshift_b(I["x"], 3)
    if lab == "relShiftStream":
        return orc.relshift_stream(I["x"], 3, 6, 20, 16, 12, 24, 8, 8, 0)
    if lab == "ewise mul + row broadcast":
        return I["a"] * I["b"]
    if lab == "add":
        return I["a"] + I["b"]
    if lab == "mul":
        return I["a"] * I["b"]
    if lab == "scale":
        return (I["x"].astype(np.float64) * -1.7).astype(np.float32)
    if lab == "silu":
        return orc.silu(I["x"])
    if lab == "relu":
        return np.maximum(I["x"], 0)
    if lab == "leakyRelu slope 0.3":
        return J.leaky_relu(I["x"], 0.3)
    if lab == "snake":
        return J.snake(I["x"], I["alpha"])
    if lab == "glu":
        return orc.glu(I["x"])
    if lab == "transpose":
        return orc.transpose(I["x"])
    if lab == "sliceCols":
        return I["x"][:, 3:9]
    if lab == "setCols":
        d = I["dst"].copy()
        d[:, 5:9] = I["src"]
        return d
    if lab == "sliceRows":
        return I["x"][3:7]
    if lab == "copyRows":
        d = I["dst"].copy()
        d[4:7] = I["src"]
        return d
    if lab == "concatRows x3":
        return np.concatenate([I["a"], I["b"], I["c"]])
    if lab == "gatherCols":
        return J.gather_cols(I["x"], I["idx"]["ints"])
    if lab == "subReshape":
        return orc.subreshape(I["x"], 5, 7, 4)
    if lab == "jbatch":
        return J.jbatch(I["enc"], 2, 5, I["pred"], 32)
    if lab == "argmaxRows":
        return J.argmax_rows(I["x"], 6, 32, 40)
    if lab == "jointArgmax":
        return J.joint_argmax(I["enc"], 1, 4, I["pred"], I["w"], I["b"], 32, 36, 44)
    if lab == "ensureTensor host literal":
        return I["x"] * 2
    if lab == "rowsView feeds matmul":
        return orc.matmul(I["c"][:6], I["b"])
    if lab == "stageDownload staged read":
        return orc.matmul(I["a"], I["b"])
    if lab.startswith("withBatch"):
        y = orc.matmul(I["a"], I["b"], act="gelu")
        cache = I["cache"].copy()
        cache[4:16] = y
        return np.concatenate([cache.reshape(-1), (y + I["d"]).reshape(-1)])
    raise KeyError(lab)


@needs_node
def test_node_backend_conformance(orc, tmp_path):
    import js_ops as J

    dump = tmp_path / "conformance.json"
    r = subprocess.run(["node", os.path.join(NODE_DIR, "conformance.js"), str(dump)], capture_output=True, text=True, timeout=110)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    cases = json.loads(dump.read_text())["cases"]
    assert len(cases) >= 55
    bad = []
    for c in cases:
        want = np.asarray(_expected(orc, J, c), np.float64).reshape(-1)
        got = np.asarray(c["output"], np.float64)
        d = float(np.abs(got - want).max()) if got.shape == want.shape else float("inf")
        print(f"{'ok  ' if d <= c['tol'] else 'FAIL'} {c['label']}: maxΔ {d:.2e} (tol {c['tol']})")
        if not d <= c["tol"]:
            bad.append(c["label"])
    assert not bad, bad
