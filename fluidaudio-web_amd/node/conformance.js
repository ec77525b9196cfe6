// HipContext against the reference's backend gates, on a GPU.
//
// 1. Structure (the check of scripts/interface-conformance.mjs:17-40): every
//    required ComputeContext method (src/gpu/compute.d.ts:106-234) is a
//    function on HipContext.prototype, and every public method is declared
//    (required or in the optional block); backend-private members start
//    with "_".
// 2. Numbers (the case list of scripts/backend-conformance.mjs:66-414): every
//    required method runs on seeded mulberry32 inputs through HipContext, or
//    is exempt as plumbing.  The reference compares two backends; here the
//    inputs, options and outputs of each case are written to a JSON file
//    (argv[2]) that tests/test_gpu_node.py checks case by case against the
//    CPU oracle with the reference's tolerances.
// Exit code: 0 = structure and coverage OK and every case ran.
"use strict";
const fs = require("fs");
const { HipContext } = require("./hip-context.js");

// compute.d.ts ComputeContext method names (required, then the optional block)
const REQUIRED = ["upload", "uploadF16", "alloc", "allocF16", "ensureTensor", "uploadBytes", "freeTensor", "pin", "pushArena", "popArena", "trimPool",
  "destroy", "download", "downloadF16", "stageDownload", "rowsView", "beginBatch", "endBatch", "withBatch", "withBatchSync", "matmul", "matmulV2",
  "matmulV3", "matmulV4", "matmulF16", "matmulInt8", "matmulNBits", "layernorm", "softmax", "conv1d", "conv1dGemm", "conv1dFast", "conv1dFastF16",
  "conv2d", "convTranspose1d", "im2col", "lstm", "bmmQK", "bmmPV", "relShift", "relShiftB", "relShiftStream", "ewise", "add", "mul", "scale", "silu",
  "relu", "leakyRelu", "snake", "glu", "adain", "transpose", "sliceCols", "setCols", "sliceRows", "copyRows", "concatRows", "gatherCols",
  "subReshape", "jbatch", "argmaxRows", "jointArgmax"];
const OPTIONAL = ["probeSubgroups", "uploadTileMajorF16", "matmulTM", "matmulF16B", "matmulF16C", "attnFused", "rowBiasAct", "startProfile",
  "endProfile", "memStatsStart", "memStats", "poolInfo"];
// plumbing without standalone numeric behaviour (backend-conformance.mjs:21-38)
const EXEMPT = new Set(["upload", "uploadF16", "alloc", "allocF16", "uploadBytes", "freeTensor", "pin", "pushArena", "popArena", "trimPool",
  "destroy", "download", "downloadF16", "beginBatch", "endBatch", "withBatchSync"]);

let failed = 0;
const proto = HipContext.prototype;
const missing = REQUIRED.filter((m) => typeof proto[m] !== "function");
const declared = new Set(REQUIRED.concat(OPTIONAL));
const undeclared = Object.getOwnPropertyNames(proto).filter((m) => m !== "constructor" && !m.startsWith("_") && typeof proto[m] === "function" && !declared.has(m));
if (missing.length) {
  failed++;
  console.log(`FAIL HipContext is missing required methods: ${missing.join(", ")}`);
} else console.log(`ok   HipContext implements all ${REQUIRED.length} required ComputeContext methods`);
if (undeclared.length) {
  failed++;
  console.log(`FAIL HipContext has public methods the interface does not declare: ${undeclared.join(", ")}`);
} else console.log("ok   no undeclared public methods");

let seed = 0x5eed;
const rand = () => {
  seed |= 0;
  seed = (seed + 0x6d2b79f5) | 0;
  let t = Math.imul(seed ^ (seed >>> 15), 1 | seed);
  t = (t + Math.imul(t ^ (t >>> 7), 61 | t)) ^ t;
  return ((t ^ (t >>> 14)) >>> 0) / 4294967296;
};
const mkData = (n) => Float32Array.from({ length: n }, () => rand() - 0.5);
const mkBytes = (n) => Uint8Array.from({ length: n }, () => Math.floor(rand() * 256));

const g = new HipContext(0);
const cases = [];
const test = (method, label, tol, fn) => cases.push({ method, label, tol, fn });
// Per case: named inputs recorded for the checker.
let rec = null;
const inp = (name, rows, cols) => {
  const d = mkData(rows * cols);
  rec[name] = { rows, cols, data: Array.from(d) };
  return g.upload(d, rows, cols);
};
const inpF16 = (name, rows, cols) => {
  const d = mkData(rows * cols);
  rec[name] = { rows, cols, data: Array.from(d) };
  return g.uploadF16(d, rows, cols);
};
const inpBytes = (name, n) => {
  const b = mkBytes(n);
  rec[name] = { bytes: Array.from(b) };
  return g.uploadBytes(b);
};
const dl = (t) => g.download(t);

for (const act of ["none", "gelu", "gelu_erf", "tanh", "relu", "silu"])
  test("matmul", `matmul bias+${act}`, 1e-3, () => dl(g.matmul(inp("a", 37, 53), inp("b", 53, 41), { bias: inp("bias", 1, 41), act })));
test("matmul", "matmul vec4 + add", 1e-3, () => dl(g.matmul(inp("a", 64, 128), inp("b", 128, 256), { act: "relu", add: inp("add", 64, 256) })));
test("matmulV2", "matmulV2", 1e-3, () => dl(g.matmulV2(inp("a", 33, 48), inp("b", 48, 52), { act: "gelu" })));
test("matmulV3", "matmulV3", 1e-3, () => dl(g.matmulV3(inp("a", 33, 64), inp("b", 64, 48))));
test("matmulV4", "matmulV4", 1e-3, () => dl(g.matmulV4(inp("a", 129, 64), inp("b", 64, 132), { bias: inp("bias", 1, 132), act: "silu" })));
test("matmulF16", "matmulF16 (f16 a/b)", 5e-2, () => g.downloadF16(g.matmulF16(inpF16("a", 40, 64), inpF16("b", 64, 64))));
test("matmul", "matmul f16-B route", 2e-2, () => dl(g.matmul(inp("a", 65, 128), inpF16("b", 128, 256), { bias: inp("bias", 1, 256), act: "silu" })));
test("matmulInt8", "matmulInt8 bias+relu", 1e-3, () =>
  dl(g.matmulInt8(inp("a", 9, 20), inpBytes("wq", 20 * 16), inp("scale", 1, 16), 16, 20, { bias: inp("bias", 1, 16), act: "relu" })));
test("matmulNBits", "matmulNBits", 1e-3, () =>
  dl(g.matmulNBits(inp("a", 7, 64), inpBytes("bq", 8 * 2 * 16), inp("scales", 1, 16), inpBytes("zp", 8 * 1 * 4), 8)));
test("layernorm", "layernorm", 1e-4, () => dl(g.layernorm(inp("x", 7, 33), inp("g", 1, 33), inp("b", 1, 33))));
test("softmax", "softmax", 1e-5, () => dl(g.softmax(inp("x", 9, 21))));
test("adain", "adain", 1e-4, () => dl(g.adain(inp("x", 5, 20), inp("scale", 1, 5), inp("shift", 1, 5))));
test("conv1d", "conv1d stride2 pad3 silu", 1e-3, () =>
  dl(g.conv1d(inp("x", 6, 25), inp("w", 1, 8 * 6 * 5), { cout: 8, k: 5, stride: 2, pad: 3, act: "silu", bias: inp("bias", 1, 8) })));
test("conv1d", "conv1d depthwise asym-pad", 1e-3, () => dl(g.conv1d(inp("x", 6, 19), inp("w", 1, 18), { cout: 6, k: 3, groups: 6, padLeft: 2, padRight: 0 })));
test("im2col", "im2col", 0, () => dl(g.im2col(inp("x", 4, 15), 3, { stride: 2, pad: 1 })));
test("conv1dGemm", "conv1dGemm", 1e-3, () => dl(g.conv1dGemm(inp("x", 4, 15), inp("w", 6, 12), 6, 3, { stride: 2, pad: 1, act: "relu" })));
test("conv1dFast", "conv1dFast bias+gelu", 1e-3, () =>
  dl(g.conv1dFast(inp("x", 4, 15), inp("w", 6, 12), 6, 3, { stride: 1, pad: 1, act: "gelu", bias: inp("bias", 1, 6) })));
test("conv1dFastF16", "conv1dFastF16", 5e-2, () => g.downloadF16(g.conv1dFastF16(inpF16("x", 4, 15), inpF16("w", 6, 12), 6, 3, { stride: 1, pad: 1, act: "silu" })));
test("conv2d", "conv2d 3x3 s2 relu", 1e-3, () =>
  dl(g.conv2d(inp("x", 3, 99), inp("w", 1, 108), { cout: 4, cin: 3, h: 9, w: 11, kh: 3, kw: 3, strideH: 2, strideW: 2, padH: 1, padW: 1, act: "relu",
    bias: inp("bias", 1, 4) })));
test("conv2d", "conv2d depthwise 3x3 s2", 1e-3, () =>
  dl(g.conv2d(inp("x", 6, 99), inp("w", 1, 54), { cout: 6, cin: 6, h: 9, w: 11, kh: 3, kw: 3, strideH: 2, strideW: 2, padH: 1, padW: 1, groups: 6,
    act: "silu" })));
test("conv2d", "conv2d cin=1 asym pad", 1e-3, () =>
  dl(g.conv2d(inp("x", 1, 120), inp("w", 1, 72), { cout: 8, cin: 1, h: 12, w: 10, kh: 3, kw: 3, strideH: 2, strideW: 2, padTop: 1, padBottom: 0,
    padLeft: 1, padRight: 0 })));
test("convTranspose1d", "convTranspose1d s2 groups2", 1e-3, () =>
  dl(g.convTranspose1d(inp("x", 4, 12), inp("w", 1, 48), { cout: 6, k: 4, stride: 2, pad: 1, groups: 2, bias: inp("bias", 1, 6) })));
test("lstm", "bidirectional lstm", 1e-3, () => dl(g.lstm(inp("x", 6, 8), inp("w", 128, 8), inp("r", 128, 16), inp("b", 2, 128), 16)));
test("bmmQK", "bmmQK W=2 +qb", 1e-4, () => dl(g.bmmQK(inp("q", 14, 48), inp("k", 18, 48), inp("qb", 1, 48), 3, 16, 2)));
test("bmmQK", "bmmQK bShared", 1e-4, () => dl(g.bmmQK(inp("q", 14, 48), inp("p", 11, 48), null, 3, 16, 2, true)));
test("bmmPV", "bmmPV W=2", 1e-4, () => dl(g.bmmPV(inp("p", 42, 9), inp("v", 18, 48), 3, 16, 2)));
test("relShift", "relShift", 0, () => dl(g.relShift(inp("x", 9, 17))));
test("relShiftB", "relShiftB", 0, () => dl(g.relShiftB(inp("x", 21, 13), 3)));
test("relShiftStream", "relShiftStream", 0, () =>
  dl(g.relShiftStream(inp("x", 18, 33), { H: 3, n: 6, Lk: 20, dMax: 16, Lc: 12, subT: 24, C: 8, left: 8, right: 0 })));
test("ewise", "ewise mul + row broadcast", 1e-6, () => dl(g.ewise(inp("a", 7, 13), inp("b", 1, 13), "mul")));
test("add", "add", 1e-6, () => dl(g.add(inp("a", 7, 13), inp("b", 7, 13))));
test("mul", "mul", 1e-6, () => dl(g.mul(inp("a", 7, 13), inp("b", 7, 13))));
test("scale", "scale", 1e-6, () => dl(g.scale(inp("x", 6, 11), -1.7)));
test("silu", "silu", 1e-5, () => dl(g.silu(inp("x", 6, 11))));
test("relu", "relu", 0, () => dl(g.relu(inp("x", 6, 11))));
test("leakyRelu", "leakyRelu slope 0.3", 1e-6, () => dl(g.leakyRelu(inp("x", 6, 11), 0.3)));
test("snake", "snake", 1e-5, () => dl(g.snake(inp("x", 4, 17), inp("alpha", 1, 4))));
test("glu", "glu", 1e-5, () => dl(g.glu(inp("x", 8, 9))));
test("transpose", "transpose", 0, () => dl(g.transpose(inp("x", 7, 13))));
test("sliceCols", "sliceCols", 0, () => dl(g.sliceCols(inp("x", 7, 13), 3, 6)));
test("setCols", "setCols", 0, () => dl(g.setCols(inp("dst", 7, 13), inp("src", 7, 4), 5)));
test("sliceRows", "sliceRows", 0, () => dl(g.sliceRows(inp("x", 10, 6), 3, 4)));
test("copyRows", "copyRows", 0, () => dl(g.copyRows(inp("dst", 10, 6), inp("src", 3, 6), 4)));
test("concatRows", "concatRows x3", 0, () => dl(g.concatRows([inp("a", 3, 6), inp("b", 2, 6), inp("c", 4, 6)])));
test("gatherCols", "gatherCols", 0, () => {
  const x = inp("x", 5, 12);
  const idx = Uint32Array.from({ length: 20 }, () => Math.floor(rand() * 12));
  rec.idx = { ints: Array.from(idx) };
  return dl(g.gatherCols(x, idx));
});
test("subReshape", "subReshape", 0, () => dl(g.subReshape(inp("x", 5, 28), 5, 7, 4)));
test("jbatch", "jbatch", 1e-6, () => dl(g.jbatch(inp("enc", 10, 32), 2, 5, inp("pred", 1, 32), 32)));
test("argmaxRows", "argmaxRows", 1e-3, () => dl(g.argmaxRows(inp("x", 6, 40), 6, 32, 40)));
test("jointArgmax", "jointArgmax", 1e-3, () =>
  dl(g.jointArgmax(inp("enc", 10, 32), 1, 4, inp("pred", 1, 32), inp("w", 32, 44), inp("b", 1, 44), 32, 36, 44)));
test("ensureTensor", "ensureTensor host literal", 1e-6, () => {
  const d = mkData(40);
  rec.x = { rows: 5, cols: 8, data: Array.from(d) };
  return dl(g.scale(g.ensureTensor({ data: d, rows: 5, cols: 8 }), 2));
});
test("rowsView", "rowsView feeds matmul", 1e-3, () => dl(g.matmul(g.rowsView(inp("c", 10, 24), 6), inp("b", 24, 12))));
test("stageDownload", "stageDownload staged read", 1e-3, () => g.stageDownload(g.matmul(inp("a", 8, 16), inp("b", 16, 8))).read());
test("withBatch", "withBatch: matmul -> copyRows -> download mid-batch -> add", 1e-3, async () => {
  const a = inp("a", 12, 16), b = inp("b", 16, 8), cache = inp("cache", 20, 8), d = inp("d", 12, 8);
  return g.withBatch(async () => {
    const y = g.matmul(a, b, { act: "gelu" });
    g.copyRows(cache, y, 4);
    const mid = await g.download(cache);
    const fin = await g.download(g.add(y, d));
    const out = new Float32Array(mid.length + fin.length);
    out.set(mid, 0);
    out.set(fin, mid.length);
    return out;
  });
});

(async () => {
  const out = [];
  const tested = new Set();
  for (const c of cases) {
    rec = {};
    try {
      const y = await c.fn();
      out.push({ method: c.method, label: c.label, tol: c.tol, inputs: rec, output: Array.from(y) });
      tested.add(c.method);
    } catch (e) {
      failed++;
      console.log(`FAIL ${c.label}: ${e.message}`);
    }
  }
  const uncovered = REQUIRED.filter((m) => !tested.has(m) && !EXEMPT.has(m));
  if (uncovered.length) {
    failed++;
    console.log(`FAIL required methods with no conformance case and no exemption: ${uncovered.join(", ")}`);
  } else console.log(`ok   ${cases.length} cases cover every required method (${EXEMPT.size} exempt as plumbing)`);
  if (process.argv[2]) fs.writeFileSync(process.argv[2], JSON.stringify({ cases: out }));
  g.destroy();
  process.exit(failed ? 1 : 0);
})().catch((e) => {
  console.error(e);
  process.exit(2);
});
