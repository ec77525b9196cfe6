// HipContext for Node: the reference's ComputeContext backend contract
// (src/gpu/compute.d.ts:106-255) on MI355X through the N-API addon
// fa_hip.node (a thin layer over include/fa_hip.h).  Same method names,
// option objects and error behaviour as GpuContext / WasmContext, so engine
// code (src/engines/asr-parakeet/raw-encoder.js) runs unchanged on it.
// CommonJS so it also loads on older Node; tensors are {h: BigInt, rows, cols}.
"use strict";
const path = require("path");
const addon = require(path.join(__dirname, "fa_hip.node"));

const ACT = { none: 0, gelu: 1, tanh: 2, relu: 3, silu: 4, gelu_erf: 5 };
const h = (t) => (t ? t.h : 0n);

class HipContext {
  constructor(device = 0) {
    this.ctx = addon.ctxCreate(device);
    this.backend = "hip";
    this.hasF16 = true;
  }
  _t(handle, rows, cols, f16 = false) {
    return { h: handle, rows, cols, f16 };
  }
  _info(handle) {
    const [rows, cols, dtype] = addon.tensorInfo(this.ctx, handle);
    return this._t(handle, rows, cols, dtype === 1);
  }
  // ── tensors & memory ──
  upload(data, rows, cols) {
    return this._t(addon.upload(this.ctx, data instanceof Float32Array ? data : Float32Array.from(data), rows, cols), rows, cols);
  }
  uploadF16(data, rows, cols) {
    return this._t(addon.uploadF16(this.ctx, data instanceof Float32Array ? data : Float32Array.from(data), rows, cols), rows, cols, true);
  }
  /** The context owns the weight format (compute.d.ts:243): f16 K-major storage. */
  uploadTileMajorF16(data, K, N) {
    return this.uploadF16(data, K, N);
  }
  alloc(rows, cols) {
    return this._t(addon.alloc(this.ctx, rows, cols), rows, cols);
  }
  allocF16(rows, cols) {
    return this._t(addon.allocF16(this.ctx, rows, cols), rows, cols, true);
  }
  ensureTensor(t) {
    return typeof t.h === "bigint" ? t : this.upload(t.data, t.rows, t.cols);
  }
  uploadBytes(typed) {
    const u8 = typed instanceof Uint8Array ? typed : new Uint8Array(typed.buffer, typed.byteOffset, typed.byteLength);
    return { h: addon.uploadBytes(this.ctx, u8), bytes: u8.length };
  }
  freeTensor(t) {
    if (t) addon.freeTensor(this.ctx, t.h);
  }
  pin(t, toParent = false) {
    addon.pin(this.ctx, t.h, toParent ? 1 : 0);
    return t;
  }
  pushArena() {
    return addon.pushArena(this.ctx);
  }
  popArena(handle) {
    addon.popArena(this.ctx, handle || 0n);
  }
  trimPool(budgetBytes) {
    addon.trimPool(this.ctx, budgetBytes === undefined ? 1 << 30 : budgetBytes);
  }
  destroy() {
    addon.ctxDestroy(this.ctx);
  }
  // ── readback ──
  async download(t) {
    return addon.download(this.ctx, t.h, t.rows * t.cols);
  }
  async downloadF16(t) {
    return this.download(t);
  }
  stageDownload(t) {
    const s = addon.stageDownload(this.ctx, t.h);
    const n = t.rows * t.cols;
    return { read: async () => addon.stagedRead(this.ctx, s, n) };
  }
  rowsView(t, rows) {
    return { ...this._t(addon.rowsView(this.ctx, t.h, rows), rows, t.cols, t.f16), view: true };
  }
  // ── batching ──
  beginBatch() {
    addon.beginBatch(this.ctx);
  }
  endBatch() {
    addon.endBatch(this.ctx);
  }
  withBatchSync(fn) {
    this.beginBatch();
    try {
      return fn();
    } finally {
      this.endBatch();
    }
  }
  async withBatch(fn) {
    this.beginBatch();
    try {
      return await fn();
    } finally {
      this.endBatch();
    }
  }
  // ── linear algebra ──
  matmul(a, b, { bias = null, act = "none", add = null } = {}) {
    return this._t(addon.matmul(this.ctx, a.h, b.h, h(bias), ACT[act], h(add)), a.rows, b.cols);
  }
  matmulV2(a, b, o) {
    return this.matmul(a, b, o);
  }
  matmulV3(a, b, o) {
    return this.matmul(a, b, o);
  }
  matmulV4(a, b, o) {
    return this.matmul(a, b, o);
  }
  matmulF16(a, b, o) {
    return this.matmul(a, b, o);
  }
  matmulTM(a, b, o) {
    return this.matmul(a, b, o);
  }
  matmulF16C(a, b, o) {
    return this.matmul(a, b, o);
  }
  matmulInt8(a, wq, scale, N, K, { bias = null, act = "none" } = {}) {
    return this._t(addon.matmulInt8(this.ctx, a.h, wq.h, scale.h, N, K, h(bias), ACT[act]), a.rows, N);
  }
  matmulNBits(a, bq, scales, zp, N, blockSize = 32) {
    return this._t(addon.matmulNBits(this.ctx, a.h, bq.h, scales.h, zp.h, N, blockSize), a.rows, N);
  }
  layernorm(x, gamma, beta, eps = 1e-5) {
    return this._t(addon.layernorm(this.ctx, x.h, gamma.h, beta.h, eps), x.rows, x.cols);
  }
  softmax(x) {
    return this._t(addon.softmax(this.ctx, x.h), x.rows, x.cols);
  }
  // ── convolution ──
  conv1d(x, w, { cout, k, bias = null, stride = 1, pad = 0, padLeft, padRight, dilation = 1, groups = 1, act = "none" } = {}) {
    const pl = padLeft === undefined ? pad : padLeft;
    const pr = padRight === undefined ? pad : padRight;
    return this._info(addon.conv1d(this.ctx, x.h, w.h, cout, k, h(bias), stride, pl, pr, dilation, groups, ACT[act]));
  }
  conv2d(x, w, o) {
    const { cout, cin, h: H, w: W_, kh, kw, bias = null, strideH = 1, strideW = 1, padH = 0, padW = 0, groups = 1, act = "none" } = o;
    const pt = o.padTop === undefined ? padH : o.padTop,
      pb = o.padBottom === undefined ? padH : o.padBottom,
      pl = o.padLeft === undefined ? padW : o.padLeft,
      pr = o.padRight === undefined ? padW : o.padRight;
    return this._info(addon.conv2d(this.ctx, x.h, w.h, cout, cin, H, W_, kh, kw, h(bias), strideH, strideW, pt, pb, pl, pr, groups, ACT[act]));
  }
  // ── attention ──
  bmmQK(q, b, qb, H, HD, W = 1, bShared = false) {
    return this._info(addon.bmmQK(this.ctx, q.h, b.h, h(qb), H, HD, W, bShared ? 1 : 0));
  }
  bmmPV(p, v, H, HD, W = 1) {
    return this._info(addon.bmmPV(this.ctx, p.h, v.h, H, HD, W));
  }
  relShift(x) {
    return this._info(addon.relShift(this.ctx, x.h));
  }
  relShiftB(x, H) {
    return this._info(addon.relShiftB(this.ctx, x.h, H));
  }
  /** compute.js relShiftStream(x, {H, n, Lk, dMax, Lc, subT, C, left, right}). */
  relShiftStream(x, { H, n, Lk, dMax, Lc, subT, C, left, right }) {
    return this._info(addon.relShiftStream(this.ctx, x.h, H, n, Lk, dMax, Lc, subT, C, left, right));
  }
  attnFused(q, k, v, pos, pbu, pbv, H, HD, W) {
    return this._info(addon.attnFused(this.ctx, q.h, k.h, v.h, pos.h, pbu.h, pbv.h, H, HD, W));
  }
  // ── elementwise & data movement ──
  ewise(a, b, op) {
    return this._t(addon.ewise(this.ctx, a.h, b.h, op === "mul" ? 1 : 0), a.rows, a.cols);
  }
  add(a, b) {
    return this.ewise(a, b, "add");
  }
  mul(a, b) {
    return this.ewise(a, b, "mul");
  }
  scale(x, s) {
    return this._t(addon.scale(this.ctx, x.h, s), x.rows, x.cols);
  }
  silu(x) {
    return this._t(addon.silu(this.ctx, x.h), x.rows, x.cols);
  }
  relu(x) {
    return this._t(addon.relu(this.ctx, x.h), x.rows, x.cols);
  }
  glu(x) {
    return this._t(addon.glu(this.ctx, x.h), x.rows / 2, x.cols);
  }
  transpose(x) {
    return this._t(addon.transpose(this.ctx, x.h), x.cols, x.rows);
  }
  sliceCols(x, col0, width) {
    return this._t(addon.sliceCols(this.ctx, x.h, col0, width), x.rows, width);
  }
  setCols(dst, src, col0) {
    addon.setCols(this.ctx, dst.h, src.h, col0);
    return dst;
  }
  sliceRows(x, row0, count) {
    return this._t(addon.sliceRows(this.ctx, x.h, row0, count), count, x.cols);
  }
  copyRows(dst, src, rowOffset) {
    addon.copyRows(this.ctx, dst.h, src.h, rowOffset);
    return dst;
  }
  concatRows(tensors) {
    return this._t(addon.concatRows(this.ctx, tensors.map((t) => t.h)), tensors.reduce((s, t) => s + t.rows, 0), tensors[0].cols);
  }
  subReshape(x, C, Tsub, F) {
    return this._t(addon.subReshape(this.ctx, x.h, C, Tsub, F), Tsub, C * F);
  }
  rowBiasAct(x, bias, act = "none") {
    return this._t(addon.rowBiasAct(this.ctx, x.h, bias.h, ACT[act]), x.rows, x.cols);
  }
  // ── TTS / decoder-side members (compute.d.ts:174-234) ──
  leakyRelu(x, slope = 0.2) {
    return this._t(addon.leakyRelu(this.ctx, x.h, slope), x.rows, x.cols);
  }
  snake(x, alpha) {
    return this._t(addon.snake(this.ctx, x.h, alpha.h), x.rows, x.cols);
  }
  adain(x, scale, shift, eps = 1e-5) {
    return this._t(addon.adain(this.ctx, x.h, scale.h, shift.h, eps), x.rows, x.cols);
  }
  im2col(x, k, { stride = 1, pad = 0, dilation = 1 } = {}) {
    return this._info(addon.im2col(this.ctx, x.h, k, stride, pad, dilation));
  }
  /** matmul(wRows [Cout, Cin*k], im2col(x)) (wasm-context.js:286-288). */
  conv1dGemm(x, wRows, cout, k, { stride = 1, pad = 0, dilation = 1, act = "none" } = {}) {
    const cols = this.im2col(x, k, { stride, pad, dilation });
    const y = this.matmul(wRows, cols, { act });
    this.freeTensor(cols);
    return y;
  }
  conv1dFast(x, wRows, cout, k, opts = {}) {
    return this.conv1d(x, wRows, Object.assign({}, opts, { cout, k }));
  }
  conv1dFastF16(x, wRows, cout, k, opts = {}) {
    return this.conv1d(x, wRows, Object.assign({}, opts, { cout, k }));
  }
  convTranspose1d(x, w, { cout, k, bias = null, stride = 1, pad = 0, dilation = 1, groups = 1, outputPadding = 0, act = "none" } = {}) {
    return this._info(addon.convTranspose1d(this.ctx, x.h, w.h, cout, k, h(bias), stride, pad, dilation, groups, outputPadding, ACT[act]));
  }
  gatherCols(x, idxMap) {
    const idx = idxMap instanceof Uint32Array ? idxMap : Uint32Array.from(idxMap);
    return this._t(addon.gatherCols(this.ctx, x.h, idx), x.rows, idx.length);
  }
  lstm(x, w, r, b, hid) {
    return this._t(addon.lstm(this.ctx, x.h, w.h, r.h, b.h, hid), x.rows, 2 * hid);
  }
  jbatch(encProj, base, B, predProj, hid) {
    return this._t(addon.jbatch(this.ctx, encProj.h, base, B, predProj.h, hid), B, hid);
  }
  argmaxRows(x, B, vocab, logits) {
    return this._t(addon.argmaxRows(this.ctx, x.h, B, vocab, logits), B, 4);
  }
  jointArgmax(encProj, frame, count, predProj, outW, outB, hidden, vocab, logits) {
    return this._t(addon.jointArgmax(this.ctx, encProj.h, frame, count, predProj.h, outW.h, outB.h, hidden, vocab, logits), count, 4);
  }
  // ── profiling ──
  startProfile(maxOps = 4096) {
    addon.profileStart(this.ctx, maxOps);
  }
  async endProfile() {
    return addon.profileEnd(this.ctx);
  }
  // ── fused encoder (one native call per window batch; backend-private, so _-prefixed) ──
  /** man: {name: {data: Float32Array, dims}} in the reference manifest naming. */
  _loadFusedEncoder(man, cfg, { format = "f16", maxT = 512 } = {}) {
    const names = Object.keys(man);
    const c = Int32Array.from(["D", "DFF", "H", "HD", "layers", "dwK", "Csub", "Fsub", "melBins"].map((k) => cfg[k]));
    const enc = addon.encoderLoad(this.ctx, c, names, names.map((k) => man[k].data), { f16: 0, int8: 1, int4: 2 }[format], maxT);
    return { enc, cfg };
  }
  /** Encode windows (list of Float32Array [melBins*T] channel-major) -> frames tensor [ΣTsub, D]. */
  _encodeFused(fused, mels, layout = "packed") {
    const mb = fused.cfg.melBins;
    const lens = Int32Array.from(mels.map((m) => m.length / mb));
    const total = lens.reduce((a, b) => a + b, 0);
    const stream = new Float32Array(mb * total);
    let off = 0;
    for (let w = 0; w < mels.length; w++) {
      const T = lens[w];
      for (let c = 0; c < mb; c++) stream.set(mels[w].subarray(c * T, (c + 1) * T), c * total + off);
      off += T;
    }
    const starts = new Int32Array(lens.length);
    for (let i = 1; i < lens.length; i++) starts[i] = starts[i - 1] + lens[i - 1];
    const feats = this.upload(stream, mb, total);
    const out = this._info(addon.encoderForwardStream(this.ctx, fused.enc, feats.h, starts, lens, layout === "packed" ? 0 : 1, -1));
    this.freeTensor(feats);
    return out;
  }
  /** Several batches [{starts, lens}] of one resident feature stream [melBins, T]:
   * each output equals encoderForwardStream of that batch, bit for bit, with
   * consecutive batches in flight on the encoder's two workspace lanes
   * (fa_encoder_forward_stream_batches); the group loop of pipeline.js:66-80. */
  _encodeFusedStreamBatches(fused, feats, batches, layout = "packed") {
    const counts = Int32Array.from(batches.map((b) => b.lens.length));
    const starts = Int32Array.from([].concat(...batches.map((b) => Array.from(b.starts))));
    const lens = Int32Array.from([].concat(...batches.map((b) => Array.from(b.lens))));
    const hs = addon.encoderForwardStreamBatches(this.ctx, fused.enc, feats.h, starts, lens, counts, layout === "packed" ? 0 : 1, -1);
    return hs.map((h) => this._info(h));
  }
  /** Log-mel features (ParakeetMel.process semantics, parakeet-mel.js:14-22) of
   * windows [starts[i], starts[i]+lens[i]) of a resident f32 sample tensor ->
   * f32 tensor [nMels, Σ floor(lens[i]/160)] in the stream layout packWindows
   * reads.  Nemotron's raw log-mel: logGuard 1e-10, normalize false. */
  _melWindows(pcm, starts, lens, nMels = 128, logGuard = 2 ** -24, normalize = true) {
    return this._info(addon.melWindows(this.ctx, pcm.h, Int32Array.from(starts), Int32Array.from(lens), nMels, logGuard, normalize ? 1 : 0));
  }
  /** Greedy TDT decoder weights (loadGpuDecoder, gpu-decoder.js:220-246): an
   * object of Float32Arrays in the decoder manifest naming. */
  _loadTdtDecoder(w) {
    const keys = ["embed", "l0_W", "l0_R", "l0_B", "l1_W", "l1_R", "l1_B", "predW", "predB", "outW", "outB"];
    return { dec: addon.tdtLoad(this.ctx, keys.map((k) => (w[k] instanceof Float32Array ? w[k] : Float32Array.from(w[k])))) };
  }
  /** gpuDecodeBatch (gpu-decoder.js:248-273): frames = tensor [Σ lens, 640] of
   * pre-projected encoder frames -> per window { ids, idFrames }. */
  _tdtDecodeBatch(d, frames, lens, cap = 4096) {
    const n = lens.length;
    const ids = new Int32Array(n * cap), fr = new Int32Array(n * cap), cnt = new Int32Array(n);
    addon.tdtDecode(this.ctx, d.dec, this.ensureTensor(frames).h, Int32Array.from(lens), cap, ids, fr, cnt);
    const out = [];
    for (let w = 0; w < n; w++) {
      const k = Math.min(cnt[w], cap);
      out.push({ ids: Array.from(ids.subarray(w * cap, w * cap + k)), idFrames: Array.from(fr.subarray(w * cap, w * cap + k)) });
    }
    return out;
  }
  _destroyTdtDecoder(d) {
    addon.tdtDestroy(d.dec);
  }
  _destroyFusedEncoder(fused) {
    addon.encoderDestroy(fused.enc);
  }
}

/** Backend factory arm (src/gpu/context.js:23-37): throws when no gfx950 GPU is present. */
function createHipContext(device = 0) {
  return new HipContext(device);
}

module.exports = { HipContext, createHipContext, ACT, version: addon.version, encoderTsub: addon.encoderTsub };
