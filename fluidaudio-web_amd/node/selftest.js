// Node self-test of the N-API addon + HipContext on a GPU: each op against an
// inline JS reference (the way scripts/gpu-verify.mjs checks WGSL kernels),
// then the fused encoder's packed-vs-standalone equality.  Exit code 0 = pass.
"use strict";
const { HipContext, version, encoderTsub } = require("./hip-context.js");
const addonRef = require("./fa_hip.node");

let seed = 0x5eed; // mulberry32, as scripts/backend-conformance.mjs:46-54
const rand = () => {
  seed |= 0;
  seed = (seed + 0x6d2b79f5) | 0;
  let t = Math.imul(seed ^ (seed >>> 15), 1 | seed);
  t = (t + Math.imul(t ^ (t >>> 7), 61 | t)) ^ t;
  return ((t ^ (t >>> 14)) >>> 0) / 4294967296;
};
const mk = (n, s = 1) => Float32Array.from({ length: n }, () => (rand() - 0.5) * s);
const maxdiff = (a, b) => a.reduce((m, v, i) => Math.max(m, Math.abs(v - b[i])), 0);
let failed = 0;
const check = (name, d, tol) => {
  const ok = d <= tol;
  if (!ok) failed++;
  console.log(`${ok ? "ok  " : "FAIL"} ${name}: maxΔ ${d.toExponential(2)} (tol ${tol})`);
};

(async () => {
  console.log("addon", version());
  const ctx = new HipContext(0);
  // matmul f32 B + bias + silu + add
  const M = 37, K = 64, N = 41;
  const a = mk(M * K), b = mk(K * N), bias = mk(N), add = mk(M * N);
  const ref = new Float32Array(M * N);
  for (let i = 0; i < M; i++)
    for (let j = 0; j < N; j++) {
      let s = 0;
      for (let k = 0; k < K; k++) s += a[i * K + k] * b[k * N + j];
      const v = s + bias[j];
      ref[i * N + j] = v / (1 + Math.exp(-Math.max(-30, Math.min(30, v)))) + add[i * N + j];
    }
  const y = ctx.matmul(ctx.upload(a, M, K), ctx.upload(b, K, N), { bias: ctx.upload(bias, 1, N), act: "silu", add: ctx.upload(add, M, N) });
  check("matmul f32 bias+silu+add", maxdiff(await ctx.download(y), ref), 1e-4);
  const y16 = ctx.matmul(ctx.upload(a, M, K), ctx.uploadF16(b, K, N), { bias: ctx.upload(bias, 1, N), act: "silu", add: ctx.upload(add, M, N) });
  check("matmul f16 weights", maxdiff(await ctx.download(y16), ref), 2e-2);
  // layernorm
  const R = 5, C = 1024, x = mk(R * C, 6), g = mk(C), be = mk(C);
  const lref = new Float32Array(R * C);
  for (let r = 0; r < R; r++) {
    let m = 0;
    for (let j = 0; j < C; j++) m += x[r * C + j];
    m /= C;
    let v = 0;
    for (let j = 0; j < C; j++) v += (x[r * C + j] - m) ** 2;
    const inv = 1 / Math.sqrt(v / C + 1e-5);
    for (let j = 0; j < C; j++) lref[r * C + j] = (x[r * C + j] - m) * inv * g[j] + be[j];
  }
  check("layernorm", maxdiff(await ctx.download(ctx.layernorm(ctx.upload(x, R, C), ctx.upload(g, 1, C), ctx.upload(be, 1, C))), lref), 1e-4);
  // relShiftB closed form
  const H = 2, t = 7, xs = mk(H * t * (2 * t - 1));
  const rs = new Float32Array(H * t * t);
  for (let hh = 0; hh < H; hh++) for (let i = 0; i < t; i++) for (let j = 0; j < t; j++) rs[(hh * t + i) * t + j] = xs[(hh * t + i) * (2 * t - 1) + t - 1 - i + j];
  check("relShiftB", maxdiff(await ctx.download(ctx.relShiftB(ctx.upload(xs, H * t, 2 * t - 1), H)), rs), 0);
  // staged read is single-use
  const st = ctx.stageDownload(y);
  await st.read();
  let threw = false;
  try {
    await st.read();
  } catch (e) {
    threw = /single-use/.test(e.message);
  }
  check("stageDownload single-use throws", threw ? 0 : 1, 0);
  // fused encoder: packed batch == standalone
  const cfg = { D: 256, DFF: 1024, H: 2, HD: 128, layers: 1, dwK: 9, Csub: 64, Fsub: 16, melBins: 128 };
  const man = {};
  const add_ = (k, n, s) => (man[k] = { data: mk(n, s) });
  for (let i = 0; i < 5; i++) {
    add_(`c${i}w`, i === 2 || i === 4 ? 64 * 64 : 64 * 9, 0.5);
    add_(`c${i}b`, 64, 0.05);
  }
  add_("linw", 64 * 16 * 256, 0.05);
  add_("linb", 256, 0.05);
  for (const ln of ["lnff1", "lnatt", "lnconv", "lnff2", "lnout"]) {
    man[`L0_${ln}_w`] = { data: Float32Array.from({ length: 256 }, () => 1 + (rand() - 0.5) * 0.04) };
    add_(`L0_${ln}_b`, 256, 0.04);
  }
  for (const k of ["ff1w1", "ff2w1"]) add_(`L0_${k}`, 256 * 1024, 0.04);
  for (const k of ["ff1w2", "ff2w2"]) add_(`L0_${k}`, 1024 * 256, 0.04);
  for (const k of ["q", "k", "v", "pos", "out"]) add_(`L0_${k}`, 256 * 256, 0.04);
  add_("L0_pbu", 256, 0.04);
  add_("L0_pbv", 256, 0.04);
  add_("L0_pw1", 512 * 256, 0.04);
  add_("L0_pw2", 256 * 256, 0.04);
  add_("L0_dw", 256 * 9, 1);
  add_("L0_dwb", 256, 0.04);
  const fused = ctx._loadFusedEncoder(man, cfg, { maxT: 64 });
  const mels = [mk(128 * 300, 2), mk(128 * 97, 2)];
  const batch = await ctx.download(ctx._encodeFused(fused, mels));
  const t0 = encoderTsub(300);
  const alone0 = await ctx.download(ctx._encodeFused(fused, [mels[0]]));
  const alone1 = await ctx.download(ctx._encodeFused(fused, [mels[1]]));
  check("fused encoder window 0 packed == alone", maxdiff(batch.subarray(0, t0 * 256), alone0), 1e-4);
  check("fused encoder window 1 packed == alone", maxdiff(batch.subarray(t0 * 256), alone1), 1e-4);
  // several batches of one resident feature stream on the encoder's two lanes == one batch at a time
  {
    const T = 900, feats = mk(128 * T, 2);
    const fs = ctx.upload(feats, 128, T);
    const batches = [{ starts: [0, 300], lens: [300, 97] }, { starts: [150], lens: [64] }, { starts: [500, 10, 800], lens: [400, 33, 100] }];
    const outs = ctx._encodeFusedStreamBatches(fused, fs, batches);
    let md2 = 0;
    for (let b = 0; b < batches.length; b++) {
      const got = await ctx.download(outs[b]);
      const ref = await ctx.download(ctx._info(addonRef.encoderForwardStream(ctx.ctx, fused.enc, fs.h, Int32Array.from(batches[b].starts),
                                                                              Int32Array.from(batches[b].lens), 0, -1)));
      md2 = Math.max(md2, got.length === ref.length ? maxdiff(got, ref) : Infinity);
    }
    check("fused encoder stream batches == one batch at a time", md2, 0);
    ctx.freeTensor(fs);
  }
  ctx._destroyFusedEncoder(fused);
  // log-mel front end: windows of one stream == each window alone; silence -> 0
  const pcmH = mk(16000 * 3, 0.2);
  const pcm = ctx.upload(pcmH, 1, pcmH.length);
  const both = await ctx.download(ctx._melWindows(pcm, [0, 16000], [16000, 32000]));
  const w0 = await ctx.download(ctx._melWindows(pcm, [0], [16000]));
  const w1 = await ctx.download(ctx._melWindows(pcm, [16000], [32000]));
  let md = 0;
  for (let m = 0; m < 128; m++)
    for (let t = 0; t < 300; t++) {
      const v = both[m * 300 + t], r = t < 100 ? w0[m * 100 + t] : w1[m * 200 + t - 100];
      md = Math.max(md, Math.abs(v - r));
    }
  check("melWindows stream == windows alone", md, 0);
  const sil = await ctx.download(ctx._melWindows(ctx.upload(new Float32Array(4800), 1, 4800), [0], [4800]));
  check("melWindows silence normalises to 0", sil.reduce((a, b) => Math.max(a, Math.abs(b)), 0), 0);
  // greedy TDT decode through the binding: constant logits (outW = 0) with
  // token 5 and duration 0 on top -> 10 symbols per frame (MAX_SYMBOLS)
  const dz = (n) => new Float32Array(n);
  const outB = dz(8198);
  outB[5] = 1;
  outB[8193] = 1;
  const tdt = ctx._loadTdtDecoder({ embed: dz(8193 * 640), l0_W: dz(2560 * 640), l0_R: dz(2560 * 640), l0_B: dz(5120), l1_W: dz(2560 * 640),
    l1_R: dz(2560 * 640), l1_B: dz(5120), predW: dz(640 * 640), predB: dz(640), outW: dz(640 * 8198), outB });
  const dres = ctx._tdtDecodeBatch(tdt, ctx.upload(dz(7 * 640), 7, 640), [7], 128)[0];
  const want = [].concat(...Array.from({ length: 7 }, (_, t) => Array(10).fill(t)));
  check("tdtDecode known answer (10 symbols per frame)", dres.ids.every((v) => v === 5) && dres.idFrames.join() === want.join() ? 0 : 1, 0);
  ctx._destroyTdtDecoder(tdt);
  ctx.destroy();
  process.exit(failed ? 1 : 0);
})().catch((e) => {
  console.error(e);
  process.exit(2);
});
