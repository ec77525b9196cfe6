"""Benchmark: the fused Parakeet FastConformer encoder on one MI355X.

Default workload: the full 24-layer encoder with
the dw-striding 8x front end over 16 windows of 15 s (1500 log-mel frames,
128 bins, ~N(0,1), seed 1), random-init f16 weights (seed 1).  One step =
the whole encoder forward over the 16 windows, read in place from the
resident channel-major feature stream (no packed copy).  value = audio-s / wall-s over the K timed steps (inputs resident in
HBM, output left on the device).  The K steps are submitted as one
fa_encoder_forward_stream_batches call, as a serving loop over a long
stream runs them: consecutive batches alternate between the encoder's two
workspace lanes, so two are in flight.  The same K steps one batch at a
time are reported beside it (timing.ms_per_step_one_batch_at_a_time).

The JSON line also carries
  roofline      the dominant kernel (by total time in the timed region),
                timed live with HIP events on the encoder's stream, against
                the MI355X dense f16 MFMA peak (or HBM peak for bandwidth
                kernels); flops/bytes are algorithmic (valid rows only);
  kernels       the same for every kernel class, and the GEMM aggregate;
  cpu_baseline  the CPU oracle (a restatement of the reference's WASM path:
                SSE f32 GEMM without FMA, JS-double LN/softmax/conv) on one
                core, on a bounded sample: preEncode of one window plus one
                conformer layer at full dims, scaled to 24 layers.

Other workloads (--workload): layer, ragged,
gemv (configs[4] GEMV), quant / quant4 (configs[4] encoder, int8 / int4
weights), copy (counter calibration).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
import __graft_entry__ as ge  # noqa: E402

MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense f16
HBM_PEAK_GBS = 8000.0
FULL = dict(D=1024, DFF=4096, H=8, HD=128, layers=24, dwK=9, Csub=256, Fsub=16, melBins=128)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ── algorithmic work per kernel launch (valid rows only) ────────────────────
# Labels that launch the same kernel on the same shape, pooled for the
# roofline (the timed region brackets exactly the class's labels).
_CLASSES = {"ff1_w1": "ff_w1", "ff2_w1": "ff_w1", "ff1_w2": "ff_w2", "ff2_w2": "ff_w2",
            "ln_ff1": "ln", "ln_att": "ln", "ln_conv": "ln", "ln_ff2": "ln"}


def kernel_class(label):
    for suf in ("_x", "_u"):
        if label.endswith(suf) and label[:-len(suf)] in _CLASSES:
            return _CLASSES[label[:-len(suf)]] + suf
    return _CLASSES.get(label, label)


def traffic_for(cls):
    """HBM bytes per launch of a kernel class, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (profiles/traffic_*.json), or None."""
    path = os.path.join(ROOT, "profiles", "traffic_encoder_24L_16x15s_f16.json")
    try:
        with open(path) as f:
            return json.load(f)["classes"].get(cls, {}).get("bytes_per_launch")
    except (OSError, ValueError, KeyError):
        return None


def kernel_work(cfg, lens, layout, fmt="f16"):
    """label -> (kind, amount per launch); kind 'flop' (MFMA) or 'byte' (HBM).
    Python ints throughout (numpy int32 lengths would overflow the products)."""
    lens = [int(t) for t in lens]
    D, DFF, C, F, MB = (int(cfg[k]) for k in ("D", "DFF", "Csub", "Fsub", "melBins"))
    s2 = lambda t: (t - 1) // 2 + 1
    T1 = [s2(t) for t in lens]
    T2 = [s2(t) for t in T1]
    T3 = [s2(t) for t in T2]
    R0, R1, R2, M = sum(lens), sum(T1), sum(T2), sum(T3)
    att = sum(2 * t * t * D * 3 for t in T3)  # (q+u)kᵀ, bd (t x t band entries used), P·V
    gemm = {"ff1_w1": 2 * M * D * DFF, "ff1_w2": 2 * M * D * DFF, "ff2_w1": 2 * M * D * DFF, "ff2_w2": 2 * M * D * DFF,
            "qkv": 2 * M * D * 3 * D, "attn_out": 2 * M * D * D, "pw1_glu": 2 * M * D * 2 * D, "pw2": 2 * M * D * D}
    w = {
        "pack_windows": ("byte", R0 * MB * 8),
        "sub_c01": ("byte", R0 * MB * 4 + R2 * (MB // 4) * C * 2 * 2),  # mel in, hi/lo pairs out
        "sub_pw2": ("flop", 2 * R2 * (MB // 4) * C * C),
        "sub_dw3": ("byte", R2 * (MB // 4) * C * 4 + M * F * C * 2 * 2),  # f32 in, hi/lo pairs out
        "sub_pw4": ("flop", 2 * M * F * C * C),
        "sub_linear": ("flop", 2 * M * F * C * D),
        "ln_out": ("byte", M * D * 8),
        "ln_out_ff1": ("byte", M * D * 10),    # f32 in + out, f16 out
        "ln_out_ff1_x": ("byte", M * D * 12),  # plus the lo plane
        "v_transpose": ("byte", M * D * 2 * 2),
        "attention": ("flop", att), "attention_x": ("flop", att),
        "dwconv": ("byte", M * D * 4), "dwconv_f32": ("byte", M * D * 6), "dwconv_lo": ("byte", M * D * 6), "dwconv_x": ("byte", M * D * 8),
        "zero_pad": ("byte", 0), "enc_src": ("byte", 0), "enc_in": ("byte", R0 * MB * 8), "enc_out": ("byte", M * D * 8),
    }
    if fmt in ("int8", "int4"):  # one layer's linears widened to f16: packed weights (+ int4 scales) in, f16 out
        nw = 4 * D * DFF + 3 * D * D + D * D + 2 * D * D + D * D
        w["dequant_w"] = ("byte", nw * 2 + (nw if fmt == "int8" else nw // 2 + nw // 32 * 2))
    for ln in ("ln_ff1", "ln_att", "ln_conv", "ln_ff2"):
        w[ln] = ("byte", M * D * 6)       # f32 in, f16 out
        w[ln + "_x"] = ("byte", M * D * 8)  # f32 in, f16 hi + lo planes out
    for k, f in gemm.items():  # algorithmic flops: a lo plane (_x) or a lo output (_u, _f32) does not add any
        for suf in ("", "_x", "_u", "_f32"):
            w[k + suf] = ("flop", f)
    return w


def summarize(recs, steps):
    """recs: (label, ms, kind, amount) per launch -> per-label summary."""
    agg = {}
    for lab, ms, kind, amt in recs:
        a = agg.setdefault(lab, [0, 0.0, kind, 0])
        a[0] += 1
        a[1] += ms
        a[3] += amt
    out = {}
    for lab, (n, ms, kind, amt) in agg.items():
        rec = {"launches": n, "avg_us": round(ms / n * 1e3, 2), "total_ms_per_step": round(ms / steps, 3)}
        if amt:
            if kind == "flop":
                tf = amt / (ms * 1e-3) / 1e12
                rec.update(tflops=round(tf, 1), frac=round(tf / MFMA_F16_PEAK_TFLOPS, 4), bound="mfma")
            else:
                gbs = amt / (ms * 1e-3) / 1e9
                rec.update(gbs=round(gbs, 1), frac=round(gbs / HBM_PEAK_GBS, 4), bound="hbm")
        rec["_work"] = amt
        out[lab] = rec
    return out


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


_CFG0_SCRIPT = r"""
import sys, time, numpy as np
sys.path.insert(0, sys.argv[1])
import oracle as orc
orc.set_threads(1)
rng = np.random.default_rng(0)
x = rng.standard_normal((750, 1024), dtype=np.float32)
w = (rng.standard_normal((1024, 4096)) * 0.02).astype(np.float16).astype(np.float32)
b = (rng.standard_normal((1, 4096)) * 0.01).astype(np.float32)
reps = int(sys.argv[2])
t0 = time.perf_counter()
for _ in range(reps):
    orc.matmul(x, w, bias=b)
print(time.perf_counter() - t0)
"""


def cpu_baseline_cfg0(instances: int, reps: int = 2):
    """X[750,1024] f32 ~N(0,1) @ W[1024,4096] (f16 values held as
    f32, as WasmContext.uploadF16 keeps them) + bias, through the oracle's
    restatement of the WASM matmul (SSE, i-k-j, no FMA), in `instances`
    independent single-threaded processes at once.  Returns (GFLOP/s of one
    instance alone, aggregate GFLOP/s of all instances)."""
    import subprocess

    odir = os.path.join(ROOT, "oracle")
    flop = 2.0 * 750 * 1024 * 4096 + 750 * 4096
    one = float(subprocess.run([sys.executable, "-c", _CFG0_SCRIPT, odir, str(reps)], capture_output=True, text=True, check=True).stdout)
    t0 = time.perf_counter()
    procs = [subprocess.Popen([sys.executable, "-c", _CFG0_SCRIPT, odir, str(reps)], stdout=subprocess.PIPE, text=True) for _ in range(instances)]
    for p in procs:
        p.communicate()
        if p.returncode:
            raise RuntimeError("configs[0] CPU instance failed")
    agg_wall = time.perf_counter() - t0
    return flop * reps / one / 1e9, flop * reps * instances / agg_wall / 1e9


def cpu_baseline():
    """Oracle on 1 core: preEncode of one 15 s window + one full-size layer,
    scaled to the 24-layer encoder; plus configs[0] (the FFN linear) on one
    core and as one single-threaded instance per host core (at most 16, the
    box's CPU share for one GPU).  Run before the GPU is touched."""
    fa = ge.load_package()
    orc = ge.load_oracle()
    orc.set_threads(1)
    cfg = dict(FULL)
    man = fa.synth.make_weights(cfg, seed=1, layers=1)
    mel = fa.synth.make_features(128, 1500, seed=1)
    t0 = time.perf_counter()
    orc.encode_batch(cfg, man, mel, layers=0)
    t_pre = time.perf_counter() - t0
    t0 = time.perf_counter()
    orc.encode_batch(cfg, man, mel, layers=1)
    t_layer = time.perf_counter() - t0 - t_pre
    per_window = t_pre + 24 * t_layer
    ncpu = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    inst = max(1, min(16, ncpu))
    g1, gagg = cpu_baseline_cfg0(inst)
    return {"value": round(15.0 / per_window, 3), "unit": "audio-s/wall-s", "cores": 1, "kind": "port",
            "sample": f"1 window x 15 s: preEncode {t_pre:.2f} s + 1 of 24 layers {t_layer:.2f} s, scaled to 24 layers "
                      f"(oracle/fa_oracle.c, single thread)",
            "cpu_model": cpu_model(), "host_cores_visible": ncpu,
            "configs0_ffn_linear": {"gflops_1core": round(g1, 2), "instances": inst, "gflops_aggregate": round(gagg, 2),
                                    "aggregate_audio_s_per_wall_s_est": round(15.0 / per_window * gagg / g1, 2),
                                    "sample": "X[750,1024] @ W[1024,4096] + bias (6.29 GFLOP), 2 reps per instance, "
                                              "oracle SSE matmul without FMA (lib.rs:59-94 order)"}}


def run_encoder(args, fa, ctx, cfg, batches, feats_h, layout, fmt="f16", seed=1):
    """batches: list of (starts, lens) into the resident feature stream feats_h
    [melBins, T].  One step = encode every batch, its windows read in place
    from the stream (fa_encoder_forward_stream)."""
    man = fa.synth.make_weights(cfg, seed=seed)
    log(f"[bench] weights generated ({sum(v.size for v in man.values()) / 1e6:.0f} M values); loading {fmt}")
    max_T = max(fa.tsub(int(t)) for _, ln in batches for t in ln)
    enc = fa.FusedEncoder(ctx, man, fmt, max_T=max_T)
    del man
    feats = ctx.upload(feats_h, feats_h.shape[0], feats_h.shape[1])
    batches = [(np.asarray(st, np.int32), np.asarray(ln, np.int32)) for st, ln in batches]
    works = [kernel_work(cfg, ln, layout, fmt) for _, ln in batches]

    def run_batch(st, ln):
        a = ctx.pushArena()
        enc.forwardStream(feats, st, ln, layout)
        ctx.popArena(a)

    def step():
        for st, ln in batches:
            run_batch(st, ln)

    def steps_pipelined(k):
        # k steps' batches in one call: consecutive batches alternate between
        # the encoder's two workspace lanes (streams of their own), so one
        # batch's kernel tails and write-backs overlap the next batch's kernels
        a = ctx.pushArena()
        enc.forwardStreamBatches(feats, batches * k, layout)
        ctx.popArena(a)

    for _ in range(args.warmup):
        step()
    steps_pipelined(2)  # both lanes capture their forward graph before the timed region
    ctx.sync()
    # timed region: K steps as a serving loop runs them (every batch one
    # captured hipGraph replay, two batches in flight on the two lanes)
    t0 = time.perf_counter()
    steps_pipelined(args.steps)
    ctx.sync()
    wall = time.perf_counter() - t0
    # the same K steps one batch at a time on the context stream (latency view)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    ctx.sync()
    wall_serial = time.perf_counter() - t0
    # discovery pass: every launch of one eager step bracketed (per batch, so
    # each launch is credited with its own batch's work)
    recs = []
    for (st, ln), work in zip(batches, works):
        ctx.startProfile(200000)
        run_batch(st, ln)
        for r in ctx.endProfile():
            kind, amt = work.get(r["label"], ("byte", 0))
            recs.append((r["label"], r["ms"], kind, amt))
    ctot = {}
    for lab, ms, _, _ in recs:
        ctot[kernel_class(lab)] = ctot.get(kernel_class(lab), 0.0) + ms
    dom = max(ctot, key=ctot.get)
    dom_labels = sorted({lab for lab, *_ in recs if kernel_class(lab) == dom})
    per_step_launches = sum(1 for lab, *_ in recs if lab in dom_labels)
    dom_work = sum(amt for lab, _, _, amt in recs if lab in dom_labels)  # per step
    # roofline region: K eager steps with only the dominant class bracketed by
    # hipExtLaunchKernelGGL start/stop events on the encoder's stream
    ctx.sync()
    ctx.startProfile(200000, only=",".join(dom_labels))
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    ctx.sync()
    wall_eager = time.perf_counter() - t0
    prof_dom = [r for r in ctx.endProfile() if r["label"] in dom_labels]
    assert len(prof_dom) == per_step_launches * args.steps, (len(prof_dom), per_step_launches)
    enc.close()
    ctx.freeTensor(feats)
    return dict(wall=wall, wall_serial=wall_serial, wall_eager=wall_eager, recs=recs, dom=dom, prof_dom=prof_dom, dom_work=dom_work, works=works)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="encoder", choices=["encoder", "layer", "ragged", "quant", "quant4", "gemv", "copy", "mel", "decode", "e2e", "stream", "oppath"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--windows", type=int, default=16, help="decode workload: windows per decode call (1..64)")
    ap.add_argument("--audio-sec", type=float, default=470.0, help="e2e workload: seconds of synthetic audio (at most 470: longer inputs faulted)")
    ap.add_argument("--streams", default="4,8,16,32", help="stream workload: concurrent stream counts timed after the single stream")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(f"bench.py: this build measures one GPU only (asked for {args.gpus}); multi-GPU runs are not part of it", file=sys.stderr)
        sys.exit(2)
    cpu = None
    if not args.no_cpu and args.workload == "encoder":
        log("[bench] CPU baseline (oracle, bounded sample) before the GPU is touched")
        cpu = cpu_baseline()
    fa = ge.load_package()
    ctx = fa.createContext("hip")
    if args.workload == "gemv":
        return bench_gemv(args, fa, ctx)
    if args.workload == "copy":
        return bench_copy(args, fa, ctx)
    if args.workload == "mel":
        return bench_mel(args, fa, ctx)
    if args.workload == "decode":
        return bench_decode(args, fa, ctx)
    if args.workload == "e2e":
        return bench_e2e(args, fa, ctx)
    if args.workload == "stream":
        return bench_stream(args, fa, ctx)
    if args.workload == "oppath":
        return bench_oppath(args, fa, ctx)
    cfg = dict(FULL)
    layout = "packed"
    rng = np.random.default_rng(1)
    if args.workload in ("encoder", "quant", "quant4", "layer"):
        n = 8 if args.workload == "layer" else 16
        lens = [1500] * n
        feats_h = rng.standard_normal((cfg["melBins"], sum(lens)), dtype=np.float32)
        batches = [(np.arange(n) * 1500, lens)]
        audio_s = 15.0 * n
        if args.workload == "layer":
            cfg["layers"] = 1
            workload = "configs[1]-shaped: one FastConformer layer (plus front end), 8 windows x 188 frames"
        else:
            workload = ("configs[2]: 24-layer FastConformer encoder + dw-striding 8x subsampling, 16 windows x 15 s "
                        "(1500 mel frames), read in place from the feature stream")
    else:
        total = 360000
        starts, lens = fa.windowing.planRaggedWindows(total, 200, 3000, 100, seed=1)
        feats_h = rng.standard_normal((cfg["melBins"], total), dtype=np.float32)
        batches = [(starts[b], lens[b]) for b in (np.asarray(g) for g in fa.windowing.packBatches(lens, 32))]
        audio_s = total * 0.01  # the stream's span: overlaps are not counted twice
        workload = (f"configs[3]: 3600 s stream cut into {len(lens)} ragged windows (2-30 s, 1 s overlap), read in place "
                    f"as {len(batches)} batches of <= 32 (sorted by length), 24 layers")
    fmt = {"quant": "int8", "quant4": "int4"}.get(args.workload, "f16")
    r = run_encoder(args, fa, ctx, cfg, batches, feats_h, layout, fmt)
    kern = summarize(r["recs"], 1)
    gemm_labels = [k for k, v in kern.items() if v.get("bound") == "mfma" and not k.startswith("attention")]
    gemm_ms = sum(kern[k]["total_ms_per_step"] for k in gemm_labels)
    gemm_flop = sum(kern[k]["_work"] for k in gemm_labels)
    gemm_tf = gemm_flop / (gemm_ms * 1e-3) / 1e12 if gemm_ms else 0.0
    for v in kern.values():
        v.pop("_work")
    prof_dom = r["prof_dom"]
    dom_ms_per_step = sum(x["ms"] for x in prof_dom) / args.steps
    dom_us = sum(x["ms"] for x in prof_dom) / len(prof_dom) * 1e3
    kind = next(k for lab, _, k, _ in r["recs"] if kernel_class(lab) == r["dom"])
    rate = r["dom_work"] / (dom_ms_per_step * 1e-3)
    if kind == "flop":
        ach = rate / 1e12
        roof = {"bound": "mfma", "achieved": round(ach, 1), "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(ach / MFMA_F16_PEAK_TFLOPS, 4)}
    else:
        ach = rate / 1e9
        roof = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4)}
    traffic = traffic_for(r["dom"]) if args.workload == "encoder" else None
    roof.update(kernel=r["dom"], traffic=traffic, avg_us=round(dom_us, 2), launches_timed=len(prof_dom),
                work_per_launch=round(r["dom_work"] * args.steps / len(prof_dom)))
    valid_frames = sum(int(fa.tsub(int(t))) for _, ln in batches for t in ln)
    res = {
        "metric": "encoder audio-s/wall-s at 1 GPU", "value": round(audio_s * args.steps / r["wall"], 1), "unit": "audio-s/wall-s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(r["wall"] / args.steps * 1e3, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f16" if fmt == "f16" else f"{fmt}-weights/f16",
        "data": "synthetic log-mel ~N(0,1) (seed 1), random-init weights (seed 1)",
        "config": {"workload": workload, "windows": sum(len(ln) for _, ln in batches), "batches": len(batches),
                   "mel_frames": int(sum(int(t) for _, ln in batches for t in ln)), "encoder_frames": valid_frames,
                   "audio_s_per_step": audio_s, "layers": cfg["layers"], "weights": fmt, "parallelism": "single GPU"},
        "timing": {"value_region": "K steps submitted as one fa_encoder_forward_stream_batches call: every batch one hipGraph replay, "
                                   "consecutive batches on the encoder's two workspace lanes (two in flight), no events",
                   "ms_per_step_one_batch_at_a_time": round(r["wall_serial"] / args.steps * 1e3, 3),
                   "roofline_region": "K further eager steps, only the dominant kernel class bracketed by HIP events",
                   "ms_per_step_eager": round(r["wall_eager"] / args.steps * 1e3, 3)},
        "roofline": roof,
        "gemm_aggregate": {"tflops": round(gemm_tf, 1), "frac": round(gemm_tf / MFMA_F16_PEAK_TFLOPS, 4), "ms_per_step": round(gemm_ms, 3)},
        "kernels": kern,  # discovery pass (every launch event-bracketed: inflated by the events)
    }
    if cpu is not None:
        res["cpu_baseline"] = cpu
    print(json.dumps(res), flush=True)


def bench_mel(args, fa, ctx):
    """The log-mel front end (fa_mel_windows) over the configs[2] windows: 16
    windows of 15 s cut at the pipeline's 13 s hop from one resident 210 s
    sample stream (synthetic: a gliding harmonic tone plus noise, seed 1).
    value = audio-s (16 x 15 s per step) / wall-s; the dominant kernel
    (mel_frames) is timed with event pairs in the timed region."""
    rng = np.random.default_rng(1)
    n_win, win, hop = 16, 240000, 208000
    n = hop * (n_win - 1) + win
    t = np.arange(n) / 16000
    pcm_h = (0.3 * np.sin(2 * np.pi * (150 + 50 * np.sin(2 * np.pi * 0.5 * t)) * t) + 0.05 * rng.standard_normal(n)).astype(np.float32)
    pcm = ctx.upload(pcm_h.reshape(1, -1), 1, n)
    starts, lens = [i * hop for i in range(n_win)], [win] * n_win

    def step():
        a = ctx.pushArena()
        ctx.melWindows(pcm, starts, lens)
        ctx.popArena(a)

    for _ in range(args.warmup):
        step()
    ctx.sync()
    ctx.startProfile(100000)
    step()
    prof_all = ctx.endProfile()
    ctx.sync()
    ctx.startProfile(100000, only="mel_frames")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    ctx.sync()
    wall = time.perf_counter() - t0
    prof = [r for r in ctx.endProfile() if r["label"] == "mel_frames"]
    frames = n_win * (win // 160)
    # algorithmic bytes of mel_frames: each window's samples (with the 200-sample
    # halo of its frames) read once, the f32 raw log-mel written once
    fbytes = n_win * (win + 400) * 4 + 128 * frames * 4
    us = sum(r["ms"] for r in prof) / len(prof) * 1e3
    kern = {}
    for r in prof_all:
        k = kern.setdefault(r["label"], {"launches": 0, "avg_us": 0.0})
        k["launches"] += 1
        k["avg_us"] += r["ms"] * 1e3
    for k in kern.values():
        k["avg_us"] = round(k["avg_us"] / k["launches"], 2)
    audio_s = n_win * win / 16000 * args.steps
    line = {"metric": "log-mel front end audio-s/wall-s at 1 GPU", "value": round(audio_s / wall, 1), "unit": "audio-s/wall-s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(wall / args.steps * 1e3, 3), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "f64", "data": "synthetic PCM: gliding harmonic tone + noise (seed 1)",
            "config": {"workload": "configs[2] windows: 16 x 15 s cut at a 13 s hop from a 210 s stream, 128 mels, per-feature normalisation",
                       "windows": n_win, "frames": frames},
            "roofline": {"bound": "hbm", "achieved": round(fbytes / us * 1e-3, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(fbytes / us * 1e-3 / HBM_PEAK_GBS, 4), "traffic": None, "kernel": "mel_frames", "avg_us": round(us, 2),
                         "launches_timed": len(prof)},
            "kernels": kern}
    if not args.no_cpu:
        orc = ge.load_oracle()
        orc.set_threads(1)
        t0 = time.perf_counter()
        for i in range(2):
            orc.mel(pcm_h[starts[i]:starts[i] + win])
        cw = time.perf_counter() - t0
        line["cpu_baseline"] = {"value": round(2 * win / 16000 / cw, 1), "unit": "audio-s/wall-s", "cores": 1, "kind": "port",
                                "sample": "2 of the 16 windows (30 s of audio) through the oracle's restatement of nemotron-mel.js (oracle/fa_oracle.c or_mel, single thread)"}
    print(json.dumps(line), flush=True)


def bench_decode(args, fa, ctx):
    """Greedy TDT decoding (fa_tdt_decode) of the configs[2] encoder output: 16
    windows x 188 pre-projected frames (synthetic ~N(0,1), seed 1; synthetic
    decoder weights with a blank bias that gives ~1 token per 3 frames).
    value = audio-s (16 x 15 s) / wall-s of the whole decode call (steps in
    lock-step on the GPU, results copied to the host)."""
    dec_w = fa.synth.make_decoder_weights(1)
    n_win, T = args.windows, 188
    frames_h = np.concatenate([fa.synth.make_projected_frames(T, seed=100 + i) for i in range(n_win)])
    frames = ctx.upload(frames_h, frames_h.shape[0], 640)
    dec = fa.TdtDecoder(ctx, dec_w)
    lens = [T] * n_win
    for _ in range(args.warmup):
        dec.decodeBatch(frames, lens)
    ctx.startProfile(200000)
    res = dec.decodeBatch(frames, lens)
    prof = ctx.endProfile()
    tokens = sum(r["count"] for r in res)
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        dec.decodeBatch(frames, lens)
    wall = time.perf_counter() - t0
    kern = {}
    for r in prof:
        k = kern.setdefault(r["label"], {"launches": 0, "total_ms": 0.0})
        k["launches"] += 1
        k["total_ms"] += r["ms"]
    for k in kern.values():
        k["avg_us"] = round(k["total_ms"] / k["launches"] * 1e3, 2)
        k["total_ms"] = round(k["total_ms"], 3)
    j = kern.get("tdt_joint", {"avg_us": 0.0, "launches": 0})
    jbytes = 640 * 8198 * 4  # the joint matrix, read once per step for the batch
    audio_s = n_win * 15.0 * args.steps
    line = {"metric": "greedy TDT decode audio-s/wall-s at 1 GPU", "value": round(audio_s / wall, 1), "unit": "audio-s/wall-s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(wall / args.steps * 1e3, 3), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic projected frames ~N(0,1), synthetic decoder weights (seed 1)",
            "config": {"workload": f"configs[2] encoder output: {n_win} windows x 188 frames, greedy TDT (durations 0..4, <= 10 symbols/frame)",
                       "windows": n_win, "frames": n_win * T, "tokens": tokens, "decode_steps": j["launches"]},
            "roofline": {"bound": "hbm", "achieved": round(jbytes / max(j["avg_us"], 1e-9) * 1e-3, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(jbytes / max(j["avg_us"], 1e-9) * 1e-3 / HBM_PEAK_GBS, 4), "traffic": None, "kernel": "tdt_joint",
                         "avg_us": j["avg_us"], "launches_timed": j["launches"]},
            "kernels": kern}
    if not args.no_cpu:
        orc = ge.load_oracle()
        t0 = time.perf_counter()
        orc.tdt_decode(dec_w, frames_h[:T])
        cw = time.perf_counter() - t0
        line["cpu_baseline"] = {"value": round(15.0 / cw, 1), "unit": "audio-s/wall-s", "cores": 1, "kind": "port",
                                "sample": "1 of the 16 windows through the oracle's restatement of decode_proj (oracle/fa_oracle.c or_tdt_decode_proj, single thread)"}
    dec.close()
    print(json.dumps(line), flush=True)


def bench_e2e(args, fa, ctx):
    """Windowed transcription end to end (pipeline.transcribeWindowed): 470 s
    of synthetic speech-like PCM (37 windows, 3 groups) -> log-mel -> 24-layer encoder (f16 weights) ->
    joint projection -> greedy TDT decode -> seam stitching; the reference's
    headline configuration is a 1 h file (README.md:10-12: 293x RTFx on
    Chrome/macOS WebGPU), whose transcription faulted here.  One step = one full transcription, stage by stage
    on the context stream (pipelined=False: the cross-stream pipelined form
    stays off, its full-size run made an illegal memory access with no cause
    shown), groups of up to 32 windows; value = audio-s / wall-s (RTFx).  One
    more pass with a synchronisation after each stage gives the stages' own
    times.  No profile window is open.  Synthetic weights: the tokens are
    meaningless, every stage does its full work."""
    import importlib
    pl = importlib.import_module(fa.__name__ + ".pipeline")
    seconds = args.audio_sec
    if seconds > 470.0:
        raise SystemExit("bench --workload e2e runs at most 470 s of audio: every transcription of the hour (64- and 32-window groups, stage "
                         "by stage and pipelined) made an illegal memory access on the GPU with no cause shown yet; 470 s ran")
    audio = fa.synth.make_pcm(seconds, seed=1)
    man = fa.synth.make_weights(dict(FULL), seed=1)
    enc = fa.FusedEncoder(ctx, man, "f16", max_T=188)
    del man
    dec_w = fa.synth.make_decoder_weights(1)
    dec = fa.TdtDecoder(ctx, dec_w)
    W, b = fa.synth.make_joint_projection(2)
    projW, projB = ctx.upload(W, W.shape[0], W.shape[1]), ctx.upload(b.reshape(1, -1), 1, b.size)
    log(f"[bench] e2e: {seconds:.0f} s of audio, weights loaded")
    for i in range(max(1, args.warmup)):
        log(f"[bench] e2e warmup transcription {i}")
        r = pl.transcribeWindowed(ctx, enc, dec, projW, projB, audio, pipelined=False)
    log(f"[bench] e2e warm: {r['stats']}")
    ctx.sync()
    t0 = time.perf_counter()
    for i in range(args.steps):
        r = pl.transcribeWindowed(ctx, enc, dec, projW, projB, audio, pipelined=False)
        log(f"[bench] e2e step {i}: {time.perf_counter() - t0:.3f} s")
    wall = (time.perf_counter() - t0) / args.steps
    # the stages' own times: every group's stages one after another, synchronised
    tsub = importlib.import_module(fa.__name__ + ".encoder").tsub
    x = np.ascontiguousarray(audio, np.float32)
    total = len(x)
    starts = pl.planWindows(total, 240000, 208000)
    groups = pl.groupWindows(starts, total, 240000, pl.MAX_WINDOWS)
    pcm = ctx.upload(x.reshape(1, -1), 1, total)
    stages = {"mel": 0.0, "encoder": 0.0, "projection": 0.0, "decode": 0.0}
    for grp in groups:
        st = [starts[i] for i in grp]
        ln = [min(s_ + 240000, total) - s_ for s_ in st]
        keep = [j for j, l in enumerate(ln) if l // 160 > 0]
        if not keep:
            continue
        st, ln = [st[j] for j in keep], [ln[j] for j in keep]
        T = [l // 160 for l in ln]
        offs = np.concatenate([[0], np.cumsum(T)[:-1]]).astype(np.int32)
        arena = ctx.pushArena()
        t = time.perf_counter()
        feats = ctx.melWindows(pcm, st, ln)
        ctx.sync()
        stages["mel"] += time.perf_counter() - t
        t = time.perf_counter()
        y = enc.forwardStream(feats, offs, T)
        ctx.sync()
        stages["encoder"] += time.perf_counter() - t
        t = time.perf_counter()
        proj = ctx.matmul(y, projW, bias=projB)
        ctx.sync()
        stages["projection"] += time.perf_counter() - t
        t = time.perf_counter()
        dec.decodeBatch(proj, [tsub(v) for v in T])
        stages["decode"] += time.perf_counter() - t
        ctx.popArena(arena)
    ctx.freeTensor(pcm)
    line = {"metric": "end-to-end transcription RTFx (audio-s/wall-s) at 1 GPU", "value": round(seconds / wall, 1), "unit": "audio-s/wall-s",
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(wall * 1e3, 2), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": round(seconds / wall / 293.0, 2), "baseline_note": "293x RTFx, 1 h file, Chrome/macOS WebGPU (README.md:10-12); other hardware",
            "dtype": "f16", "data": "synthetic speech-like PCM, random-init encoder/decoder/projection weights",
            "config": {"workload": f"{seconds:.0f} s PCM, 15 s windows at 13 s hop, groups of up to {pl.MAX_WINDOWS} windows, Parakeet TDT 0.6B shapes "
                                   "(24 layers), stage by stage on one stream",
                       "windows": r["stats"]["windows"], "groups": r["stats"]["groups"], "tokens": r["stats"]["tokens"]},
            "stages_ms": {k: round(v * 1e3, 2) for k, v in stages.items()}}
    if not args.no_cpu:
        # one window through the oracle: mel + preEncode + 1 layer (scaled to 24) + decode of the window's frames
        orc = ge.load_oracle()
        orc.set_threads(1)
        seg = audio[:240000]
        t0 = time.perf_counter()
        orc.mel(seg, 128, 2.0 ** -24, True)
        t_mel = time.perf_counter() - t0
        enc_cpu = cpu_baseline()
        t_enc = 15.0 / enc_cpu["value"]
        frames = fa.synth.make_projected_frames(188, seed=9)
        t0 = time.perf_counter()
        orc.tdt_decode(dec_w, frames)
        t_dec = time.perf_counter() - t0
        per_window = t_mel + t_enc + t_dec
        line["cpu_baseline"] = {"value": round(13.0 / per_window, 3), "unit": "audio-s/wall-s", "cores": 1, "kind": "port",
                                "sample": f"one 15 s window (13 s of new audio per window): mel {t_mel:.2f} s + encoder {t_enc:.1f} s "
                                          f"(preEncode + 1 layer scaled to 24) + decode {t_dec:.2f} s, oracle/fa_oracle.c single thread"}
    dec.close()
    enc.close()
    print(json.dumps(line), flush=True)


def bench_oppath(args, fa, ctx):
    """configs[2] through the reference's own op sequence (parakeetEncodeBatch,
    raw-encoder.js:235-386, on the ComputeContext ops: ~700 launches per
    batch) with f16 weights (uploadF16, the probed uploadTileMajorF16 of a Node
    host), beside the fused encoder on the same windows: the throughput an
    unchanged engine gets from this backend.  Timed twice: the multi-op
    attention chain, and the reference's opt-in attnFused member."""
    man = fa.synth.make_weights(dict(FULL), seed=1)
    mels = fa.synth.make_features(FULL["melBins"], 1500, seed=1, W=16)
    enc = fa.loadParakeetEncoder(ctx, man, weights="f16")
    del man
    line_kern = {}

    def run(fused):
        a = ctx.pushArena()
        y, _ = fa.parakeetEncodeBatch(ctx, enc, mels, attnFused=fused)
        ctx.sync()
        ctx.popArena(a)

    res = {}
    for fused in (False, True):
        for _ in range(max(1, args.warmup)):
            run(fused)
        t0 = time.perf_counter()
        for _ in range(args.steps):
            run(fused)
        wall = (time.perf_counter() - t0) / args.steps
        res["attnFused" if fused else "chain"] = {"ms_per_step": round(wall * 1e3, 2), "value": round(240.0 / wall, 1)}
        log(f"[bench] op path, attnFused={fused}: {wall * 1e3:.1f} ms per 16 x 15 s")
    # launches per batch and the op path's busiest kernels, from one profiled batch
    ctx.startProfile(20000)
    run(True)
    prof = ctx.endProfile()
    for r in prof:
        k = line_kern.setdefault(r["label"], {"launches": 0, "ms": 0.0})
        k["launches"] += 1
        k["ms"] += r["ms"]
    top = sorted(line_kern.items(), key=lambda kv: -kv[1]["ms"])[:12]
    best = max(res.values(), key=lambda v: v["value"])
    line = {"metric": "encoder audio-s/wall-s at 1 GPU (reference op sequence)", "value": best["value"], "unit": "audio-s/wall-s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": best["ms_per_step"], "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "f16", "data": "synthetic log-mel ~N(0,1) (seed 1), random-init weights (seed 1)",
            "config": {"workload": "configs[2] (24 layers, 16 x 15 s) through parakeetEncodeBatch's ComputeContext calls, f16 weights, one "
                                   "withBatchSync per batch", "launches_per_batch": len(prof)},
            "variants": res,
            "kernels_top": {k: {"launches": v["launches"], "ms_per_batch": round(v["ms"], 3)} for k, v in top}}
    print(json.dumps(line), flush=True)


def bench_stream(args, fa, ctx):
    """Streaming encode (the native stream: fa_stream_* over the fused encoder,
    device-resident K/V and conv caches) of 30 s of synthetic log-mel pushed
    160 ms at a time (16 mel frames = one chunk of 2 encoder frames), with
    this path's Parakeet shapes (24 layers, d_model 1024, f16 weights) and the
    EOU streaming config (eou-parakeet/config.js: chunk 2, left 70, causal conv
    with LayerNorm, subsampling pads t2 b1 l2 r1).  value = audio-s / wall-s
    of one stream; per-chunk latency in the config."""
    cfg = dict(FULL, subPad={"t": 2, "b": 1, "l": 2, "r": 1}, convCausal=True, attChunk=2, attLeft=70, Fsub=17)
    man = fa.synth.make_weights(cfg, seed=1)
    enc = fa.FusedEncoder(ctx, man, "f16", max_T=128, cfg=cfg)
    seconds, piece = 30.0, 16
    mel = fa.synth.make_features(128, int(seconds * 100), seed=2)[0]

    def run():
        st = fa.createEncodeStream(ctx, enc)
        n = 0
        for t in range(0, mel.shape[1], piece):
            o = fa.encodeStreamPush(ctx, st, mel[:, t:t + piece])
            n += 0 if o is None else o.shape[0]
        o = fa.encodeStreamFlush(ctx, st)
        n += 0 if o is None else o.shape[0]
        fa.disposeEncodeStream(ctx, st)
        return n

    for _ in range(args.warmup):
        frames = run()
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        frames = run()
    wall = (time.perf_counter() - t0) / args.steps
    chunks = mel.shape[1] // piece
    # per-kernel GPU time of steady-state chunk passes, eager under HIP events
    # (a profiled pass is not graph-replayed)
    st = fa.createEncodeStream(ctx, enc)
    for t in range(0, 64 * piece, piece):  # past the first pass and the cache fill
        fa.encodeStreamPush(ctx, st, mel[:, t:t + piece])
    ctx.sync()
    ctx.startProfile(200000)
    prof_chunks = 8
    for t in range(64 * piece, (64 + prof_chunks) * piece, piece):
        fa.encodeStreamPush(ctx, st, mel[:, t:t + piece])
    prof = ctx.endProfile()
    fa.disposeEncodeStream(ctx, st)
    kern = {}
    for r in prof:
        k = kern.setdefault(r["label"], {"launches": 0, "ms": 0.0})
        k["launches"] += 1
        k["ms"] += r["ms"]
    kern = {lab: {"launches_per_chunk": v["launches"] // prof_chunks, "us_per_chunk": round(v["ms"] * 1e3 / prof_chunks, 1)}
            for lab, v in sorted(kern.items(), key=lambda kv: -kv[1]["ms"])}
    # several streams in flight: each 160 ms tick pushes one piece to every
    # stream in one fa_stream_push_many call; streams at the same point run as
    # one batched pass (up to 16 per pass, passes on the encoder's lanes)
    def run_many(n):
        sts = [fa.createEncodeStream(ctx, enc) for _ in range(n)]
        for t in range(0, mel.shape[1], piece):
            fa.encodeStreamsPush(ctx, sts, [mel[:, t:t + piece]] * n)
        for st in sts:
            fa.encodeStreamFlush(ctx, st)
            fa.disposeEncodeStream(ctx, st)

    concurrent = {}
    for n in [int(v) for v in args.streams.split(",") if v.strip()]:
        run_many(n)
        ctx.sync()
        t0 = time.perf_counter()
        run_many(n)
        ctx.sync()
        wn = time.perf_counter() - t0
        concurrent[str(n)] = {"aggregate_audio_s_per_wall_s": round(n * seconds / wn, 1), "per_stream_x_real_time": round(seconds / wn, 1),
                              "ms_per_tick": round(wn * 1e3 / chunks, 3)}
        log(f"[bench] {n} streams: {concurrent[str(n)]}")
    line = {"metric": "streaming encode audio-s/wall-s per stream at 1 GPU", "value": round(seconds / wall, 1), "unit": "audio-s/wall-s",
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(wall * 1e3, 2), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "f16", "data": "synthetic log-mel ~N(0,1), random-init weights",
            "config": {"workload": "30 s pushed in 160 ms pieces, 24 layers d_model 1024, chunk 2 / left 70 (EOU streaming config), native fused stream",
                       "frames": frames, "chunks": chunks, "ms_per_chunk": round(wall * 1e3 / chunks, 3)},
            "concurrent_streams": concurrent,
            "kernels_eager_per_chunk": kern,
            "kernel_us_per_chunk_eager": round(sum(v["us_per_chunk"] for v in kern.values()), 1)}
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import np_ref
        import torch
        torch.set_num_threads(1)
        seg = mel[:, :300]  # 3 s
        t0 = time.perf_counter()
        np_ref.encode(cfg, man, [seg])
        cw = time.perf_counter() - t0
        line["cpu_baseline"] = {"value": round(3.0 / cw, 2), "unit": "audio-s/wall-s", "cores": 1, "kind": "port",
                                "sample": "3 s offline chunked-causal encode (the function the stream computes) through oracle/np_ref.py, float64 torch, 1 thread"}
    enc.close()
    print(json.dumps(line), flush=True)


def bench_copy(args, fa, ctx):
    """Calibration for the rocprofv3 FETCH_SIZE / WRITE_SIZE counters: a plain
    device-to-device copy of a known 256 MiB (copyRows -> the runtime's copy
    kernel), so counter KiB per dispatch can be scaled to bytes moved."""
    rows, cols = 65536, 1024  # 256 MiB of f32
    src = ctx.upload(np.ones((rows, cols), np.float32), rows, cols)
    dst = ctx.alloc(rows, cols)
    for _ in range(args.warmup):
        ctx.copyRows(dst, src, 0)
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ctx.copyRows(dst, src, 0)
    ctx.sync()
    wall = time.perf_counter() - t0
    nbytes = rows * cols * 4
    print(json.dumps({"metric": "copy GB/s (counter calibration)", "value": round(2 * nbytes * args.steps / wall / 1e9, 1), "unit": "GB/s",
                      "bytes_read_per_launch": nbytes, "bytes_written_per_launch": nbytes, "steps": args.steps}), flush=True)


def bench_gemv(args, fa, ctx):
    """configs[4] GEMV: M in {1,4,16} x K=1024 x N=4096, int8 / int4 weights,
    distinct weight buffers rotated (> 256 MB total) so the MALL cannot serve
    them: one call per buffer (fa_gemv_quant), and all buffers in one batched
    call (fa_gemv_quant_batch, launches of <= 48 buffers).  gbs = algorithmic
    bytes (weights + scales + activations + outputs) / kernel time; wall_gbs
    over the host-timed calls."""
    K, N = 1024, 4096
    rng = np.random.default_rng(1)
    out = {}
    for fmt, code, wbytes in (("int8", 1, K * N), ("int4", 2, K * N // 2)):
        nbuf = max(2, (320 << 20) // wbytes + 1)
        sbytes = N * 4 if code == 1 else N * (K // 32) * 2
        ws = [ctx.uploadBytes(rng.integers(0, 256, wbytes, dtype=np.uint8)) for _ in range(nbuf)]
        if code == 1:
            ss = [ctx.upload(rng.random(N, dtype=np.float32) * 0.01, 1, N) for _ in range(nbuf)]
        else:
            ss = [ctx.uploadBytes((rng.random(N * K // 32, dtype=np.float32) * 0.01).astype(np.float16)) for _ in range(nbuf)]
        for M in (1, 4, 16):
            a = ctx.upload(rng.standard_normal((M, K), dtype=np.float32), M, K)
            def call(i):
                ar = ctx.pushArena()
                ctx.gemvQuant(a, ws[i], ss[i], code, N, K)
                ctx.popArena(ar)

            for i in range(nbuf):
                call(i)
            ctx.sync()
            ctx.startProfile(100000)
            t0 = time.perf_counter()
            reps = 4
            for _ in range(reps):
                for i in range(nbuf):
                    call(i)
            ctx.sync()
            wall = time.perf_counter() - t0
            prof = ctx.endProfile()
            ms = [r["ms"] for r in prof if r["label"].startswith("gemv")]
            avg = sum(ms) / len(ms)
            by = wbytes + sbytes + M * K * 4 + M * N * 4
            out[f"{fmt}_M{M}"] = {"avg_us": round(avg * 1e3, 2), "gbs": round(by / (avg * 1e-3) / 1e9, 1),
                                  "frac": round(by / (avg * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                  "wall_us_per_call": round(wall / (reps * nbuf) * 1e6, 2), "buffers": nbuf}
            # all buffers in one batched call (launches of <= 48 weight buffers)
            alist = [a] * nbuf

            def bcall():
                ar = ctx.pushArena()
                ctx.gemvQuantBatch(alist, ws, ss, code, N, K)
                ctx.popArena(ar)

            bcall()
            ctx.sync()
            ctx.startProfile(100000)
            t0 = time.perf_counter()
            for _ in range(reps):
                bcall()
            ctx.sync()
            bwall = time.perf_counter() - t0
            prof = ctx.endProfile()
            kms = sum(r["ms"] for r in prof if r["label"].startswith("gemv_batch"))
            nl = sum(1 for r in prof if r["label"].startswith("gemv_batch"))
            btot = by * nbuf * reps
            out[f"{fmt}_M{M}_batched"] = {"launches_per_call": nl // reps, "kernel_us_per_launch": round(kms / nl * 1e3, 2),
                                          "gbs": round(btot / (kms * 1e-3) / 1e9, 1), "frac": round(btot / (kms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                          "wall_gbs": round(btot / bwall / 1e9, 1), "buffers": nbuf}
    print(json.dumps({"metric": "weight-only quantised GEMV HBM GB/s", "workload": "configs[4] GEMV K=1024 N=4096", "results": out}), flush=True)


if __name__ == "__main__":
    main()
