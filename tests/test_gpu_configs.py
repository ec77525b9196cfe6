"""Every BASELINE config at its full size on the GPU, through the C ABI.

configs[0]  the FFN linear X[750,1024] @ W[1024,4096] + bias on the f16 route
            (and the int8 weight route) against the oracle's restatement of
            the reference's CPU matmul and a float64 product;
configs[1]  the fused encoder with one layer on 8 x 15 s windows (M = 1504
            frames) against the oracle at full dims;
configs[2]  all 16 windows of the 24-layer batch against the oracle's
            24-layer encode of the same windows;
configs[3]  a full 32-window ragged batch (the first packed batch of the
            3600 s stream) equal to 32 standalone encodes, and the whole hour
            (8 batches, 233 windows) equal to standalone encodes;
configs[4]  the 24-layer int8 and int4 encoders on 16 x 15 s against the HIP
            fp32 op path loaded with the same weights quantised and
            dequantised, and window 0 against the oracle's 24-layer encode
            with those weights (the quantiser is pinned bit-exact to the
            oracle on the CPU, test_oracle.py).
North-star bar for the encoder: rel-L2 <= 1e-2 vs the fp32 path and
frame-wise argmax of R [1024, 64] ~ N(0,1) (seed 2) identical on >= 99.9 %
of frames.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

FULL = dict(D=1024, DFF=4096, H=8, HD=128, layers=24, dwK=9, Csub=256, Fsub=16, melBins=128)


def rel_l2(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))


def flips(a, b, seed=2):
    R = np.random.default_rng(seed).standard_normal((a.shape[1], 64)).astype(np.float32)
    return int(np.sum(np.argmax(a @ R, 1) != np.argmax(b @ R, 1)))


@pytest.fixture(scope="module")
def full_weights(fa):
    return fa.synth.make_weights(FULL, seed=1)


# ── configs[0] ──────────────────────────────────────────────────────────────
def test_config0_ffn_linear(ctx, orc):
    rng = np.random.default_rng(0)
    x = rng.standard_normal((750, 1024), dtype=np.float32)
    w = (rng.standard_normal((1024, 4096)) * 0.02).astype(np.float16).astype(np.float32)
    b = (rng.standard_normal((1, 4096)) * 0.01).astype(np.float32)
    got = ctx.download(ctx.matmul(ctx.upload(x, 750, 1024), ctx.uploadF16(w, 1024, 4096), bias=ctx.upload(b, 1, 4096))).reshape(750, 4096)
    cpu = orc.matmul(x, w, bias=b)  # the reference's CPU path (lib.rs:59-94 + JS bias)
    r = rel_l2(got, cpu)
    # the f16 route rounds A to f16 (compute.js:413-416) and accumulates in f32:
    # against float64 of exactly that product it is f32-accurate
    x16 = x.astype(np.float16).astype(np.float64)
    exact = x16 @ w.astype(np.float64) + b.astype(np.float64)
    e = float(np.abs(got - exact).max() / np.abs(exact).max())
    print(f"configs[0] f16 route: rel-L2 vs CPU path {r:.2e}, max err vs f64 of the f16-rounded product {e:.2e}")
    assert r <= 1e-2 and e < 1e-5


def test_config0_ffn_linear_int8(ctx, orc):
    rng = np.random.default_rng(0)
    x = rng.standard_normal((750, 1024), dtype=np.float32)
    w = (rng.standard_normal((1024, 4096)) * 0.02).astype(np.float32)
    b = (rng.standard_normal((1, 4096)) * 0.01).astype(np.float32)
    q, s = orc.quantize_int8_cols(w)
    got = ctx.download(ctx.matmulInt8(ctx.upload(x, 750, 1024), ctx.uploadBytes(q), ctx.upload(s, 1, 4096), 4096, 1024,
                                      bias=ctx.upload(b, 1, 4096))).reshape(750, 4096)
    ref = orc.matmul_int8(x, q, s, 4096, 1024, bias=b)
    r = rel_l2(got, ref)
    print(f"configs[0] int8 route: rel-L2 vs oracle matmul_int8 {r:.2e}")
    assert r <= 1e-2


# ── configs[1] ──────────────────────────────────────────────────────────────
def test_config1_one_layer_vs_oracle(ctx, fa, orc):
    cfg = dict(FULL, layers=1)
    man = fa.synth.make_weights(cfg, seed=1)
    mels = fa.synth.make_features(128, 1500, seed=11, W=8)
    enc = fa.FusedEncoder(ctx, man, "f16", max_T=188)
    got = np.concatenate(enc.encode(mels))
    enc.close()
    ref = orc.encode_batch(cfg, man, mels, layers=1)
    assert got.shape == ref.shape == (8 * 188, 1024)
    r, f = rel_l2(got, ref), flips(got, ref)
    print(f"configs[1] (1 layer, M=1504): rel-L2 {r:.2e}, argmax disagreements {f}/{len(got)}")
    assert r <= 1e-2 and f <= 0.001 * len(got)


# ── configs[2] ──────────────────────────────────────────────────────────────
def test_config2_all_16_windows_vs_oracle_24_layers(ctx, fa, orc, full_weights):
    """Every window of the 16-window, 24-layer batch against the oracle's
    24-layer encode of the same 16 windows (the oracle's threads run the
    windows in parallel)."""
    mels = fa.synth.make_features(128, 1500, seed=12, W=16)
    enc = fa.FusedEncoder(ctx, full_weights, "f16", max_T=188)
    got = enc.encode(mels)
    enc.close()
    ref = orc.encode_batch(FULL, full_weights, mels)
    g = np.concatenate(got)
    assert g.shape == ref.shape == (16 * 188, 1024)
    worst = max(rel_l2(g[i * 188:(i + 1) * 188], ref[i * 188:(i + 1) * 188]) for i in range(16))
    f = flips(g, ref)
    print(f"configs[2] all 16 windows, 24 layers: rel-L2 vs oracle {rel_l2(g, ref):.2e} (worst window {worst:.2e}), "
          f"argmax disagreements {f}/{len(ref)}")
    assert worst <= 1e-2 and f <= 0.001 * len(ref)


# ── configs[3] ──────────────────────────────────────────────────────────────
def test_config3_full_32_window_batch_equals_standalone(ctx, fa, full_weights):
    starts, lens = fa.windowing.planRaggedWindows(360000, 200, 3000, 100, seed=1)
    idx = fa.windowing.packBatches(lens, 32)[0]
    assert len(idx) == 32
    rng = np.random.default_rng(3)
    mels = [rng.standard_normal((128, int(lens[i]))).astype(np.float32) for i in idx]
    enc = fa.FusedEncoder(ctx, full_weights, "f16", max_T=375)
    batch = enc.encode(mels)
    worst = 0.0
    for m, b in zip(mels, batch):
        alone = enc.encode([m])[0]
        assert b.shape == alone.shape
        worst = max(worst, float(np.abs(b - alone).max()))
    enc.close()
    print(f"configs[3] 32-window batch ({sum(len(b) for b in batch)} frames): max |batch - standalone| = {worst:.2e}")
    assert worst < 1e-4


def test_encoder_refuses_more_than_32_windows(ctx, fa):
    cfg = dict(D=256, DFF=1024, H=2, HD=128, layers=1, dwK=9, Csub=64, Fsub=16, melBins=128)
    man = fa.synth.make_weights(cfg, seed=1)
    enc = fa.FusedEncoder(ctx, man, "f16", max_T=64)
    mels = [np.zeros((128, 40), np.float32)] * 33
    with pytest.raises(fa.FaError, match="33 windows"):
        enc.encode(mels)
    assert len(enc.encode(mels[:32])) == 32
    enc.close()


def test_config3_hour_all_batches_equal_standalone(ctx, fa, full_weights, monkeypatch):
    """The whole 3600 s configs[3] plan: its 233 ragged windows in 8 packed
    batches of <= 32 (two encoder lanes), read in place from one feature
    stream, equal each window encoded alone (eager, so no graph per length)."""
    total = 360000
    starts, lens = fa.windowing.planRaggedWindows(total, 200, 3000, 100, seed=1)
    batches = [(starts[b], lens[b]) for b in (np.asarray(g) for g in fa.windowing.packBatches(lens, 32))]
    assert len(batches) == 8 and sum(len(b[0]) for b in batches) == len(lens)
    feats_h = np.random.default_rng(5).standard_normal((128, total), dtype=np.float32)
    feats = ctx.upload(feats_h, 128, total)
    enc = fa.FusedEncoder(ctx, full_weights, "f16", max_T=375)
    outs = enc.forwardStreamBatches(feats, batches)
    got = []
    for o, (st, ln) in zip(outs, batches):
        h = ctx.download(o).reshape(-1, 1024)
        ctx.freeTensor(o)
        off = 0
        for s_, l_ in zip(st, ln):
            t = fa.encoder.tsub(int(l_))
            got.append((int(s_), int(l_), h[off:off + t]))
            off += t
    monkeypatch.setenv("FA_GRAPH", "0")
    worst = 0.0
    for s_, l_, g in got:
        alone = enc.encode([feats_h[:, s_:s_ + l_]])[0]
        assert alone.shape == g.shape
        worst = max(worst, float(np.abs(g - alone).max()))
    enc.close()
    ctx.freeTensor(feats)
    print(f"configs[3] hour: {len(got)} windows in 8 batches, max |batch - standalone| = {worst:.2e}")
    assert worst < 1e-4


# ── configs[4] ──────────────────────────────────────────────────────────────
def _dequantized(orc, man, fmt):
    """The manifest with every conformer linear (and the positional weights)
    replaced by its quantise -> dequantise round trip, as the fused encoder
    stores them (per output column; pw1/pw2 are [out, in] in the manifest)."""
    out = dict(man)
    for k, v in man.items():
        if not k.startswith("L"):
            continue
        name = k[k.index("_") + 1:]
        if name not in ("ff1w1", "ff1w2", "ff2w1", "ff2w2", "q", "k", "v", "out", "pos", "pw1", "pw2"):
            continue
        w = v.reshape(v.shape[0], v.shape[1]).astype(np.float32)
        kn = w.T.copy() if name in ("pw1", "pw2") else w  # [K, N]
        if fmt == "int8":
            q, s = orc.quantize_int8_cols(kn)
            d = orc.dequant_int8_cols(q, s)
        else:
            bq, sh, _, _ = orc.quantize_int4_g32(kn)
            d = orc.dequant_int4_g32(bq, sh, kn.shape[0], kn.shape[1])
        d = d.T if name in ("pw1", "pw2") else d
        out[k] = np.ascontiguousarray(d, np.float32).reshape(v.shape)
    return out


@pytest.mark.parametrize("fmt", ["int8", "int4"])
def test_config4_quantized_encoder_vs_fp32_path(ctx, fa, orc, full_weights, fmt):
    mels = fa.synth.make_features(128, 1500, seed=13, W=16)
    enc = fa.FusedEncoder(ctx, full_weights, fmt, max_T=188)
    got = np.concatenate(enc.encode(mels))
    enc.close()
    deq = _dequantized(orc, full_weights, fmt)
    ref32 = fa.loadParakeetEncoder(ctx, deq, weights="f32")
    a = ctx.pushArena()
    y, _ = fa.parakeetEncodeBatch(ctx, ref32, mels)
    ref = ctx.download(y).reshape(-1, FULL["D"])
    ctx.popArena(a)
    assert got.shape == ref.shape == (16 * 188, 1024)
    r, f = rel_l2(got, ref), flips(got, ref)
    print(f"configs[4] {fmt} encoder, 24 layers x 16 x 15 s: rel-L2 vs fp32 path (dequantised weights) {r:.2e}, "
          f"argmax disagreements {f}/{len(got)}")
    assert r <= 1e-2 and f <= 0.001 * len(got)
    # window 0 against the oracle's own 24-layer encode with the dequantised weights
    ro = orc.encode_batch(FULL, deq, [mels[0]])
    r0, f0 = rel_l2(got[:188], ro), flips(got[:188], ro)
    print(f"configs[4] {fmt} window 0 vs oracle (dequantised weights): rel-L2 {r0:.2e}, argmax disagreements {f0}/188")
    assert r0 <= 1e-2 and f0 <= 1


@pytest.mark.parametrize("fmt", ["int8", "int4"])
def test_quantized_widened_route_equals_fused_route(ctx, fa, full_weights, fmt):
    """Batches of >= 512 encoder rows widen each layer's quantised weights to
    f16 once and run the f16 GEMMs; smaller batches dequantise inside the GEMM
    tiles.  Both compute the same f16 weight values and the same K-ordered
    sums, so two windows encoded alone (376 rows, fused route) equal the same
    windows inside a 4-window batch (752 rows, widened route)."""
    lw = {k: v for k, v in full_weights.items() if not (k.startswith("L") and int(k[1:k.index("_")]) >= 4)}
    mels = fa.synth.make_features(128, 1500, seed=21, W=4)
    enc = fa.FusedEncoder(ctx, lw, fmt, max_T=188)
    small = enc.encode(mels[:2])
    big = enc.encode(mels)
    enc.close()
    for a, b in zip(small, big[:2]):
        d = float(np.abs(a - b).max() / np.abs(b).max())
        print(f"{fmt}: fused vs widened route, max rel diff {d:.2e}")
        assert d <= 1e-5
