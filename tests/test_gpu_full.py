"""Full-size checks (BASELINE configs[2]/[3]) through size-independent
properties: the fused f16 encoder against the HIP fp32 op-by-op path (the
reference's parakeetEncodeBatch op sequence on fp32 MFMA kernels, itself
pinned op by op to the oracle), and ragged-batch invariance."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
FULL = dict(D=1024, DFF=4096, H=8, HD=128, layers=24, dwK=9, Csub=256, Fsub=16, melBins=128)


@pytest.fixture(scope="module")
def full_weights(fa):
    return fa.synth.make_weights(FULL, seed=1)


def _ref_path(ctx, fa, ref32, mels):
    a = ctx.pushArena()
    y, T = fa.parakeetEncodeBatch(ctx, ref32, mels)
    ref = ctx.download(y).reshape(-1, FULL["D"])
    ctx.popArena(a)
    return ref


def test_config3_fused_f16_vs_fp32_path(ctx, fa, full_weights):
    """north_star bar at configs[2]: rel-L2 <= 1e-2 per batch, and frame-wise
    argmax of R [1024, 64] ~ N(0,1) (seed 2) identical on >= 99.9 % of frames.
    The disagreement rate is a property of the f16 path (~0.07 % with the
    default operand precision); one batch of 3008 frames would estimate it
    with +-0.05 % noise, so it is measured over 8 batches (24,064 frames,
    feature seeds 1..8)."""
    enc = fa.FusedEncoder(ctx, full_weights, "f16", max_T=188)
    ref32 = fa.loadParakeetEncoder(ctx, full_weights, weights="f32")
    R = np.random.default_rng(2).standard_normal((1024, 64)).astype(np.float32)
    flips = frames = 0
    for seed in range(1, 9):
        mels = fa.synth.make_features(128, 1500, seed=seed, W=16)
        got = np.concatenate(enc.encode(mels))
        ref = _ref_path(ctx, fa, ref32, mels)
        assert got.shape == ref.shape == (16 * 188, 1024)
        rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
        f = int(np.sum(np.argmax(got @ R, 1) != np.argmax(ref @ R, 1)))
        print(f"configs[2] seed {seed}: rel-L2 {rel:.3e}, argmax disagreements {f}/{len(got)}")
        assert rel <= 1e-2
        flips += f
        frames += len(got)
    enc.close()
    agree = 1.0 - flips / frames
    print(f"configs[2]: projected argmax agreement {agree:.5f} over {frames} frames")
    assert agree >= 0.999


def test_exact_operands_track_fp32_path(ctx, fa, full_weights):
    """Every operand carried as an exact f16 pair (fa_encoder_set_exact with all
    bits, all layers): the f16 route then differs from the fp32 path only by
    f32 accumulation order and f16 attention internals -> rel-L2 well under
    1e-4 at full width (4 layers, 4 windows); plain f16 operands are ~10x
    further away.  Pins the two-plane GEMM, LayerNorm, attention and
    depthwise-conv paths against the fp32 reference."""
    lw = {k: v for k, v in full_weights.items() if not (k.startswith("L") and int(k[1:k.index("_")]) >= 4)}
    mels = fa.synth.make_features(128, 1500, seed=3, W=4)
    enc = fa.FusedEncoder(ctx, lw, "f16", max_T=188)
    ref = _ref_path(ctx, fa, fa.loadParakeetEncoder(ctx, lw, weights="f32"), mels)
    enc.setExact(31)
    assert all(enc.exact(l) == 31 for l in range(4))
    exact = np.concatenate(enc.encode(mels))
    enc.setExact(0)
    plain = np.concatenate(enc.encode(mels))
    enc.close()
    r_exact = np.linalg.norm(exact - ref) / np.linalg.norm(ref)
    r_plain = np.linalg.norm(plain - ref) / np.linalg.norm(ref)
    print(f"4 layers: rel-L2 exact operands {r_exact:.2e}, plain f16 {r_plain:.2e}")
    assert r_exact < 5e-5
    assert r_plain > 3 * r_exact


def test_set_exact_validation(ctx, fa, full_weights):
    lw = {k: v for k, v in full_weights.items() if not (k.startswith("L") and int(k[1:k.index("_")]) >= 2)}
    enc = fa.FusedEncoder(ctx, lw, "f16", max_T=64)
    assert enc.exact(1) == 29 and enc.exact(5) == -1  # default tail (all but FF hidden) covers both layers of a 2-layer model
    with pytest.raises(fa.FaError):
        enc.setExact(64)
    with pytest.raises(fa.FaError):
        enc.setExact(1, 1, 5)
    enc.close()
    for fmt in ("int8", "int4"):  # quantised weights take the same masks; their default tail is all-exact
        q = fa.FusedEncoder(ctx, lw, fmt, max_T=64)
        assert q.exact(0) == 31 and q.exact(1) == 31
        q.setExact(1)
        assert q.exact(0) == 1
        q.close()


def test_config4_ragged_batch_equals_standalone(ctx, fa, full_weights):
    starts, lens = fa.windowing.planRaggedWindows(360000, 200, 3000, 100, seed=1)
    idx = fa.windowing.packBatches(lens, 32)[0]
    rng = np.random.default_rng(1)
    mels = [rng.standard_normal((128, int(lens[i]))).astype(np.float32) for i in idx[:8]]
    enc = fa.FusedEncoder(ctx, full_weights, "f16", max_T=375)
    batch = enc.encode(mels)
    worst = 0.0
    for m, b in zip(mels, batch):
        alone = enc.encode([m])[0]
        worst = max(worst, float(np.abs(b - alone).max()))
    enc.close()
    print(f"ragged: max |batch - standalone| = {worst:.2e}")
    assert worst < 1e-4
