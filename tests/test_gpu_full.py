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


def test_config3_fused_f16_vs_fp32_path(ctx, fa, full_weights):
    mels = fa.synth.make_features(128, 1500, seed=1, W=16)
    enc = fa.FusedEncoder(ctx, full_weights, "f16", max_T=188)
    got = np.concatenate(enc.encode(mels))
    enc.close()
    ref32 = fa.loadParakeetEncoder(ctx, full_weights, weights="f32")
    a = ctx.pushArena()
    y, T = fa.parakeetEncodeBatch(ctx, ref32, mels)
    ref = ctx.download(y).reshape(-1, FULL["D"])
    ctx.popArena(a)
    assert got.shape == ref.shape == (16 * 188, 1024)
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    R = np.random.default_rng(2).standard_normal((1024, 64)).astype(np.float32)
    agree = np.mean(np.argmax(got @ R, 1) == np.argmax(ref @ R, 1))
    print(f"configs[2]: rel-L2 {rel:.3e}, projected argmax agreement {agree:.5f}")
    assert rel <= 1e-2
    assert agree >= 0.999


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
