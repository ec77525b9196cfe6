"""ComputeContext ops through the C ABI vs the CPU oracle (same seeded inputs).
Tolerances mirror the reference's conformance gate
(scripts/backend-conformance.mjs:66-414): matmul 1e-3 (f32 B), f16-B route
2e-2, layernorm 1e-4, softmax 1e-5, index ops exact."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

rng = np.random.default_rng(0x5EED)


def rnd(*shape):
    return (rng.random(shape, dtype=np.float32) - 0.5).astype(np.float32)


def dl(ctx, t):
    return ctx.download(t).reshape(t.rows, t.cols)


ACTS = ["none", "gelu", "gelu_erf", "tanh", "relu", "silu"]


@pytest.mark.parametrize("act", ACTS)
def test_matmul_f32_odd_shape(ctx, orc, act):
    a, b, bias = rnd(37, 53), rnd(53, 41), rnd(1, 41)
    got = dl(ctx, ctx.matmul(ctx.upload(a, 37, 53), ctx.upload(b, 53, 41), bias=ctx.upload(bias, 1, 41), act=act))
    ref = orc.matmul(a, b, bias, act)
    assert np.abs(got - ref).max() < 1e-3


@pytest.mark.parametrize("shape", [(64, 128, 256), (300, 256, 640), (1, 1024, 64)])
def test_matmul_f32_mfma_with_add(ctx, orc, shape):
    M, K, N = shape
    a, b, d = rnd(M, K), rnd(K, N), rnd(M, N)
    got = dl(ctx, ctx.matmul(ctx.upload(a, M, K), ctx.upload(b, K, N), act="relu", add=ctx.upload(d, M, N)))
    ref = orc.matmul(a, b, None, "relu", d)
    assert np.abs(got - ref).max() < 1e-3


@pytest.mark.parametrize("shape", [(64, 128, 256), (300, 1024, 1024), (3008, 1024, 4096), (17, 64, 80)])
def test_matmul_f16_weights(ctx, orc, shape):
    M, K, N = shape
    a, b, bias, d = rnd(M, K), rnd(K, N), rnd(1, N), rnd(M, N)
    b16 = b.astype(np.float16).astype(np.float32)
    got = dl(ctx, ctx.matmul(ctx.upload(a, M, K), ctx.uploadF16(b, K, N), bias=ctx.upload(bias, 1, N), act="silu", add=ctx.upload(d, M, N)))
    ref = orc.matmul(a, b16, bias, "silu", d)
    err = np.abs(got - ref).max() / max(1.0, np.abs(ref).max())
    assert err < 2e-2, err


@pytest.mark.parametrize("cfg", ["auto", "1", "2", "3", "4", "5", "0"])
@pytest.mark.parametrize("shape", [(3008, 1024, 4096), (3008, 4096, 1024), (1504, 1024, 2048), (515, 512, 576), (203, 256, 256), (1, 64, 128)])
def test_matmul_f16_activations(ctx, orc, monkeypatch, cfg, shape):
    """f16 A x f16 B (the encoder's GEMM route: direct-to-LDS kernels, each
    configuration pinned in turn, M tails included) vs float64 dot products of
    the same f16-rounded operands; bias + residual epilogue."""
    M, K, N = shape
    if cfg != "auto":
        monkeypatch.setenv("FA_GEMM_DMA", cfg)
    a, b, bias, d = rnd(M, K) * 4, rnd(K, N) * 0.1, rnd(1, N), rnd(M, N)
    a16, b16 = a.astype(np.float16), b.astype(np.float16)
    got = dl(ctx, ctx.matmul(ctx._uploadF16Rows(a, M, K), ctx.uploadF16(b, K, N), bias=ctx.upload(bias, 1, N), add=ctx.upload(d, M, N)))
    ref = a16.astype(np.float64) @ b16.astype(np.float64) + bias.astype(np.float64) + d
    err = np.abs(got - ref).max() / np.abs(ref).max()
    assert err < 1e-5, (cfg, shape, err)


@pytest.mark.parametrize("cfg", ["auto", "1", "2", "3", "4", "5", "6"])
@pytest.mark.parametrize("shape", [(3008, 1024, 4096), (3008, 4096, 1024), (1504, 1024, 2048), (515, 512, 576), (203, 128, 256), (1, 64, 128)])
def test_matmul_two_plane_activations(ctx, orc, monkeypatch, cfg, shape):
    """A carried as exact f16 hi + lo planes (the encoder's exact-operand route,
    every two-plane configuration pinned in turn, M tails included) vs float64
    dot products of hi + lo with the f16 weights: f32-level agreement, far
    tighter than the one-plane route allows."""
    M, K, N = shape
    if cfg != "auto":
        monkeypatch.setenv("FA_GEMM_DMA", cfg)
    a, b, bias, d = rnd(M, K) * 4, rnd(K, N) * 0.1, rnd(1, N), rnd(M, N)
    hi = a.astype(np.float16)
    lo = (a - hi.astype(np.float32)).astype(np.float16)
    got = dl(ctx, ctx._matmulPair(ctx._uploadF16Rows(hi.astype(np.float32), M, K), ctx._uploadF16Rows(lo.astype(np.float32), M, K),
                                  ctx.uploadF16(b, K, N), bias=ctx.upload(bias, 1, N), add=ctx.upload(d, M, N)))
    b16 = b.astype(np.float16).astype(np.float64)
    ref = (hi.astype(np.float64) + lo.astype(np.float64)) @ b16 + bias.astype(np.float64) + d
    one_plane = hi.astype(np.float64) @ b16 + bias.astype(np.float64) + d
    err = np.abs(got - ref).max() / np.abs(ref).max()
    assert err < 2e-6, (cfg, shape, err)
    if M * N > 1000:  # the lo plane is carried: the one-plane product is much further away
        assert np.abs(one_plane - ref).max() / np.abs(ref).max() > 20 * err


def test_layernorm(ctx, orc):
    for R, Cc in [(5, 1024), (33, 77)]:
        x, g, b = rnd(R, Cc) * 3 + 1, rnd(1, Cc) + 1, rnd(1, Cc)
        got = dl(ctx, ctx.layernorm(ctx.upload(x, R, Cc), ctx.upload(g, 1, Cc), ctx.upload(b, 1, Cc)))
        assert np.abs(got - orc.layernorm(x, g, b)).max() < 1e-4


def test_softmax(ctx, orc):
    x = rnd(40, 188) * 8
    got = dl(ctx, ctx.softmax(ctx.upload(x, 40, 188)))
    assert np.abs(got - orc.softmax(x)).max() < 1e-5


def test_index_ops_exact(ctx, orc):
    H, t = 3, 11
    x = rnd(H * t, 2 * t - 1)
    assert np.array_equal(dl(ctx, ctx.relShiftB(ctx.upload(x, H * t, 2 * t - 1), H)), orc.relshift_b(x, H))
    y = rnd(7, 13)
    assert np.array_equal(dl(ctx, ctx.transpose(ctx.upload(y, 7, 13))), orc.transpose(y))
    C_, Ts, F = 4, 5, 3
    z = rnd(C_, Ts * F)
    assert np.array_equal(dl(ctx, ctx.subReshape(ctx.upload(z, C_, Ts * F), C_, Ts, F)), orc.subreshape(z, C_, Ts, F))


def test_glu_silu_ewise(ctx, orc):
    x = rnd(16, 9) * 6
    assert np.abs(dl(ctx, ctx.glu(ctx.upload(x, 16, 9))) - orc.glu(x)).max() < 1e-5
    assert np.abs(dl(ctx, ctx.silu(ctx.upload(x, 16, 9))) - orc.silu(x)).max() < 1e-5
    a, b = rnd(6, 10), rnd(1, 10)
    assert np.abs(dl(ctx, ctx.add(ctx.upload(a, 6, 10), ctx.upload(b, 1, 10))) - (a + b)).max() == 0


def test_conv2d_subsampling_shapes(ctx, orc):
    Cc, T, F = 8, 21, 16
    x = rnd(1, T * F)
    w0, b0 = rnd(Cc, 1, 3, 3), rnd(Cc)
    got = dl(ctx, ctx.conv2d(ctx.upload(x, 1, T * F), ctx.upload(w0, 1, w0.size), Cc, 1, T, F, 3, 3, bias=ctx.upload(b0, 1, Cc), strideH=2,
                             strideW=2, padTop=1, padBottom=1, padLeft=1, padRight=1, act="relu"))
    ref = orc.conv2d(x, w0, Cc, 1, T, F, 3, 3, b0, 2, 2, 1, 1, 1, 1, 1, "relu")
    assert np.abs(got - ref).max() < 1e-5
    T1, F1 = (T - 1) // 2 + 1, (F - 1) // 2 + 1
    w1 = rnd(Cc, 1, 3, 3)
    got1 = dl(ctx, ctx.conv2d(ctx.upload(ref, Cc, T1 * F1), ctx.upload(w1, 1, w1.size), Cc, Cc, T1, F1, 3, 3, strideH=2, strideW=2, padTop=1,
                              padBottom=1, padLeft=1, padRight=1, groups=Cc))
    ref1 = orc.conv2d(ref, w1, Cc, Cc, T1, F1, 3, 3, None, 2, 2, 1, 1, 1, 1, Cc, "none")
    assert np.abs(got1 - ref1).max() < 1e-5


def test_conv1d_depthwise(ctx, orc):
    D, T = 32, 50
    x, w, b = rnd(D, T), rnd(D, 1, 9), rnd(D)
    got = dl(ctx, ctx.conv1d(ctx.upload(x, D, T), ctx.upload(w, 1, w.size), D, 9, bias=ctx.upload(b, 1, D), padLeft=4, padRight=4, groups=D,
                             act="silu"))
    assert np.abs(got - orc.conv1d_grouped(x, w, D, 9, b, 1, 4, 4, 1, D, "silu")).max() < 1e-5


def test_bmm_and_fused_attention(ctx, orc):
    H, HD, W, T = 2, 128, 3, 70
    D = H * HD
    q, k, v = rnd(W * T, D), rnd(W * T, D), rnd(W * T, D)
    p = rnd(2 * T - 1, D)
    u, vb = rnd(1, D) * 0.1, rnd(1, D) * 0.1
    tq, tk, tv, tp, tu, tvb = (ctx.upload(a, *a.shape) for a in (q, k, v, p, u, vb))
    ac = orc.bmm_qk(q, k, u, H, HD, W)
    assert np.abs(dl(ctx, ctx.bmmQK(tq, tk, tu, H, HD, W)) - ac).max() < 1e-4
    bdr = orc.bmm_qk(q, p, vb, H, HD, W, True)
    bd = orc.relshift_b(bdr, W * H)
    probs = orc.softmax(ac + bd)
    ref = orc.bmm_pv(probs, v, H, HD, W)
    assert np.abs(dl(ctx, ctx.bmmPV(ctx.upload(probs, *probs.shape), tv, H, HD, W)) - ref).max() < 1e-4
    fused = dl(ctx, ctx.attnFused(tq, tk, tv, tp, tu, tvb, H, HD, W))
    rel = np.linalg.norm(fused - ref) / np.linalg.norm(ref)
    assert rel < 1e-2, rel


def test_rel_shift_stream_matches_oracle(ctx, orc):
    """relShiftStream (the streaming encoder's chunked-causal rel_shift) vs the
    oracle, bit for bit: negative key positions, clamped distances on both
    sides, right context, and a streaming position mid-stream."""
    rng = np.random.default_rng(3)
    for H, n, Lk, P, dMax, Lc, subT, C, left, right in [(8, 4, 74, 77, 73, 70, 140, 4, 70, 0), (2, 5, 30, 9, 3, 20, 7, 3, 6, 2),
                                                        (1, 1, 1, 1, 0, 0, 0, 1, 0, 0), (4, 16, 100, 120, 119, 84, 0, 16, 70, 3)]:
        x = rng.standard_normal((H * n, P)).astype(np.float32)
        opts = dict(H=H, n=n, Lk=Lk, dMax=dMax, Lc=Lc, subT=subT, C=C, left=left, right=right)
        got = dl(ctx, ctx.relShiftStream(ctx.upload(x, H * n, P), opts))
        assert np.array_equal(got, orc.relshift_stream(x, H, n, Lk, dMax, Lc, subT, C, left, right)), opts


def test_ops_failing_after_allocation_release_their_output(ctx):
    """An op that rejects its inputs after allocating its output releases it:
    repeated failing calls inside an arena draw no new buffers from the device.
    matmul (f16 activations with f32 weights) and matmulNBits (scales too
    small) check those inputs only once the output exists."""
    rng = np.random.default_rng(3)
    a16 = ctx.allocF16(64, 128)
    b32 = ctx.upload(rng.standard_normal((128, 64)).astype(np.float32), 128, 64)
    a32 = ctx.upload(rng.standard_normal((8, 64)).astype(np.float32), 8, 64)
    N, nblk = 32, 2
    bq = ctx.uploadBytes(np.zeros(N * nblk * 16, np.uint8))
    small = ctx.upload(np.ones((1, 4), np.float32), 1, 4)
    zp = ctx.uploadBytes(np.full(N, 0x88, np.uint8))
    arena = ctx.pushArena()

    def fail_both():
        with pytest.raises(Exception, match="f16 B"):
            ctx.matmul(a16, b32)
        with pytest.raises(Exception, match="too small"):
            ctx.matmulNBits(a32, bq, small, zp, N)

    fail_both()
    ctx.memStatsStart()
    for _ in range(3):
        fail_both()
    assert ctx.memStats()["created"] == 0
    ctx.popArena(arena)
    for t in (a16, b32, a32, bq, small, zp):
        ctx.freeTensor(t)
