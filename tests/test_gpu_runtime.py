"""ComputeContext runtime semantics through the C ABI: arenas, pin, pool
reuse, staged reads, batching, error paths, ragged packing index maps."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
rng = np.random.default_rng(77)


def test_arena_pool_reuse_and_stale_handles(ctx, fa):
    x = ctx.upload(rng.standard_normal((64, 64)).astype(np.float32), 64, 64)
    ctx.memStatsStart()
    for _ in range(3):  # the same scratch shapes recycle through the pool (gpu-memory-check.mjs:32-54)
        a = ctx.pushArena()
        t = ctx.transpose(ctx.scale(x, 2.0))
        ctx.popArena(a)
    st = ctx.memStats()
    assert st["reused"] >= 4 and st["created"] <= 2
    with pytest.raises(fa.FaError, match="stale"):
        ctx.download(t)


def test_pin_promotes_to_parent(ctx, fa):
    x = ctx.upload(np.ones((4, 4), np.float32), 4, 4)
    outer = ctx.pushArena()
    inner = ctx.pushArena()
    y = ctx.scale(x, 3.0)
    z = ctx.scale(x, 5.0)
    ctx.pin(y, True)
    ctx.popArena(inner)
    assert np.all(ctx.download(y) == 3.0)
    with pytest.raises(fa.FaError):
        ctx.download(z)
    ctx.popArena(outer)
    with pytest.raises(fa.FaError):
        ctx.download(y)


def test_staged_read_single_use_and_batch_nesting(ctx, fa):
    x = ctx.upload(np.arange(6, dtype=np.float32), 2, 3)
    s = ctx.stageDownload(ctx.scale(x, 2.0))
    assert np.array_equal(s.read(), np.arange(6, dtype=np.float32) * 2)
    with pytest.raises(fa.FaError, match="single-use"):
        s.read()
    ctx.beginBatch()
    with pytest.raises(fa.FaError, match="already open"):
        ctx.beginBatch()
    ctx.endBatch()
    with pytest.raises(fa.FaError):
        ctx.endBatch()


def test_shape_errors_raise(ctx, fa):
    a = ctx.upload(np.zeros((3, 5), np.float32), 3, 5)
    b = ctx.upload(np.zeros((4, 2), np.float32), 4, 2)
    with pytest.raises(fa.FaError, match="matmul"):
        ctx.matmul(a, b)
    with pytest.raises(fa.FaError):
        ctx.relShiftB(a, 2)


@pytest.mark.parametrize("layout", ["packed", "padded"])
def test_pack_windows_and_row_maps_bitexact(ctx, layout):
    mb, T = 16, 500
    feats = rng.standard_normal((mb, T)).astype(np.float32)
    starts = np.array([0, 90, 180, 181, 420], np.int32)
    lens = np.array([100, 95, 3, 200, 80], np.int32)  # overlapping windows
    got = ctx.download(ctx.packWindows(ctx.upload(feats, mb, T), starts, lens, layout)).reshape(-1, mb)
    tmax = lens.max()
    parts = []
    for s, l in zip(starts, lens):
        w = feats[:, s:s + l].T
        if layout == "padded":
            w = np.concatenate([w, np.zeros((tmax - l, mb), np.float32)])
        parts.append(w)
    assert np.array_equal(got, np.concatenate(parts))
    for stage in range(4):
        ls = lens.copy()
        for _ in range(stage):
            ls = (ls - 1) // 2 + 1
        m = ctx.windowRowMap(lens, layout, stage)
        if layout == "packed":
            exp = np.concatenate([np.full(l, i, np.int32) for i, l in enumerate(ls)])
        else:
            exp = np.concatenate([np.where(np.arange(ls.max()) < l, i, -1).astype(np.int32) for i, l in enumerate(ls)])
        assert np.array_equal(m, exp)


def test_encoder_input_validation(ctx, fa):
    cfg = dict(D=256, DFF=1024, H=2, HD=128, layers=1, dwK=9, Csub=64, Fsub=16, melBins=128)
    enc = fa.FusedEncoder(ctx, fa.synth.make_weights(cfg, seed=1), "f16", max_T=32)
    mel = ctx.upload(np.zeros((1000, 128), np.float32), 1000, 128)
    with pytest.raises(fa.FaError, match="max_T"):
        enc.forward(mel, [999])  # subsamples to 125 > 32
    with pytest.raises(fa.FaError, match="rows"):
        enc.forward(mel, [200, 200, 200, 200, 201])
    with pytest.raises(fa.FaError, match="windows"):
        enc.forward(mel, [10] * 65)
    enc.close()
