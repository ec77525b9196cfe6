"""Weight-only quantised paths through the C ABI vs the oracle.
Dequant is bit-exact; GEMMs/GEMVs meet the reference's gpu-verify tolerances
(int8 1e-2, int4 1e-3 relative to the output scale; scripts/gpu-verify.mjs)."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
rng = np.random.default_rng(55)


def lib_quant(fa, w, fmt):
    K, N = w.shape
    if fmt == 1:
        q, s = np.empty((N, K), np.int8), np.empty(N, np.float32)
    else:
        nb = -(-K // 32)
        q, s = np.empty((N, nb, 16), np.uint8), np.empty((N, nb), np.uint16)
    assert fa.lib().fa_quantize_weights(fmt, np.ascontiguousarray(w).ctypes.data_as(C.POINTER(C.c_float)), K, N,
                                        q.ctypes.data_as(C.c_void_p), s.ctypes.data_as(C.c_void_p)) == 0
    return q, s


def rel(a, b):
    return float(np.abs(a - b).max() / max(1e-30, np.abs(b).max()))


def test_dequant_bitexact(ctx, fa, orc):
    K, N = 96, 40
    w = (rng.standard_normal((K, N)) * 0.05).astype(np.float32)
    q, s = orc.quantize_int8_cols(w)
    got = ctx.download(ctx.dequantInt8(ctx.uploadBytes(q), ctx.upload(s, 1, N), K, N)).reshape(K, N)
    assert np.array_equal(got, orc.dequant_int8_cols(q, s))
    bq, sh, _, _ = orc.quantize_int4_g32(w)
    got4 = ctx.download(ctx.dequantInt4(ctx.uploadBytes(bq), ctx.uploadBytes(sh), K, N)).reshape(K, N)
    assert np.array_equal(got4, orc.dequant_int4_g32(bq, sh, K, N))


@pytest.mark.parametrize("M", [1, 4, 16, 40])
@pytest.mark.parametrize("fmt", [1, 2])
def test_gemv_quant(ctx, fa, orc, M, fmt):
    K, N = 1024, 4096
    w = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    a = rng.standard_normal((M, K)).astype(np.float32)
    q, s = lib_quant(fa, w, fmt)
    if fmt == 1:
        ref = orc.matmul_int8(a, q.T.copy(), s, N, K)
        st = ctx.upload(s, 1, N)
    else:
        bq, sh, sf, zp = orc.quantize_int4_g32(w)
        assert np.array_equal(bq, q) and np.array_equal(sh, s)
        ref = orc.matmul_nbits(a, bq, sf, zp, N)
        st = ctx.uploadBytes(s)
    got = ctx.download(ctx.gemvQuant(ctx.upload(a, M, K), ctx.uploadBytes(q), st, fmt, N, K)).reshape(M, N)
    assert rel(got, ref) < (1e-2 if fmt == 1 else 2e-3)


@pytest.mark.parametrize("M", [1, 16])
@pytest.mark.parametrize("fmt", [1, 2])
def test_gemv_quant_batch_equals_single_calls(ctx, fa, M, fmt):
    """One launch over 50 items (two launches of <= 48) gives each item's
    single-call result (checked against the oracle in test_gemv_quant) up to
    f32 summation order: the batched tile runs the whole K in one wave, the
    single call splits it over four."""
    K, N, n = 1024, 512, 50
    items = []
    for i in range(n):
        w = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
        q, s = lib_quant(fa, w, fmt)
        st = ctx.upload(s, 1, N) if fmt == 1 else ctx.uploadBytes(s)
        items.append((ctx.upload(rng.standard_normal((M, K)).astype(np.float32), M, K), ctx.uploadBytes(q), st))
    got = ctx.download(ctx.gemvQuantBatch([t[0] for t in items], [t[1] for t in items], [t[2] for t in items], fmt, N, K)).reshape(n, M, N)
    for i, (a, q, st) in enumerate(items):
        one = ctx.download(ctx.gemvQuant(a, q, st, fmt, N, K)).reshape(M, N)
        assert np.abs(got[i] - one).max() <= 1e-5 * max(1.0, np.abs(one).max()), i


def test_gemv_quant_batch_rejects(ctx, fa):
    K, N = 1024, 256
    q = ctx.uploadBytes(np.zeros(K * N, np.uint8))
    s = ctx.upload(np.ones(N, np.float32), 1, N)
    a1, a2 = ctx.upload(np.zeros((1, K), np.float32), 1, K), ctx.upload(np.zeros((2, K), np.float32), 2, K)
    with pytest.raises(fa.FaError):
        ctx.gemvQuantBatch([a1, a2], [q, q], [s, s], 1, N, K)  # mixed M
    with pytest.raises(fa.FaError):
        ctx.gemvQuantBatch([a1], [q], [s], 1, N, 1000)  # K not a multiple of 64
    small = ctx.uploadBytes(np.zeros(16, np.uint8))
    with pytest.raises(fa.FaError):
        ctx.gemvQuantBatch([a1], [small], [s], 1, N, K)


@pytest.mark.parametrize("M", [3, 300])
def test_matmul_int8_reference_layout(ctx, orc, M):
    K, N = 256, 192
    w = (rng.standard_normal((K, N)) * 0.05).astype(np.float32)
    q, s = orc.quantize_int8_cols(w)  # [K, N] row-major bytes (gemm.js:697-701)
    a, bias = rng.standard_normal((M, K)).astype(np.float32), rng.standard_normal(N).astype(np.float32) * 0.1
    got = ctx.download(ctx.matmulInt8(ctx.upload(a, M, K), ctx.uploadBytes(q), ctx.upload(s, 1, N), N, K,
                                      bias=ctx.upload(bias, 1, N), act="relu")).reshape(M, N)
    assert rel(got, orc.matmul_int8(a, q, s, N, K, bias, "relu")) < 1e-2


@pytest.mark.parametrize("M", [2, 256])
def test_matmul_nbits_asymmetric(ctx, orc, M):
    K, N = 128, 96
    nblk, zpb = K // 32, (K // 32 + 1) // 2
    bq = rng.integers(0, 256, (N, nblk, 16), dtype=np.uint8)
    sc = (rng.random((N, nblk)) * 0.01).astype(np.float32)
    zp = rng.integers(0, 256, (N, zpb), dtype=np.uint8)
    a = rng.standard_normal((M, K)).astype(np.float32)
    got = ctx.download(ctx.matmulNBits(ctx.upload(a, M, K), ctx.uploadBytes(bq), ctx.upload(sc, 1, sc.size), ctx.uploadBytes(zp), N)).reshape(M, N)
    assert rel(got, orc.matmul_nbits(a, bq, sc, zp, N)) < 2e-3
