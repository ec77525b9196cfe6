"""fa_mel_windows_static (the allocation-free entry point) through the C ABI,
against fa_mel_windows on the same windows: bit-identical output on two
calls in a row (the second smaller, so the shared static array still holds
the first call's statistics), on a third call with another bin count (its
tables replace the 128-bin ones), and back; size limits rejected clearly.
Device buffers come from hipMalloc called by the test itself (the caller's
memory; the entry point allocates none)."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


class DevBuf:
    """A caller-owned device buffer (hipMalloc through the HIP runtime the
    library itself links)."""
    hip = None

    def __init__(self, nbytes):
        if DevBuf.hip is None:
            DevBuf.hip = C.CDLL("libamdhip64.so.7")
        self.ptr = C.c_void_p()
        assert DevBuf.hip.hipMalloc(C.byref(self.ptr), C.c_size_t(nbytes)) == 0
        self.nbytes = nbytes

    def put(self, arr):
        a = np.ascontiguousarray(arr)
        assert a.nbytes <= self.nbytes
        assert DevBuf.hip.hipMemcpy(self.ptr, a.ctypes.data_as(C.c_void_p), C.c_size_t(a.nbytes), 1) == 0  # host -> device
        return self

    def get(self, shape, dtype=np.float32):
        a = np.empty(shape, dtype)
        assert DevBuf.hip.hipMemcpy(a.ctypes.data_as(C.c_void_p), self.ptr, C.c_size_t(a.nbytes), 2) == 0  # device -> host
        return a

    def free(self):
        DevBuf.hip.hipFree(self.ptr)


def _static(fa, ctx, pcm_dev, nsamp, starts, lens, n_mels, guard, normalize, out_dev, cols):
    st = np.ascontiguousarray(starts, np.int32)
    ln = np.ascontiguousarray(lens, np.int32)
    return fa.lib().fa_mel_windows_static(ctx._p, C.c_void_p(pcm_dev), nsamp, st.ctypes.data_as(C.POINTER(C.c_int32)),
                                          ln.ctypes.data_as(C.POINTER(C.c_int32)), len(st), n_mels, guard, normalize,
                                          C.c_void_p(out_dev), cols)


def test_mel_windows_static_matches_allocating_entry(ctx, fa):
    rng = np.random.default_rng(7)
    nsamp = 16000 * 60
    t = np.arange(nsamp) / 16000
    pcm_h = (0.3 * np.sin(2 * np.pi * 220 * t) + 0.05 * rng.standard_normal(nsamp)).astype(np.float32)
    pcm_d = DevBuf(pcm_h.nbytes).put(pcm_h)
    pcm_t = ctx.upload(pcm_h.reshape(1, -1), 1, nsamp)
    cases = [
        ([0, 208000, 416000, 5000], [240000, 240000, 240000, 100000], 128, 2.0 ** -24, 1),  # first call
        ([1000, 30000], [40000, 7777], 128, 2.0 ** -24, 1),                                  # smaller second call
        ([0, 50000, 90000], [64000, 12345, 160], 80, 1e-10, 0),                               # other bin count, raw
        ([300], [48000], 128, 2.0 ** -24, 1),                                                 # back to 128 bins
    ]
    for starts, lens, nm, guard, norm in cases:
        cols = sum(l // 160 for l in lens)
        want = ctx.download(ctx.melWindows(pcm_t, starts, lens, nm, guard, bool(norm))).reshape(nm, cols)
        out = DevBuf(nm * cols * 4).put(np.full(nm * cols, np.nan, np.float32))
        rc = _static(fa, ctx, pcm_d.ptr.value, nsamp, starts, lens, nm, guard, norm, out.ptr.value, cols)
        assert rc == 0, fa.lib().fa_last_error(ctx._p)
        ctx.sync()
        got = out.get((nm, cols))
        out.free()
        print(f"static mel: {len(lens)} windows, {nm} bins, {cols} frames: max |diff| = {np.abs(got - want).max():.1e}")
        assert np.array_equal(got, want)
    pcm_d.free()


def test_mel_windows_static_rejects_sizes(ctx, fa):
    out = DevBuf(128 * 65 * 4)
    pcm = DevBuf(16000 * 10 * 4).put(np.zeros(16000 * 10, np.float32))
    n = 16000 * 10
    assert _static(fa, ctx, pcm.ptr.value, n, [0] * 65, [160] * 65, 128, 2.0 ** -24, 1, out.ptr.value, 65) == 5  # > 64 windows
    assert b"64" in fa.lib().fa_last_error(ctx._p)
    assert _static(fa, ctx, pcm.ptr.value, n, [0], [1600], 129, 2.0 ** -24, 1, out.ptr.value, 10) == 1     # > 128 bins
    assert _static(fa, ctx, pcm.ptr.value, n, [0], [1600], 128, 2.0 ** -24, 1, out.ptr.value, 11) == 1     # wrong out size
    assert _static(fa, ctx, pcm.ptr.value, n, [159000], [1600], 128, 2.0 ** -24, 1, out.ptr.value, 10) == 1  # outside the stream
    out.free()
    pcm.free()


def test_mel_windows_static_serves_one_context_per_device(ctx, fa):
    """A second context on the same GPU is refused (FA_E_STATE) while the
    first one owns the static array."""
    nsamp = 16000 * 2
    pcm_h = np.random.default_rng(3).standard_normal(nsamp).astype(np.float32) * 0.1
    pcm_d = DevBuf(pcm_h.nbytes).put(pcm_h)
    out_d = DevBuf(128 * 200 * 4)
    assert _static(fa, ctx, pcm_d.ptr.value, nsamp, [0], [32000], 128, 2.0 ** -24, 1, out_d.ptr.value, 200) == 0
    other = fa.createContext("hip")
    assert _static(fa, other, pcm_d.ptr.value, nsamp, [0], [32000], 128, 2.0 ** -24, 1, out_d.ptr.value, 200) == fa._lib.FA_E_STATE
    assert b"another context" in fa.lib().fa_last_error(other._p)
    other.destroy()
    pcm_d.free()
    out_d.free()
