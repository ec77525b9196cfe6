"""HipContext: the reference's `ComputeContext` backend contract
(src/gpu/compute.d.ts:106-255) on MI355X, through the C ABI.

Method names, argument meaning and error behaviour follow the d.ts so engine
code written against GpuContext/WasmContext reads the same:
  - tensors are opaque {rows, cols} handles, row-major f32 (weights uploaded
    with uploadF16 are f16 and route matmul to the f16-compute kernels, as
    GpuContext does, compute.js:413-416);
  - upload() is persistent; alloc() draws from the pool inside the newest
    arena; popArena() recycles; pin() exempts or promotes to the parent arena
    (buffer-pool.js:49-126);
  - beginBatch() nests -> error; stageDownload().read() is single-use;
  - misuse raises FaError (the reference throws Error).
Every required member of the d.ts is implemented; the TTS and decoder-side
ops (lstm, snake, adain, convTranspose1d, im2col, conv1dGemm/conv1dFast*,
gatherCols, leakyRelu, jbatch, argmaxRows, jointArgmax) are plain kernels with
the CPU backend's arithmetic (wasm-context.js), off the encoder's hot path.
"""
from __future__ import annotations

import ctypes as C
from contextlib import contextmanager

import numpy as np

from . import _lib as L
from ._lib import ACT, FaError, check, lib


class HipTensor:
    """Opaque device tensor {rows, cols}."""

    __slots__ = ("ctx", "h", "rows", "cols", "f16", "view")

    def __init__(self, ctx, h, rows, cols, f16=False, view=False):
        self.ctx, self.h, self.rows, self.cols, self.f16, self.view = ctx, h, rows, cols, f16, view

    def __repr__(self):
        return f"HipTensor([{self.rows}, {self.cols}]{' f16' if self.f16 else ''})"


class PackedBytes:
    """Handle from uploadBytes (int8 / int4 payloads)."""

    __slots__ = ("ctx", "h", "nbytes")

    def __init__(self, ctx, h, nbytes):
        self.ctx, self.h, self.nbytes = ctx, h, nbytes


class StagedRead:
    """Single-use staged readback (compute.d.ts:39-45)."""

    def __init__(self, ctx, h, n):
        self._ctx, self._h, self._n = ctx, h, n

    def read(self) -> np.ndarray:
        out = np.empty(self._n, np.float32)
        check(self._ctx._p, lib().fa_staged_read(self._ctx._p, self._h, out.ctypes.data_as(L.F32P)))
        return out


def _f32(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


class NativeHandle:
    """One native object's pointer and destructor; released at most once,
    by its owner's close() or by the context's destroy(), whichever is first."""

    __slots__ = ("_owner", "p", "_destroy")

    def __init__(self, owner, p, destroy):
        self._owner, self.p, self._destroy = owner, p, destroy

    def release(self):
        if self.p:
            p, self.p = self.p, None
            self._owner._owned.pop(id(self), None)
            self._destroy(p)


class HipContext:
    """ComputeContext on one gfx950 GPU (one HIP stream, in-order)."""

    backend = "hip"
    hasF16 = True

    def __init__(self, device: int = 0):
        p = L.P()
        st = lib().fa_ctx_create(device, C.byref(p))
        if st != L.FA_OK:
            raise FaError(st, f"fa_ctx_create(device={device}) failed with status {st} (no gfx950 GPU visible?)")
        self._p = p
        self._destroyed = False
        self._owned = {}  # id -> NativeHandle: objects that free device memory through this context

    def _own(self, ptr, destroy) -> "NativeHandle":
        """Register a native object (encoder, decoder, stream) created on this
        context; destroy() releases every one still live before the context.
        The registry holds plain cells, not weak references, so interpreter
        shutdown (which clears weak references before running finalizers)
        cannot destroy the context ahead of its objects."""
        h = NativeHandle(self, ptr, destroy)
        self._owned[id(h)] = h
        return h

    # ── lifecycle ─────────────────────────────────────────────────────────
    def destroy(self):
        if not self._destroyed:
            for h in reversed(list(self._owned.values())):  # newest first (a stream before its encoder); they free device memory through the context
                h.release()
            lib().fa_ctx_destroy(self._p)
            self._destroyed = True

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass

    def sync(self):
        check(self._p, lib().fa_sync(self._p))

    def _out(self):
        return L.T()

    def _t(self, h, rows=None, cols=None, f16=False, view=False):
        if rows is None:
            r, c, d = C.c_int(), C.c_int(), C.c_int()
            check(self._p, lib().fa_tensor_info(self._p, h, C.byref(r), C.byref(c), C.byref(d)))
            rows, cols, f16 = r.value, c.value, d.value == 1
        return HipTensor(self, h, rows, cols, f16, view)

    @staticmethod
    def _h(t):
        return 0 if t is None else t.h

    # ── tensors & memory ──────────────────────────────────────────────────
    def upload(self, data, rows, cols):
        d = _f32(data).reshape(-1)
        if d.size != rows * cols:
            raise FaError(L.FA_E_INVALID, f"upload: {d.size} values for [{rows},{cols}]")
        o = self._out()
        check(self._p, lib().fa_upload(self._p, d.ctypes.data_as(L.F32P), rows, cols, C.byref(o)))
        return HipTensor(self, o.value, rows, cols)

    def uploadF16(self, data, rows, cols):
        d = _f32(data).reshape(-1)
        if d.size != rows * cols:
            raise FaError(L.FA_E_INVALID, f"uploadF16: {d.size} values for [{rows},{cols}]")
        o = self._out()
        check(self._p, lib().fa_upload_f16(self._p, d.ctypes.data_as(L.F32P), rows, cols, C.byref(o)))
        return HipTensor(self, o.value, rows, cols, f16=True)

    def _uploadF16Rows(self, data, rows, cols):
        """Row-major f16 activations (no ComputeContext counterpart; feeds matmul's f16 x f16 route)."""
        d = _f32(data).reshape(-1)
        if d.size != rows * cols:
            raise FaError(L.FA_E_INVALID, f"_uploadF16Rows: {d.size} values for [{rows},{cols}]")
        o = self._out()
        check(self._p, lib().fa_upload_f16_rows(self._p, d.ctypes.data_as(L.F32P), rows, cols, C.byref(o)))
        return HipTensor(self, o.value, rows, cols, f16=True)

    def alloc(self, rows, cols):
        o = self._out()
        check(self._p, lib().fa_alloc(self._p, rows, cols, C.byref(o)))
        return HipTensor(self, o.value, rows, cols)

    def allocF16(self, rows, cols):
        o = self._out()
        check(self._p, lib().fa_alloc_f16(self._p, rows, cols, C.byref(o)))
        return HipTensor(self, o.value, rows, cols, f16=True)

    def ensureTensor(self, t):
        if isinstance(t, HipTensor):
            return t
        return self.upload(t["data"], t["rows"], t["cols"])

    def uploadBytes(self, typed):
        b = np.ascontiguousarray(np.asarray(typed)).view(np.uint8).reshape(-1)
        o = self._out()
        check(self._p, lib().fa_upload_bytes(self._p, b.ctypes.data_as(C.c_void_p), b.size, C.byref(o)))
        return PackedBytes(self, o.value, b.size)

    def freeTensor(self, t):
        if t is not None:
            check(self._p, lib().fa_free_tensor(self._p, t.h))

    def pin(self, t, toParent=False):
        check(self._p, lib().fa_pin(self._p, t.h, int(bool(toParent))))
        return t

    def pushArena(self):
        o = self._out()
        check(self._p, lib().fa_push_arena(self._p, C.byref(o)))
        return o.value

    def popArena(self, handle=None):
        check(self._p, lib().fa_pop_arena(self._p, handle or 0))

    def trimPool(self, budgetBytes=None):
        check(self._p, lib().fa_trim_pool(self._p, (1 << 30) if budgetBytes is None else int(budgetBytes)))

    def poolInfo(self):
        b = C.c_size_t()
        check(self._p, lib().fa_pool_info(self._p, C.byref(b), None, None, None))
        return {"bytes": b.value}

    def memStatsStart(self):
        self._mem0 = self._memraw()

    def _memraw(self):
        cr, cb, ru = C.c_uint64(), C.c_uint64(), C.c_uint64()
        check(self._p, lib().fa_pool_info(self._p, None, C.byref(cr), C.byref(cb), C.byref(ru)))
        return cr.value, cb.value, ru.value

    def memStats(self):
        if not hasattr(self, "_mem0"):
            return None
        a, b = self._mem0, self._memraw()
        return {"created": b[0] - a[0], "createdBytes": b[1] - a[1], "reused": b[2] - a[2]}

    # ── readback ──────────────────────────────────────────────────────────
    def download(self, t) -> np.ndarray:
        out = np.empty(t.rows * t.cols, np.float32)
        check(self._p, lib().fa_download(self._p, t.h, out.ctypes.data_as(L.F32P)))
        return out

    downloadF16 = download

    def stageDownload(self, t) -> StagedRead:
        o = self._out()
        check(self._p, lib().fa_stage_download(self._p, t.h, C.byref(o)))
        return StagedRead(self, o.value, t.rows * t.cols)

    def rowsView(self, t, rows):
        o = self._out()
        check(self._p, lib().fa_rows_view(self._p, t.h, rows, C.byref(o)))
        return HipTensor(self, o.value, rows, t.cols, t.f16, view=True)

    # ── batching ──────────────────────────────────────────────────────────
    def beginBatch(self):
        check(self._p, lib().fa_begin_batch(self._p))

    def endBatch(self):
        check(self._p, lib().fa_end_batch(self._p))

    def withBatchSync(self, fn):
        self.beginBatch()
        try:
            return fn()
        finally:
            self.endBatch()

    withBatch = withBatchSync

    # ── linear algebra ────────────────────────────────────────────────────
    def matmul(self, a, b, bias=None, act="none", add=None):
        o = self._out()
        check(self._p, lib().fa_matmul(self._p, a.h, b.h, self._h(bias), ACT[act], self._h(add), C.byref(o)))
        return HipTensor(self, o.value, a.rows, b.cols)

    def matmulV2(self, a, b, bias=None, act="none"):
        return self.matmul(a, b, bias=bias, act=act)

    matmulV3 = matmulV4 = matmulF16 = matmulV2

    def _matmulPair(self, a_hi, a_lo, b, bias=None, add=None):
        """(A_hi + A_lo) · B with A as two exact f16 planes (no ComputeContext counterpart)."""
        o = self._out()
        check(self._p, lib().fa_matmul_pair(self._p, a_hi.h, a_lo.h, b.h, self._h(bias), self._h(add), C.byref(o)))
        return HipTensor(self, o.value, a_hi.rows, b.cols)

    def matmulInt8(self, a, wq, scale, N, K, bias=None, act="none"):
        o = self._out()
        check(self._p, lib().fa_matmul_int8(self._p, a.h, wq.h, scale.h, N, K, self._h(bias), ACT[act], C.byref(o)))
        return HipTensor(self, o.value, a.rows, N)

    def matmulNBits(self, a, bq, scales, zp, N, blockSize=32):
        o = self._out()
        check(self._p, lib().fa_matmul_nbits(self._p, a.h, bq.h, scales.h, zp.h, N, blockSize, C.byref(o)))
        return HipTensor(self, o.value, a.rows, N)

    def layernorm(self, x, gamma, beta, eps=1e-5):
        o = self._out()
        check(self._p, lib().fa_layernorm(self._p, x.h, gamma.h, beta.h, eps, C.byref(o)))
        return HipTensor(self, o.value, x.rows, x.cols)

    def softmax(self, x):
        o = self._out()
        check(self._p, lib().fa_softmax(self._p, x.h, C.byref(o)))
        return HipTensor(self, o.value, x.rows, x.cols)

    # ── convolution ───────────────────────────────────────────────────────
    def conv1d(self, x, w, cout, k, bias=None, stride=1, pad=0, padLeft=None, padRight=None, dilation=1, groups=1, act="none"):
        pl = pad if padLeft is None else padLeft
        pr = pad if padRight is None else padRight
        o = self._out()
        check(self._p, lib().fa_conv1d(self._p, x.h, w.h, cout, k, self._h(bias), stride, pl, pr, dilation, groups, ACT[act], C.byref(o)))
        return self._t(o.value)

    def conv2d(self, x, w, cout, cin, h, w_, kh, kw, bias=None, strideH=1, strideW=1, padH=0, padW=0, padTop=None, padBottom=None,
               padLeft=None, padRight=None, groups=1, act="none"):
        pt = padH if padTop is None else padTop
        pb = padH if padBottom is None else padBottom
        pl = padW if padLeft is None else padLeft
        pr = padW if padRight is None else padRight
        o = self._out()
        check(self._p, lib().fa_conv2d(self._p, x.h, w.h, cout, cin, h, w_, kh, kw, self._h(bias), strideH, strideW, pt, pb, pl, pr, groups,
                                       ACT[act], C.byref(o)))
        return self._t(o.value)

    # ── attention ─────────────────────────────────────────────────────────
    def bmmQK(self, q, b, qb, H, HD, W=1, bShared=False):
        o = self._out()
        check(self._p, lib().fa_bmm_qk(self._p, q.h, b.h, self._h(qb), H, HD, W, int(bool(bShared)), C.byref(o)))
        return self._t(o.value)

    def bmmPV(self, p, v, H, HD, W=1):
        o = self._out()
        check(self._p, lib().fa_bmm_pv(self._p, p.h, v.h, H, HD, W, C.byref(o)))
        return self._t(o.value)

    def relShift(self, x):
        o = self._out()
        check(self._p, lib().fa_rel_shift(self._p, x.h, C.byref(o)))
        return self._t(o.value)

    def relShiftB(self, x, H):
        o = self._out()
        check(self._p, lib().fa_rel_shift_b(self._p, x.h, H, C.byref(o)))
        return self._t(o.value)

    def relShiftStream(self, x, opts=None, **kw):
        """compute.js relShiftStream(x, {H, n, Lk, dMax, Lc, subT, C, left, right})."""
        o_ = dict(opts or {}, **kw)
        o = self._out()
        check(self._p, lib().fa_rel_shift_stream(self._p, x.h, *(int(o_[k]) for k in ("H", "n", "Lk", "dMax", "Lc", "subT", "C", "left", "right")),
                                                 C.byref(o)))
        return self._t(o.value)

    def attnFused(self, q, k, v, pos, pbu, pbv, H, HD, W):
        o = self._out()
        check(self._p, lib().fa_attn_fused(self._p, q.h, k.h, v.h, pos.h, pbu.h, pbv.h, H, HD, W, C.byref(o)))
        return self._t(o.value)

    # ── elementwise & data movement ───────────────────────────────────────
    def ewise(self, a, b, op):
        o = self._out()
        check(self._p, lib().fa_ewise(self._p, a.h, b.h, 1 if op == "mul" else 0, C.byref(o)))
        return HipTensor(self, o.value, a.rows, a.cols)

    def add(self, a, b):
        return self.ewise(a, b, "add")

    def mul(self, a, b):
        return self.ewise(a, b, "mul")

    def _unary(self, fn, x, *extra):
        o = self._out()
        check(self._p, fn(self._p, x.h, *extra, C.byref(o)))
        return HipTensor(self, o.value, x.rows, x.cols)

    def scale(self, x, s):
        return self._unary(lib().fa_scale, x, C.c_float(s))

    def silu(self, x):
        return self._unary(lib().fa_silu, x)

    def relu(self, x):
        return self._unary(lib().fa_relu, x)

    def glu(self, x):
        o = self._out()
        check(self._p, lib().fa_glu(self._p, x.h, C.byref(o)))
        return HipTensor(self, o.value, x.rows // 2, x.cols)

    def transpose(self, x):
        o = self._out()
        check(self._p, lib().fa_transpose(self._p, x.h, C.byref(o)))
        return HipTensor(self, o.value, x.cols, x.rows)

    def sliceCols(self, x, col0, width):
        o = self._out()
        check(self._p, lib().fa_slice_cols(self._p, x.h, col0, width, C.byref(o)))
        return HipTensor(self, o.value, x.rows, width)

    def setCols(self, dst, src, col0):
        check(self._p, lib().fa_set_cols(self._p, dst.h, src.h, col0))
        return dst

    def sliceRows(self, x, row0, count):
        o = self._out()
        check(self._p, lib().fa_slice_rows(self._p, x.h, row0, count, C.byref(o)))
        return HipTensor(self, o.value, count, x.cols)

    def copyRows(self, dst, src, rowOffset):
        check(self._p, lib().fa_copy_rows(self._p, dst.h, src.h, rowOffset))
        return dst

    def concatRows(self, tensors):
        hs = (L.T * len(tensors))(*[t.h for t in tensors])
        o = self._out()
        check(self._p, lib().fa_concat_rows(self._p, hs, len(tensors), C.byref(o)))
        return HipTensor(self, o.value, sum(t.rows for t in tensors), tensors[0].cols)

    def subReshape(self, x, C_, Tsub, F):
        o = self._out()
        check(self._p, lib().fa_sub_reshape(self._p, x.h, C_, Tsub, F, C.byref(o)))
        return HipTensor(self, o.value, Tsub, C_ * F)

    def rowBiasAct(self, x, bias, act="none"):
        o = self._out()
        check(self._p, lib().fa_row_bias_act(self._p, x.h, bias.h, ACT[act], C.byref(o)))
        return HipTensor(self, o.value, x.rows, x.cols)

    # ── TTS / decoder-side members (compute.d.ts:174-234) ──────────────────
    def leakyRelu(self, x, slope=0.2):
        return self._unary(lib().fa_leaky_relu, x, C.c_double(slope))

    def snake(self, x, alpha):
        return self._unary(lib().fa_snake, x, alpha.h)

    def adain(self, x, scale, shift, eps=1e-5):
        return self._unary(lib().fa_adain, x, scale.h, shift.h, C.c_double(eps))

    def im2col(self, x, k, stride=1, pad=0, dilation=1):
        o = self._out()
        check(self._p, lib().fa_im2col(self._p, x.h, k, stride, pad, dilation, C.byref(o)))
        return self._t(o.value)

    def conv1dGemm(self, x, wRows, cout, k, stride=1, pad=0, dilation=1, act="none"):
        """wasm-context.js:286-288: matmul(wRows [Cout, Cin*k], im2col(x))."""
        cols = self.im2col(x, k, stride=stride, pad=pad, dilation=dilation)
        y = self.matmul(wRows, cols, act=act)
        self.freeTensor(cols)
        return y

    def conv1dFast(self, x, wRows, cout, k, **opts):
        """wasm-context.js:265-267: conv1d with wRows as the [Cout, Cin*k] weight."""
        return self.conv1d(x, wRows, cout, k, **opts)

    def conv1dFastF16(self, x, wRows, cout, k, **opts):
        return self.conv1d(x, wRows, cout, k, **opts)

    def convTranspose1d(self, x, w, cout, k, bias=None, stride=1, pad=0, dilation=1, groups=1, outputPadding=0, act="none"):
        o = self._out()
        check(self._p, lib().fa_conv_transpose1d(self._p, x.h, w.h, cout, k, self._h(bias), stride, pad, dilation, groups, outputPadding,
                                                 ACT[act], C.byref(o)))
        return self._t(o.value)

    def gatherCols(self, x, idxMap):
        idx = np.ascontiguousarray(idxMap, np.uint32)
        o = self._out()
        check(self._p, lib().fa_gather_cols(self._p, x.h, idx.ctypes.data_as(C.POINTER(C.c_uint32)), len(idx), C.byref(o)))
        return HipTensor(self, o.value, x.rows, len(idx))

    def lstm(self, x, w, r, b, hid):
        o = self._out()
        check(self._p, lib().fa_lstm(self._p, x.h, w.h, r.h, b.h, hid, C.byref(o)))
        return HipTensor(self, o.value, x.rows, 2 * hid)

    def jbatch(self, encProj, base, B, predProj, hid):
        o = self._out()
        check(self._p, lib().fa_jbatch(self._p, encProj.h, base, B, predProj.h, hid, C.byref(o)))
        return HipTensor(self, o.value, B, hid)

    def argmaxRows(self, x, B, vocab, logits):
        o = self._out()
        check(self._p, lib().fa_argmax_rows(self._p, x.h, B, vocab, logits, C.byref(o)))
        return HipTensor(self, o.value, B, 4)

    def jointArgmax(self, encProj, frame, count, predProj, outW, outB, hidden, vocab, logits):
        o = self._out()
        check(self._p, lib().fa_joint_argmax(self._p, encProj.h, frame, count, predProj.h, outW.h, outB.h, hidden, vocab, logits, C.byref(o)))
        return HipTensor(self, o.value, count, 4)

    # ── profiling (compute.d.ts:250-251) ──────────────────────────────────
    def startProfile(self, maxOps=4096, only=None):
        """Bracket launches with HIP events; `only` restricts it to a comma-separated
        list of exact labels (an entry ending in '*' matches a prefix)."""
        self._prof_cap = maxOps
        check(self._p, lib().fa_profile_only(self._p, (only or "").encode()))
        check(self._p, lib().fa_profile_start(self._p, maxOps))

    def endProfile(self):
        cap = getattr(self, "_prof_cap", 4096)
        labels = (C.c_char * (48 * cap))()
        ms = (C.c_float * cap)()
        n = C.c_int()
        check(self._p, lib().fa_profile_end(self._p, cap, labels, ms, C.byref(n)))
        raw = bytes(labels)
        return [{"label": raw[48 * i:48 * i + 48].split(b"\0", 1)[0].decode(), "ms": float(ms[i])} for i in range(min(n.value, cap))]

    # ── quantised-weight helpers (no ComputeContext counterpart) ──────────
    def dequantInt8(self, wq, scale, K, N):
        o = self._out()
        check(self._p, lib().fa_dequant_int8(self._p, wq.h, scale.h, K, N, C.byref(o)))
        return HipTensor(self, o.value, K, N)

    def dequantInt4(self, bq, scales_f16, K, N):
        o = self._out()
        check(self._p, lib().fa_dequant_int4(self._p, bq.h, scales_f16.h, K, N, C.byref(o)))
        return HipTensor(self, o.value, K, N)

    def gemvQuant(self, a, w, scales, fmt, N, K):
        o = self._out()
        check(self._p, lib().fa_gemv_quant(self._p, a.h, w.h, scales.h, fmt, N, K, C.byref(o)))
        return HipTensor(self, o.value, a.rows, N)

    def gemvQuantBatch(self, a_list, w_list, s_list, fmt, N, K):
        """len(w_list) independent GEMVs in one launch per 48 items; returns
        [count*M, N] (item i at rows i*M ..)."""
        n = len(w_list)
        if not (len(a_list) == len(s_list) == n):
            raise ValueError("gemvQuantBatch: one a, w and scales per item")
        arr = lambda xs: (L.T * n)(*[x.h for x in xs])
        o = self._out()
        check(self._p, lib().fa_gemv_quant_batch(self._p, n, arr(a_list), arr(w_list), arr(s_list), fmt, N, K, C.byref(o)))
        return HipTensor(self, o.value, n * a_list[0].rows, N)

    # ── ragged windows ────────────────────────────────────────────────────
    def packWindows(self, feats, starts, lens, layout="packed"):
        s = np.ascontiguousarray(starts, np.int32)
        l = np.ascontiguousarray(lens, np.int32)
        o = self._out()
        check(self._p, lib().fa_pack_windows(self._p, feats.h, s.ctypes.data_as(L.I32P), l.ctypes.data_as(L.I32P), len(l),
                                             0 if layout == "packed" else 1, C.byref(o)))
        return self._t(o.value)

    def melWindows(self, pcm, starts, lens, nMels=128, logGuard=2.0 ** -24, normalize=True):
        """Log-mel features of windows [starts[i], starts[i]+lens[i]) of a
        resident f32 sample stream -> f32 [nMels, Σ floor(lens[i]/160)]
        (fa_mel_windows), the layout packWindows reads."""
        s = np.ascontiguousarray(starts, np.int32)
        l = np.ascontiguousarray(lens, np.int32)
        o = self._out()
        check(self._p, lib().fa_mel_windows(self._p, pcm.h, s.ctypes.data_as(L.I32P), l.ctypes.data_as(L.I32P), len(l), int(nMels),
                                            float(logGuard), int(bool(normalize)), C.byref(o)))
        return self._t(o.value)

    def windowRowMap(self, lens, layout="packed", stage=0):
        l = np.ascontiguousarray(lens, np.int32)
        lay = 0 if layout == "packed" else 1
        rows = C.c_int()
        check(self._p, lib().fa_window_row_map(self._p, l.ctypes.data_as(L.I32P), len(l), lay, stage, None, C.byref(rows)))
        m = np.empty(rows.value, np.int32)
        check(self._p, lib().fa_window_row_map(self._p, l.ctypes.data_as(L.I32P), len(l), lay, stage, m.ctypes.data_as(L.I32P), C.byref(rows)))
        return m



def createContext(backend: str = "hip", device: int = 0) -> HipContext:
    """Backend factory (src/gpu/context.js:23-37) with the `hip` arm.  Raises
    when no gfx950 GPU is available: there is no silent CPU fallback."""
    if backend not in ("hip", "auto"):
        raise ValueError(f"createContext: backend {backend!r} is not provided by this package (only 'hip')")
    return HipContext(device)
