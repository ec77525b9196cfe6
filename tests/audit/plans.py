"""Scenarios run against the launch-audit build (build_audit.py), one per
process:

    FA_LIB_PATH=.../libfa_hip_audit.so FA_AUDIT_KERNARGS=.../kernargs.txt \
        python tests/audit/plans.py <scenario>

Each prints one JSON line: the stand-in runtime's violations and counters.
Kernels do not run, so device buffers hold what the host wrote (zeros after
allocation); only host-side control flow that reads device results (the TDT
decoder's live-window count) sees those zeros and ends early.
"""
from __future__ import annotations

import ctypes as C
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

FULL = dict(D=1024, DFF=4096, H=8, HD=128, layers=24, dwK=9, Csub=256, Fsub=16, melBins=128)
# FA_AUDIT_LAYERS: fewer encoder layers (same shapes per layer, fewer launches) for quicker plans
if os.environ.get("FA_AUDIT_LAYERS"):
    FULL["layers"] = int(os.environ["FA_AUDIT_LAYERS"])


def report(L, extra=None):
    buf = C.create_string_buffer(1 << 20)
    cnt = (C.c_ulonglong * 4)()
    L.audit_report.restype = C.c_int
    n = L.audit_report(buf, len(buf), cnt)
    out = {"violations": [v for v in buf.value.decode().splitlines() if v], "count": n, "launches": cnt[0], "graph_replays": cnt[1],
           "replayed_launches": cnt[2], "allocations": cnt[3]}
    ub = C.create_string_buffer(1 << 16)
    chk = C.c_ulonglong()
    L.audit_extent_report.restype = C.c_int
    L.audit_extent_report(ub, len(ub), C.byref(chk))
    out["extent_checks"] = chk.value
    out["unmodelled"] = [u for u in ub.value.decode().splitlines() if u]
    rb = C.create_string_buffer(1 << 16)
    L.audit_race_report.restype = C.c_int
    L.audit_race_report(rb, len(rb), C.byref(chk))
    out["order_checks"] = chk.value
    out["races"] = [r for r in rb.value.decode().splitlines() if r]
    out.update(extra or {})
    print(json.dumps(out), flush=True)


class Dim3(C.Structure):
    _fields_ = [("x", C.c_uint32), ("y", C.c_uint32), ("z", C.c_uint32)]


def controls(L):
    """Negative controls: each misuse below must be reported."""
    V = C.c_void_p
    L.hipMalloc.argtypes = [C.POINTER(V), C.c_size_t]
    L.hipFree.argtypes = [V]
    L.hipMemcpy.argtypes = [V, V, C.c_size_t, C.c_int]
    L.hipEventCreate.argtypes = [C.POINTER(V)]
    L.hipEventDestroy.argtypes = [V]
    L.hipEventRecord.argtypes = [V, V]
    L.hipStreamCreateWithFlags.argtypes = [C.POINTER(V), C.c_uint]
    L.hipStreamBeginCapture.argtypes = [V, C.c_int]
    L.hipStreamEndCapture.argtypes = [V, C.POINTER(V)]
    L.hipGraphInstantiateWithFlags.argtypes = [C.POINTER(V), V, C.c_ulonglong]
    L.hipGraphLaunch.argtypes = [V, V]
    L.hipLaunchKernel.argtypes = [V, Dim3, Dim3, C.POINTER(V), C.c_size_t, V]
    got = {}

    def step(name, fn):
        L.audit_clear()
        fn()
        buf = C.create_string_buffer(1 << 16)
        got[name] = L.audit_report(buf, len(buf), None)

    a, b = V(), V()
    L.hipMalloc(C.byref(a), 4096)
    L.hipMalloc(C.byref(b), 4096)
    host = (C.c_char * 8192)()
    # copy into a freed block; a copy running past its block's end
    L.hipFree(b)
    step("copy_into_freed_block", lambda: L.hipMemcpy(b, host, 16, 1))
    step("copy_past_block_end", lambda: L.hipMemcpy(a, host, 8192, 1))
    # an event recorded after destruction
    ev = V()
    L.hipEventCreate(C.byref(ev))
    L.hipEventDestroy(ev)
    step("event_after_destroy", lambda: L.hipEventRecord(ev, None))
    # a kernel whose pointer argument lies in a freed block (f32_to_f16_kernel(src, dst, n))
    kern = C.addressof(C.c_char.in_dll(L, "_ZN2fa17f32_to_f16_kernelEPKfPDF16_l"))
    n = C.c_long(16)
    args = (V * 3)(C.cast(C.pointer(b), V), C.cast(C.pointer(a), V), C.cast(C.pointer(n), V))
    step("kernel_arg_in_freed_block", lambda: L.hipLaunchKernel(kern, Dim3(1, 1, 1), Dim3(64, 1, 1), args, 0, None))
    # a block size above the kernel's maximum
    args2 = (V * 3)(C.cast(C.pointer(a), V), C.cast(C.pointer(a), V), C.cast(C.pointer(n), V))
    step("block_above_max", lambda: L.hipLaunchKernel(kern, Dim3(1, 1, 1), Dim3(2048, 1, 1), args2, 0, None))
    # a graph whose captured pointer is freed before a replay
    s, g, x, c = V(), V(), V(), V()
    L.hipStreamCreateWithFlags(C.byref(s), 0)
    L.hipMalloc(C.byref(c), 4096)
    args3 = (V * 3)(C.cast(C.pointer(c), V), C.cast(C.pointer(a), V), C.cast(C.pointer(n), V))
    L.hipStreamBeginCapture(s, 0)
    L.hipLaunchKernel(kern, Dim3(1, 1, 1), Dim3(64, 1, 1), args3, 0, s)
    L.hipStreamEndCapture(s, C.byref(g))
    L.hipGraphInstantiateWithFlags(C.byref(x), g, 0)
    step("graph_replay_clean", lambda: L.hipGraphLaunch(x, s))
    L.hipFree(c)
    step("graph_replay_after_free", lambda: L.hipGraphLaunch(x, s))
    # extent models: copy_f4_kernel(src, dst, n4) inside its blocks, then one
    # 16-byte vector past the end of the destination's 4096 bytes
    cp = C.addressof(C.c_char.in_dll(L, "_ZN2fa14copy_f4_kernelEPK15HIP_vector_typeIfLj4EEPS1_l"))
    d, e = V(), V()
    L.hipMalloc(C.byref(d), 8192)
    L.hipMalloc(C.byref(e), 4096)
    n4_ok, n4_over = C.c_long(256), C.c_long(257)
    a_ok = (V * 3)(C.cast(C.pointer(d), V), C.cast(C.pointer(e), V), C.cast(C.pointer(n4_ok), V))
    a_over = (V * 3)(C.cast(C.pointer(d), V), C.cast(C.pointer(e), V), C.cast(C.pointer(n4_over), V))
    step("extent_clean", lambda: L.hipLaunchKernel(cp, Dim3(1, 1, 1), Dim3(256, 1, 1), a_ok, 0, None))
    step("extent_write_past_block_end", lambda: L.hipLaunchKernel(cp, Dim3(1, 1, 1), Dim3(256, 1, 1), a_over, 0, None))
    # ordering: two non-blocking streams write the same block, first with an
    # event between them (ordered), then without; a synchronous copy on the
    # null stream into a block a queued kernel writes; the same after a
    # stream synchronisation
    L.hipStreamWaitEvent.argtypes = [V, V, C.c_uint]
    L.hipStreamSynchronize.argtypes = [V]
    s1, s2, ev2 = V(), V(), V()
    L.hipStreamCreateWithFlags(C.byref(s1), 1)
    L.hipStreamCreateWithFlags(C.byref(s2), 1)
    L.hipEventCreate(C.byref(ev2))

    def ordered():
        L.hipLaunchKernel(cp, Dim3(1, 1, 1), Dim3(256, 1, 1), a_ok, 0, s1)
        L.hipEventRecord(ev2, s1)
        L.hipStreamWaitEvent(s2, ev2, 0)
        L.hipLaunchKernel(cp, Dim3(1, 1, 1), Dim3(256, 1, 1), a_ok, 0, s2)

    def unordered():
        L.hipLaunchKernel(cp, Dim3(1, 1, 1), Dim3(256, 1, 1), a_ok, 0, s1)
        L.hipLaunchKernel(cp, Dim3(1, 1, 1), Dim3(256, 1, 1), a_ok, 0, s2)

    def null_copy(sync):
        def f():
            L.hipLaunchKernel(cp, Dim3(1, 1, 1), Dim3(256, 1, 1), a_ok, 0, s1)
            if sync:
                L.hipStreamSynchronize(s1)
            L.hipMemcpy(e, host, 64, 1)
        return f

    L.hipStreamSynchronize(None)
    step("streams_ordered_by_event", ordered)
    L.hipStreamSynchronize(s2)
    step("streams_unordered_write_write", unordered)
    L.hipStreamSynchronize(s2)
    L.hipStreamSynchronize(s1)
    step("null_stream_copy_after_sync", null_copy(True))
    step("null_stream_copy_over_queued_kernel", null_copy(False))
    L.audit_clear()
    print(json.dumps({"controls": got}), flush=True)


def e2e(L, fa, wb: int, seconds: float, profile: bool, pipelined: bool = True):
    """pipeline.transcribeWindowed over `seconds` of synthetic PCM in groups of
    `wb` windows with the full encoder (f16): one pass with captured graphs,
    then one pass with a profile window of 400,000 launches open."""
    import importlib
    pl = importlib.import_module(fa.__name__ + ".pipeline")
    pl.MAX_WINDOWS = max(pl.MAX_WINDOWS, wb)  # the audit build's encoder takes wb windows
    ctx = fa.createContext("hip")
    man = fa.synth.make_weights(dict(FULL), seed=1)
    enc = fa.FusedEncoder(ctx, man, "f16", max_T=188)
    del man
    dec = fa.TdtDecoder(ctx, fa.synth.make_decoder_weights(1))
    W, b = fa.synth.make_joint_projection(2)
    projW, projB = ctx.upload(W, W.shape[0], W.shape[1]), ctx.upload(b.reshape(1, -1), 1, b.size)
    audio = fa.synth.make_pcm(seconds, seed=1)
    r = pl.transcribeWindowed(ctx, enc, dec, projW, projB, audio, wb=wb, pipelined=pipelined, untested=True)
    n_prof = 0
    if profile:
        ctx.startProfile(400000)
        r = pl.transcribeWindowed(ctx, enc, dec, projW, projB, audio, wb=wb, pipelined=pipelined, untested=True)
        n_prof = len(ctx.endProfile())
    stats = r["stats"]
    enc.close()
    dec.close()
    ctx.destroy()
    report(L, {"windows": stats["windows"], "groups": stats["groups"], "profiled_launches": n_prof})


def ragged(L, fa):
    """the hour's ragged windows in packed batches of up to 32,
    every batch through fa_encoder_forward_stream_batches (two lanes)."""
    import numpy as np
    ctx = fa.createContext("hip")
    man = fa.synth.make_weights(dict(FULL), seed=1)
    enc = fa.FusedEncoder(ctx, man, "f16", max_T=375)
    del man
    total = 360000
    starts, lens = fa.windowing.planRaggedWindows(total, 200, 3000, 100, seed=1)
    batches = [(starts[b], lens[b]) for b in (np.asarray(g) for g in fa.windowing.packBatches(lens, 32))]
    feats = ctx.upload(np.zeros((128, total), np.float32), 128, total)
    for _ in range(2):
        for o in enc.forwardStreamBatches(feats, batches, "packed"):
            ctx.freeTensor(o)
    enc.close()
    ctx.destroy()
    report(L, {"batches": len(batches)})


def quant(L, fa):
    """the quantised encoder (int8, int4) on both of its routes:
    4 windows of 15 s (752 rows: each layer's weights widened once by
    wdq_kernel, then the f16 GEMMs) and 2 windows of 8 s (200 rows: the
    dequantisation inside the GEMM)."""
    ctx = fa.createContext("hip")
    man = fa.synth.make_weights(dict(FULL), seed=1)
    for fmt in ("int8", "int4"):
        enc = fa.FusedEncoder(ctx, man, fmt, max_T=188)
        for T, W in ((1500, 4), (800, 2)):
            enc.encode(fa.synth.make_features(128, T, seed=3, W=W))
        enc.close()
    ctx.destroy()
    report(L, {"formats": 2})


def oppath(L, fa):
    """The reference's op sequence (parakeetEncodeBatch over ComputeContext
    ops) with f16 and f32 weights, with and without the attnFused member, on
    2 windows; then the fused encoder's packed and padded forwards from
    packWindows."""
    import numpy as np
    ctx = fa.createContext("hip")
    man = fa.synth.make_weights(dict(FULL), seed=1)
    mels = fa.synth.make_features(128, 400, seed=5, W=2)
    for weights in ("f16", "f32"):
        enc = fa.loadParakeetEncoder(ctx, man, weights=weights)
        for fused in (False, True):
            a = ctx.pushArena()
            fa.parakeetEncodeBatch(ctx, enc, mels, attnFused=fused)
            ctx.popArena(a)
    fe = fa.FusedEncoder(ctx, man, "f16", max_T=188)
    stream_ = np.concatenate(mels, axis=1)
    feats = ctx.upload(stream_, 128, stream_.shape[1])
    for layout in ("packed", "padded"):
        a = ctx.pushArena()
        packed = ctx.packWindows(feats, [0, 400], [400, 400], layout)
        fe.forward(packed, [400, 400], layout)
        ctx.popArena(a)
    fe.close()
    ctx.destroy()
    report(L, {"routes": 5})


def stream(L, fa, profile: bool):
    """The stream workload (EOU config): one stream pushed 160 ms at a time,
    then 16 streams pushed together, with or without a profile window."""
    cfg = dict(FULL, subPad={"t": 2, "b": 1, "l": 2, "r": 1}, convCausal=True, attChunk=2, attLeft=70, Fsub=17)
    ctx = fa.createContext("hip")
    man = fa.synth.make_weights(cfg, seed=1)
    enc = fa.FusedEncoder(ctx, man, "f16", max_T=128, cfg=cfg)
    del man
    mel = fa.synth.make_features(128, 800, seed=2)[0]
    if profile:
        ctx.startProfile(200000)
    st = fa.createEncodeStream(ctx, enc)
    for t in range(0, mel.shape[1], 16):
        fa.encodeStreamPush(ctx, st, mel[:, t:t + 16])
    fa.encodeStreamFlush(ctx, st)
    fa.disposeEncodeStream(ctx, st)
    sts = [fa.createEncodeStream(ctx, enc) for _ in range(16)]
    for t in range(0, mel.shape[1], 16):
        fa.encodeStreamsPush(ctx, sts, [mel[:, t:t + 16]] * 16)
    for s in sts:
        fa.encodeStreamFlush(ctx, s)
        fa.disposeEncodeStream(ctx, s)
    if profile:
        ctx.endProfile()
    enc.close()
    ctx.destroy()
    report(L)


def stream_failures(L, fa):
    """Error paths of stream pushes, with failures injected into the stand-in
    runtime: an allocation that fails before a pass is queued leaves the
    stream as it was (the next push emits the frames of both pushes), a
    launch that fails while a pass is queued marks the stream failed (later
    pushes are refused with FA_E_STATE)."""
    cfg = dict(FULL, layers=2, subPad={"t": 2, "b": 1, "l": 2, "r": 1}, convCausal=True, attChunk=2, attLeft=70, Fsub=17)
    ctx = fa.createContext("hip")
    man = fa.synth.make_weights(cfg, seed=1)
    enc = fa.FusedEncoder(ctx, man, "f16", max_T=128, cfg=cfg)
    mel = fa.synth.make_features(128, 320, seed=2)[0]
    pieces = [mel[:, t:t + 32] for t in range(0, 320, 32)]

    def frames(o):
        return 0 if o is None else o.shape[0]

    ref = fa.createEncodeStream(ctx, enc)
    ref_counts = [frames(fa.encodeStreamPush(ctx, ref, p)) for p in pieces]
    fa.disposeEncodeStream(ctx, ref)
    out = {"reference_frames": sum(ref_counts)}
    # allocation failure on push 3: nothing moves, push 4 catches up
    st = fa.createEncodeStream(ctx, enc)
    got, err = [], None
    for i, p in enumerate(pieces):
        if i == 3:
            ctx.trimPool(0)
            L.audit_fail_alloc(0)
            try:
                fa.encodeStreamPush(ctx, st, p)
            except fa.FaError as e:
                err = e.code
            L.audit_fail_alloc(-1)
            continue
        got.append(frames(fa.encodeStreamPush(ctx, st, p)))
    out["alloc_failure_code"] = err
    out["alloc_failure_frames"] = sum(got)
    fa.disposeEncodeStream(ctx, st)
    # launch failure inside a pass: the stream is refused afterwards
    st = fa.createEncodeStream(ctx, enc)
    fa.encodeStreamPush(ctx, st, pieces[0])
    L.audit_fail_launch(5)
    try:
        fa.encodeStreamPush(ctx, st, pieces[1])
        out["launch_failure_code"] = 0
    except fa.FaError as e:
        out["launch_failure_code"] = e.code
    L.audit_fail_launch(-1)
    try:
        fa.encodeStreamPush(ctx, st, pieces[2])
        out["after_failure_code"] = 0
    except fa.FaError as e:
        out["after_failure_code"] = e.code
    fa.disposeEncodeStream(ctx, st)
    enc.close()
    ctx.destroy()
    L.audit_clear()
    print(json.dumps(out), flush=True)


def abi(L, fa):
    """The library's host-side semantics and error paths through its Python
    bindings, with no GPU (results read back are whatever the stand-in holds:
    only control flow, bookkeeping and validation are checked): arenas and
    pool reuse, pin, staged reads, batch nesting, shape errors, encoder /
    decoder / log-mel / transcription argument checks, the allocation-free
    entry point's size limits and its one-context-per-device rule."""
    import ctypes as C
    import importlib
    import numpy as np
    pl = importlib.import_module(fa.__name__ + ".pipeline")
    ctx = fa.createContext("hip")
    got = {}

    def check(name, fn):
        try:
            fn()
            got[name] = "ok"
        except Exception as e:  # noqa: BLE001 (reported per check)
            got[name] = f"{type(e).__name__}: {e}"

    def raises(fn, match=""):
        try:
            fn()
        except (fa.FaError, ValueError) as e:
            if match and match not in str(e):
                raise AssertionError(f"error without {match!r}: {e}")
            return
        raise AssertionError("no error")

    def arenas():
        x = ctx.upload(np.ones((64, 64), np.float32), 64, 64)
        ctx.memStatsStart()
        t = None
        for _ in range(3):
            a = ctx.pushArena()
            t = ctx.transpose(ctx.scale(x, 2.0))
            ctx.popArena(a)
        st = ctx.memStats()
        assert st["reused"] >= 4 and st["created"] <= 2, st
        raises(lambda: ctx.download(t), "stale")

    def pin():
        x = ctx.upload(np.ones((4, 4), np.float32), 4, 4)
        outer = ctx.pushArena()
        inner = ctx.pushArena()
        y = ctx.scale(x, 3.0)
        z = ctx.scale(x, 5.0)
        ctx.pin(y, True)
        ctx.popArena(inner)
        ctx.download(y)
        raises(lambda: ctx.download(z))
        ctx.popArena(outer)
        raises(lambda: ctx.download(y))

    def staged():
        x = ctx.upload(np.arange(6, dtype=np.float32), 2, 3)
        s = ctx.stageDownload(ctx.scale(x, 2.0))
        s.read()
        raises(s.read, "single-use")
        ctx.beginBatch()
        raises(ctx.beginBatch, "already open")
        ctx.endBatch()
        raises(ctx.endBatch)

    def shapes():
        a = ctx.upload(np.zeros((3, 5), np.float32), 3, 5)
        b = ctx.upload(np.zeros((4, 2), np.float32), 4, 2)
        raises(lambda: ctx.matmul(a, b), "matmul")
        raises(lambda: ctx.relShiftB(a, 2))

    def encoder():
        cfg = dict(D=256, DFF=1024, H=2, HD=128, layers=1, dwK=9, Csub=64, Fsub=16, melBins=128)
        enc = fa.FusedEncoder(ctx, fa.synth.make_weights(cfg, seed=1), "f16", max_T=32)
        mel = ctx.upload(np.zeros((1000, 128), np.float32), 1000, 128)
        raises(lambda: enc.forward(mel, [999]), "max_T")
        raises(lambda: enc.forward(mel, [200, 200, 200, 200, 201]), "rows")
        raises(lambda: enc.forward(mel, [10] * 65), "windows")
        enc.close()

    def decoder():
        d = fa.TdtDecoder(ctx, fa.synth.make_decoder_weights(1))
        raises(lambda: d.decodeBatch(ctx.upload(np.zeros((10, 100), np.float32), 10, 100), [10]))  # not 640 wide
        raises(lambda: d.decodeBatch(ctx.upload(np.zeros((10, 640), np.float32), 10, 640), [11]))  # more frames than rows
        raises(lambda: d.decodeBatch(ctx.upload(np.zeros((10, 640), np.float32), 10, 640), [-1]))  # negative length
        d.close()

    def mel():
        pcm = ctx.upload(np.zeros((1, 1000), np.float32), 1, 1000)
        raises(lambda: ctx.melWindows(pcm, [0], [2000]))
        raises(lambda: ctx.melWindows(pcm, [0], [1000], nMels=129))
        raises(lambda: ctx.melWindows(pcm, [-1], [10]))

    def transcription():
        raises(lambda: pl.transcribeWindowed(None, None, None, None, None, np.zeros(16000, np.float32), wb=0), "wb")
        raises(lambda: pl.transcribeWindowed(None, None, None, None, None, np.zeros(int(471 * 16000), np.float32)), "faulted the GPU")

    def mel_static():
        L.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        pcm, out = C.c_void_p(), C.c_void_p()
        n = 16000 * 10
        L.hipMalloc(C.byref(pcm), n * 4)
        L.hipMalloc(C.byref(out), 128 * 200 * 4)

        def call(c, starts, lens, n_mels, cols):
            st = np.ascontiguousarray(starts, np.int32)
            ln = np.ascontiguousarray(lens, np.int32)
            return fa.lib().fa_mel_windows_static(c._p, pcm, n, st.ctypes.data_as(C.POINTER(C.c_int32)), ln.ctypes.data_as(C.POINTER(C.c_int32)),
                                                  len(st), n_mels, 2.0 ** -24, 1, out, cols)
        assert call(ctx, [0] * 65, [160] * 65, 128, 65) == fa._lib.FA_E_UNSUPPORTED  # > 64 windows
        assert call(ctx, [0], [1600], 129, 10) == fa._lib.FA_E_INVALID  # > 128 bins
        assert call(ctx, [0], [1600], 128, 11) == fa._lib.FA_E_INVALID  # wrong output size
        assert call(ctx, [159000], [1600], 128, 10) == fa._lib.FA_E_INVALID  # outside the stream
        assert call(ctx, [0], [32000], 128, 200) == 0
        other = fa.createContext("hip")
        assert call(other, [0], [32000], 128, 200) == fa._lib.FA_E_STATE  # the array serves one context per device
        assert b"another context" in fa.lib().fa_last_error(other._p)
        other.destroy()

    for name, fn in [("arenas", arenas), ("pin", pin), ("staged", staged), ("shapes", shapes), ("encoder", encoder), ("decoder", decoder),
                     ("mel", mel), ("transcription", transcription), ("mel_static", mel_static)]:
        check(name, fn)
    ctx.destroy()
    report(L, {"checks": got})


def main():
    import __graft_entry__ as ge
    fa = ge.load_package()
    L = fa._lib.lib()
    what = sys.argv[1]
    if what == "controls":
        controls(L)
    elif what.startswith("e2e"):
        # e2e<wb>[s][p] [seconds]: s = stage by stage, p = a profiled pass too
        wb = int(what[3:].rstrip("ps"))
        e2e(L, fa, wb, float(sys.argv[2]) if len(sys.argv) > 2 else 3600.0, what.endswith("p"), "s" not in what[3:])
    elif what == "ragged":
        ragged(L, fa)
    elif what == "quant":
        quant(L, fa)
    elif what == "oppath":
        oppath(L, fa)
    elif what == "abi":
        abi(L, fa)
    elif what == "stream_failures":
        stream_failures(L, fa)
    elif what in ("stream", "streamp"):
        stream(L, fa, what == "streamp")
    else:
        raise SystemExit(f"unknown scenario {what}")


if __name__ == "__main__":
    main()
