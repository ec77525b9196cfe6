"""Host-side launch audit (CPU): the library's own objects linked against a
stand-in HIP runtime (tests/audit/launch_audit.cpp) that runs no kernel and
checks every call instead -- kernel pointer arguments (read with each
kernel's argument layout from its code-object metadata) inside live device
blocks at launch and at every graph replay, block sizes against the kernels'
launch bounds, static LDS against 160 KB, copies and fills inside their
blocks, and streams / events / graphs not used after destruction.

The plans audited are the ones whose GPU runs failed or matter most: the
one-hour windowed transcription in 64-window groups with a 400,000-launch
profile window open (the run that faulted the GPU; the audit build lifts the
encoder's 32-window limit for it), the same hour in 32-window groups
pipelined and stage by stage, configs[3]'s ragged batches on two lanes, and
the stream workload with and without a profile window (the workload whose
rocprofv3 trace crashed in the host).  Each path kernel also has an extent
model (tests/audit/extents.cpp): from its arguments and grid it derives the
byte span every pointer argument is read or written over and checks that span
against the block, so a launch whose index ranges run past a buffer is caught
as well.  Those ranges also feed a happens-before check across streams
(vector clocks over stream order, events, synchronisations and hipFree): a
write and another access to overlapping bytes from two streams with no
ordering between them is reported as a race.  The "abi" scenario runs the bindings' host semantics and argument
validation (arenas, pin, staged reads, batches, shape and size errors, the
allocation-free log-mel entry point's limits) against the same stand-in,
and the N-API addon is built against it too, so the Node host's conformance
cases and self-test run through the addon on the CPU."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
AUD = os.path.join(ROOT, "tests", "audit")
OBJ = os.path.join(ROOT, "fluidaudio-web_amd", "csrc", "_build")


@pytest.fixture(scope="module")
def builds():
    if not os.path.isdir(OBJ) or not any(f.endswith(".o") for f in os.listdir(OBJ)):
        pytest.skip("no library objects: run __graft_entry__.build() first")
    sys.path.insert(0, AUD)
    import build_audit
    return {None: build_audit.build(), 64: build_audit.build(64)}


def run(builds, scenario, *args, max_windows=None, layers=None):
    lib = builds[max_windows]
    tag = "" if max_windows is None else f"_w{max_windows}"
    env = dict(os.environ, FA_LIB_PATH=lib, FA_AUDIT_KERNARGS=os.path.join(AUD, "_build", f"kernargs{tag}.txt"))
    if layers:
        env["FA_AUDIT_LAYERS"] = str(layers)
    r = subprocess.run([sys.executable, os.path.join(AUD, "plans.py"), scenario, *map(str, args)], env=env, capture_output=True, text=True,
                       timeout=600)
    assert r.returncode == 0, r.stderr[-3000:]
    return json.loads(r.stdout.strip().splitlines()[-1])


def test_stand_in_reports_each_misuse(builds):
    got = run(builds, "controls")["controls"]
    assert got.pop("graph_replay_clean") == 0
    assert got.pop("extent_clean") == 0
    assert got.pop("streams_ordered_by_event") == 0
    assert got.pop("null_stream_copy_after_sync") == 0
    assert all(v >= 1 for v in got.values()), got  # a kernel's misuse can also show in its extents


def test_hour_in_64_window_groups_with_profile_window(builds):
    """The plan of the faulted run: 3600 s, 277 windows in 64-window groups,
    a graph-replayed pass, then a pass under a 400,000-launch profile window."""
    r = run(builds, "e2e64sp", 3600, max_windows=64)  # stage by stage, as that run was
    print(r)
    assert r["windows"] == 277 and r["groups"] == 6 and r["profiled_launches"] > 1000
    assert r["violations"] == []


@pytest.mark.parametrize("scenario", ["e2e32", "e2e32sp"])
def test_windowed_transcription_32_window_groups(builds, scenario):
    r = run(builds, scenario, 900, layers=2)
    assert r["groups"] >= 2 and r["graph_replays"] >= 2
    assert r["violations"] == []
    assert r["extent_checks"] > 0 and _unmodelled_on_path(r) == []


def _unmodelled_on_path(r):
    # kernels launched without an extent model
    return list(r["unmodelled"])


def test_hour_stage_by_stage_kernel_extents(builds):
    """The plan of the second faulted run, with every kernel's read / write
    ranges (extents.cpp) checked: 3600 s, 24 layers, 32-window groups stage
    by stage (10 groups: 8 x 32, 20, and one 1200-frame window)."""
    r = run(builds, "e2e32s", 3600)
    assert r["windows"] == 277 and r["groups"] == 10
    assert r["violations"] == []
    assert r["extent_checks"] > 50000 and _unmodelled_on_path(r) == []
    assert r["races"] == [] and r["order_checks"] > 50000


def test_hour_pipelined_stream_ordering(builds):
    """The plan of the pipelined hour that faulted: 3600 s, 24 layers,
    32-window groups with group g + 1's log-mel, encoder and projection on an
    encoder lane while group g decodes on the context stream.  Every range
    each kernel, copy and fill touches is ordered against the other streams'
    earlier accesses to the same bytes: no race."""
    r = run(builds, "e2e32", 3600)
    assert r["windows"] == 277 and r["launches"] > 2000
    assert r["violations"] == [] and _unmodelled_on_path(r) == []
    assert r["races"] == [] and r["order_checks"] > 50000


def test_ragged_batches_on_two_lanes(builds):
    r = run(builds, "ragged", layers=2)
    assert r["batches"] == 8 and r["graph_replays"] >= 8
    assert r["violations"] == []
    assert r["extent_checks"] > 0 and _unmodelled_on_path(r) == []
    assert r["races"] == [] and r["order_checks"] > 10000


def test_quantized_encoder_routes(builds):
    """configs[4]'s int8 and int4 encoder on both routes (weights widened once
    per layer for 752 rows; dequantisation inside the GEMM for 200 rows):
    every kernel modelled, inside its blocks, no unordered access."""
    r = run(builds, "quant", layers=2)
    assert r["launches"] > 100
    assert r["violations"] == [] and _unmodelled_on_path(r) == [] and r["races"] == []
    assert r["extent_checks"] > 500


def test_reference_op_sequence_and_packed_forwards(builds):
    """parakeetEncodeBatch's ComputeContext ops (f16 and f32 weights, with and
    without attnFused) and the fused encoder's packed / padded forwards from
    packWindows: every kernel modelled, inside its blocks."""
    r = run(builds, "oppath", layers=2)
    assert r["launches"] > 300
    assert r["violations"] == [] and _unmodelled_on_path(r) == [] and r["races"] == []
    assert r["extent_checks"] > 1000


@pytest.mark.parametrize("scenario", ["stream", "streamp"])
def test_stream_workload(builds, scenario):
    r = run(builds, scenario, layers=4)
    assert r["launches"] > 2000
    assert r["violations"] == []
    assert r["extent_checks"] > 10000 and _unmodelled_on_path(r) == []
    assert r["races"] == [] and r["order_checks"] > 10000


def test_stream_push_failures_leave_consistent_state(builds):
    """An allocation that fails before a stream pass is queued changes nothing
    (the next push emits both pushes' frames: the reference total); a launch
    that fails while a pass is queued marks the stream failed, and the next
    push is refused with FA_E_STATE."""
    r = run(builds, "stream_failures")
    assert r["alloc_failure_code"] == 4  # FA_E_OOM
    assert r["alloc_failure_frames"] == r["reference_frames"] > 0
    assert r["launch_failure_code"] == 3  # FA_E_DEVICE
    assert r["after_failure_code"] == 2  # FA_E_STATE


def test_host_semantics_and_argument_checks(builds):
    """Arena reuse and stale handles, pin, single-use staged reads, batch
    nesting, shape errors, encoder / decoder / log-mel / transcription
    argument checks and the allocation-free log-mel entry point's limits and
    one-context-per-device rule, with no GPU; the calls that pass validation
    launch inside their blocks."""
    r = run(builds, "abi")
    assert r["checks"] == {k: "ok" for k in ("arenas", "pin", "staged", "shapes", "encoder", "decoder", "mel", "transcription", "mel_static")}
    assert r["violations"] == [] and r["launches"] > 0


def _node_report(builds, script, tmp_path):
    import shutil
    import build_audit
    if shutil.which("node") is None:
        pytest.skip("node not installed")
    ndir = build_audit.build_node(builds[None])
    if ndir is None:
        pytest.skip("Node headers not installed")
    rep = tmp_path / f"{script}.txt"
    env = dict(os.environ, FA_AUDIT_KERNARGS=os.path.join(AUD, "_build", "kernargs.txt"), FA_AUDIT_REPORT=str(rep))
    r = subprocess.run(["node", os.path.join(ndir, f"{script}.js"), str(tmp_path / "dump.json")], env=env, capture_output=True, text=True, timeout=300)
    lines = rep.read_text().splitlines()
    counts = {k: int(v) for k, v in (ln.split(" ", 1) for ln in lines if ln.split(" ", 1)[0] in ("launches", "replays", "extent_checks", "order_checks"))}
    bad = [ln for ln in lines if ln.startswith(("violation", "race"))]
    return r, counts, bad


def test_node_addon_conformance_cases(builds, tmp_path):
    """The N-API addon (node/fa_napi.c) and HipContext (hip-context.js) run
    every required ComputeContext method's conformance case against the
    stand-in runtime: the addon's argument marshalling, tensor handles and
    error paths make no launch, copy or handle error and no unordered access
    (the numbers are not checked: kernels do not run)."""
    r, counts, bad = _node_report(builds, "conformance", tmp_path)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "58 cases cover every required method" in r.stdout
    assert counts["launches"] > 50 and counts["extent_checks"] > 100 and bad == []
    assert not any(ln.startswith("unmodelled") for ln in (tmp_path / "conformance.txt").read_text().splitlines())


def test_node_addon_selftest_runs_to_the_end(builds, tmp_path):
    """The Node self-test (fused encoder, log-mel windows, TDT decode through
    the addon) runs to its last case against the stand-in (exit 1 = only
    numeric checks failed, as kernels do not run; 2 would be an exception),
    with graph replays and no violation."""
    r, counts, bad = _node_report(builds, "selftest", tmp_path)
    assert r.returncode in (0, 1), r.stdout[-2000:] + r.stderr[-2000:]
    assert "tdtDecode known answer" in r.stdout
    assert counts["launches"] > 200 and counts["replays"] > 0 and counts["extent_checks"] > 1000 and bad == []

