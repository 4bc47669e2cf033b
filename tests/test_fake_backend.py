"""librelx's pipeline on the CPU, over a stand-in for the HIP runtime.

tests/native/pipeline_driver links the library's host sources (plan,
program, runtime, workers, indexed, transfer, capi) against
tests/native/hip_fake.cpp, under ThreadSanitizer, and runs C-ABI scenarios
over cases written here (plan bytes, bindings, source, the oracle's result).
The stand-in runs streams as worker threads, events as stream markers, and
every relayout launch with the element-wise kernel's semantics; it checks
each access to device memory, page-locked memory and registered host
buffers against the ordering HIP guarantees (stream order, events, host
synchronization), so a missing wait is reported whatever the timing.

Covered here, the way the reference's host backend and fault shim cover
its transfer engine (libreloc/include/reloc/HostBackend.h:27-75,
libreloc/test/TransferTestSupport.h:83-164):
  * ring and event ordering: every chunk size, ring depth, worker count,
    host-stage boundary, pageable and pinned sources, no_wait calls,
    caller streams (none, the null stream, a stream of their own), groups,
    submitted groups in flight together, device-to-host, device-resident
    relayouts, the allocation-free upload; results equal the oracle's and
    no access is unordered, with delays and jitter on every operation;
  * resources: parameter tables found by content across fresh bindings,
    and the ring and wire arena released down to max_retained_bytes once
    the context's calls have completed;
  * faults: allocation failures, copies, launches, event records and
    stream waits refused when submitted, copies and kernels that fault on
    their stream (a sticky device error), a synchronize that fails, and a
    device whose completion cannot be proven: the error code and the
    completion the C ABI reports, whether the context is quarantined, and
    what the next call and the close do;
  * the checker itself: a device-to-host call told of no producer stream
    reads a source still being written, which the checker reports.
"""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from oracle import relx_oracle as O
from sym_amd import encoder as EN
from sym_amd import workloads as W
from tests import fuzz_plans as F

HERE = os.path.dirname(os.path.abspath(__file__))
NATIVE = os.path.join(HERE, "native")
DRIVER = os.path.join(NATIVE, "_build", "pipeline_driver")


@pytest.fixture(scope="module")
def driver():
    if shutil.which("g++") is None or not os.path.isdir("/opt/rocm/include/hip"):
        pytest.skip("g++ or the HIP headers are missing")
    r = subprocess.run(["make", "-s", "-j8", "-C", NATIVE], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    return DRIVER


def run(driver, lines, timeout=240):
    """Run scenario lines; returns the parsed results (ThreadSanitizer
    findings fail the test)."""
    env = dict(os.environ, TSAN_OPTIONS="halt_on_error=0 exitcode=66 report_signal_unsafe=0")
    r = subprocess.run([driver], input="\n".join(lines) + "\n", capture_output=True, text=True,
                       timeout=timeout, env=env)
    assert "ThreadSanitizer" not in r.stderr, r.stderr[-6000:]
    assert r.returncode == 0, (r.returncode, r.stderr[-3000:])
    out = [json.loads(l) for l in r.stdout.splitlines() if l.startswith("{")]
    assert len(out) == len(lines), r.stdout[-2000:]
    return out


# ------------------------------------------------------------------ cases

def write_case(root, name, blob, src, want=None, syms=None, params=None, index=None):
    """params: {name: (kind, bits, array)}; index: (bits, array)."""
    d = os.path.join(str(root), name)
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "plan.bin"), "wb") as f:
        f.write(blob)
    lines = ["sym %s %d" % (k, v) for k, v in (syms or {}).items()]
    for i, (pname, (kind, bits, arr)) in enumerate((params or {}).items()):
        fn = "param%d.bin" % i
        arr = np.ascontiguousarray(arr)
        with open(os.path.join(d, fn), "wb") as f:
            f.write(arr.tobytes())
        lines.append("param %s %d %d %d %d %s" % (pname, kind, bits, arr.ndim, arr.size, fn))
    if index is not None:
        bits, arr = index
        with open(os.path.join(d, "index.bin"), "wb") as f:
            f.write(np.ascontiguousarray(arr).tobytes())
        lines.append("index 2 %d 1 %d index.bin" % (bits, len(arr)))
    with open(os.path.join(d, "bind.txt"), "w") as f:
        f.write("\n".join(lines) + "\n")
    with open(os.path.join(d, "src.bin"), "wb") as f:
        f.write(np.ascontiguousarray(src).tobytes())
    if want is not None:
        with open(os.path.join(d, "want.bin"), "wb") as f:
            f.write(bytes(want))
    return d


@pytest.fixture(scope="module")
def cases(tmp_path_factory):
    root = tmp_path_factory.mktemp("fake_cases")
    c = {}
    # C1 (layout only): 2^18 f32, transpose [4096, 64] -> [64, 4096]
    n = 1 << 18
    x = W.c1_input(n)
    blob = W.c1_plan().blob
    want = O.execute_layout(O.bind(O.decode_plan(blob), {"s0": n}), x.tobytes())
    c["c1"] = write_case(root, "c1", blob, x, want, {"s0": n})
    # C1 at 16 MiB: chunks of several MiB
    n = 1 << 22
    x = W.c1_input(n)
    want = O.execute_layout(O.bind(O.decode_plan(blob), {"s0": n}), x.tobytes())
    c["c1big"] = write_case(root, "c1big", blob, x, want, {"s0": n})
    # C2 (typed, one per-tensor cast): the host applies it at boundary 1
    shape = (2, 3, 32, 48)
    x = W.c2_input(*shape)
    blob = W.c2_plan(*shape).blob
    c["c2"] = write_case(root, "c2", blob, x, O.run_typed(blob, {}, {}, x).tobytes())
    # C5 (a per-head quantize on the device: results not emulated)
    b, s = 2, 64
    x, scale = W.c5_input(b, s)
    c["c5"] = write_case(root, "c5", W.c5_plan().blob, x, None, {"B": b, "S": s},
                         {"scale": (0, 32, scale)})
    # indexed: rows of an f32 table (copy gather)
    rng = np.random.default_rng(5)
    table = rng.standard_normal((4096, 64)).astype(np.float32)
    idx = rng.integers(0, 4096, 3000).astype(np.int64)
    iplan = EN.encode_index_select(["N", "D"], "float32", "M", "int64", "float32")
    syms = {"N": 4096, "D": 64, "M": len(idx)}
    c["ix"] = write_case(root, "ix", iplan, table, table[idx].tobytes(), syms, index=(64, idx))
    # a (128, 96) f16 transpose: a tile kernel and an edge kernel read the
    # one chunk
    src = np.random.default_rng(255).standard_normal((128, 96)).astype(np.float16)
    plan = EN.encode([128, 96], "float16", [EN.Transpose((1, 0))])
    c["edge"] = write_case(root, "edge", plan.blob, src, src.T.tobytes())
    # random layout plans (pads, transposes, reshapes) from the fuzz set
    k = 0
    for seed in range(0, 200):
        r = F.make_plan(seed)
        if r is None or r[0].typed:
            continue
        plan, src, _ = r
        try:
            want = O.execute_layout(O.bind(O.decode_plan(plan.blob), {}), src.tobytes())
        except (O.BindError, O.ExecutionError):
            continue
        c["fz%d" % k] = write_case(root, "fz%d" % seed, plan.blob, src, want)
        k += 1
        if k == 6:
            break
    return c


def ok(res):
    """Every call succeeded, results matched, no unordered access."""
    assert not res["setup_error"], res
    assert all(cl["rc"] == 0 for cl in res["calls"]), res["calls"]
    assert res["close"]["rc"] == 0, res["close"]
    assert res["mismatches"] == 0, res["notes"]
    assert not res["violations"], res["violations"][:5]
    assert not res["quarantined"]


# ------------------------------------------------------------ ordering

DELAYS = "delay_copy=300 delay_kernel=300 jitter=1"


def test_upload_orders_and_results(driver, cases):
    lines = []
    for name in ("c1", "fz0", "fz1", "fz2", "fz3", "fz4", "fz5"):
        for pinned in (0, 1):
            for chunk, nbuf in ((0, 0), (65536, 2), (16384, 3)):
                lines.append("h2d %s pinned=%d chunk=%d nbuf=%d threads=3 seed=%d %s"
                             % (cases[name], pinned, chunk, nbuf, len(lines), DELAYS))
    res = run(driver, lines)
    for r in res:
        ok(r)
        assert r["checked"] == 2
    chunked = [r for r in res if "chunk=16384" in lines[res.index(r)]]
    assert max(r["report"]["chunks"] for r in chunked) >= 8


def test_report_describes_the_schedule(driver, cases):
    """The host side of the report (reference Report::hostChunkBytes,
    hostBuffers and the staging rows) against the schedule each call ran:
    16 MiB of f32 wire in 2 MiB chunks staged through a 3-slot ring (the
    second call reuses it), sent by direct DMA, staged as one chunk (a ring
    of one slot, as the reference sizes it: min(n_buffers, chunks)), and on
    one copy stream."""
    c = cases["c1big"]
    M = 1 << 20
    lines = ["h2d %s pinned=0 chunk=%d nbuf=3 threads=4 %s" % (c, 2 * M, DELAYS),
             "h2d %s pinned=1 chunk=%d nbuf=3 threads=4 %s" % (c, 2 * M, DELAYS),
             "h2d %s pinned=0 chunk=%d nbuf=2 threads=4 %s" % (c, 16 * M, DELAYS),
             "h2d %s pinned=0 chunk=%d nbuf=2 threads=4 streams=1 %s" % (c, 2 * M, DELAYS),
             "d2h %s pinned=0 chunk=%d nbuf=3 threads=4 %s" % (c, 4 * M, DELAYS)]
    res = run(driver, lines)
    for r in res:
        ok(r)
        assert r["checked"] == 2
    rep = [r["report"] for r in res]
    assert rep[0]["wire_bytes"] == 16 * M
    assert (rep[0]["chunks"], rep[0]["host_chunk_bytes"], rep[0]["host_buffers"]) == (8, 2 * M, 3)
    assert (rep[0]["staging_slots"], rep[0]["staging_bytes"], rep[0]["staging_reused"]) == (3, 6 * M, 1)
    assert rep[0]["copy_streams"] == 2 and rep[0]["direct_dma"] == 0
    assert (rep[1]["chunks"], rep[1]["host_chunk_bytes"], rep[1]["host_buffers"]) == (8, 2 * M, 0)
    assert (rep[1]["staging_slots"], rep[1]["staging_bytes"], rep[1]["direct_dma"]) == (0, 0, 1)
    assert (rep[2]["chunks"], rep[2]["host_chunk_bytes"], rep[2]["host_buffers"]) == (1, 16 * M, 1)
    assert (rep[2]["staging_slots"], rep[2]["staging_bytes"], rep[2]["copy_streams"]) == (1, 16 * M, 1)
    assert res[2]["pinned_bytes"] == 16 * M  # one slot: the ring the call needed, no more
    assert (rep[3]["chunks"], rep[3]["copy_streams"], rep[3]["host_buffers"]) == (8, 1, 2)
    assert (rep[4]["chunks"], rep[4]["host_chunk_bytes"], rep[4]["host_buffers"]) == (4, 4 * M, 3)
    assert rep[4]["staging_slots"] == 3 and rep[4]["copy_streams"] == 2


def test_large_chunks_and_the_last_batch(driver, cases):
    """16 MiB of source in chunks of 2 to 16 MiB: kernel batches of several
    chunks, the last chunk a batch of its own."""
    lines = ["h2d %s pinned=%d chunk=%d nbuf=2 threads=4 repeat=2 %s" % (cases["c1big"], pinned, ch, DELAYS)
             for pinned in (0, 1) for ch in (16 << 20, 2 << 20)]
    res = run(driver, lines)
    for r in res:
        ok(r)
        assert r["checked"] == 2
    # 8 chunks of 2 MiB: batches of two chunks up to the last, which is
    # alone: [0,2) [2,4) [4,6) [6,7) [7,8)
    assert [r["report"]["kernel_launches"] for r in res] == [1, 5, 1, 5]


def test_host_stages_and_device_stages(driver, cases):
    lines = ["h2d %s hs=1 chunk=%d nbuf=2 threads=4 seed=%d %s" % (cases["c2"], ch, i, DELAYS)
             for i, ch in enumerate((0, 8192, 65536))]
    # device value stages: ordering only (the stand-in does not run stages)
    lines += ["h2d %s chunk=%d check=0 seed=%d %s" % (cases["c5"], ch, i, DELAYS)
              for i, ch in enumerate((0, 32768))]
    lines += ["h2d %s hs=0 check=0 chunk=8192 %s" % (cases["c2"], DELAYS)]
    res = run(driver, lines)
    for r in res:
        ok(r)
    assert all(r["report"]["wire_boundary"] == 1 and r["checked"] == 2 for r in res[:3])
    assert all(r["counts"]["unemulated"] > 0 for r in res[3:])


@pytest.mark.parametrize("caller", ["none", "null", "stream"])
def test_no_wait_and_caller_streams(driver, cases, caller):
    lines = ["h2d %s caller=%s nowait=%d chunk=32768 nbuf=2 repeat=3 seed=%d %s"
             % (cases[n], caller, nw, i, DELAYS)
             for i, (n, nw) in enumerate(((n, nw) for n in ("c1", "fz2") for nw in (0, 1)))]
    for r in run(driver, lines):
        ok(r)


@pytest.mark.parametrize("caller", ["none", "stream"])
def test_no_wait_calls_back_to_back(driver, cases, caller):
    """Calls in flight together: each call's copies overwrite the wire arena
    the call before may still be reading, and its kernels the destination
    that call writes."""
    lines = ["h2d %s caller=%s nowait=1 burst=1 pinned=%d chunk=%d nbuf=2 repeat=4 seed=%d %s"
             % (cases[n], caller, pinned, chunk, i, DELAYS)
             for i, (n, pinned, chunk) in enumerate(
                 (n, p, ch) for n in ("c1", "fz2") for p in (0, 1) for ch in (0, 16384, 65536))]
    res = run(driver, lines)
    for r in res:
        ok(r)
        assert r["checked"] == 1


def test_groups_and_submissions(driver, cases):
    lines = ["group %s members=3 chunk=32768 nbuf=2 %s" % (cases["c1"], DELAYS),
             "group %s members=4 hs=1 chunk=8192 nbuf=3 %s" % (cases["c2"], DELAYS),
             "submit %s members=2 chunk=32768 %s" % (cases["c1"], DELAYS),
             "submit %s members=2 chunk=16384 nbuf=2 twice=1 %s" % (cases["fz1"], DELAYS),
             "submit %s members=2 pinned=1 twice=1 %s" % (cases["c1"], DELAYS)]
    res = run(driver, lines)
    for r in res:
        ok(r)
    assert res[0]["checked"] == 3 and res[3]["checked"] == 4


def test_indexed_uploads(driver, cases):
    lines = ["h2d %s chunk=%d nbuf=2 seed=%d %s" % (cases["ix"], ch, i, DELAYS)
             for i, ch in enumerate((0, 65536, 4096))]
    lines.append("h2d %s pinned=1 %s" % (cases["ix"], DELAYS))
    res = run(driver, lines)
    for r in res:
        ok(r)
    assert {r["report"]["implementation"] for r in res} >= {"hip_table_gather"} or \
        all(r["report"]["implementation"].startswith("hip_relayout") for r in res)


def test_device_to_host_and_device_resident(driver, cases):
    lines = []
    for name in ("c1", "fz0", "fz3"):
        for pinned in (0, 1):
            for chunk in (0, 16384):
                lines.append("d2h %s pinned=%d chunk=%d nbuf=2 caller=stream %s"
                             % (cases[name], pinned, chunk, DELAYS))
        for caller in ("null", "stream"):
            lines.append("device %s caller=%s %s" % (cases[name], caller, DELAYS))
    lines.append("d2h %s caller=null %s" % (cases["c1"], DELAYS))
    # an indexed plan's rows gathered from a device-resident table
    lines += ["device %s caller=%s %s" % (cases["ix"], caller, DELAYS) for caller in ("null", "stream")]
    res = run(driver, lines)
    for r in res:
        ok(r)
    assert all(r["checked"] == 2 for r in res)


def test_allocation_free_upload(driver, cases):
    lines = ["static %s %s" % (cases["c1"], DELAYS), "static %s %s" % (cases["fz2"], DELAYS)]
    for r in run(driver, lines):
        ok(r)


def test_allocation_free_calls_from_two_contexts(driver, cases):
    """no_wait static calls alternating between two contexts on one device
    share the device's static scratch: each call's copies into it wait for
    the previous static call's end, whichever context made it (the checker
    reports a copy that overwrites the scratch while a kernel of the other
    context still reads it)."""
    lines = ["static_pair %s repeat=%d %s" % (cases[name], n, DELAYS)
             for name in ("c1", "fz2") for n in (2, 5)]
    for r in run(driver, lines):
        ok(r)
        assert r["checked"] >= 2, r


def test_parameter_tables_uploaded_once_per_context(driver, cases):
    """A fresh binding per call finds its parameter tables in the context:
    the calls allocate the wire arena and one table block, however many
    bindings run (each binding's own pair of tables would be two more per
    call)."""
    for name in ("c5", "c1"):
        res = run(driver, ["h2d %s check=0 repeat=4 rebind=%d %s" % (cases[name], rb, DELAYS)
                           for rb in (0, 1)])
        for r in res:
            ok(r)
            assert r["counts"]["mallocs"] == 2, r["counts"]
        assert res[0]["counts"] == res[1]["counts"]


def test_retained_scratch_bound(driver, cases):
    """max_retained_bytes: after each blocking call the ring (3 slots of
    1 MiB) and then the wire arena (2 MiB) are released until what is kept
    fits; the next call allocates them again. A negative bound keeps both
    (reference DispatchResources.h:57-61)."""
    base = "h2d %s repeat=3 chunk=65536 nbuf=3 %s" % (cases["c1"], DELAYS)
    res = run(driver, [base + " retained=%d" % lim for lim in (-1, 0, 2 << 20, 5 << 20)])
    for r in res:
        ok(r)
        assert r["checked"] == 3
    kept = [(r["pinned_bytes"], r["device_bytes"]) for r in res]
    assert kept == [(3 << 20, 2 << 20), (0, 0), (0, 2 << 20), (3 << 20, 2 << 20)]
    # device blocks: wire arena per call when it is released, plus the table block
    assert [r["counts"]["mallocs"] for r in res] == [2, 4, 2, 2]
    assert [r["counts"]["host_mallocs"] for r in res] == [3, 9, 9, 3]
    # a no_wait call keeps its scratch until the synchronize that completes it
    r = run(driver, ["h2d %s nowait=1 repeat=2 chunk=65536 nbuf=3 retained=0 %s"
                     % (cases["c1"], DELAYS)])[0]
    ok(r)
    assert (r["pinned_bytes"], r["device_bytes"]) == (0, 0)
    assert r["counts"]["mallocs"] == 3, r["counts"]
    # device-to-host calls release their result buffer and ring the same way
    res = run(driver, ["d2h %s repeat=3 retained=0 pinned=%d %s" % (cases["c1"], p, DELAYS)
                       for p in (0, 1)])
    for r in res:
        ok(r)
        assert (r["pinned_bytes"], r["device_bytes"]) == (0, 0)
        assert r["counts"]["mallocs"] == 4, r["counts"]  # a result buffer per call + the tables
    # the 1 MiB result crosses as one chunk: a ring of one slot per call
    assert [r["counts"]["host_mallocs"] for r in res] == [3, 0]


def test_small_staged_uploads_read_their_slot(driver, cases):
    """A staged upload of one chunk of at most 1 MiB of wire: its kernel
    reads the ring slot (zero-copy), with no copy ahead of it; a pinned
    source keeps its direct copy, and a chunked upload its copies. Blocking
    calls back to back, no_wait calls and calls from several threads all
    reuse the slot in order, with the results of the oracle, also where
    several kernels of one call read the slot."""
    lines = ["h2d %s repeat=3 %s" % (cases["c1"], DELAYS),
             "h2d %s repeat=3 pinned=1 %s" % (cases["c1"], DELAYS),
             "h2d %s repeat=3 chunk=65536 nbuf=2 %s" % (cases["c1"], DELAYS),
             "h2d %s repeat=4 nowait=1 burst=1 %s" % (cases["c1"], DELAYS),
             "h2d %s repeat=2 %s" % (cases["c2"], DELAYS),
             "h2d %s repeat=2 %s" % (cases["ix"], DELAYS),
             "threads %s threads_n=3 repeat=3 shared=1 %s" % (cases["c1"], DELAYS),
             "h2d %s repeat=3 %s" % (cases["edge"], DELAYS),
             "h2d %s repeat=3 nowait=1 burst=1 %s" % (cases["edge"], DELAYS)]
    res = run(driver, lines)
    for r in res:
        ok(r)
    zc = [r["counts"]["zero_copy"] for r in res]
    assert zc[:6] == [3, 0, 0, 4, 2, 2], zc
    assert zc[6] == 9, zc
    # two kernels per call read the one staging of its chunk
    assert [r["report"]["kernel_launches"] for r in res[7:]] == [2, 2], res[7:]
    assert zc[7:] == [6, 6], zc


def test_random_layout_plans_under_delays(driver, tmp_path):
    """Random layout plans from the fuzz set (seeds 200..420: pads,
    transposes with edge tiles, reshapes), each uploaded blocking from
    pageable and pinned sources, in no_wait calls back to back and in small
    chunks, evicted device-to-host and relaid on the device, under jittered
    delays: the oracle's results and no unordered access."""
    lines = []
    for seed in range(200, 420):
        r = F.make_plan(seed)
        if r is None or r[0].typed:
            continue
        plan, src, _ = r
        try:
            want = O.execute_layout(O.bind(O.decode_plan(plan.blob), {}), src.tobytes())
        except (O.BindError, O.ExecutionError):
            continue
        d = write_case(str(tmp_path), "f%d" % seed, plan.blob, src, want)
        dl = "delay_copy=200 delay_kernel=200 jitter=1 seed=%d" % seed
        lines += ["h2d %s repeat=2 %s" % (d, dl), "h2d %s repeat=2 pinned=1 %s" % (d, dl),
                  "h2d %s repeat=3 nowait=1 burst=1 %s" % (d, dl),
                  "h2d %s repeat=2 chunk=4096 nbuf=2 %s" % (d, dl),
                  "d2h %s repeat=2 %s" % (d, dl), "device %s %s" % (d, dl)]
    assert len(lines) >= 60, len(lines)
    for r in run(driver, lines, timeout=600):
        ok(r)


def test_checker_reports_a_missing_wait(driver, cases):
    """The device source is written on the caller's stream, but the call is
    told of no producer stream: the relayout reads it unordered."""
    res = run(driver, ["d2h %s caller=stream_untold %s" % (cases["c1"], DELAYS)])[0]
    assert any("relayout kernel" in v and "unordered" in v for v in res["violations"]), res


# --------------------------------------------------------------- faults

def fault(driver, case, knob, extra=""):
    return run(driver, ["h2d %s chunk=32768 nbuf=2 repeat=2 %s %s" % (case, knob, extra)])[0]


def test_faults_when_submitted(driver, cases):
    """A call refused when submitted fails with backend_failure; the
    context drains (completion known), stays usable, and closes."""
    for knob in ("fail_copy_at=3", "fail_launch_at=2", "fail_record_at=4", "fail_wait_at=2"):
        r = fault(driver, cases["c1"], knob, DELAYS)
        first = r["calls"][0]
        assert first["rc"] == 1 and first["code"] == "backend_failure", (knob, r)
        assert first["completion"] == 1, (knob, first)  # drained: complete
        assert not r["quarantined"] and r["close"]["rc"] == 0, (knob, r)
        assert not r["violations"], (knob, r["violations"][:3])
        # the next call on the same context succeeds and is right
        assert r["calls"][1]["rc"] == 0 and r["checked"] == 1 and r["mismatches"] == 0, (knob, r)


def test_allocation_failures(driver, cases):
    # the wire arena (first device allocation of the call) cannot be made
    r = fault(driver, cases["c1"], "fail_malloc_at=1")
    assert r["calls"][0]["code"] == "backend_failure" and "OutOfMemory" in r["calls"][0]["message"]
    assert r["calls"][0]["completion"] == 1 and not r["quarantined"] and r["close"]["rc"] == 0
    # the pinned ring cannot be made (pageable source)
    r = fault(driver, cases["c1"], "fail_host_malloc_at=1")
    assert r["calls"][0]["code"] == "backend_failure" and "OutOfMemory" in r["calls"][0]["message"]
    assert not r["quarantined"]
    # the context itself cannot be made
    r = run(driver, ["h2d %s fail_host_malloc_at=1 knobs_first=1" % cases["c1"]])[0]
    assert r["create"]["rc"] == 1 and r["create"]["code"] == "backend_failure"


def test_faults_on_the_stream_quarantine(driver, cases):
    """A copy or kernel that faults on its stream leaves a sticky device
    error: the call fails, the drain cannot prove completion, the context
    is quarantined and refuses later calls; closing reports the unknown
    completion."""
    for knob in ("fail_copy_async_at=2", "fail_kernel_async_at=1"):
        r = fault(driver, cases["c1"], knob, DELAYS)
        first = r["calls"][0]
        assert first["rc"] == 1 and first["code"] == "completion_unknown", (knob, r)
        assert "backend_failure" in first["message"] and "quarantined" in first["message"]
        assert first["completion"] == 2, (knob, first)  # unknown
        assert r["quarantined"] == 1
        assert r["close"]["rc"] == 1 and r["close"]["code"] == "completion_unknown"


def test_unknown_completion_quarantines(driver, cases):
    """Every synchronize fails (the reference's quiesce returning Unknown):
    the call fails with an unknown completion, the context is quarantined,
    and close keeps its memory."""
    r = fault(driver, cases["c1"], "sync_unknown=1", DELAYS)
    first = r["calls"][0]
    assert first["code"] == "completion_unknown" and first["completion"] == 2
    assert r["quarantined"] == 1 and r["close"]["code"] == "completion_unknown"
    assert not [v for v in r["violations"] if "hipFree" in v or "hipHostFree" in v]


def test_a_failed_synchronize_once(driver, cases):
    """One synchronize fails, the rest work: the call reports the failure,
    the drain succeeds, the context stays usable and closes cleanly."""
    r = fault(driver, cases["c1"], "fail_sync_at=1", DELAYS)
    first = r["calls"][0]
    assert first["rc"] == 1 and first["code"] == "backend_failure"
    assert first["completion"] == 1 and not r["quarantined"]
    assert r["close"]["rc"] == 0


def test_submitted_group_failures(driver, cases):
    """A submitted group the device fails: the completion's query or wait
    reports it; a sticky fault cannot be drained (completion_unknown, the
    context quarantined), a failed wait on a healthy device can
    (backend_failure, complete); the outcome is kept."""
    line = "submit %s members=2 chunk=32768 pinned=1 %s"
    r = run(driver, [line % (cases["c1"], "fail_kernel_async_at=1 " + DELAYS)])[0]
    codes = [cl["code"] for cl in r["calls"] if cl["rc"]]
    assert codes and codes[-1] == "completion_unknown", r["calls"]
    assert [cl for cl in r["calls"] if cl["rc"]][-1]["completion"] == 2
    assert r["quarantined"] == 1 and r["close"]["code"] == "completion_unknown"
    r = run(driver, [line % (cases["c1"], "fail_sync_at=1")])[0]
    bad = [cl for cl in r["calls"] if cl["rc"]]
    assert [cl["code"] for cl in bad] == ["backend_failure"], r["calls"]
    assert bad[0]["completion"] == 1 and "hipEventSynchronize" in bad[0]["message"]
    assert not r["quarantined"] and r["close"]["rc"] == 0


def test_device_to_host_failures(driver, cases):
    line = "d2h %s chunk=16384 nbuf=2 pinned=%d repeat=2 %s"
    # refused launch: drained, the next call works
    r = run(driver, [line % (cases["c1"], 0, "fail_launch_at=1 " + DELAYS)])[0]
    assert r["calls"][0]["code"] == "backend_failure" and r["calls"][0]["completion"] == 1
    assert r["calls"][1]["rc"] == 0 and r["checked"] == 1 and r["mismatches"] == 0
    assert not r["quarantined"] and r["close"]["rc"] == 0 and not r["violations"]
    # a copy that faults on its stream: quarantined
    r = run(driver, [line % (cases["c1"], 1, "fail_copy_async_at=3 " + DELAYS)])[0]
    assert r["calls"][0]["code"] == "completion_unknown" and r["calls"][0]["completion"] == 2
    assert r["quarantined"] == 1 and len(r["calls"]) == 1
    assert r["close"]["code"] == "completion_unknown"


def test_device_resident_and_static_failures(driver, cases):
    # a refused relayout launch is reported; the context stays usable
    r = run(driver, ["device %s caller=stream repeat=2 fail_launch_at=1 %s" % (cases["c1"], DELAYS)])[0]
    assert r["calls"][0]["code"] == "backend_failure"
    assert all(cl["rc"] == 0 for cl in r["calls"][1:]) and r["checked"] == 1
    assert not r["violations"] and r["close"]["rc"] == 0
    # the allocation-free upload: a refused copy drains; a faulting one quarantines
    r = run(driver, ["static %s repeat=2 fail_copy_at=1 %s" % (cases["c1"], DELAYS)])[0]
    assert r["calls"][0]["code"] == "backend_failure" and r["calls"][0]["completion"] == 1
    assert r["calls"][1]["rc"] == 0 and r["checked"] == 1 and r["mismatches"] == 0
    r = run(driver, ["static %s repeat=2 fail_copy_async_at=1 %s" % (cases["c1"], DELAYS)])[0]
    assert r["calls"][0]["code"] == "completion_unknown" and r["calls"][0]["completion"] == 2
    assert r["quarantined"] == 1 and r["close"]["code"] == "completion_unknown"


def test_quarantined_context_refuses_calls(driver, cases):
    """After a quarantine every call is refused with resources_closed."""
    r = run(driver, ["h2d %s chunk=32768 repeat=3 persist=1 fail_copy_async_at=1 %s"
                     % (cases["c1"], DELAYS)])[0]
    assert r["quarantined"] == 1 and len(r["calls"]) == 3
    assert [cl["code"] for cl in r["calls"]] == ["completion_unknown"] + ["resources_closed"] * 2
    assert [cl["completion"] for cl in r["calls"]] == [2, 0, 0]
    r = run(driver, ["group %s members=2 chunk=32768 fail_kernel_async_at=1 %s" % (cases["c1"], DELAYS)])[0]
    assert r["calls"][0]["code"] == "completion_unknown" and r["calls"][0]["completion"] == 2
    assert r["quarantined"] == 1


@pytest.mark.parametrize("shared", [1, 0])
def test_threads_upload_at_once(driver, cases, shared):
    """Host threads upload at once through one context (the library
    serializes its calls) or one context each, all sharing the bound
    plans and their device caches; results right, nothing unordered, no
    data race."""
    lines = ["threads %s threads_n=4 shared=%d repeat=3 chunk=%d nbuf=2 threads=2 %s"
             % (cases[n], shared, ch, DELAYS) for n, ch in (("c1", 32768), ("fz2", 16384), ("c2", 8192))]
    for r in run(driver, lines):
        ok(r)
        assert r["checked"] == 12 and len(r["calls"]) == 12
