#!/usr/bin/env python3
"""Benchmark of the libreloc plan-execution hot path on one MI355X.

Headline: the metric of BASELINE.json (effective GB/s of output, fused
relayout + H2D) on its largest single-GPU configuration, C5 at B=64,
S=4096: f16 [64,4096,32,128] in host memory -> permute to [B,32,S,128] ->
f32 -> int8 quantize (per-head scale) in HBM; 2 GiB cross PCIe, 1 GiB is
written.

* A step is one blocking call of the reference-shaped dispatch API from a
  pageable host tensor: fresh output allocation, bind, prepare, execute and
  completion, as the reference times its typed H2D rows.
* `value`: output bytes x steps / wall time of the K steps.
* `pcie`: the same steps in wire bytes against the measured pinned H2D
  ceiling, plus the pinned-source (direct DMA) rate.
* `roofline`: the dominant kernel, the permute over one kernel batch of the
  upload (16 batch entries), run back to back on one stream over buffers
  spanning 2 GiB; algorithmic bytes per launch over its mean duration (two
  events bracketing the timed launches, over their count; the mean of an
  event pair per launch, which adds the events' own cost to each launch,
  is reported beside it), against 8 TB/s. `in_pipeline` times the same launches inside the timed
  steps. `traffic` comes from the committed rocprofv3 PMC summary
  (profiles/traffic.json; PMC counters need a profiler run of their own).
* `cpu_baseline`: the reference's own cpu_reference row (oracle/_ref: CPU
  transform into a 2-slot pinned ring, then H2D) on the same batch and host.

`--report` prints one JSON line per config (C1..C5, device-resident kernel
rates, and the indexed-plan gathers ix_*) instead.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


def log(*a):
    """Progress on stderr (the JSON line is the only stdout output)."""
    print("[bench]", *a, file=sys.stderr, flush=True)


METRIC ="effective GB/s (output bytes/s) fused relayout+H2D; % of PCIe and HBM roofline"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--e2e-samples", type=int, default=40)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-table", action="store_true",
                    help="skip the per-config table of the bench line")
    ap.add_argument("--table-samples", type=int, default=TABLE_SAMPLES,
                    help="timed calls per config and source in the per-config table")
    ap.add_argument("--report", action="store_true", help="one JSON line per config")
    ap.add_argument("--configs", default="c1,c2,c3,c4,c5")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="run a plain copy of known size, then each config's kernel (for rocprofv3 --pmc)")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="turn two rocprofv3 --pmc runs of --traffic-probe into profiles/traffic.json")
    ap.add_argument("--summarize-trace", metavar="TRACE_DIR",
                    help="per-call copy/kernel/staging timeline of a rocprofv3 marker + memory-copy "
                         "+ kernel trace of the headline (RELX_TRACE=1), or of a --trace-configs run "
                         "(its output line saved as TRACE_DIR/plan.json)")
    ap.add_argument("--summarize-stats", metavar="TRACE_DIR",
                    help="per-config kernel durations from a rocprofv3 --kernel-trace run of "
                         "--traffic-probe (its output line saved as TRACE_DIR/probe.json)")
    ap.add_argument("--summarize-line", metavar="BENCH_LINE_FILE",
                    help="markdown table of the per-config table (`configs`) of a saved bench line")
    ap.add_argument("--summarize-report", metavar="REPORT_FILE",
                    help="markdown tables (profiles/configs_report.md) from the saved output of "
                         "--report")
    ap.add_argument("--trace-configs", metavar="CONFIGS",
                    help="end-to-end uploads of these configs only, pageable then pinned (8 warm-up "
                         "calls and 6 timed calls each), for a rocprofv3 trace; prints the call plan")
    return ap.parse_args()


# ------------------------------------------------------------------ setup

def torch_mod():
    import torch
    if not torch.cuda.is_available():
        sys.exit("bench.py needs a GPU (torch.cuda.is_available() is False)")
    return torch


class Case:
    """One workload: a bound plan plus host inputs for it."""

    def __init__(self, name, workload, blob, symbols, params, src, extra=None, widths=(0, 0)):
        from sym_amd import pyreloc as P
        self.name, self.workload = name, workload
        self.plan = P.Plan(blob)
        self.bound = P.Bound(self.plan, symbols, params if self.plan.typed else None)
        self.blob, self.symbols, self.params = blob, symbols, params
        self.src = np.ascontiguousarray(src)
        self.extra = extra or {}
        b = self.bound
        self.out_bytes = b.destination_bytes if self.plan.typed else b.total_bytes
        self.wire_bytes = self.src.nbytes  # boundary-0 wire (device programs start there)
        self.kernel = b.kernel
        self.win, self.wout = widths  # element bytes of the wire and the result


def make_case(name):
    from sym_amd import workloads as W
    if name == "c4":
        pool = W.c4_pool(experts=1)
        q, sc = pool[0][0]
        return Case(name, "C4 MoE expert matrix int8 gate [14336,4096] -> per-row dequant -> f16",
                    W.c4_plan().blob, {"s0": q.shape[0], "s1": q.shape[1]}, W.param("scale", sc), q,
                    widths=(1, 2))
    if name == "c1":
        n = 16777216
        return Case(name, "C1 README plan f32[N=16777216] -> [N/64,64] -> transpose [64,N/64]",
                    W.c1_plan().blob, {"s0": n}, None, W.c1_input(n), widths=(4, 4))
    if name == "c2":
        return Case(name, "C2 image batch f32 NCHW [32,3,224,224] -> pad C 3->4 -> NHWC -> f16",
                    W.c2_plan().blob, {}, {}, W.c2_input(), widths=(4, 2))
    if name == "c3":
        q, s = W.c3_input()
        return Case(name, "C3 int8 weight [4096,11008] -> dequant(scale[11008]) -> f16 -> [11008,4096]",
                    W.c3_plan().blob, {"s0": 4096, "s1": 11008}, W.param("scale", s), q,
                    widths=(1, 2))
    if name.startswith("c5"):
        b, s = (64, 4096) if name == "c5" else tuple(int(v) for v in name[3:].split("x"))
        x, sc = W.c5_input(b, s)
        return Case(name, "C5 f16 [%d,%d,32,128] -> [B,32,S,128] -> f32 -> int8 (per-head scale)"
                    % (b, s), W.c5_plan().blob, {"B": b, "S": s}, W.param("scale", sc), x,
                    {"B": b, "S": s}, widths=(2, 1))
    raise ValueError(name)


# ------------------------------------------------------ indexed plans

# index_select (axis 0) + cast workloads: table shape, source dtype, result
# dtype, selected rows (random, with repeats).
IX = {"ix_f32f16": ((1 << 20, 1024), "float32", "float16", 65536),
      "ix_f16f32": ((1 << 20, 1024), "float16", "float32", 65536),
      "ix_i8": ((1 << 20, 4096), "int8", "int8", 65536),
      "ix_row5": ((1 << 23, 5), "float32", "float16", 1 << 22)}
IX_SETS = 8  # index sets rotated per step
_W = {"float32": 4, "float16": 2, "int8": 1}
_NP = {"float32": np.float32, "float16": np.float16, "int8": np.int8}
SEED = 20260710


def ix_bound(P, name, rows=None, seed=SEED):
    from sym_amd.encoder import encode_index_select
    shape, sd, rd, count = IX[name]
    shape = ((rows,) + shape[1:]) if rows else shape
    idx = np.random.default_rng(seed).integers(0, shape[0], count).astype("<i8")
    b = P.bind_indexed(P.load_indexed_plan(encode_index_select(list(shape), sd, count, "int64", rd)),
                       {}, ("int64", [count], idx.tobytes()))
    return b, shape, sd, rd, idx


def ix_kernel(name):
    """The gather kernel instance a config launches (GatherOp, source bytes
    per item) for 256-byte aligned buffers, as the library selects it."""
    shape, sd, rd, _ = IX[name]
    row = int(np.prod(shape[1:]))
    if sd == rd:
        nb = 16
        while nb > 1 and (row * _W[sd]) % nb:
            nb //= 2
        return 0, nb
    v = 4
    while v > 1 and row % v:
        v //= 2
    return (1 if sd == "float32" else 2), v * _W[sd]


def ix_alg_bytes(b, sd, rd, count):
    """Algorithmic HBM bytes of one gather: selected rows read, 4-byte
    device indices read, result written."""
    return count * b.row_elements * (_W[sd] + _W[rd]) + 4 * count


def gather_rate(torch, ctx, bounds, table, out_bytes, steps, warmup):
    """K back-to-back device gathers into rotating outputs, each step with
    the next of `bounds` (index sets drawn with different seeds, so that the
    rows one step reads are not still in the 256 MB Infinity Cache from the
    step before); returns (ms per step over the bracketed region, mean
    per-launch ms)."""
    sets = max(2, min(8, int(np.ceil(600e6 / out_bytes))))
    outs = [torch.empty(out_bytes, dtype=torch.uint8, device="cuda") for _ in range(sets)]
    stream = torch.cuda.Stream()
    sp = stream.cuda_stream
    tb = table.numel() * table.element_size()

    def run(i):
        ctx.index_select_device(bounds[i % len(bounds)], table.data_ptr(), tb,
                                outs[i % sets].data_ptr(), out_bytes, stream=sp)
    for i in range(warmup):
        run(i)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for i in range(steps):
        run(i)
    t1.record(stream)
    torch.cuda.synchronize()
    ms_step = t0.elapsed_time(t1) / steps
    n = min(steps, 200)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for i in range(n):
        ev[i][0].record(stream)
        run(i)
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    kms = float(np.mean([a.elapsed_time(b) for a, b in ev]))
    del outs
    return ms_step, kms


def device_table(torch, shape, sd):
    g = torch.Generator(device="cuda")
    g.manual_seed(SEED)
    if sd == "int8":
        return torch.randint(-128, 128, shape, dtype=torch.int8, device="cuda", generator=g)
    return torch.randn(shape, dtype=getattr(torch, sd), device="cuda", generator=g)


def ix_config(torch, ctx, P, name, args, h2d_ceiling):
    """Device gather from an HBM-resident table (relx_index_select_device),
    then the host-table upload (host gather into the pinned ring + device
    cast), pageable and pinned, and the reference CPU executor on the same
    host table."""
    b, shape, sd, rd, idx = ix_bound(P, name)
    count = len(idx)
    table = device_table(torch, shape, sd)
    out_bytes = b.destination_bytes
    bounds = [b] + [ix_bound(P, name, seed=SEED + s)[0] for s in range(1, IX_SETS)]
    ms_step, kms = gather_rate(torch, ctx, bounds, table, out_bytes, max(50, args.steps // 20), 10)
    alg = ix_alg_bytes(b, sd, rd, count)
    del table
    res = {"config": name, "workload": "index_select %s %s -> %d rows -> %s" % (sd, list(shape), count, rd),
           "kernel": "gather<%d, %d>" % ix_kernel(name),
           "device": {"ms_per_step": round(ms_step, 5), "kernel_ms_per_launch_events": round(kms, 5),
                      "output_GBps": round(out_bytes / ms_step / 1e6, 1),
                      "algorithmic_bytes": alg, "achieved_GBps": round(alg / ms_step / 1e6, 1),
                      "hbm_frac": round(alg / ms_step / 1e6 / HBM_PEAK_GBS, 4),
                      "traffic": traffic_for(name, alg)}}
    # upload from a host table a quarter the size (same selected rows)
    rows = max(shape[0] // 4, 1)
    hb, hshape, _, _, hidx = ix_bound(P, name, rows=rows)
    rng = np.random.default_rng(SEED)
    host = (rng.standard_normal(hshape, dtype=np.float32).astype(_NP[sd]) if sd != "int8"
            else rng.integers(-128, 128, hshape, dtype=np.int8))
    out = torch.empty(out_bytes, dtype=torch.uint8, device="cuda")
    for pinned in (False, True):
        src = torch.from_numpy(host.view(np.uint8).reshape(-1)).pin_memory() if pinned else None
        ptr, nb = (src.data_ptr(), src.numel()) if pinned else (host.ctypes.data, host.nbytes)
        for _ in range(3):
            rep = ctx.execute_h2d(hb, ptr, nb, out.data_ptr(), out_bytes)
        ts = []
        for _ in range(max(10, args.e2e_samples // 4)):
            t = time.perf_counter()
            rep = ctx.execute_h2d(hb, ptr, nb, out.data_ptr(), out_bytes)
            ts.append(time.perf_counter() - t)
        p50 = float(np.percentile(ts, 50))
        res["e2e_pinned" if pinned else "e2e_pageable"] = {
            "table_bytes": host.nbytes, "p50_ms": round(p50 * 1e3, 3),
            "effective_GBps": round(out_bytes / p50 / 1e9, 2), "wire_bytes": rep["wire_bytes"],
            "pcie_frac": round(rep["wire_bytes"] / p50 / 1e9 / h2d_ceiling, 4),
            "implementation": rep["implementation"], "chunks": rep["chunks"]}
        del src
    from oracle import ref
    if ref.available() and not args.no_cpu:
        from sym_amd.encoder import encode_index_select
        blob = encode_index_select(list(hshape), sd, count, "int64", rd)
        r = ref.IndexedRef(blob, {}, "int64", [count], hidx.tobytes(), threads=8)
        o = np.empty(out_bytes, np.uint8)
        r.execute(host, o)
        n, t0 = 0, time.perf_counter()
        while True:
            r.execute(host, o)
            n += 1
            el = time.perf_counter() - t0
            if el >= min(args.cpu_seconds, 5.0) and n >= 3:
                break
        res["cpu_baseline"] = {"value": round(out_bytes * n / el / 1e9, 3), "unit": "GB/s",
                               "cores": 8, "kind": "reference",
                               "sample": "%d x typed::executeHost (indexed rows) over the host table" % n}
    return res


# ----------------------------------------------------------- measurements

# Bytes the rotating buffer sets of a device-rate measurement span: eight
# times the MI355X's 256 MB Infinity Cache (MALL). With fewer, a launch
# rewrites result lines still held there from the previous pass, which never
# reach HBM -- cached stores then look faster than they are (C5 8x4096 over
# two sets: 65.9 us cached, 72.8 us streaming; over eight: 75.2 and 73.4).
ROTATE_BYTES = 2 << 30
# the library's kernel-batch rule (kKernelBatchBytes, runtime.h): a launch
# takes whole chunks up to this much wire, at most a quarter of the call's
KERNEL_BATCH_BYTES = 512 << 20


def batch_units(B, S):
    """Batch entries per full kernel batch of the C5 [B, S] upload in
    chunks of one entry (S*4096 f16 elements)."""
    return max(1, min(KERNEL_BATCH_BYTES // (S * 4096 * 2), B // 4))


def device_rate(torch, ctx, bound, wire_bytes, out_bytes, steps, warmup, sets=None):
    """K back-to-back device relayouts over rotating buffer sets spanning
    ROTATE_BYTES, at least one pass over every set in each timed region.
    Returns (ms_per_step over the bracketed region, mean per-launch kernel
    ms)."""
    per = wire_bytes + out_bytes
    sets = sets or max(2, -(-ROTATE_BYTES // per))
    steps = max(steps, sets)
    wires = [torch.empty(wire_bytes, dtype=torch.uint8, device="cuda") for _ in range(sets)]
    outs = [torch.empty(out_bytes, dtype=torch.uint8, device="cuda") for _ in range(sets)]
    for w in wires:
        w.random_(0, 256)
    # a dedicated (non-null) stream: the kernels and the events must share it
    stream = torch.cuda.Stream()
    sp = stream.cuda_stream
    assert sp != 0
    for i in range(warmup):
        ctx.relayout_device(bound, wires[i % sets].data_ptr(), outs[i % sets].data_ptr(), stream=sp)
    torch.cuda.synchronize()
    # and at least 30 ms of back-to-back launches: after idle stretches (the
    # latency-bound end-to-end calls before it) the clocks take a few ms to
    # come back, which a short timed region would see
    t_warm = time.perf_counter()
    while time.perf_counter() - t_warm < 0.03:
        for i in range(50):
            ctx.relayout_device(bound, wires[i % sets].data_ptr(), outs[i % sets].data_ptr(), stream=sp)
        torch.cuda.synchronize()
    # whole-job: K steps bracketed by synchronize
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record(stream)
    for i in range(steps):
        ctx.relayout_device(bound, wires[i % sets].data_ptr(), outs[i % sets].data_ptr(), stream=sp)
    t1.record(stream)
    torch.cuda.synchronize()
    ms_step = t0.elapsed_time(t1) / steps
    # per-launch durations on the launch stream
    n = min(steps, max(400, sets))
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for i in range(n):
        ev[i][0].record(stream)
        ctx.relayout_device(bound, wires[i % sets].data_ptr(), outs[i % sets].data_ptr(), stream=sp)
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    kms = float(np.mean([a.elapsed_time(b) for a, b in ev]))
    torch.cuda.synchronize()
    del wires, outs
    return ms_step, kms


def e2e_rate(torch, ctx, case, samples, pinned, host_stages=-1):
    out = torch.empty(case.out_bytes, dtype=torch.uint8, device="cuda")
    if pinned:
        src_t = torch.from_numpy(case.src.view(np.uint8).reshape(-1)).pin_memory()
        ptr, nb = src_t.data_ptr(), src_t.numel()
    else:
        ptr, nb = case.src.ctypes.data, case.src.nbytes
    for _ in range(8):  # reference protocol: 8 warmups, then samples
        rep = ctx.execute_h2d(case.bound, ptr, nb, out.data_ptr(), case.out_bytes,
                              host_stages=host_stages, source_pinned=1 if pinned else 0)
    ts = []
    for _ in range(samples):
        t = time.perf_counter()
        rep = ctx.execute_h2d(case.bound, ptr, nb, out.data_ptr(), case.out_bytes,
                              host_stages=host_stages, source_pinned=1 if pinned else 0)
        ts.append(time.perf_counter() - t)
    p50, p95 = float(np.percentile(ts, 50)), float(np.percentile(ts, 95))
    return p50, p95, rep


def first_call_ms(torch, P, case):
    """A cold call: new context, bind, first upload (ring, wire arena and
    parameter upload allocated on the way), completion; pageable source."""
    out = torch.empty(case.out_bytes, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    t = time.perf_counter()
    ctx = P.Context(0)
    b = P.Bound(case.plan, case.symbols, case.params if case.plan.typed else None)
    ctx.execute_h2d(b, case.src.ctypes.data, case.src.nbytes, out.data_ptr(), case.out_bytes)
    ms = (time.perf_counter() - t) * 1e3
    ctx.close()
    return round(ms, 3)


def host_info():
    """The host's CPU as /proc/cpuinfo and sysfs describe it: the model
    string in full (with family/model/stepping, since a virtual machine may
    report only "AMD EPYC"), and how the affinity mask's CPUs map onto
    physical cores (SMT siblings share a core's load/store units and its
    memory bandwidth)."""
    info, first = {}, True
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if not line.strip():
                    first = False
                if first and ":" in line:
                    k, v = (s.strip() for s in line.split(":", 1))
                    if k in ("model name", "cpu family", "model", "stepping", "cpu MHz",
                             "cache size", "siblings", "cpu cores"):
                        info[k] = v
    except OSError:
        pass
    cpus = sorted(os.sched_getaffinity(0))
    cores = set()
    for c in cpus:
        try:
            base = "/sys/devices/system/cpu/cpu%d/topology/" % c
            with open(base + "physical_package_id") as f:
                pkg = f.read().strip()
            with open(base + "core_id") as f:
                cores.add((pkg, f.read().strip()))
        except OSError:
            cores.add(("?", str(c)))
    mem = None
    try:
        with open("/proc/meminfo") as f:
            mem = int(f.readline().split()[1]) * 1024
    except (OSError, ValueError, IndexError):
        pass
    return {"cpu_model": info.get("model name", ""),
            "cpu_id": "family %s model %s stepping %s" % (info.get("cpu family", "?"),
                                                          info.get("model", "?"),
                                                          info.get("stepping", "?")),
            "cpu_mhz": info.get("cpu MHz"), "cache": info.get("cache size"),
            "nproc": os.cpu_count(), "affinity_cpus": len(cpus),
            "affinity_physical_cores": len(cores), "host_memory_bytes": mem}


def hbm_copy_ceiling(torch, nbytes=1 << 30, iters=20):
    a = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    a.random_(0, 256)
    for _ in range(3):
        b.copy_(a)
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(iters):
        b.copy_(a)
    e.record()
    torch.cuda.synchronize()
    return 2 * nbytes * iters / (s.elapsed_time(e) * 1e-3) / 1e9


def cpu_baseline(case, seconds, threads):
    """The reference libreloc CPU executor (oracle/_ref) timed on this host:
    repeated typed::executeHost / executeH2DThreaded over the config."""
    from oracle import ref
    if not ref.available():
        return None
    if case.plan.typed:
        r = ref.TypedRef(case.blob, case.symbols, case.params, threads=threads)
    else:
        r = ref.LayoutRef(case.blob, case.symbols, threads=threads)
    out = np.empty(case.out_bytes, np.uint8)
    r.execute(case.src, out)
    n, t0 = 0, time.perf_counter()
    while True:
        r.execute(case.src, out)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds and n >= 3:
            break
    return {"value": round(case.out_bytes * n / el / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "reference",
            "sample": "%d x typed::executeHost of the full %s batch (%d output bytes each) in %.1f s"
                      % (n, case.name.upper(), case.out_bytes, el)}


def traffic_for(config, algorithmic_bytes=None):
    """HBM bytes per launch of the config's kernel from the committed PMC
    summary (profiles/traffic.json), or None; None too when the summary's
    launch moved other algorithmic bytes than the one measured now."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        entry = json.load(f).get("configs", {}).get(config)
    if entry is None or (algorithmic_bytes is not None and entry["algorithmic_bytes"] != algorithmic_bytes):
        return None
    return entry["traffic_bytes"]


# Calibration copy of the traffic probe: one device-to-device copy of this
# many bytes reads and writes exactly this many bytes of HBM.
CALIBRATION_BYTES = 256 << 20


# Launches per config in --traffic-probe: warm-up launches (not counted by
# the summaries), then timed ones, each config then a copy of its bytes.
PROBE_WARM, PROBE_LAUNCHES = 20, 100


def probe_bound(name):
    """A config's bound plan and its boundary-0 wire and result bytes, for a
    device-resident probe (no host input is generated)."""
    from sym_amd import pyreloc as P
    from sym_amd import workloads as W
    rng = np.random.default_rng(SEED)
    if name.startswith("c5_"):
        b, s = (int(v) for v in name[3:].split("x"))
        sc = rng.uniform(0.02, 0.05, 32).astype(np.float32)
        bound = P.Bound(P.Plan(W.c5_plan().blob), {"B": b, "S": s}, W.param("scale", sc))
        return bound, b * s * 4096 * 2, b * s * 4096, (2, 1)
    case = make_case(name)
    return case.bound, case.wire_bytes, case.out_bytes, (case.win, case.wout)


def probe_launches(torch, ctx, bound, wire_bytes, out_bytes, warm, n):
    """`warm` + `n` device relayouts back to back over rotating buffer sets
    spanning ROTATE_BYTES (every launch reads and writes HBM), `n` raised to
    one pass over the sets; returns the launches made."""
    per = wire_bytes + out_bytes
    sets = max(2, -(-ROTATE_BYTES // per))
    n = warm + max(n, sets)
    wires = [torch.empty(wire_bytes, dtype=torch.uint8, device="cuda") for _ in range(sets)]
    outs = [torch.empty(out_bytes, dtype=torch.uint8, device="cuda") for _ in range(sets)]
    for w in wires:
        w.random_(0, 256)
    stream = torch.cuda.Stream()
    for i in range(n):
        ctx.relayout_device(bound, wires[i % sets].data_ptr(), outs[i % sets].data_ptr(),
                            stream=stream.cuda_stream)
    torch.cuda.synchronize()
    del wires, outs
    return n


def traffic_probe(torch, ctx, names):
    """A plain copy of known size (the PMC calibration), then per config
    PROBE_WARM + PROBE_LAUNCHES launches of its kernel over rotating buffer
    sets and a 16-byte copy of the same algorithmic bytes; prints, in that
    order, which kernel each config launches and how many times, for the
    summaries of a rocprofv3 run of this probe (_assign)."""
    from sym_amd import pyreloc as P
    a = torch.empty(CALIBRATION_BYTES, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    a.random_(0, 256)
    for _ in range(5):
        b.copy_(a)
    torch.cuda.synchronize()
    del a, b
    kernels = {}
    for name in names:
        if name == "c5_e2e":
            # the headline steps: each kernel batch's k_permute launch inside
            # the upload (the summaries keep the full batches, the most
            # common grid)
            from sym_amd import workloads as W
            x, sc = W.c5_input(HEADLINE_B, HEADLINE_S)
            plan = P.load_typed_plan(W.c5_plan().blob)
            bound = P.bind_typed(plan, {"B": HEADLINE_B, "S": HEADLINE_S}, W.param("scale", sc))
            out = torch.empty(x.size, dtype=torch.int8, device="cuda")
            calls = 3
            for _ in range(calls):
                rep = ctx.execute_h2d(bound, x.ctypes.data, x.nbytes, out.data_ptr(), x.size)
            units = batch_units(HEADLINE_B, HEADLINE_S)
            kernels[name] = {"family": "permute", "win": 2, "wout": 1, "output_bytes": x.size,
                             "algorithmic_bytes": units * HEADLINE_S * 4096 * 3 + sc.nbytes,
                             "launches_per_call": rep["kernel_launches"],
                             "dispatches": calls * rep["kernel_launches"]}
            del out, x
            continue
        if name in IX:
            b, shape, sd, rd, idx = ix_bound(P, name)
            table = device_table(torch, shape, sd)
            bounds = [b] + [ix_bound(P, name, seed=SEED + s)[0] for s in range(1, IX_SETS)]
            gather_rate(torch, ctx, bounds, table, b.destination_bytes, 20, 2)
            del table
            op, nbi = ix_kernel(name)
            kernels[name] = {"family": "gather", "pattern": "k_gather<%d, %d," % (op, nbi),
                             "output_bytes": b.destination_bytes,
                             "algorithmic_bytes": ix_alg_bytes(b, sd, rd, len(idx)),
                             "dispatches": 2 + 20 + 20, "skip": 2}  # gather_rate's launches
            continue
        bound, wire, out_bytes, (win, wout) = probe_bound(name)
        launched = probe_launches(torch, ctx, bound, wire, out_bytes, PROBE_WARM, PROBE_LAUNCHES)
        alg = wire + out_bytes + bound.parameter_bytes
        copy_bytes = max(16, alg // 2 // 16 * 16)
        copy = P.measure_copy(0, copy_bytes, 20, 3)
        kernels[name] = {"family": bound.kernel, "wire_bytes": wire, "output_bytes": out_bytes,
                         "algorithmic_bytes": alg, "win": win, "wout": wout,
                         "dispatches": launched, "skip": PROBE_WARM,
                         "copy_bytes": copy_bytes, "copy_GBps_events": round(copy, 1)}
    print(json.dumps({"calibration_bytes": CALIBRATION_BYTES, "kernels": kernels}), flush=True)


def _pmc_rows(d, counter):
    """The rows of one counter (values in KiB per dispatch) from a rocprofv3
    --pmc CSV directory."""
    import csv
    import glob
    rows = []
    for path in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
        with open(path) as f:
            rows += [r for r in csv.DictReader(f) if r.get("Counter_Name") == counter]
    return rows


def _csv_rows(d, suffix):
    import csv
    import glob
    rows = []
    for path in glob.glob(os.path.join(d, "**", "*" + suffix), recursive=True):
        with open(path) as f:
            rows += list(csv.DictReader(f))
    return rows


def _union(intervals):
    """Total length of the union of (start, end) intervals."""
    total, cur_s, cur_e = 0, None, None
    for s, e in sorted(intervals):
        if cur_e is None or s > cur_e:
            if cur_e is not None:
                total += cur_e - cur_s
            cur_s, cur_e = s, e
        else:
            cur_e = max(cur_e, e)
    return total + (cur_e - cur_s if cur_e is not None else 0)


TRACE_WARMUP, TRACE_SAMPLES = 8, 6


def trace_configs(torch, ctx, names, h2d_ceiling):
    """The end-to-end calls a --trace-configs trace covers, in call order."""
    entries = []
    for name in names:
        case = make_case(name)
        for pinned in (False, True):
            _, _, rep = e2e_rate(torch, ctx, case, TRACE_SAMPLES, pinned=pinned)
            entries.append({"config": name, "source": "pinned" if pinned else "pageable",
                            "warmup": TRACE_WARMUP, "samples": TRACE_SAMPLES,
                            "wire_bytes": rep["wire_bytes"], "chunks": rep["chunks"],
                            "implementation": rep["implementation"]})
    return {"pinned_h2d_ceiling_GBps": round(h2d_ceiling, 2), "entries": entries}


def _median(v):
    v = sorted(v)
    return v[len(v) // 2] if v else float("nan")


def summarize_calls(d, plan):
    """Where each end-to-end call's time goes, from the library's
    `relx.h2d.call` ranges (host entry to return) of a --trace-configs run:
    per config and source, medians over the timed calls of the wall time,
    its ideal at the PCIe ceiling (wire bytes / pinned ceiling), the time
    before the first copy starts (staging of the first chunk, call set-up),
    the DMA engines' busy time and the gaps between copies, and the tail
    after the last copy lands (last kernels and the host's wake-up)."""
    marks = _csv_rows(d, "marker_api_trace.csv")
    calls = sorted((int(r["Start_Timestamp"]), int(r["End_Timestamp"]))
                   for r in marks if r["Function"].startswith("relx.h2d.call"))
    copies = sorted((int(r["Start_Timestamp"]), int(r["End_Timestamp"]))
                    for r in _csv_rows(d, "memory_copy_trace.csv")
                    if r["Direction"] == "MEMORY_COPY_HOST_TO_DEVICE")
    kernels = [(int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"])
               for r in _csv_rows(d, "kernel_trace.csv") if "relx::" in r["Kernel_Name"]]
    stage = [(int(r["Start_Timestamp"]), int(r["End_Timestamp"]))
             for r in marks if r["Function"].startswith("relx.h2d.stage")]
    ceiling = plan["pinned_h2d_ceiling_GBps"]
    lines = ["| config | source | chunks | wall us | ideal us | PCIe frac | before first copy us | "
             "DMA busy us | gaps between copies us | tail after last copy us | host staging us | kernels |",
             "|---|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|"]
    i = 0
    for e in plan["entries"]:
        rows = []
        for j in range(e["warmup"] + e["samples"]):
            if i >= len(calls):
                break
            t0, t1 = calls[i]
            i += 1
            if j < e["warmup"]:
                continue
            cs = [c for c in copies if t0 <= c[0] < t1]
            ks = [k for k in kernels if t0 <= k[0] < t1]
            if not cs:
                continue
            busy = _union(cs)
            first, last = min(c[0] for c in cs), max(c[1] for c in cs)
            rows.append({"wall": (t1 - t0) / 1e3, "before": (first - t0) / 1e3, "busy": busy / 1e3,
                         "gaps": (last - first - busy) / 1e3, "tail": (t1 - last) / 1e3,
                         "stage": sum(b - a for a, b in stage if t0 <= a < t1) / 1e3, "kernels": len(ks)})
        if not rows:
            continue
        m = {k: _median([r[k] for r in rows]) for k in rows[0]}
        ideal = e["wire_bytes"] / ceiling / 1e3
        lines.append("| %s | %s | %d | %.1f | %.1f | %.3f | %.1f | %.1f | %.1f | %.1f | %.1f | %d |" % (
            e["config"], e["source"], e["chunks"], m["wall"], ideal, ideal / m["wall"], m["before"],
            m["busy"], m["gaps"], m["tail"], m["stage"], m["kernels"]))
    print("\n".join(lines))


def summarize_trace(d):
    """Per-call timeline of the headline upload from a rocprofv3
    --kernel-trace --memory-copy-trace --marker-trace run with RELX_TRACE=1:
    host staging ranges, H2D copies and relayout kernels of each call, the
    share of the call the DMA engines were busy, and how much of each
    kernel ran under a copy. Prints a markdown table."""
    marks = _csv_rows(d, "marker_api_trace.csv")
    copies = [(int(r["Start_Timestamp"]), int(r["End_Timestamp"]))
              for r in _csv_rows(d, "memory_copy_trace.csv")
              if r["Direction"] == "MEMORY_COPY_HOST_TO_DEVICE"]
    kernels = [(int(r["Start_Timestamp"]), int(r["End_Timestamp"]))
               for r in _csv_rows(d, "kernel_trace.csv") if "k_permute" in r["Kernel_Name"]]
    # calls begin at chunk 0 of a staged ("stage") or direct ("submit") upload
    starts = sorted((int(r["Start_Timestamp"]), r["Function"].split()[0])
                    for r in marks if r["Function"].endswith(" chunk=0") and
                    r["Function"].split()[0] in ("relx.h2d.stage", "relx.h2d.submit"))
    stage = [(int(r["Start_Timestamp"]), int(r["End_Timestamp"]))
             for r in marks if r["Function"].startswith("relx.h2d.stage")]
    waits = [(int(r["Start_Timestamp"]), int(r["End_Timestamp"]))
             for r in marks if r["Function"].startswith("relx.h2d.slot_wait")]
    lines = ["| call | source | span ms | first copy after ms | copies | DMA busy | host staging ms | "
             "slot waits ms | kernels | kernel time under a copy | tail after last copy us |",
             "|---|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|"]
    for i, (t0, kind) in enumerate(starts):
        t1 = starts[i + 1][0] if i + 1 < len(starts) else float("inf")
        cs = [c for c in copies if t0 <= c[0] < t1]
        if not cs:
            continue
        # the call's kernels: those issued before its last copy landed, and
        # the batch that follows it (later launches belong to other work)
        last = max(c[1] for c in cs)
        ks = [k for k in kernels if t0 <= k[0] < min(t1, last + 1000000)]
        if not ks:
            continue
        end = max(k[1] for k in ks)
        span = end - t0
        busy = _union(cs)
        under = sum(_union([(max(k[0], c[0]), min(k[1], c[1])) for c in cs if c[0] < k[1] and c[1] > k[0]])
                    for k in ks)
        ktime = sum(k[1] - k[0] for k in ks)
        st = sum(e - s for s, e in stage if t0 <= s < end)
        wt = sum(e - s for s, e in waits if t0 <= s < end)
        lines.append("| %d | %s | %.3f | %.3f | %d | %.1f%% | %.2f | %.2f | %d | %.1f%% | %.1f |" % (
            i, "pageable (staged)" if kind == "relx.h2d.stage" else "pinned (direct DMA)",
            span / 1e6, (min(c[0] for c in cs) - t0) / 1e6, len(cs), 100.0 * busy / span,
            st / 1e6, wt / 1e6, len(ks), 100.0 * under / max(1, ktime),
            (end - max(c[1] for c in cs)) / 1e3))
    print("\n".join(lines))


def _kernel_pattern(info):
    """The kernel names a probed config launches: the gather instance it
    names, or its family at its element widths (the one-level interleave,
    k_interleave1p, the permute's eight-wave and direct forms and the
    transpose's byte-tile forms included)."""
    import re
    if info.get("pattern"):
        return re.compile(re.escape(info["pattern"]))
    return re.compile(r"k_%s(1p|8|_direct8?|_b8?)?<%d, %d" % (info["family"], info["win"], info["wout"]))


def _by_dispatch(rows):
    return sorted(rows, key=lambda r: int(r["Dispatch_Id"]))


def _assign(rows, probe):
    """Each probed config's dispatches, in the probe's order: rows (one per
    dispatch, in dispatch order) are walked once; a config takes the next
    `dispatches` rows whose kernel name matches it (the first `skip` of them
    are warm-up launches), then the run of k_copy16 dispatches of its
    same-bytes copy that follows. Configs that share one kernel instance
    (the C5 shapes) are told apart by this order."""
    cur, out = 0, {}
    for name, info in probe["kernels"].items():
        pat, n = _kernel_pattern(info), info.get("dispatches")
        taken, i = [], cur
        while i < len(rows) and (n is None or len(taken) < n):
            if pat.search(rows[i]["Kernel_Name"]):
                taken.append(rows[i])
            i += 1
        copies = []
        if info.get("copy_bytes"):
            while i < len(rows) and "k_copy16" not in rows[i]["Kernel_Name"]:
                i += 1
            while i < len(rows) and "k_copy16" in rows[i]["Kernel_Name"]:
                copies.append(rows[i])
                i += 1
        cur = i
        out[name] = (taken[info.get("skip", 0):], copies)
    return out


def _grid(r):
    return int(r.get("Grid_Size_X") or r.get("Grid_Size"))


def _mode_grid(rows):
    """The most common launch grid (threads) of the rows, and the rows of it."""
    if not rows:
        return 0, []
    grids = [_grid(r) for r in rows]
    g = max(set(grids), key=grids.count)
    return g, [r for r in rows if _grid(r) == g]


def summarize_stats(d, probe):
    """Per-config kernel durations from a rocprofv3 --kernel-trace run of
    --traffic-probe (its output line saved as d/probe.json): each config's
    timed dispatches (assigned in dispatch order, _assign) at their most
    common grid, their mean and median duration, the algorithmic bytes over
    the mean against 8 TB/s, and the 16-byte copy of the same bytes that the
    probe ran right after them (median duration, the same bytes over it, and
    the kernel's rate as a fraction of the copy's; of its two forms, one
    and two vectors per lane, the faster). Prints a markdown table."""
    rows = _by_dispatch(_csv_rows(d, "kernel_trace.csv"))
    us = lambda r: (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    lines = ["| config | kernel | grid (threads) | dispatches | mean us | median us | algorithmic "
             "bytes | achieved GB/s | of 8 TB/s | copy median us | copy GB/s | of copy |",
             "|---|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|"]
    for name, (krows, crows) in _assign(rows, probe).items():
        grid, krows = _mode_grid(krows)
        if not krows:
            continue
        info = probe["kernels"][name]
        kernel = krows[0]["Kernel_Name"].replace("void relx::(anonymous namespace)::", "")
        t = [us(r) for r in krows]
        mean, alg = float(np.mean(t)), info["algorithmic_bytes"]
        gbs = alg / mean / 1e3
        copy = "| | |"
        if crows:
            # the copy runs in two forms (one and two vectors per lane): the
            # faster form's median
            forms = {}
            for r in crows:
                forms.setdefault(r["Kernel_Name"], []).append(us(r))
            cm = min(float(np.median(v)) for v in forms.values())
            cgbs = alg / cm / 1e3
            copy = "%.2f | %.1f | %.3f |" % (cm, cgbs, gbs / cgbs)
        lines.append("| %s | `%s` | %d | %d | %.2f | %.2f | %d | %.1f | %.3f | %s" % (
            name, kernel.split("(")[0], grid, len(t), mean, float(np.median(t)), alg, gbs,
            gbs / HBM_PEAK_GBS, copy))
    print("\n".join(lines))


def summarize_pmc(fetch_dir, write_dir, probe):
    """Scale each kernel's FETCH_SIZE / WRITE_SIZE by what the counters read
    for the calibration copy and write profiles/traffic.json."""
    out = {"calibration_bytes": probe["calibration_bytes"], "configs": {}}
    med = {}
    for counter, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        rows = _by_dispatch(_pmc_rows(d, counter))
        cal = [float(r["Counter_Value"]) * 1024.0 for r in rows if "copyBuffer" in r["Kernel_Name"]
               and float(r["Counter_Value"]) * 1024.0 > probe["calibration_bytes"] / 4]
        if not cal:
            raise SystemExit("no calibration copy dispatches for %s in %s" % (counter, d))
        factor = probe["calibration_bytes"] / float(np.median(cal))
        out[counter + "_calibration_factor"] = round(factor, 4)
        for name, (krows, _) in _assign(rows, probe).items():
            grid, krows = _mode_grid(krows)
            if krows:
                vals = [float(r["Counter_Value"]) * 1024.0 for r in krows]
                med.setdefault(name, {})[counter] = float(np.median(vals)) * factor
                med[name]["kernel"] = krows[0]["Kernel_Name"]
                med[name]["dispatches"] = len(vals)
                med[name]["grid"] = grid
    for name, m in med.items():
        if "FETCH_SIZE" in m and "WRITE_SIZE" in m:
            alg = probe["kernels"][name]["algorithmic_bytes"]
            t = m["FETCH_SIZE"] + m["WRITE_SIZE"]
            out["configs"][name] = {"kernel": m["kernel"], "dispatches": m["dispatches"],
                                    "grid_threads": m["grid"],
                                    "fetch_factor": out["FETCH_SIZE_calibration_factor"],
                                    "write_factor": out["WRITE_SIZE_calibration_factor"],
                                    "fetch_bytes": round(m["FETCH_SIZE"]),
                                    "write_bytes": round(m["WRITE_SIZE"]),
                                    "traffic_bytes": round(t), "algorithmic_bytes": alg,
                                    "traffic_over_algorithmic": round(t / alg, 4)}
    return out


# --------------------------------------------------------------- report

def one_config(torch, ctx, P, name, args, h2d_ceiling):
    case = make_case(name)
    ms_step, kms = device_rate(torch, ctx, case.bound, case.wire_bytes, case.out_bytes,
                               max(50, args.steps // 10), 20)
    alg = case.wire_bytes + case.out_bytes + case.bound.parameter_bytes
    p50, p95, rep = e2e_rate(torch, ctx, case, max(10, args.e2e_samples // 2), pinned=False)
    q50, q95, prep = e2e_rate(torch, ctx, case, max(10, args.e2e_samples // 2), pinned=True)
    return {"config": name, "workload": case.workload, "kernel": case.kernel,
            "device": {"ms_per_step": round(ms_step, 5),
                       "output_GBps": round(case.out_bytes / ms_step / 1e6, 1),
                       "algorithmic_bytes": alg, "achieved_GBps": round(alg / ms_step / 1e6, 1),
                       "hbm_frac": round(alg / ms_step / 1e6 / HBM_PEAK_GBS, 4)},
            "e2e_pageable": {"p50_ms": round(p50 * 1e3, 3), "p95_ms": round(p95 * 1e3, 3),
                             "effective_GBps": round(case.out_bytes / p50 / 1e9, 2),
                             "wire_bytes": rep["wire_bytes"],
                             "pcie_frac": round(rep["wire_bytes"] / p50 / 1e9 / h2d_ceiling, 4),
                             "implementation": rep["implementation"], "chunks": rep["chunks"]},
            "e2e_pinned": {"p50_ms": round(q50 * 1e3, 3), "p95_ms": round(q95 * 1e3, 3),
                           "effective_GBps": round(case.out_bytes / q50 / 1e9, 2),
                           "wire_bytes": prep["wire_bytes"],
                           "pcie_frac": round(prep["wire_bytes"] / q50 / 1e9 / h2d_ceiling, 4),
                           "implementation": prep["implementation"], "chunks": prep["chunks"]}}


def d2h_config(torch, ctx, name, args, d2h_ceiling):
    """The device-to-host direction (KV eviction): the config's source is
    resident on the device, the result lands in host memory (pageable or
    pinned); wire bytes are the result's."""
    case = make_case(name)
    src = torch.from_numpy(case.src.view(np.uint8).reshape(-1)).cuda()
    out = {}
    for pinned in (False, True):
        dst = torch.empty(case.out_bytes, dtype=torch.uint8)
        if pinned:
            dst = dst.pin_memory()
        for _ in range(3):
            ctx.execute_d2h(case.bound, src.data_ptr(), src.numel(), dst.data_ptr(), case.out_bytes,
                            source_pinned=1 if pinned else 0)
        ts = []
        for _ in range(max(10, args.e2e_samples // 2)):
            t = time.perf_counter()
            rep = ctx.execute_d2h(case.bound, src.data_ptr(), src.numel(), dst.data_ptr(),
                                  case.out_bytes, source_pinned=1 if pinned else 0)
            ts.append(time.perf_counter() - t)
        p50 = float(np.percentile(ts, 50))
        out["pinned" if pinned else "pageable"] = {
            "p50_ms": round(p50 * 1e3, 3), "effective_GBps": round(case.out_bytes / p50 / 1e9, 2),
            "pcie_frac": round(case.out_bytes / p50 / 1e9 / d2h_ceiling, 4), "chunks": rep["chunks"]}
    del src
    return {"config": name + "_d2h", "workload": case.workload + " (device -> host)",
            "kernel": case.kernel, "pinned_d2h_ceiling_GBps": round(d2h_ceiling, 2), **out}


def c4_report(torch, ctx, P, args, h2d_ceiling):
    """C4: two experts (6 matrices) per step as one grouped transfer."""
    from sym_amd import workloads as W
    pool = W.c4_pool()
    steps = W.c4_steps(20)
    plan = P.Plan(W.c4_plan().blob)
    bounds = {}
    for e in range(8):
        for j, (q, s) in enumerate(pool[e]):
            bounds[(e, j)] = P.Bound(plan, {"s0": q.shape[0], "s1": q.shape[1]}, W.param("scale", s))
    # gate, up and down hold the same element count: one output buffer per slot
    dst = [torch.empty(bounds[(0, 0)].destination_bytes, dtype=torch.uint8, device="cuda")
           for _ in range(6)]

    def step(experts, pinned=None):
        bl, sl, dl = [], [], []
        k = 0
        for e in experts:
            for j in range(3):
                q, _ = pool[e][j]
                bl.append(bounds[(e, j)])
                sl.append((pinned[(e, j)].data_ptr(), q.nbytes) if pinned else (q.ctypes.data, q.nbytes))
                dl.append((dst[k].data_ptr(), dst[k].numel()))
                k += 1
        return ctx.execute_group_h2d(bl, sl, dl, source_pinned=1 if pinned else 0)

    def timed(pinned=None):
        for ex in steps[:3]:
            step(ex, pinned)
        ts = []
        for ex in steps:
            t = time.perf_counter()
            _, tot = step(ex, pinned)
            ts.append(time.perf_counter() - t)
        return float(np.percentile(ts, 50)), tot

    p50, total = timed()
    # the same steps from an expert pool in page-locked memory (direct DMA)
    pinned_pool = {key: torch.from_numpy(pool[key[0]][key[1]][0]).pin_memory() for key in bounds}
    p50_pinned, total_pinned = timed(pinned_pool)
    del pinned_pool
    # device-only: one matrix per launch over resident wires
    b = bounds[(0, 0)]
    q = pool[0][0][0]
    ms_step, kms = device_rate(torch, ctx, b, q.nbytes, b.destination_bytes, 200, 20)
    alg = q.nbytes + b.destination_bytes + b.parameter_bytes
    return {"config": "c4", "workload": "C4 MoE: 2 of 8 experts x {gate,up [14336,4096], down [4096,14336]} int8 -> per-row dequant -> f16",
            "kernel": b.kernel,
            "device": {"matrix": "gate [14336,4096]", "ms_per_step": round(ms_step, 5),
                       "output_GBps": round(b.destination_bytes / ms_step / 1e6, 1),
                       "achieved_GBps": round(alg / ms_step / 1e6, 1),
                       "hbm_frac": round(alg / ms_step / 1e6 / HBM_PEAK_GBS, 4)},
            "e2e_pageable": {"p50_ms": round(p50 * 1e3, 3),
                             "effective_GBps": round(total["destination_bytes"] / p50 / 1e9, 2),
                             "wire_bytes": total["wire_bytes"],
                             "pcie_frac": round(total["wire_bytes"] / p50 / 1e9 / h2d_ceiling, 4),
                             "steps": len(steps)},
            "e2e_pinned": {"p50_ms": round(p50_pinned * 1e3, 3),
                           "effective_GBps": round(total_pinned["destination_bytes"] / p50_pinned / 1e9, 2),
                           "wire_bytes": total_pinned["wire_bytes"],
                           "pcie_frac": round(total_pinned["wire_bytes"] / p50_pinned / 1e9 / h2d_ceiling, 4),
                           "steps": len(steps)}}


# ------------------------------------------------------- per-config table

# The reference's measurement protocol: 8 warm-up calls, then 100 samples,
# p50 and p95 (bench/results/typed-h2d-221/README.md:23-26).
TABLE_WARMUP, TABLE_SAMPLES = 8, 100


def _calls(fn, samples, warmup=TABLE_WARMUP):
    for _ in range(warmup):
        rep = fn()
    ts = []
    for _ in range(samples):
        t = time.perf_counter()
        rep = fn()
        ts.append(time.perf_counter() - t)
    return float(np.percentile(ts, 50)), float(np.percentile(ts, 95)), rep


def _e2e_row(p50, p95, rep, out_bytes, ceiling, samples):
    return {"p50_ms": round(p50 * 1e3, 4), "p95_ms": round(p95 * 1e3, 4),
            "effective_GBps": round(out_bytes / p50 / 1e9, 2), "wire_bytes": rep["wire_bytes"],
            "pcie_frac": round(rep["wire_bytes"] / p50 / 1e9 / ceiling, 4),
            "chunks": rep["chunks"], "implementation": rep["implementation"], "samples": samples}


def config_table(torch, P, args, h2d_ceiling, c5_headline):
    """BASELINE.json's five configs at full size, each measured in this run:

    * `e2e_pageable` / `e2e_pinned`: relx_execute_h2d of the config's bound
      plan from a pageable and from a page-locked copy of its source, with
      the library's automatic choices, 8 warm-up calls, then p50/p95 of
      `samples` calls; pcie_frac = wire bytes / p50 / the pinned H2D ceiling
      measured at the start of this run. C4 is the grouped step (2 of 8
      experts, 6 matrices) over 20 drawn steps, as the reference reports it;
      C1 adds its small-N latencies on the one plan.
    * `kernel`: the device relayout alone over resident buffers, launched
      back to back on one stream between two events (`us`), against 8 TB/s
      in algorithmic bytes (wire read + result written + parameters), and
      against a 16-byte vector copy of the same bytes run in the same
      process (`copy_GBps`, `of_copy`).

    A fresh context; every end-to-end leg runs before any kernel or copy
    leg, since large device frees can slow later pinned copies on streams
    created before them."""
    from sym_amd import workloads as W
    samples = args.table_samples
    ctx = P.Context(0)
    names = ["c1", "c2", "c3"] + ["c5_%dx%d" % bs for bs in W.C5_SHAPES]
    rows, kernels = {}, []
    for name in names:
        log("table: %s end to end" % name)
        if name == "c5_%dx%d" % (HEADLINE_B, HEADLINE_S):
            x, sc = c5_headline
            case = Case(name, "C5 f16 [64,4096,32,128] -> [B,32,S,128] -> f32 -> int8 (per-head scale)",
                        W.c5_plan().blob, {"B": HEADLINE_B, "S": HEADLINE_S}, W.param("scale", sc), x,
                        widths=(2, 1))
        else:
            case = make_case(name)
        big = case.wire_bytes >= (1 << 30)
        n = max(10, samples // 4) if big else samples  # 2 GiB calls: 25 samples (40 ms each)
        row = {"workload": case.workload, "kernel": case.kernel}
        out = torch.empty(case.out_bytes, dtype=torch.uint8, device="cuda")
        for pinned in (False, True):
            if pinned:
                held = torch.from_numpy(case.src.view(np.uint8).reshape(-1)).pin_memory()
                ptr, nb = held.data_ptr(), held.numel()
            else:
                held, ptr, nb = None, case.src.ctypes.data, case.src.nbytes
            p50, p95, rep = _calls(lambda: ctx.execute_h2d(case.bound, ptr, nb, out.data_ptr(),
                                                           case.out_bytes,
                                                           source_pinned=1 if pinned else 0), n)
            row["e2e_pinned" if pinned else "e2e_pageable"] = _e2e_row(p50, p95, rep, case.out_bytes,
                                                                       h2d_ceiling, n)
            del held
        del out
        if name == "c1":
            lat = {}
            for small in (128, 192, 256):
                sc1 = Case("c1", "C1 N=%d" % small, W.c1_plan().blob, {"s0": small}, None,
                           W.c1_input(small))
                o1 = torch.empty(sc1.out_bytes, dtype=torch.uint8, device="cuda")
                p50, p95, _ = _calls(lambda: ctx.execute_h2d(sc1.bound, sc1.src.ctypes.data,
                                                             sc1.src.nbytes, o1.data_ptr(),
                                                             sc1.out_bytes), samples)
                lat[str(small)] = {"p50_us": round(p50 * 1e6, 1), "p95_us": round(p95 * 1e6, 1)}
            row["small_n_latency"] = lat
        rows[name] = row
        kernels.append((name, case.bound, case.wire_bytes, case.out_bytes))
        del case
    log("table: c4 grouped steps")
    rows["c4"], c4_kernel = c4_table(torch, ctx, P, h2d_ceiling)
    kernels.append(c4_kernel)
    for name, bound, wire, out_bytes in kernels:
        log("table: %s kernel" % name)
        ms_step, kms = device_rate(torch, ctx, bound, wire, out_bytes, 200, 20)
        alg = wire + out_bytes + bound.parameter_bytes
        rows[name]["kernel"] = {"name": rows[name]["kernel"], "us": round(ms_step * 1e3, 3),
                                "us_event_per_launch": round(kms * 1e3, 3),
                                "algorithmic_bytes": alg,
                                "GBps": round(alg / ms_step / 1e6, 1),
                                "hbm_frac": round(alg / ms_step / 1e6 / HBM_PEAK_GBS, 4)}
    for name, bound, wire, out_bytes in kernels:
        k = rows[name]["kernel"]
        copy = P.measure_copy(0, max(16, k["algorithmic_bytes"] // 2), 100, 3)
        k["copy_GBps"] = round(copy, 1)
        k["of_copy"] = round(k["GBps"] / copy, 4)
    ctx.close()
    order = ["c1", "c2", "c3", "c4"] + ["c5_%dx%d" % bs for bs in W.C5_SHAPES]
    return {"protocol": "per config: %d warm-up calls, then p50/p95 of %d calls (25 for the 2 GiB "
                        "C5 shape; C4: 20 grouped steps), pageable and page-locked sources; kernel: "
                        "200 back-to-back launches between events over resident buffers, and a "
                        "16-byte copy of the same bytes in the same run" % (TABLE_WARMUP, samples),
            "pinned_h2d_ceiling_GBps": round(h2d_ceiling, 2),
            "rows": {k: rows[k] for k in order}}


def c4_table(torch, ctx, P, h2d_ceiling):
    """C4 per step: 2 of 8 experts drawn uniformly, their 6 int8 matrices as
    one grouped transfer (p50/p95 over 20 drawn steps after 3 warm-up
    steps), from a pageable and from a page-locked expert pool; the kernel
    leg is one gate matrix."""
    from sym_amd import workloads as W
    pool = W.c4_pool()
    steps = W.c4_steps(20)
    plan = P.Plan(W.c4_plan().blob)
    bounds = {(e, j): P.Bound(plan, {"s0": q.shape[0], "s1": q.shape[1]}, W.param("scale", s))
              for e in range(8) for j, (q, s) in enumerate(pool[e])}
    dst = [torch.empty(bounds[(0, 0)].destination_bytes, dtype=torch.uint8, device="cuda")
           for _ in range(6)]

    def run(experts, pinned):
        bl, sl, dl = [], [], []
        for k, (e, j) in enumerate((e, j) for e in experts for j in range(3)):
            q = pool[e][j][0]
            bl.append(bounds[(e, j)])
            sl.append((pinned[(e, j)].data_ptr(), q.nbytes) if pinned else (q.ctypes.data, q.nbytes))
            dl.append((dst[k].data_ptr(), dst[k].numel()))
        return ctx.execute_group_h2d(bl, sl, dl, source_pinned=1 if pinned else 0)[1]

    row = {"workload": "C4 MoE: 2 of 8 experts x {gate,up [14336,4096], down [4096,14336]} int8 "
                       "-> per-row dequant -> f16 (one grouped transfer per step)",
           "kernel": bounds[(0, 0)].kernel}
    for pinned in (None, True):
        held = ({key: torch.from_numpy(pool[key[0]][key[1]][0]).pin_memory() for key in bounds}
                if pinned else None)
        for ex in steps[:3]:
            run(ex, held)
        ts = []
        for ex in steps:
            t = time.perf_counter()
            tot = run(ex, held)
            ts.append(time.perf_counter() - t)
        p50, p95 = float(np.percentile(ts, 50)), float(np.percentile(ts, 95))
        r = _e2e_row(p50, p95, tot, tot["destination_bytes"], h2d_ceiling, len(steps))
        r["implementation"] = "hip_relayout_group (6 matrices)"
        row["e2e_pinned" if pinned else "e2e_pageable"] = r
        del held
    del dst
    b, q = bounds[(0, 0)], pool[0][0][0]
    return row, ("c4", b, q.nbytes, b.destination_bytes)


# ------------------------------------------------------------- headline

HEADLINE_B, HEADLINE_S = 64, 4096  # C5 at its largest shape: 2 GiB f16 in, 1 GiB int8 out
# Staging of the headline's pageable source: the 8 worker threads the
# reference's typed transfers use (reloc_torch execute_typed_transfer passes
# the template's threads, 8), and this library's 3-slot pinned ring (measured
# 98.7-99.4% of the PCIe ceiling on C5 64x4096; with the chunks left to the
# library, reloc_torch's 2 slots run as 3 as well).
GATHER_THREADS, RING_SLOTS = 8, 3


def host_view(P, a):
    return P.BufferView(a.ctypes.data, a.nbytes, 0, list(a.shape),
                        [st // a.dtype.itemsize for st in a.strides], a.dtype.itemsize, "host")


def device_view(P, t):
    return P.BufferView(t.data_ptr(), t.numel() * t.element_size(), 0, list(t.shape),
                        list(t.stride()), t.element_size(), "cuda", t.device.index)


def cpu_reference_h2d(torch, blob, symbols, params, src, out_bytes, seconds, threads, device=0):
    """The reference's own `cpu_reference` H2D row (oracle/_ref): its CPU
    transform of every stage into a 2-slot pinned ring, each slot's H2D on a
    HIP copy stream (libreloc/src/Dispatch.cpp:452-546,1983-2046;
    bench/results/typed-h2d-221/README.md:23-36), timed on this host over
    whole calls until `seconds` have passed (at least two)."""
    from oracle import ref
    if not ref.hip_available():
        return None
    r = ref.CpuH2dRef(blob, symbols, params, threads=threads, buffers=2, queues=1, device=device)
    out = torch.empty(out_bytes, dtype=torch.uint8, device="cuda:%d" % device)
    r.execute(src.ctypes.data, src.nbytes, out.data_ptr(), out_bytes)  # warm: ring, pool
    n, t0 = 0, time.perf_counter()
    while True:
        r.execute(src.ctypes.data, src.nbytes, out.data_ptr(), out_bytes)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds and n >= 2:
            break
    del r, out
    return {"value": round(out_bytes * n / el / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "reference",
            "sample": "%d whole calls in %.1f s of the reference's cpu_reference H2D row "
                      "(CPU transform into 2 pinned slots, then H2D) on the full headline batch"
                      % (n, el)}


def headline(torch, P, args, h2d_ceiling, inputs):
    """C5 at B=64, S=4096 end to end: one step is one blocking call of the
    reference-shaped dispatch API from a pageable host tensor (fresh output
    allocation, bind, prepare, execute, completion), as the reference times
    its typed H2D rows (bench/results/typed-h2d-221/README.md:31-35)."""
    from sym_amd import workloads as W
    B, S = HEADLINE_B, HEADLINE_S
    x, sc = inputs
    blob = W.c5_plan().blob
    plan = P.load_typed_plan(blob)
    syms = {"B": B, "S": S}
    params = W.param("scale", sc)
    E = B * S * 4096
    out_bytes, wire_bytes = E, 2 * E
    src_view = host_view(P, x)
    stream = torch.cuda.current_stream().cuda_stream
    res = P.Resources(0)

    def step(view=src_view, resources=res, slots=RING_SLOTS):
        out = torch.empty((B, 32, S, 128), dtype=torch.int8, device="cuda")
        bound = P.bind_typed(plan, syms, params)
        req = P.prepare_dispatch(bound, view, device_view(P, out), "h2d")
        rep = P.execute_dispatch(req, caller_stream=stream, resources=resources,
                                 gather_threads=GATHER_THREADS, n_buffers=slots)
        return out, rep

    torch.cuda.synchronize()
    t = time.perf_counter()
    out, rep = step()  # the cold call: ring, wire arena and parameters allocated on the way
    first_ms = round((time.perf_counter() - t) * 1e3, 3)
    for _ in range(max(0, args.warmup - 1)):
        out, rep = step()
    del out
    log("first call %.1f ms; %d warmup steps done" % (first_ms, args.warmup))
    res.time_kernels(True)
    ts = []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ta = time.perf_counter()
        out, rep = step()
        ts.append(time.perf_counter() - ta)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    kt = res.kernel_times()
    res.time_kernels(False)
    log("%d timed steps: %.2f ms per step" % (args.steps, elapsed / args.steps * 1e3))
    del out
    ms_step = elapsed / args.steps * 1e3
    value = out_bytes * args.steps / elapsed / 1e9
    p50, p95 = float(np.percentile(ts, 50)), float(np.percentile(ts, 95))

    # The dominant kernel: k_permute, one launch per kernel batch of the
    # upload. A batch takes whole batch entries (the chunks) up to 512 MiB of
    # wire, at most a quarter of the call, and the last chunk is a batch of
    # its own. The roofline takes the full batch's launch, the same box over
    # B' entries, back to back on one stream between two events (an event
    # pair per launch, which adds the events' cost, is reported beside it).
    # The launches inside the steps are timed by event pairs on their copy
    # stream, which also count the wait from the batch's last copy to the
    # kernel's start.
    units = batch_units(B, S)
    launches_per_call = kt["launches"] // max(1, kt["calls"])
    expected = -(-(B - 1) // units) + 1 if units > 1 else B
    assert launches_per_call == expected, (B, units, launches_per_call)
    unit_bytes = S * 4096 * 3  # one batch entry: 2 B of f16 read + 1 B of int8 written per element
    alg_per_launch = units * unit_bytes + sc.nbytes
    # in the steps: every launch's bytes over every launch's time
    pipeline_bytes = kt["calls"] * (B * unit_bytes + launches_per_call * sc.nbytes)
    pipeline_gbs = pipeline_bytes / (kt["ms"] * 1e-3) / 1e9
    ub = P.bind_typed(plan, {"B": units, "S": S}, params)
    kernel_ms, pair_ms = device_rate(torch, res, ub, 2 * units * S * 4096, units * S * 4096,
                               max(100, 4 * args.steps), 10)
    achieved = alg_per_launch / (kernel_ms * 1e-3) / 1e9
    copy_gbs = P.measure_copy(0, alg_per_launch // 2, 200, 3)

    # the same steps from a pinned source (direct DMA)
    pinned = torch.from_numpy(x).pin_memory()
    pview = P.BufferView(pinned.data_ptr(), x.nbytes, 0, list(x.shape),
                         [st // 2 for st in x.strides], 2, "host")
    out, prep_rep = step(pview)
    pts = []
    for _ in range(max(5, args.steps // 2)):
        ta = time.perf_counter()
        out, prep_rep = step(pview)
        pts.append(time.perf_counter() - ta)
    q50 = float(np.percentile(pts, 50))
    del out, pinned
    res.close()
    torch.cuda.synchronize()

    # reloc_torch's default ring depth (execute_typed_transfer n_buffers=2,
    # libreloc/python/reloc_torch/dispatch.py:260) on resources of their
    # own, so that the ring holds what that depth asks for
    res2 = P.Resources(0)
    for _ in range(3):
        out, rep2 = step(resources=res2, slots=2)
    del out
    ts2 = []
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    for _ in range(max(5, args.steps // 2)):
        ta = time.perf_counter()
        out, rep2 = step(resources=res2, slots=2)
        ts2.append(time.perf_counter() - ta)
    torch.cuda.synchronize()
    el2 = time.perf_counter() - t2
    del out
    res2.close()
    torch.cuda.synchronize()
    log("two ring slots: %.2f ms per step" % (el2 / len(ts2) * 1e3))

    log("pinned source p50 %.2f ms" % (q50 * 1e3))
    cpu = cpu_all = None
    if not args.no_cpu:
        log("cpu baseline")
        cpu = cpu_reference_h2d(torch, blob, syms, params, x, out_bytes, args.cpu_seconds, 8)
        cores = len(os.sched_getaffinity(0))
        cpu_all = (cpu_reference_h2d(torch, blob, syms, params, x, out_bytes, args.cpu_seconds,
                                     cores) if cores != 8 else cpu)
    traffic = traffic_for("c5_e2e", alg_per_launch)
    return {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seed 20260710: activations N(0,1) as f16, per-head scales U[0.02,0.05])",
        "config": {"workload": "C5 f16 [64,4096,32,128] -> [B,32,S,128] -> f32 -> int8 "
                               "(per-head scale, zero-point 0), pageable host source -> HBM",
                   "B": B, "S": S, "output_bytes": out_bytes, "wire_bytes_per_step": rep["wire_bytes"],
                   "implementation": rep["implementation"], "chunks_per_step": rep["host_chunks"],
                   "kernel_launches_per_step": rep["kernel_launches"],
                   "gather_threads": GATHER_THREADS, "ring_slots": RING_SLOTS,
                   "step": "torch.empty output + bind_typed + prepare_dispatch + execute_dispatch "
                           "(blocking, ordered after torch's stream)",
                   "value_definition": "output bytes x steps / wall time of the steps"},
        "pcie": {"pinned_h2d_ceiling_GBps": round(h2d_ceiling, 2),
                 "wire_GBps": round(rep["wire_bytes"] * args.steps / elapsed / 1e9, 2),
                 "frac": round(rep["wire_bytes"] * args.steps / elapsed / 1e9 / h2d_ceiling, 4),
                 "p50_ms": round(p50 * 1e3, 3), "p95_ms": round(p95 * 1e3, 3),
                 "first_call_ms": first_ms,
                 "pinned_source": {"p50_ms": round(q50 * 1e3, 3),
                                   "effective_GBps": round(out_bytes / q50 / 1e9, 2),
                                   "frac": round(prep_rep["wire_bytes"] / q50 / 1e9 / h2d_ceiling, 4),
                                   "implementation": prep_rep["implementation"]},
                 "two_ring_slots": {"steps": len(ts2), "value": round(out_bytes * len(ts2) / el2 / 1e9, 2),
                                    "p50_ms": round(float(np.percentile(ts2, 50)) * 1e3, 3),
                                    "frac": round(rep2["wire_bytes"] * len(ts2) / el2 / 1e9 / h2d_ceiling, 4),
                                    "host_buffers": rep2["host_buffers"],
                                    "note": "n_buffers=2, reloc_torch's default ring depth, on "
                                            "resources of their own (with the chunks left to the "
                                            "library a ring has at least three slots)"},
                 "staging": rep["staging"], "host_chunk_bytes": rep["host_chunk_bytes"],
                 "host_buffers": rep["host_buffers"]},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": "profiles/traffic.json, committed: FETCH_SIZE + WRITE_SIZE "
                                       "per dispatch of this launch from two rocprofv3 --pmc runs of "
                                       "bench.py --traffic-probe --configs c5_e2e (counters need a "
                                       "profiler run of their own; not measured in this run)",
                     "kernel": "k_permute_direct8<2, 1, 6> (f16 -> f32 -> int8, [B,S,32,128] -> [B,32,S,128], eight waves per SIMD, streaming stores)",
                     "launch": "one kernel batch of the upload: %d batch entries [%d,%d,32,128]"
                               % (units, units, S),
                     "kernel_ms_per_launch": round(kernel_ms, 5),
                     "kernel_ms_definition": "two events on the launch stream bracketing the timed "
                                             "region's back-to-back launches, over their count",
                     "kernel_ms_per_launch_event_pairs": round(pair_ms, 5),
                     "algorithmic_bytes_per_launch": alg_per_launch,
                     "algorithmic_bytes_per_unit": unit_bytes, "units_per_launch": units,
                     "in_pipeline": {"launches_timed": kt["launches"],
                                     "launches_per_call": launches_per_call,
                                     "kernel_ms_per_call_events": round(kt["ms"] / max(1, kt["calls"]), 4),
                                     "achieved": round(pipeline_gbs, 1)},
                     "copy_ceiling": {"GBps": round(copy_gbs, 1), "bytes": alg_per_launch,
                                      "kernel": "16-byte vector copy of the same bytes, the faster of one and two vectors per lane",
                                      "frac": round(achieved / copy_gbs, 4)}},
        "cpu_baseline": cpu,
        "cpu_baseline_all_cores": cpu_all,
        "host": host_info(),
    }


def summarize_line(path):
    """Markdown tables of the per-config table of a saved bench line (the
    `configs` key of the default run's JSON line)."""
    with open(path) as f:
        d = json.loads([l for l in f.read().splitlines() if l.startswith("{")][-1])
    t = d["configs"]
    out = ["Protocol: %s. Pinned H2D ceiling measured in the same run: **%.2f GB/s**." % (
        t["protocol"], t["pinned_h2d_ceiling_GBps"]), "",
        "| config | pageable p50 ms | p95 ms | PCIe frac | pinned p50 ms | p95 ms | PCIe frac | "
        "output GB/s (pinned) | kernel us | of 8 TB/s | same-run copy GB/s | of copy |",
        "|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|"]
    for name, r in t["rows"].items():
        a, b, k = r["e2e_pageable"], r["e2e_pinned"], r["kernel"]
        out.append("| %s | %.3f | %.3f | %.3f | %.3f | %.3f | %.3f | %.2f | %.2f | %.3f | %.0f | %.3f |" % (
            name, a["p50_ms"], a["p95_ms"], a["pcie_frac"], b["p50_ms"], b["p95_ms"], b["pcie_frac"],
            b["effective_GBps"], k["us"], k["hbm_frac"], k["copy_GBps"], k["of_copy"]))
    lat = t["rows"]["c1"].get("small_n_latency")
    if lat:
        out += ["", "C1 small N (latency-bound), end-to-end p50 / p95 us: " + ", ".join(
            "N=%s: %.1f / %.1f" % (n, v["p50_us"], v["p95_us"]) for n, v in lat.items())]
    print("\n".join(out))


def summarize_report(path):
    """The per-config tables of profiles/configs_report.md from the saved
    output of --report: device-resident kernel rates, end-to-end uploads from
    pageable and pinned sources, downloads, and C1's small-N latencies.
    Prints markdown."""
    with open(path) as f:
        rows = [json.loads(l) for l in f if l.startswith("{")]
    head = {}
    for r in rows:
        if "pinned_h2d_ceiling_GBps" in r and "config" not in r:
            head.update(r)
        if "hbm_copy_GBps" in r:
            head.update(r)
    vc = head.get("vector_copy_GBps") or {}
    out = ["Measured pinned H2D ceiling: **%.2f GB/s**; torch 1 GiB device copy: %.1f GB/s%s." % (
        head["pinned_h2d_ceiling_GBps"], head.get("hbm_copy_GBps", float("nan")),
        ("; librelx 16-byte vector copy: " + ", ".join("%s %.0f GB/s" % kv for kv in vc.items())) if vc else ""),
        "", "| config | kernel | device us | achieved GB/s | HBM frac | e2e pageable p50 ms | PCIe frac | "
        "e2e pinned p50 ms | PCIe frac |", "|---|---|---:|---:|---:|---:|---:|---:|---:|"]
    cell = lambda d, k: d.get(k, "-") if d else "-"
    for r in rows:
        if "device" not in r or r.get("config", "").endswith("_d2h"):
            continue
        d, a, b = r["device"], r.get("e2e_pageable"), r.get("e2e_pinned")
        out.append("| %s | %s | %.2f | %.1f | %.3f | %s | %s | %s | %s |" % (
            r["config"], r["kernel"], d["ms_per_step"] * 1e3, d["achieved_GBps"], d["hbm_frac"],
            cell(a, "p50_ms"), cell(a, "pcie_frac"), cell(b, "p50_ms"), cell(b, "pcie_frac")))
    d2h = [r for r in rows if r.get("config", "").endswith("_d2h")]
    if d2h:
        out += ["", "Device -> host (KV eviction: the C5 source resident on the device, the int8 result "
                "into host memory; PCIe fraction against the measured pinned D2H ceiling, **%.2f GB/s**):"
                % d2h[0]["pinned_d2h_ceiling_GBps"], "",
                "| config | pageable p50 ms | GB/s | PCIe frac | pinned p50 ms | GB/s | PCIe frac | chunks |",
                "|---|---:|---:|---:|---:|---:|---:|---:|"]
        for r in d2h:
            a, b = r["pageable"], r["pinned"]
            out.append("| %s | %s | %s | %s | %s | %s | %s | %s |" % (
                r["config"], a["p50_ms"], a["effective_GBps"], a["pcie_frac"], b["p50_ms"],
                b["effective_GBps"], b["pcie_frac"], a["chunks"]))
    lat = [r for r in rows if "e2e_latency_us_p50" in r]
    if lat:
        out += ["", "C1 small N (latency-bound), end-to-end p50 / p95 us: " + ", ".join(
            "N=%d: %.1f / %.1f" % (r["N"], r["e2e_latency_us_p50"], r["e2e_latency_us_p95"]) for r in lat)]
    print("\n".join(out))


def main():
    args = parse()
    if args.summarize_report:
        summarize_report(args.summarize_report)
        return
    if args.summarize_line:
        summarize_line(args.summarize_line)
        return
    if args.summarize_stats:
        with open(os.path.join(args.summarize_stats, "probe.json")) as f:
            summarize_stats(args.summarize_stats, json.loads(f.read().strip().splitlines()[-1]))
        return
    if args.summarize_trace:
        plan_path = os.path.join(args.summarize_trace, "plan.json")
        if os.path.exists(plan_path):
            with open(plan_path) as f:
                summarize_calls(args.summarize_trace, json.loads(f.read().strip().splitlines()[-1]))
        else:
            summarize_trace(args.summarize_trace)
        return
    if args.summarize_pmc:
        probe = None
        for d in args.summarize_pmc:
            p = os.path.join(d, "probe.json")
            if os.path.exists(p):
                with open(p) as f:
                    probe = json.load(f)
        if probe is None:
            sys.exit("probe.json (the --traffic-probe output line) missing from the PMC directories")
        res = summarize_pmc(args.summarize_pmc[0], args.summarize_pmc[1], probe)
        path = os.path.join(ROOT, "profiles", "traffic.json")
        if os.path.exists(path):  # keep the configs this probe did not cover
            with open(path) as f:
                old = json.load(f)
            merged = dict(old.get("configs", {}))
            merged.update(res["configs"])
            res["configs"] = merged
        with open(path, "w") as f:
            json.dump(res, f, indent=1)
        print(json.dumps(res))
        return
    if args.gpus != 1:
        sys.exit("bench.py measures one GPU: this build runs the path on one MI355X only "
                 "(every GPU box here has one GPU); got --gpus %d" % args.gpus)
    torch = torch_mod()
    from sym_amd import pyreloc as P
    ctx = P.Context(0)
    h2d_ceiling = P.measure_h2d(0, 256 << 20, 20, 3)

    if args.trace_configs:
        print(json.dumps(trace_configs(torch, ctx, args.trace_configs.split(","), h2d_ceiling)), flush=True)
        ctx.close()
        return

    if args.traffic_probe:
        traffic_probe(torch, ctx, args.configs.split(","))
        ctx.close()
        return

    if args.report:
        print(json.dumps({"pinned_h2d_ceiling_GBps": round(h2d_ceiling, 2)}), flush=True)
        for name in args.configs.split(","):
            if name == "c4":
                print(json.dumps(c4_report(torch, ctx, P, args, h2d_ceiling)), flush=True)
            elif name == "c1":
                print(json.dumps(one_config(torch, ctx, P, "c1", args, h2d_ceiling)), flush=True)
                for n in (128, 192, 256):
                    from sym_amd import workloads as W
                    case = Case("c1", "C1 N=%d" % n, W.c1_plan().blob, {"s0": n}, None, W.c1_input(n))
                    p50, p95, rep = e2e_rate(torch, ctx, case, 50, pinned=False)
                    print(json.dumps({"config": "c1", "N": n, "e2e_latency_us_p50": round(p50 * 1e6, 1),
                                      "e2e_latency_us_p95": round(p95 * 1e6, 1)}), flush=True)
            elif name in IX:
                print(json.dumps(ix_config(torch, ctx, P, name, args, h2d_ceiling)), flush=True)
            elif name == "c5":
                from sym_amd import workloads as W
                for b, s in W.C5_SHAPES:
                    print(json.dumps(one_config(torch, ctx, P, "c5_%dx%d" % (b, s), args, h2d_ceiling)),
                          flush=True)
                d2h_ceiling = P.measure_d2h(0, 256 << 20, 20, 3)
                for b, s in ((8, 1024), (8, 4096), (64, 1024)):
                    print(json.dumps(d2h_config(torch, ctx, "c5_%dx%d" % (b, s), args, d2h_ceiling)),
                          flush=True)
            else:
                print(json.dumps(one_config(torch, ctx, P, name, args, h2d_ceiling)), flush=True)
        # The HBM copy ceilings come last: after hundreds of MB of device
        # allocations are freed, later host->device copies from pinned memory
        # on streams created before can run at half speed (a plain HIP probe
        # shows it too), which would skew the configs' end-to-end rates.
        print(json.dumps({"hbm_copy_GBps": round(hbm_copy_ceiling(torch), 1),
                          "vector_copy_GBps": {str(n >> 20) + "MiB": round(P.measure_copy(0, n, 50, 3), 1)
                                               for n in (16 << 20, 64 << 20, 256 << 20, 1 << 30)}}),
              flush=True)
        ctx.close()
        return

    from sym_amd import workloads as W
    log("generating the C5 %dx%d input" % (HEADLINE_B, HEADLINE_S))
    inputs = W.c5_input(HEADLINE_B, HEADLINE_S)
    line = headline(torch, P, args, h2d_ceiling, inputs)
    ctx.close()
    if not args.no_table:
        line["configs"] = config_table(torch, P, args, h2d_ceiling, inputs)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
