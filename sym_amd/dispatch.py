"""Typed dispatch in the shape of the reference's pyreloc dispatch API.

The reference prepares a single-use request from a bound typed plan and two
buffer views, selects one "implementation row", and executes it
(libreloc/python/PyDispatch.cpp:86-235,517-901; libreloc/src/Dispatch.cpp:
1147-1218,1382-1532,1983-2046). Its rows include CPU executors; this build
has exactly one kind of row, the device relayout, offered at each wire
boundary a host may reach with per-tensor stages:

    hip_relayout        the source bytes cross PCIe; every stage on the GPU
    hip_relayout@k      the host applies stages [0, k) while staging

The device-to-host direction has one row, `hip_relayout`: the device runs
the relayout and every stage and the result crosses PCIe (the reference's
cuda_stages_then_cpu rows with every stage on the device).

Indexed (wire v2) plans go through `prepare_index_select_program(bound,
source_view)` (reference prepareIndexSelect, libreloc/src/Dispatch.cpp:
1269-1283): the source view is the whole host table; the host gathers the
selected rows while staging and the device runs the rest. The automatic
row sends the table itself instead when the selection is long (2^16 rows
or more) and the table is no larger than the gathered rows; the device
then gathers the rows (report implementation `hip_table_gather`). They
have no device-to-host row.

Names, argument meaning and error codes follow the reference so that
`reloc_torch.dispatch` can call these functions in place of `_pyreloc`'s.
Requests whose policy asks for a CPU executor ("original_cpu") or a forced
row this build lacks raise TransferError("implementation_unavailable").
"""
import math
import threading

from . import pyreloc as P
from .pyreloc import TransferError
from .transfer import (BufferView, DispatchResources, GatherPool,  # noqa: F401
                       _gather_threads, context_for)

POLICIES = ("auto", "original_cpu")


class Calibration:
    """A parsed cost-model calibration (reference pyreloc.Calibration,
    libreloc/python/PyReloc.cpp:658-672; the file format of
    libreloc/src/CostModel.cpp:29-76). The reference's `auto` policy uses it
    to choose between CPU and device rows; this build has only device rows,
    so a calibration is accepted wherever the reference takes one and
    changes no selection."""

    __slots__ = ("_machine", "_values")

    def __init__(self, machine, values):
        self._machine = machine
        self._values = dict(values)

    @property
    def machine(self):
        return self._machine

    def value(self, key):
        """The calibrated figure under `key`, or None."""
        return self._values.get(key)

    def __repr__(self):
        return "Calibration(machine=%r, %d values)" % (self._machine, len(self._values))


def _strtod(s):
    """A whole-string C strtod: decimal and hexadecimal floats, inf and nan;
    NaN for anything else (the caller rejects non-finite values)."""
    if "_" in s:  # Python's float() takes digit separators, strtod does not
        return math.nan
    try:
        return float(s)
    except ValueError:
        pass
    body = s[1:] if s[:1] in "+-" else s
    if body[:2] in ("0x", "0X"):
        try:
            return float.fromhex(s)
        except ValueError:
            pass
    return math.nan


def parse_calibration(text):
    """Parse a "# costmodel calibration v0" file; ValueError names the
    offending line, as the reference's CostModel::parse does."""
    machine, values, saw_version = "", {}, False
    for line_no, line in enumerate(text.split("\n"), 1):
        raw = line.strip(" \t\r\n")
        if not raw:
            continue
        if not saw_version:
            if raw != "# costmodel calibration v0":
                raise ValueError("calibration: first non-blank line must be the v0 version "
                                 "header (line %d)" % line_no)
            saw_version = True
            continue
        if raw.startswith("#"):
            if raw.startswith("# machine:"):
                machine = raw[len("# machine:"):].strip(" \t\r\n")
            continue
        fields = raw.split("#", 1)[0].split()
        if len(fields) < 2:
            raise ValueError("calibration: expected 'key value' at line %d" % line_no)
        if len(fields) > 2:
            raise ValueError("calibration: trailing junk at line %d" % line_no)
        key, text_value = fields
        v = _strtod(text_value)
        if not math.isfinite(v):
            raise ValueError("calibration: non-numeric value at line %d" % line_no)
        if key in values:
            raise ValueError("calibration: duplicate key '%s' at line %d" % (key, line_no))
        values[key] = v
    if not saw_version:
        raise ValueError("calibration: empty file (no version header)")
    return Calibration(machine, values)


def load_calibration(path):
    """Load a calibration file (reference pyreloc.load_calibration,
    libreloc/python/PyReloc.cpp:662-672)."""
    try:
        with open(path) as f:
            text = f.read()
    except OSError:
        raise ValueError("calibration: cannot read " + str(path)) from None
    return parse_calibration(text)


def _check_calibration(calibration):
    if calibration is not None and not isinstance(calibration, Calibration):
        raise TypeError("calibration must be pyreloc.Calibration or None")


def _label(k):
    return "hip_relayout" if k == 0 else "hip_relayout@%d" % k


def _row(bound, k):
    wire = bound.info.wire_bytes_at[k]  # the source layout, staged to boundary k
    return {"implementation": _label(k), "wire_boundary": k, "wire_result_layout": False,
            "wire_bytes": wire, "device_temp_bytes": wire, "method": "device_relayout"}


class IndexSelectProgram:
    """A bound indexed plan checked against its host table view (reference
    prepareIndexSelect's Program, libreloc/src/Dispatch.cpp:1269-1283)."""

    def __init__(self, bound, source):
        self.bound = bound
        self.source = source


def _check_table_view(bound, view):
    """The source-view checks of checkView for an indexed program
    (libreloc/src/Dispatch.cpp:161-201)."""
    if view.kind == "cuda":
        raise TransferError("direction_mismatch", "host-to-device source must be host memory")
    view.span_bytes  # noqa: B018 - the checked span raises for a bad view
    if view.element_size != bound.info.source_width:
        raise TransferError("plan_mismatch", "source element size differs from the typed "
                            "program's source type")
    if not view.is_dense():
        raise TransferError("unsupported_layout", "source view must be dense row-major")
    if view.extents != bound.source_extents:
        raise TransferError("plan_mismatch", "indexed source requires the prepared host row shape")


def prepare_index_select_program(bound, source):
    """Check a bound indexed plan against its host table view (reference
    prepare_index_select_program, libreloc/python/PyDispatch.cpp:518-528)."""
    if not isinstance(bound, P.IndexedBound):
        raise TypeError("prepare_index_select_program needs a bound indexed plan")
    _check_table_view(bound, source)
    return IndexSelectProgram(bound, source)


def _unwrap(plan):
    return plan.bound if isinstance(plan, IndexSelectProgram) else plan


def query_capability(bound, direction, device):
    """Eligible and excluded rows (reference query_capability,
    libreloc/src/Dispatch.cpp:1382-1532)."""
    bound = _unwrap(bound)
    if device not in ("host", "cuda"):
        raise ValueError("device must be 'host' or 'cuda', got '%s'" % device)
    if direction not in ("h2d", "d2h"):
        raise ValueError("direction must be 'h2d' or 'd2h', got '%s'" % direction)
    if not bound.typed:
        raise TransferError("typed_unsupported", "layout plans dispatch through execute_transfer")
    if device == "host":
        return {"eligible": [], "excluded": [{"implementation": "hip_relayout",
                                              "reason": "host_destination"}]}
    if direction == "d2h" and bound.indexed:
        # indexed sources are host rows (libreloc/src/Dispatch.cpp:1397-1404)
        return {"eligible": [], "excluded": [{"implementation": "hip_relayout",
                                              "reason": "host_index_select"}]}
    if direction == "d2h":
        out = bound.destination_bytes
        return {"eligible": [{"implementation": "hip_relayout", "wire_boundary": bound.stage_count,
                              "wire_result_layout": True, "wire_bytes": out,
                              "device_temp_bytes": out, "method": "device_relayout"}],
                "excluded": []}
    rows = [_row(bound, k) for k in range(bound.info.host_stages_max + 1)]
    excluded = [{"implementation": _label(k), "reason": "per_channel_stage_on_host"}
                for k in range(bound.info.host_stages_max + 1, bound.stage_count + 1)]
    return {"eligible": rows, "excluded": excluded}


class DispatchTemplate:
    """Bound plan + selected row, reusable for many views (reference
    DispatchTemplate, libreloc/include/reloc/Dispatch.h:104-124)."""

    def __init__(self, bound, direction, capability, selection, threads):
        self.bound = bound
        self.program = bound
        self.direction = direction
        self.capability = capability
        self.selection = selection
        self.threads = threads


class DispatchRequest:
    """Single-use request: template + validated views (reference
    DispatchRequest, libreloc/include/reloc/Dispatch.h:126-175)."""

    def __init__(self, template, source, destination):
        self.template = template
        self.source = source
        self.destination = destination
        self.selected = dict(template.selection)
        self.report = {}
        self.executing = False
        self.consumed = False
        self._lock = threading.Lock()


def _select(bound, direction, capability, policy, implementation):
    if policy not in POLICIES:
        raise ValueError("policy must be 'auto' or 'original_cpu', got '%s'" % policy)
    if policy == "original_cpu":
        raise TransferError("implementation_unavailable",
                            "no CPU executor row: every plan runs on the device")
    labels = [r["implementation"] for r in capability["eligible"]]
    if not labels:
        raise TransferError("implementation_unavailable", "no eligible row (%s)" % ", ".join(
            "%s: %s" % (r["implementation"], r["reason"]) for r in capability["excluded"]))
    if implementation:
        if implementation not in labels:
            raise TransferError("implementation_unavailable",
                                "row '%s' is not eligible (eligible: %s)" % (implementation,
                                                                           ", ".join(labels)))
        return {"implementation": implementation, "policy": policy, "placement_reason": "forced",
                "host_stages": labels.index(implementation) if direction == "h2d" else 0}
    if direction == "d2h":
        return {"implementation": "hip_relayout", "policy": policy,
                "placement_reason": "device_relayout", "host_stages": 0}
    auto = bound.info.host_stages_auto
    return {"implementation": _label(auto), "policy": policy,
            "placement_reason": "device_relayout", "host_stages": -1}


def prepare_dispatch_template(bound, direction, device="cuda", *, policy="auto", calibration=None,
                              threads=8, implementation=""):
    """Validate the program, enumerate the rows and select one; allocates
    and launches nothing (reference prepare_dispatch_template)."""
    if int(threads) < 1:
        raise ValueError("threads must be >= 1")
    _check_calibration(calibration)
    bound = _unwrap(bound)
    capability = query_capability(bound, direction, device)
    selection = _select(bound, direction, capability, policy, implementation)
    return DispatchTemplate(bound, direction, capability, selection, int(threads))


def select_dispatch(bound, direction, device="host", *, policy="auto", calibration=None, threads=8,
                    implementation=""):
    """The row the policy picks for this program, direction and device end,
    without buffers: the row's fields plus 'policy' and 'placement_reason'
    (reference select_dispatch, libreloc/python/PyDispatch.cpp:438-462,
    845-864). A bridge fixes the row here and forces it in prepare_dispatch
    once the destination exists."""
    if device not in ("host", "cuda"):
        raise ValueError("device must be 'host' or 'cuda', got '%s'" % device)
    if int(threads) < 1:
        raise ValueError("threads must be >= 1")
    _check_calibration(calibration)
    bound = _unwrap(bound)
    capability = query_capability(bound, direction, device)
    selection = _select(bound, direction, capability, policy, implementation)
    row = next(r for r in capability["eligible"] if r["implementation"] == selection["implementation"])
    out = dict(row)
    out["policy"] = selection["policy"]
    out["placement_reason"] = selection["placement_reason"]
    return out


def _check_view(bound, view, is_source, direction):
    """checkView (libreloc/src/Dispatch.cpp:162-219): a CUDA view on the
    device end of its direction, the checked span, the program's element
    size, dense row-major, and exactly the program's bytes (an indexed
    source: the prepared host row shape)."""
    info = bound.info
    what = "source" if is_source else "destination"
    if direction == "h2d" and is_source and view.kind == "cuda":
        raise TransferError("direction_mismatch", "host-to-device source must be host memory")
    if direction == "d2h" and not is_source and view.kind == "cuda":
        raise TransferError("direction_mismatch", "device-to-host destination must be host memory")
    span = view.span_bytes
    if view.element_size != (info.source_width if is_source else info.result_width):
        raise TransferError("plan_mismatch", "%s element size differs from the typed program's "
                            "%s type" % (what, "source" if is_source else "result"))
    if not view.is_dense():
        raise TransferError("unsupported_layout", "%s view must be dense row-major" % what)
    if is_source and bound.indexed:
        if direction != "h2d" or view.extents != bound.source_extents:
            raise TransferError("plan_mismatch", "indexed source requires the prepared host row shape")
        return
    # the source layout's bytes at boundary 0 (pads enter later), the result's
    expected = info.wire_bytes_at[0] if is_source else bound.destination_bytes
    if span != expected:
        raise TransferError("plan_mismatch", "%s view spans %d bytes but the typed program needs %d"
                            % (what, span, expected))
    if is_source:
        elements = 1
        for e in view.extents:
            elements *= e
        want = 1
        for e in info.source_extents[:info.source_rank]:
            want *= e
        if elements != want:
            raise TransferError("plan_mismatch", "source view element count differs from the "
                                "program's source descriptor")


def _check_views(bound, source, destination, direction):
    _check_view(bound, source, True, direction)
    _check_view(bound, destination, False, direction)
    # this library's rows move data between host and device memory only
    device_end = destination if direction == "h2d" else source
    if device_end.kind != "cuda":
        raise TransferError("backend_mismatch", "%s rows need the %s in device memory"
                            % (direction, "destination" if direction == "h2d" else "source"))


def prepare_dispatch_from_template(template, source, destination):
    _check_views(template.bound, source, destination, template.direction)
    return DispatchRequest(template, source, destination)


def prepare_dispatch(bound, source, destination, direction, *, policy="auto", calibration=None,
                     threads=8, implementation=""):
    """Template + views in one step (reference prepare_dispatch,
    libreloc/python/PyDispatch.cpp:131-157)."""
    t = prepare_dispatch_template(bound, direction, "cuda", policy=policy, calibration=calibration,
                                  threads=threads, implementation=implementation)
    return prepare_dispatch_from_template(t, source, destination)


class Resources(P.Context):
    """Retained streams, pinned ring and device wire scratch of one device,
    reused across requests (reference dispatch::Resources,
    libreloc/src/DispatchResources.cpp:44,552-686). `DispatchResources` is
    the per-device cache of them that the reference's constructor builds."""


def _resources_for(resources, device):
    return context_for(resources, max(0, device))


def _staging_options(pinning, min_pinned_bytes):
    """Validate the reference's staging options (parsePinning,
    libreloc/python/PyPinning.h:6-15; min_pinned_bytes is an optional
    size_t, libreloc/include/reloc/Transfer.h:136-141).

    Here they choose nothing: this library stages every staged chunk
    through its one retained ring of page-locked slots (the reference
    allocates staging per call, page-locked or not by this policy, and its
    unconfigured default is pageable). A staged source is read by the host
    and sent from the ring; a page-locked source is sent by direct DMA when
    direct_dense_upload allows it, whatever the policy. The values are
    echoed in the report's staging rows."""
    if pinning not in ("auto", "pinned", "pageable"):
        raise ValueError("pinning must be auto, pinned or pageable")
    if min_pinned_bytes is not None:
        if isinstance(min_pinned_bytes, bool) or not hasattr(min_pinned_bytes, "__index__"):
            raise TypeError("min_pinned_bytes must be an integer or None")
        if not 0 <= min_pinned_bytes.__index__() < 1 << 64:
            raise TypeError("min_pinned_bytes must be a byte count (0 <= n < 2**64)")
    return pinning, min_pinned_bytes


def _retained_limit(resources):
    """The owner's max_retained_bytes (None: no bound)."""
    limits = getattr(resources, "_limits", None) or {}
    return limits.get("retained_bytes")


def _staging_rows(rep, staging):
    """The staging row of a call that staged chunks (reference
    StagingDecision rows, libreloc/python/PyPinning.h:16-36): the ring it
    cycled through. memory_kind is always "pinned" (see _staging_options);
    the reason is "forced_pinned" when the caller asked for that, else
    "retained_pinned_ring"."""
    if not rep["staging_slots"]:
        return []
    pinning, min_pinned_bytes, retained = staging
    cap = rep["staging_bytes"]
    return [{"policy": pinning, "memory_kind": "pinned", "wire_bytes": rep["wire_bytes"],
             "staging_capacity_bytes": cap, "buffer_count": rep["staging_slots"],
             "min_pinned_bytes": min_pinned_bytes,
             "reason": "forced_pinned" if pinning == "pinned" else "retained_pinned_ring",
             "retention_eligible": retained is None or cap <= retained,
             "reused": bool(rep["staging_reused"])}]


def _report(rep, request, staging):
    sel = request.selected
    return {"implementation": rep["implementation"], "policy": sel["policy"],
            "placement_reason": sel["placement_reason"], "method": "device_relayout",
            "wire_boundary": rep["wire_boundary"], "source_bytes": rep["source_bytes"],
            "wire_bytes": rep["wire_bytes"], "destination_bytes": rep["destination_bytes"],
            "parameter_bytes": rep["parameter_bytes"],
            "payload_bytes_transferred": rep["payload_bytes_transferred"],
            "device_temp_bytes": rep["wire_bytes"],
            "artifact_version": 2 if request.template.bound.indexed else 1, "executed": True,
            "host_pipeline": "pinned_ring" if not rep["direct_dma"] else "direct_dma",
            "host_kernel": "copy" if rep["implementation"] == "hip_table_gather" else
            "index_select" if request.template.bound.indexed else
            "host_stages" if rep["wire_boundary"] else "copy",
            "host_chunks": rep["chunks"], "host_chunk_bytes": rep["host_chunk_bytes"],
            "host_buffers": rep["host_buffers"], "copy_streams": rep["copy_streams"],
            "kernel_launches": rep["kernel_launches"], "staging": _staging_rows(rep, staging)}


def execute_dispatch(request, *, caller_stream=None, n_buffers=2, n_streams=2, gather_threads=1,
                     gather_pool=None, pinning="auto", min_pinned_bytes=None,
                     direct_dense_upload=True, pipeline=True, chunk_size=0, resources=None,
                     owners=None):
    """Run the selected row and block until it completed; returns the report
    (reference execute_dispatch, libreloc/python/PyDispatch.cpp:159-235)."""
    if not request._lock.acquire(blocking=False) or request.executing:
        raise TransferError("already_executed", "typed request is executing")
    try:
        if request.consumed:
            raise TransferError("already_executed", "typed request was already executed")
        if n_buffers < 1:
            raise ValueError("n_buffers must be >= 1")
        if n_streams < 1:
            raise ValueError("n_streams must be >= 1")
        staging = _staging_options(pinning, min_pinned_bytes) + (_retained_limit(resources),)
        if gather_threads < 0:
            raise ValueError("gather_threads must be >= 0 (0 = all cores)")
        gather_threads = _gather_threads(gather_threads, gather_pool)
        live = _live_limit(resources)
        if live is not None and request.template.direction == "h2d" and _request_wire(request) > live:
            request.consumed = True
            raise TransferError("insufficient_capacity",
                                "typed scratch live-byte limit exceeded: the wire takes %d bytes, "
                                "max_live_bytes is %d" % (_request_wire(request), live))
        request.executing = True
        src, dst = request.source, request.destination
        d2h = request.template.direction == "d2h"
        device = src.device if d2h else dst.device
        ctx = _resources_for(resources, device)
        run = ctx.execute_d2h if d2h else ctx.execute_h2d
        # direct_dense_upload=False: a dense pinned source is staged through
        # the ring instead of sent by direct DMA; pipeline=False: the whole
        # buffer is staged, then sent as one chunk (reference
        # TransferOptions, libreloc/include/reloc/Transfer.h:129-134)
        # the source's own memory kind is probed (-1) unless direct DMA is off
        source_pinned = -1 if direct_dense_upload or d2h else 0
        chunk = int(chunk_size or 0) if pipeline else 1 << 62
        rep = run(request.template.bound, src.address, src.capacity_bytes - src.offset_bytes,
                  dst.address, dst.capacity_bytes - dst.offset_bytes,
                  n_buffers=n_buffers, chunk_bytes=chunk,
                  host_stages=request.selected["host_stages"],
                  gather_threads=gather_threads, source_pinned=source_pinned,
                  caller_stream=caller_stream, n_streams=n_streams)
        request.consumed = True
        request.report = _report(rep, request, staging)
        return dict(request.report)
    finally:
        request.executing = False
        request._lock.release()


class GroupRequest:
    """Members executed as one schedule with one completion (reference
    GroupRequest, libreloc/include/reloc/Dispatch.h:177-214)."""

    def __init__(self, items):
        self.items = items
        self.consumed = False
        self.executing = False
        self.report = {}


def prepare_dispatch_group(entries):
    """entries: (template or bound plan, source view, destination view,
    direction) tuples (reference prepare_dispatch_group)."""
    items = []
    for plan, source, destination, direction in entries:
        if direction != "h2d":
            raise TransferError("direction_mismatch", "groups move host-to-device members")
        t = plan if isinstance(plan, DispatchTemplate) else prepare_dispatch_template(plan, direction)
        items.append(prepare_dispatch_from_template(t, source, destination))
    if not items:
        raise TransferError("invalid_options", "an empty group")
    if len(items) > 256:
        raise TransferError("invalid_options", "a group holds at most 256 items")
    return GroupRequest(items)


def _request_wire(r):
    """Device wire bytes a request stages (its selected host boundary)."""
    b, k = _unwrap(r.template.bound), r.selected["host_stages"]
    return int(b.info.wire_bytes_at[k if k >= 0 else b.info.host_stages_auto])


def _live_limit(resources):
    """The live-byte cap of a DispatchResources owner (None: no cap)."""
    limits = getattr(resources, "_limits", None) or {}
    v = limits.get("live_bytes")
    return v if v else None


def _check_group_scratch(group, max_scratch_bytes):
    """The group's members hold their wire in the device arena together
    until the group completes (each 256-byte aligned): a group whose wire
    exceeds max_scratch_bytes is refused before anything is enqueued, and
    its requests are spent, as the reference's owner refuses scratch past
    its live-byte limit (libreloc/src/DispatchResources.cpp:120-137;
    the group is consumed, libreloc/python/tests/torch_frontend/test_group.py:176-179)."""
    need = sum((_request_wire(r) + 255) // 256 * 256 for r in group.items)
    if need > max_scratch_bytes:
        group.consumed = True
        for r in group.items:
            r.consumed = True
        raise TransferError("insufficient_capacity",
                            "typed scratch live-byte limit exceeded: the group's wire takes %d bytes, "
                            "max_scratch_bytes is %d" % (need, max_scratch_bytes))


def execute_dispatch_group(group, *, caller_stream=None, gather_threads=8, gather_pool=None,
                           pinning="auto", min_pinned_bytes=None, max_scratch_bytes=64 << 20,
                           resources=None, owners=None, device_layout=False, n_buffers=1,
                           chunked_members=False):
    """All members through one ring and one barrier; returns the group
    report with per-item reports (reference execute_dispatch_group,
    libreloc/src/Dispatch.cpp:1833-1981; defaults of
    libreloc/python/PyDispatch.cpp:648-655)."""
    if group.executing or group.consumed:
        raise TransferError("already_executed", "group is executing or already executed")
    if gather_threads < 1 or not max_scratch_bytes:
        raise ValueError("gather_threads and max_scratch_bytes must be positive")
    gather_threads = _gather_threads(gather_threads, gather_pool)
    staging = _staging_options(pinning, min_pinned_bytes) + (_retained_limit(resources),)
    _check_group_scratch(group, min(max_scratch_bytes, _live_limit(resources) or max_scratch_bytes))
    group.executing = True
    try:
        dev = max(0, group.items[0].destination.device)
        ctx = _resources_for(resources, dev)
        bounds = [r.template.bound for r in group.items]
        srcs = [(r.source.address, r.source.capacity_bytes - r.source.offset_bytes) for r in group.items]
        dsts = [(r.destination.address, r.destination.capacity_bytes - r.destination.offset_bytes)
                for r in group.items]
        reps, total = ctx.execute_group_h2d(bounds, srcs, dsts, n_buffers=n_buffers,
                                            gather_threads=gather_threads,
                                            caller_stream=caller_stream)
        items = []
        for r, rep in zip(group.items, reps):
            r.consumed = True
            r.report = _report(rep, r, staging)
            items.append(dict(r.report))
        group.consumed = True
        group.report = {"logical_transfers": len(items), "request_count": 1,
                        "completion_granularity": "group",
                        "payload_copy_calls": sum(i["host_chunks"] for i in items),
                        "kernel_launches": sum(i["kernel_launches"] for i in items),
                        "output_bytes": total["destination_bytes"],
                        "staging": _staging_rows(total, staging), "items": items}
        return dict(group.report)
    finally:
        group.executing = False


class DispatchCompletion:
    """Completion of a submitted group (reference pyreloc.DispatchCompletion,
    libreloc/python/PyDispatch.cpp:659-695): wait(), query() and
    wait_stream(stream). The group report is filled in once it completed."""

    def __init__(self, group, native, items, staging):
        self.group = group
        self._native = native
        self._items = items
        self._staging = staging

    def _finish(self):
        if self.group.consumed:
            return
        items = []
        for r, rep in zip(self._items, self._native.reports):
            r.consumed = True
            r.report = _report(rep, r, self._staging)
            items.append(dict(r.report))
        self.group.consumed = True
        self.group.report = {"logical_transfers": len(items), "request_count": 1,
                             "completion_granularity": "group",
                             "payload_copy_calls": sum(i["host_chunks"] for i in items),
                             "kernel_launches": sum(i["kernel_launches"] for i in items),
                             "output_bytes": self._native.total["destination_bytes"],
                             "staging": _staging_rows(self._native.total, self._staging),
                             "items": items}

    def wait(self):
        try:
            self._native.wait()
        finally:
            self.group.executing = False
        self._finish()
        return dict(self.group.report)

    def query(self):
        done = self._native.query()
        if done:
            self.group.executing = False
            self._finish()
        return done

    def wait_stream(self, stream):
        self._native.wait_stream(stream)

    def close(self):
        self._native.close()
        self.group.executing = False

    def __reduce_ex__(self, protocol):
        raise TypeError("dispatch completions cannot be serialized")


def submit_dispatch_group(group, *, caller_stream=None, gather_threads=8, gather_pool=None,
                          pinning="auto", min_pinned_bytes=None, max_scratch_bytes=64 << 20,
                          resources=None, owners=None, device_layout=False, n_buffers=2,
                          chunked_members=False):
    """Enqueue a group and return its completion; host staging of pageable
    sources happens before this returns (reference submit_dispatch_group)."""
    if group.executing or group.consumed:
        raise TransferError("already_executed", "group is executing or already executed")
    if owners is None or not isinstance(owners, tuple) or len(owners) not in (2, 3):
        raise ValueError("owners must be (source owners, destination owners[, extra owners])")
    if gather_threads < 1 or not max_scratch_bytes:
        raise ValueError("gather_threads and max_scratch_bytes must be positive")
    gather_threads = _gather_threads(gather_threads, gather_pool)
    staging = _staging_options(pinning, min_pinned_bytes) + (_retained_limit(resources),)
    _check_group_scratch(group, min(max_scratch_bytes, _live_limit(resources) or max_scratch_bytes))
    dev = max(0, group.items[0].destination.device)
    ctx = _resources_for(resources, dev)
    bounds = [r.template.bound for r in group.items]
    srcs = [(r.source.address, r.source.capacity_bytes - r.source.offset_bytes) for r in group.items]
    dsts = [(r.destination.address, r.destination.capacity_bytes - r.destination.offset_bytes)
            for r in group.items]
    group.executing = True
    try:
        native = ctx.submit_group_h2d(bounds, srcs, dsts, owners=owners, n_buffers=n_buffers,
                                      gather_threads=gather_threads,
                                      caller_stream=caller_stream)
    except Exception:
        group.executing = False
        raise
    return DispatchCompletion(group, native, group.items, staging)
