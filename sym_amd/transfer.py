"""Layout transfers in the shape of the reference's pyreloc transfer API
(libreloc/python/PyTransfer.cpp:312-461), over librelx's C-ABI.

`reloc_torch.transport` (libreloc/python/reloc_torch/transport.py:92-209)
calls these names: `BufferView` (with its checked `span_bytes`),
`validate_transfer_source`, `make_transfer` -> `TransferRequest`,
`execute_transfer`, `TransferResourceCache`, `cuda_enabled` and
`cuda_pointer_device`. The checks and reason codes are the reference's
(libreloc/src/Transfer.cpp:65-279, restated in sym_amd/csrc/transfer.cpp);
execution runs the layout plan through this library's upload or download
pipeline on the GPU. Host-to-host transfers, which the reference runs on
its host backend, are rejected with "backend_mismatch".

The per-device resource caches (`TransferResourceCache`,
`DispatchResources`) create one retained context per device on first use
and take the reference's constructor arguments.
"""
import ctypes
import os
import threading

from . import _native as N
from .pyreloc import TransferError, _options

_DIRECTIONS = {"h2d": 0, "d2h": 1}
_COMPLETION = {0: "not_launched", 1: "complete", 2: "unknown"}


def _fail(err):
    """Every transfer failure is a TransferError('<code>: <detail>'), as the
    reference's transfer bindings raise (PyTransfer.cpp:34-36)."""
    raise TransferError(err.code.decode(errors="replace"), err.message.decode(errors="replace"),
                        _COMPLETION.get(err.completion, "unknown"))

# librelx is built for gfx950 only: the device paths are always compiled in
# (the reference's RELOC_ENABLE_CUDA build flag).
cuda_enabled = True


def _direction(direction):
    if direction not in _DIRECTIONS:
        raise ValueError("direction must be 'h2d' or 'd2h', got '%s'" % (direction,))
    return _DIRECTIONS[direction]


def _integer(name, v, lo, hi):
    """An integer argument in [lo, hi); anything else raises TypeError."""
    if isinstance(v, bool) or not hasattr(v, "__index__"):
        raise TypeError("BufferView: %s must be an integer, got %r" % (name, v))
    v = v.__index__()
    if not lo <= v < hi:
        raise TypeError("BufferView: %s = %d is outside [%d, %d)" % (name, v, lo, hi))
    return v


class BufferView:
    """A framework buffer: the allocation it lives in (base, capacity) plus
    the logical view (offset, extents, element strides). kind is 'host' or
    'cuda'; device is the device ordinal (-1 for host). Reference
    pyreloc.BufferView (libreloc/python/PyTransfer.cpp:312-331)."""

    __slots__ = ("base", "capacity_bytes", "offset_bytes", "extents", "strides", "element_size",
                 "kind", "device")

    def __init__(self, base, capacity_bytes, offset_bytes, extents, strides, element_size,
                 kind, device=-1):
        if kind == "device":
            kind = "cuda"
        if kind not in ("host", "cuda"):
            raise ValueError("kind must be 'host' or 'cuda', got '%s'" % (kind,))
        # the reference binds uintptr_t base, size_t capacity and offset,
        # int64 extents and strides, uint32 element size and int device: a
        # value those types cannot hold is refused as its binding refuses it
        # (TypeError), never wrapped into range
        self.base = _integer("base", base, 0, 1 << 64)
        self.capacity_bytes = _integer("capacity_bytes", capacity_bytes, 0, 1 << 64)
        self.offset_bytes = _integer("offset_bytes", offset_bytes, 0, 1 << 64)
        self.extents = [_integer("extents", e, -(1 << 63), 1 << 63) for e in extents]
        self.strides = [_integer("strides", s, -(1 << 63), 1 << 63) for s in strides]
        self.element_size = _integer("element_size", element_size, 0, 1 << 32)
        self.kind = kind
        self.device = _integer("device", device, -(1 << 31), 1 << 31)

    @property
    def address(self):
        """Address of logical element 0."""
        return self.base + self.offset_bytes

    def native(self):
        v = N.relx_view()
        v.base, v.capacity_bytes, v.offset_bytes = self.base, self.capacity_bytes, self.offset_bytes
        v.rank = len(self.extents) if len(self.extents) == len(self.strides) else -1
        for i, (e, s) in enumerate(list(zip(self.extents, self.strides))[:N.RELX_MAX_VIEW_RANK]):
            v.extents[i], v.strides[i] = e, s
        v.element_size = self.element_size
        v.kind = 1 if self.kind == "cuda" else 0
        v.device = self.device
        return v

    @property
    def span_bytes(self):
        """Checked byte span from element 0; raises TransferError for empty,
        overlapping or overflowing views (reference viewSpanBytes)."""
        if len(self.extents) != len(self.strides):
            raise TransferError("invalid_view", "view extents/strides rank mismatch")
        span = ctypes.c_uint64(0)
        err = N.relx_err()
        v = self.native()
        if N.lib().relx_view_span_bytes(ctypes.byref(v), b"view", ctypes.byref(span),
                                        ctypes.byref(err)):
            _fail(err)
        return span.value

    def is_dense(self):
        """Row-major dense over its extents."""
        running = 1
        for e, s in zip(reversed(self.extents), reversed(self.strides)):
            if e != 1 and s != running:
                return False
            running *= e
        return True

    def __repr__(self):
        return "BufferView(%s, extents=%s, strides=%s, element_size=%d)" % (
            self.kind, self.extents, self.strides, self.element_size)


def validate_transfer_source(bound, source, direction):
    """Preflight: prove the bound plan's source accesses fit `source` and
    that the view is admissible for `direction`. Returns the source span in
    bytes; raises TransferError('<code>: <detail>'). Allocates and launches
    nothing (reference validate_transfer_source)."""
    d = _direction(direction)
    if len(source.extents) != len(source.strides):
        raise TransferError("invalid_view", "source extents/strides rank mismatch")
    span = ctypes.c_uint64(0)
    err = N.relx_err()
    v = source.native()
    if N.lib().relx_validate_transfer_source(bound._h, ctypes.byref(v), d, ctypes.byref(span),
                                             ctypes.byref(err)):
        _fail(err)
    return span.value


class TransferRequest:
    """A validated, single-use forward transfer owning copies of the bound
    plan and both views (reference pyreloc.TransferRequest,
    libreloc/python/PyTransfer.cpp:333-366)."""

    def __init__(self, bound, source, destination, direction, source_span_bytes,
                 destination_bytes):
        self.bound = bound
        self._source = source
        self._destination = destination
        self._direction = direction
        self._source_span_bytes = source_span_bytes
        self._destination_bytes = destination_bytes
        self._consumed = False
        self._executing = False
        self._staging = []

    direction = property(lambda self: self._direction)
    source_span_bytes = property(lambda self: self._source_span_bytes)
    destination_bytes = property(lambda self: self._destination_bytes)
    source = property(lambda self: self._source)
    destination = property(lambda self: self._destination)

    @property
    def consumed(self):
        return self._executing or self._consumed

    @property
    def staging(self):
        if self._executing:
            raise ValueError("staging report is unavailable during execution")
        return [dict(s) for s in self._staging]


def make_transfer(bound, source, destination, direction):
    """Full validation with the dense destination view; returns the
    single-use TransferRequest (reference make_transfer)."""
    d = _direction(direction)
    for role, view in (("source", source), ("destination", destination)):
        if len(view.extents) != len(view.strides):
            raise TransferError("invalid_view", "%s extents/strides rank mismatch" % role)
    s, t = source.native(), destination.native()
    span, out = ctypes.c_uint64(0), ctypes.c_uint64(0)
    err = N.relx_err()
    if N.lib().relx_validate_transfer(bound._h, ctypes.byref(s), ctypes.byref(t), d,
                                      ctypes.byref(span), ctypes.byref(out), ctypes.byref(err)):
        _fail(err)
    return TransferRequest(bound, source, destination, direction, span.value, out.value)


def cuda_pointer_device(pointer):
    """Device ordinal owning `pointer`; raises TransferError for host or
    unknown memory (reference cuda_pointer_device)."""
    dev = ctypes.c_int(-1)
    err = N.relx_err()
    if N.lib().relx_pointer_device(ctypes.c_void_p(int(pointer)), ctypes.byref(dev),
                                   ctypes.byref(err)):
        _fail(err)
    return dev.value


# ------------------------------------------------------------ resources

def _check_limit(name, v):
    """A resource limit is a non-negative integer that fits 64 bits, as the
    reference's size_t/unsigned arguments (test_transfer_resources.py:87-94)."""
    if isinstance(v, bool) or not isinstance(v, int):
        raise TypeError("%s must be an integer" % name)
    if v < 0:
        raise ValueError("%s must be >= 0" % name)
    if v >= 1 << 64:
        raise OverflowError("%s does not fit 64 bits" % name)


class _ContextCache:
    """Retained per-device contexts created on first use: the role of the
    reference's TransferResourceCache and dispatch::Resources owners
    (libreloc/src/TransferResourceCache.cpp, DispatchResources.cpp:552-686).
    A context serializes the calls made on it; `clear()` retires idle
    contexts, `close()` all of them. Construction touches no GPU."""

    def __init__(self, max_retained_bytes, limits):
        # None: no bound (the module's own contexts)
        if max_retained_bytes is not None:
            _check_limit("max_retained_bytes", max_retained_bytes)
        for name, v in limits.items():
            if v is not None:
                _check_limit(name, v)
        self._max_retained = max_retained_bytes
        self._limits = dict(limits, retained_bytes=self._max_retained)
        self._pid = os.getpid()
        self._lock = threading.Lock()
        self._contexts = {}
        self._closed = False
        self._requests = self._hits = self._creations = 0

    def _check_process(self):
        if os.getpid() != self._pid:
            raise TransferError("process_mismatch", "resource cache belongs to another process")

    def context(self, device):
        """The retained context of `device`, created on first use."""
        self._check_process()
        from .pyreloc import Context
        with self._lock:
            if self._closed:
                raise TransferError("resources_closed", "resource cache is closed")
            self._requests += 1
            ctx = self._contexts.get(device)
            if ctx is None:
                ctx = self._contexts[device] = Context(device, self._max_retained)
                self._creations += 1
            else:
                self._hits += 1
            return ctx

    @property
    def closed(self):
        self._check_process()
        return self._closed

    def clear(self):
        """Retire every retained context (the next call creates a new one)."""
        self._check_process()
        with self._lock:
            contexts, self._contexts = self._contexts, {}
        for ctx in contexts.values():
            ctx.close()

    def close(self):
        self._check_process()
        with self._lock:
            self._closed = True
        self.clear()

    def _usage(self):
        rows = []
        for dev, ctx in sorted(self._contexts.items()):
            s = ctx.stats()
            rows.append({"device": dev, "kind": "cuda", "pinned_bytes": s["pinned_bytes"],
                         "device_bytes": s["device_bytes"], "calls": s["calls"],
                         "failures": s["failures"], "quarantined": s["quarantined"]})
        return rows

    def __enter__(self):
        self._check_process()
        if self._closed:
            raise TransferError("resources_closed", "resource cache is closed")
        return self

    def __exit__(self, *exc):
        self.close()
        return False

    def __reduce_ex__(self, protocol):
        raise TypeError("transfer resources cannot be serialized")


class TransferResourceCache(_ContextCache):
    """Explicit lazy transfer resource cache for layout transfers (reference
    pyreloc.TransferResourceCache, libreloc/python/PyTransfer.cpp:368-394);
    no GPU initialization until execution."""

    def __init__(self, *, max_retained_bytes=256 << 20, max_contexts=4, max_contexts_per_device=2,
                 max_background_workers=64, max_live_staging_bytes=None, acquire_timeout_ms=None):
        super().__init__(max_retained_bytes, {
            "contexts": max_contexts, "contexts_per_device": max_contexts_per_device,
            "background_workers": max_background_workers,
            "live_staging_bytes": max_live_staging_bytes, "acquire_timeout_ms": acquire_timeout_ms})

    def stats(self):
        self._check_process()
        with self._lock:
            devices = self._usage()
        staged = sum(d["pinned_bytes"] for d in devices)
        return {"contexts": len(devices), "idle": len(devices), "leased": 0, "building": 0,
                "retiring": 0, "quarantined": sum(1 for d in devices if d["quarantined"]),
                "allocated_staging_bytes": staged, "retained_allocated_bytes": staged,
                "requests": self._requests, "hits": self._hits, "misses": self._creations,
                "failures": sum(d["failures"] for d in devices), "closed": self._closed,
                "process_valid": os.getpid() == self._pid, "limits": dict(self._limits),
                "devices": devices}


class DispatchResources(_ContextCache):
    """Retained typed-dispatch resources per device (reference
    pyreloc.DispatchResources, libreloc/python/PyDispatch.cpp:710-800)."""

    def __init__(self, *, max_retained_bytes=64 << 20, max_live_bytes=0, max_background_workers=64,
                 max_streams=8, max_contexts=1, max_contexts_per_device=1, acquire_timeout_ms=None):
        super().__init__(max_retained_bytes, {
            "live_bytes": max_live_bytes, "background_workers": max_background_workers,
            "streams": max_streams, "contexts": max_contexts,
            "contexts_per_device": max_contexts_per_device, "acquire_timeout_ms": acquire_timeout_ms})

    def stats(self):
        self._check_process()
        with self._lock:
            devices = self._usage()
        return {"requests": self._requests, "hits": self._hits,
                "context_creations": self._creations,
                "device_bytes": sum(d["device_bytes"] for d in devices),
                "host_bytes": sum(d["pinned_bytes"] for d in devices),
                "retained_bytes": sum(d["device_bytes"] + d["pinned_bytes"] for d in devices),
                "closed": self._closed, "quarantined": any(d["quarantined"] for d in devices),
                "process_valid": os.getpid() == self._pid, "active_contexts": len(devices),
                "limits": dict(self._limits), "contexts": devices}


_default_cache = None
_default_lock = threading.Lock()


def default_resources():
    """The module's own per-device contexts, for calls given no resources."""
    global _default_cache
    with _default_lock:
        if _default_cache is None:
            _default_cache = _ContextCache(None, {})
        return _default_cache


def context_for(resources, device):
    """The context a call on `device` runs on: `resources` is None (the
    module's contexts), a resource cache, or a context itself."""
    if resources is None:
        return default_resources().context(device)
    if isinstance(resources, _ContextCache):
        return resources.context(device)
    if getattr(resources, "device", device) != device:
        raise TransferError("device_mismatch", "resources run on device %d, the view is on %d"
                            % (resources.device, device))
    return resources


# ------------------------------------------------------------ execution

class GatherPool:
    """A host worker pool handle (reference pyreloc.GatherPool,
    libreloc/python/PyReloc.cpp:731-760): `threads` 0 means every core.
    Passed as `gather_pool`, its thread count sets the staging workers of
    the call (librelx keeps its worker threads inside each context). A
    closed pool is refused with ValueError, as the reference does."""

    def __init__(self, threads=0):
        threads = int(threads)
        if threads < 0:
            raise ValueError("threads must be >= 0 (0 = all cores)")
        self._threads = threads or (os.cpu_count() or 1)
        self._closed = False

    @property
    def threads(self):
        return self._threads

    @property
    def closed(self):
        return self._closed

    def close(self):
        """Idempotent."""
        self._closed = True

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
        return False


def _gather_threads(gather_threads, gather_pool):
    """The staging workers of a call: the pool's count when one is given."""
    if gather_pool is None:
        return gather_threads
    if not isinstance(gather_pool, GatherPool):
        raise TypeError("gather_pool must be pyreloc.GatherPool or None")
    if gather_pool.closed:
        raise ValueError("gather_pool is closed")
    return gather_pool.threads


def execute_transfer(request, *, caller_stream=None, n_buffers=4, n_streams=2, gather_threads=1,
                     gather_pool=None, resources=None, owners=None, pinning="auto",
                     min_pinned_bytes=None):
    """Run the forward transfer and block until this request's work has
    completed (reference execute_transfer,
    libreloc/python/PyTransfer.cpp:120-219). caller_stream (a hipStream_t
    handle; 0 is the legacy default stream, None means no producer to order
    after) is recorded before any private stream touches shared storage."""
    if isinstance(resources, _ContextCache):
        resources._check_process()
    if request._executing:
        raise TransferError("already_executed", "transfer request is already executing")
    request._executing = True
    try:
        if n_buffers < 1:
            raise ValueError("n_buffers must be >= 1")
        if n_streams < 1:
            raise ValueError("n_streams must be >= 1")
        if gather_threads < 0:
            raise ValueError("gather_threads must be >= 0 (0 = all cores)")
        gather_threads = _gather_threads(gather_threads, gather_pool)
        if pinning not in ("auto", "pinned", "pageable"):
            raise ValueError("pinning must be auto, pinned or pageable")
        if resources is not None or owners is not None:
            if (not isinstance(owners, tuple) or len(owners) != 2 or owners[0] is None or
                    owners[1] is None):
                raise ValueError("owners must be a (source, destination) tuple of strong owners")
        if request._consumed:
            raise TransferError("already_executed", "transfer request was already executed")
        src, dst = request.source, request.destination
        dev_view = dst if request.direction == "h2d" else src
        device = dev_view.device if dev_view.kind == "cuda" else 0
        ctx = context_for(resources, device)
        request._consumed = True
        threads = gather_threads if gather_threads > 0 else (os.cpu_count() or 8)
        opt = _options(n_buffers=n_buffers, gather_threads=threads, host_stages=0,
                       caller_stream=caller_stream, n_streams=n_streams)
        s, t = src.native(), dst.native()
        rep = N.relx_report()
        err = N.relx_err()
        if N.lib().relx_execute_transfer(ctx._h, request.bound._h, ctypes.byref(s),
                                         ctypes.byref(t), _DIRECTIONS[request.direction],
                                         ctypes.byref(opt), ctypes.byref(rep), ctypes.byref(err)):
            _fail(err)
        r = rep.as_dict()
        # the ring a staged transfer cycled through (none for direct DMA);
        # this library's ring is always page-locked, whatever `pinning`
        retained = (getattr(resources, "_limits", None) or {}).get("retained_bytes")
        request._staging = [] if not r["staging_slots"] else [{
            "policy": pinning, "memory_kind": "pinned", "wire_bytes": r["wire_bytes"],
            "staging_capacity_bytes": r["staging_bytes"], "buffer_count": r["staging_slots"],
            "min_pinned_bytes": min_pinned_bytes,
            "reason": "forced_pinned" if pinning == "pinned" else "retained_pinned_ring",
            "retention_eligible": retained is None or r["staging_bytes"] <= retained,
            "reused": bool(r["staging_reused"])}]
        request.report = r
        return None
    finally:
        request._executing = False
