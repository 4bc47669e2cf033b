"""Python surface over librelx, mirroring the reference's `pyreloc` module
(libreloc/python/PyReloc.cpp:596-987, PyDispatch.cpp:517-901,
PyTransfer.cpp:312-461) for the H2D plan-execution path.

Names and argument meaning follow the reference: `wire_version`,
`load_plan`, `load_typed_plan`, `load_indexed_plan`, `bind`, `bind_typed`,
`bind_indexed`, `bind_indexed_from_pointer`, and errors raised as
`DecodeError`, `BindError` or `TransferError("<code>: <detail>")`. Buffers
cross as (pointer, nbytes) pairs; ctypes releases the GIL during each call.
"""
import ctypes

from . import _native as N
from ._native import RelxError

DTYPE_KINDS = {
    "float32": (0, 32), "float16": (0, 16), "float64": (0, 64), "bfloat16": (1, 16),
    "int8": (2, 8), "int16": (2, 16), "int32": (2, 32), "int64": (2, 64), "uint8": (2, 8),
}


class DecodeError(ValueError):
    def __init__(self, message, offset=-1):
        super().__init__(message)
        self.offset = offset


class BindError(ValueError):
    pass


class TransferError(RuntimeError):
    def __init__(self, code, detail, completion="not_launched"):
        super().__init__("%s: %s" % (code, detail))
        self.code = code
        self.detail = detail
        self.completion = completion


_BIND_CODES = {"bind_error", "unsupported_stage", "invalid_parameter", "unsupported_layout",
               "pads_not_settled", "fill_crosses_channel_stage", "mixed_fills_unsupported",
               "fill_mismatch", "invalid_boundary"}


def _raise(err):
    code = err.code.decode(errors="replace")
    msg = err.message.decode(errors="replace")
    if code == "decode_error":
        raise DecodeError("%s (at byte %d)" % (msg, err.offset), err.offset)
    if code in _BIND_CODES:
        raise BindError("%s: %s" % (code, msg) if code != "bind_error" else msg)
    raise TransferError(code, msg, {0: "not_launched", 1: "complete", 2: "unknown"}.get(
        err.completion, "unknown"))


def version():
    return N.lib().relx_version().decode()


def wire_version(blob):
    """Wire version of a plan blob (bytes 4..8), or None if it is not a plan."""
    blob = bytes(blob)
    v = N.lib().relx_wire_version(blob, len(blob))
    return None if v < 0 else v


class Plan:
    """A decoded, immutable plan (v0 layout or v1 typed)."""

    def __init__(self, blob):
        self.blob = bytes(blob)
        err = N.relx_err()
        h = ctypes.c_void_p()
        if N.lib().relx_plan_load(self.blob, len(self.blob), ctypes.byref(h), ctypes.byref(err)):
            _raise(err)
        self._h = h
        self._free = N.lib().relx_plan_free  # kept: module globals may be gone at exit

    @property
    def typed(self):
        return bool(N.lib().relx_plan_is_typed(self._h))

    @property
    def symbols(self):
        L = N.lib()
        return [L.relx_plan_symbol(self._h, i).decode() for i in range(L.relx_plan_symbol_count(self._h))]

    @property
    def num_stages(self):
        return N.lib().relx_plan_stage_count(self._h)

    @property
    def stages(self):
        """Decoded value stages (reference TypedPlanHandle.stages,
        libreloc/python/PyReloc.cpp:241-259): transform, policy, input and
        output dtypes with signedness, rank, axis and channel presence."""
        out = []
        for i in range(self.num_stages):
            s = N.relx_plan_stage_info()
            N.lib().relx_plan_stage(self._h, i, ctypes.byref(s))
            out.append({"transform": _TRANSFORM_NAMES[s.transform],
                        "policy": _POLICY_NAMES.get(s.policy, "unknown"),
                        "input": _DTYPE_NAMES.get((s.in_kind, s.in_bits), "unknown"),
                        "input_signedness": _SIGNEDNESS[s.in_signedness],
                        "output": _DTYPE_NAMES.get((s.out_kind, s.out_bits), "unknown"),
                        "output_signedness": _SIGNEDNESS[s.out_signedness],
                        "rank": s.rank, "axis": s.axis, "has_channel": bool(s.has_channel),
                        "scale": _PARAM_KINDS[s.scale_kind],
                        "zero_point": _PARAM_KINDS[s.zero_point_kind]})
        return out

    @property
    def fills(self):
        return N.lib().relx_plan_fill_count(self._h)

    @property
    def parameters(self):
        """Runtime parameter declarations in first-declaration order
        (reference TypedPlanHandle.parameters, PyReloc.cpp:263-288)."""
        L = N.lib()
        out = []
        for i in range(L.relx_plan_parameter(self._h, -1, None, None, None, None, None, None)):
            name = ctypes.c_char_p()
            kind, bits, rank, stage, role = (ctypes.c_int() for _ in range(5))
            L.relx_plan_parameter(self._h, i, ctypes.byref(name), ctypes.byref(kind),
                                  ctypes.byref(bits), ctypes.byref(rank), ctypes.byref(stage),
                                  ctypes.byref(role))
            out.append({"name": name.value.decode(),
                        "dtype": _DTYPE_NAMES.get((kind.value, bits.value), "unknown"),
                        "rank": rank.value, "stage": stage.value,
                        "role": "scale" if role.value == 0 else "zero_point"})
        return out

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._free(h)
            self._h = None


def load_plan(blob):
    """Decode a layout (v0) plan; a v1 blob is rejected like the reference's
    decodePlan does (unsupported wire format version at byte 4)."""
    if wire_version(blob) not in (0, None):
        raise DecodeError("unsupported wire format version (at byte 4)", 4)
    return Plan(blob)


def load_typed_plan(blob):
    """Decode a typed (v1) plan; a v0 blob is rejected at byte 4."""
    if wire_version(blob) not in (1, None):
        raise DecodeError("unsupported wire format version (at byte 4)", 4)
    return Plan(blob)


def load_indexed_plan(blob):
    """Decode an indexed (v2) plan (reference load_indexed_plan,
    libreloc/python/PyReloc.cpp:863-875); a v0 or v1 blob is rejected at
    byte 4."""
    if wire_version(blob) not in (2, None):
        raise DecodeError("unsupported wire format version (at byte 4)", 4)
    return IndexedPlan(blob)


_DTYPE_NAMES = {(0, 32): "float32", (0, 16): "float16", (0, 64): "float64", (1, 16): "bfloat16",
                (2, 8): "int8", (2, 16): "int16", (2, 32): "int32", (2, 64): "int64"}
_POLICY_NAMES = {0: "ieee_rne", 1: "exact", 2: "symmetric_rne", 3: "affine"}
_TRANSFORM_NAMES = {0: "cast", 1: "quantize", 2: "dequantize"}
_SIGNEDNESS = {0: "signless", 1: "signed", 2: "unsigned"}
_PARAM_KINDS = {0: None, 1: "inline", 2: "binding"}


def _indexed_metadata(blob):
    """Descriptor shapes, dtypes, axis and policy of a decoded v2 blob, as
    the reference's IndexedPlanHandle.metadata (PyReloc.cpp:177-238):
    expressions become nested lists (['const', v], ['symbol', name],
    ['add'|'mul', lhs, rhs], ['floordiv'|'mod', lhs, constant]; a
    subtraction reads as lhs + (-1 * rhs))."""
    import struct
    off = [8]

    def u32():
        v = struct.unpack_from("<I", blob, off[0])[0]
        off[0] += 4
        return v

    def u8():
        v = blob[off[0]]
        off[0] += 1
        return v

    symbols = []
    for _ in range(u32()):
        n = u32()
        symbols.append(blob[off[0]:off[0] + n].decode())
        off[0] += n

    def expr():
        stack = []
        for _ in range(u32()):
            op = u8()
            if op == 1:
                stack.append(["const", struct.unpack_from("<q", blob, off[0])[0]])
                off[0] += 8
            elif op == 0:
                stack.append(["symbol", symbols[u32()]])
            else:
                rhs, lhs = stack.pop(), stack.pop()
                if op == 2:
                    stack.append(["add", lhs, rhs])
                elif op == 3:
                    stack.append(["add", lhs, ["mul", ["const", -1], rhs]])
                elif op == 4:
                    stack.append(["mul", lhs, rhs])
                else:
                    if rhs[0] != "const":
                        raise ValueError("indexed metadata requires constant divisors")
                    stack.append(["floordiv" if op == 5 else "mod", lhs, rhs[1]])
        return stack[-1]

    def desc():
        shape = [expr() for _ in range(u32())]
        for _ in range(u32()):
            expr()
        expr()
        kind = u8()
        bits = u32()
        return {"shape": shape, "dtype": _DTYPE_NAMES.get((kind, bits), "unknown")}

    out = {"source": desc(), "indices": desc(), "result": desc()}
    out["axis"] = u32()
    out["policy"] = _POLICY_NAMES.get(u8(), "unknown")
    return out


class IndexedPlan(Plan):
    """A decoded indexed plan (reference IndexedPlanHandle,
    libreloc/python/PyReloc.cpp:852-854)."""

    @property
    def metadata(self):
        return _indexed_metadata(self.blob)


class Bound:
    """A bound plan with its prepared device program."""

    def __init__(self, plan, symbols, parameters=None):
        self.plan = plan
        names = list(symbols)
        n = len(names)
        sn = (ctypes.c_char_p * max(1, n))(*[s.encode() for s in names])
        sv = (ctypes.c_int64 * max(1, n))(*[int(symbols[s]) for s in names])
        params = parameters or {}
        keep = []
        arr = (N.relx_param * max(1, len(params)))()
        for i, (name, value) in enumerate(params.items()):
            dtype, extents, data = value
            kind, bits = DTYPE_KINDS[dtype]
            data = bytes(data)
            buf = ctypes.create_string_buffer(data, len(data))
            keep += [buf, name.encode()]
            arr[i] = N.relx_param(keep[-1], kind, bits, len(extents),
                                  int(extents[0]) if extents else 1,
                                  ctypes.cast(buf, ctypes.c_void_p), len(data))
        err = N.relx_err()
        h = ctypes.c_void_p()
        if N.lib().relx_bind(plan._h, sn, sv, n, arr, len(params), ctypes.byref(h), ctypes.byref(err)):
            _raise(err)
        self._adopt(h)

    def _adopt(self, h):
        self._h = h
        self._free = N.lib().relx_bound_free  # kept: module globals may be gone at exit
        info = N.relx_bound_info()
        N.lib().relx_bound_query(h, ctypes.byref(info))
        self.info = info

    @property
    def typed(self):
        return bool(self.info.typed)

    @property
    def indexed(self):
        return bool(self.info.indexed)

    @property
    def extents(self):
        return list(self.info.extents[:self.info.rank])

    @property
    def src_strides(self):
        return list(self.info.src_strides[:self.info.rank])

    @property
    def dst_strides(self):
        return list(self.info.dst_strides[:self.info.rank])

    @property
    def element_size(self):
        return self.info.element_size

    @property
    def total_bytes(self):
        return self.info.total_bytes

    @property
    def source_bytes(self):
        return self.info.source_bytes

    @property
    def destination_bytes(self):
        return self.info.destination_bytes

    @property
    def parameter_bytes(self):
        return self.info.parameter_bytes

    @property
    def stage_count(self):
        return self.info.stages

    @property
    def kernel(self):
        return self.info.kernel.decode()

    @property
    def permute_direct(self):
        """True when every whole-box launch of a permute program runs the
        direct body (shift indexing, parameters by channel coordinate)."""
        return bool(self.info.permute_direct)

    @property
    def transpose_tile_q(self):
        """q width of a transpose program's tiles (128 for one-byte sources
        whose source-contiguous extent allows it, else 64; 0 for other
        kernel families)."""
        return self.info.transpose_tile_q

    @property
    def transpose_tile_c(self):
        """c width of a transpose program's tiles (128 for a one-byte source
        with two- or four-byte results whose q and c extents allow it, else
        64; 0 for other kernel families)."""
        return self.info.transpose_tile_c

    @property
    def transpose_row_params(self):
        """True when every tile launch of a transpose program indexes its
        dequantize parameters by destination row."""
        return bool(self.info.transpose_row_params)

    def bytes_at(self, boundary):
        return self.info.bytes_at[boundary]

    def footprints(self):
        return [self.info.bytes_at[k] for k in range(self.info.stages + 1)]

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._free(h)
            self._h = None


class IndexedBound(Bound):
    """A bound indexed plan (reference IndexedBoundPlan,
    libreloc/python/PyReloc.cpp:855-862): `source_extents` is the table's
    shape, `result_extents` the selected rows', `indices` the bound,
    range-checked row indices (a copy). The device program relocates the
    selected rows (identity) through the plan's cast."""

    def __init__(self, plan, symbols, dtype, extents, data):
        if dtype not in DTYPE_KINDS:
            raise ValueError("unsupported index dtype %r" % (dtype,))
        self.plan = plan
        kind, bits = DTYPE_KINDS[dtype]
        names = list(symbols)
        n = len(names)
        sn = (ctypes.c_char_p * max(1, n))(*[s.encode() for s in names])
        sv = (ctypes.c_int64 * max(1, n))(*[int(symbols[s]) for s in names])
        ext = [int(e) for e in extents]
        ea = (ctypes.c_int64 * max(1, len(ext)))(*ext)
        data = bytes(data)
        buf = ctypes.create_string_buffer(data, max(1, len(data)))
        err = N.relx_err()
        h = ctypes.c_void_p()
        if N.lib().relx_bind_indexed(plan._h, sn, sv, n, kind, bits, ea, len(ext),
                                     ctypes.cast(buf, ctypes.c_void_p), len(data),
                                     ctypes.byref(h), ctypes.byref(err)):
            _raise(err)
        self._adopt(h)
        self._index_bytes = data
        self._index_bits = bits

    @property
    def source_extents(self):
        i = self.info
        return [i.table_rows] + list(i.result_extents[1:i.result_rank])

    @property
    def result_extents(self):
        return list(self.info.result_extents[:self.info.result_rank])

    @property
    def row_elements(self):
        return self.info.row_elements

    @property
    def table_bytes(self):
        return self.info.table_bytes

    @property
    def indices(self):
        import array
        a = array.array("q" if self._index_bits == 64 else "i")
        a.frombytes(self._index_bytes)
        return list(a)


def bind(plan, symbols):
    """bind (Bind.cpp:176-384) for a layout plan."""
    return Bound(plan, symbols)


def bind_indexed(plan, symbols, indices):
    """bindIndexed (Bind.cpp:701-819): `indices` is the (dtype, extents,
    little-endian bytes) operand, as the reference's pyreloc.bind_indexed."""
    if not isinstance(indices, tuple) or len(indices) != 3:
        raise ValueError("indices must be a (dtype, extents, bytes) tuple")
    dtype, extents, data = indices
    return IndexedBound(plan, symbols, dtype, extents, data)


def bind_indexed_from_pointer(plan, symbols, dtype, extents, pointer, nbytes):
    """bind_indexed over a caller-owned little-endian index buffer at
    `pointer` (reference bind_indexed_from_pointer, PyReloc.cpp:894-919);
    the buffer is read during this call only."""
    if not pointer and nbytes:
        raise ValueError("index pointer must not be null")
    data = ctypes.string_at(pointer, int(nbytes)) if nbytes else b""
    return IndexedBound(plan, symbols, dtype, extents, data)


def bind_typed(plan, symbols, parameters):
    """bindTyped (Bind.cpp:494-699): parameters are {name: (dtype, extents,
    little-endian bytes)} exactly as the reference's pyreloc.bind_typed."""
    return Bound(plan, symbols, parameters)


def _options(n_buffers=0, chunk_bytes=0, host_stages=-1, gather_threads=0, source_pinned=-1,
             caller_stream=None, no_wait=False, n_streams=0):
    """Per-call options. `caller_stream` is a hipStream_t handle the call is
    ordered after (0 is the legacy null stream, torch's default stream);
    None means no producer stream, as the reference's caller_stream=None
    (libreloc/python/PyDispatch.cpp:199-202). `n_streams`: 1 runs the call
    on one copy stream; 0 (default) or more uses the context's two."""
    has = caller_stream is not None
    return N.relx_options(int(n_buffers), int(chunk_bytes), int(host_stages), int(gather_threads),
                          int(source_pinned), int(caller_stream) if has else 0,
                          1 if no_wait else 0, 1 if has else 0, int(n_streams))


class Context:
    """A retained per-device execution context (streams, pinned ring, device
    wire scratch): the role of the reference's TransferResources /
    dispatch::Resources owners. `max_retained_bytes` bounds the ring and
    wire arena kept once the context's calls have completed (None: no
    bound; 0 keeps none)."""

    def __init__(self, device=0, max_retained_bytes=None):
        if max_retained_bytes is not None and int(max_retained_bytes) < 0:
            raise ValueError("max_retained_bytes must be >= 0")
        limit = -1 if max_retained_bytes is None else min(int(max_retained_bytes), (1 << 63) - 1)
        err = N.relx_err()
        h = ctypes.c_void_p()
        if N.lib().relx_ctx_create(int(device), limit, ctypes.byref(h), ctypes.byref(err)):
            _raise(err)
        self._h = h
        self.device = device

    def execute_h2d(self, bound, src_ptr, src_nbytes, dst_ptr, dst_nbytes, **options):
        """Run one bound plan host -> device; returns the report dict."""
        rep = N.relx_report()
        err = N.relx_err()
        opt = _options(**options)
        if N.lib().relx_execute_h2d(self._h, bound._h, src_ptr, src_nbytes, dst_ptr, dst_nbytes,
                                    ctypes.byref(opt), ctypes.byref(rep), ctypes.byref(err)):
            _raise(err)
        return rep.as_dict()

    def execute_h2d_static(self, bound, src_ptr, src_nbytes, dst_ptr, dst_nbytes, **options):
        """The allocation-free upload (relx_execute_h2d_static): a page-locked
        source, the wire staged in the library's static device scratch."""
        rep = N.relx_report()
        err = N.relx_err()
        opt = _options(**options)
        if N.lib().relx_execute_h2d_static(self._h, bound._h, src_ptr, src_nbytes, dst_ptr,
                                           dst_nbytes, ctypes.byref(opt), ctypes.byref(rep),
                                           ctypes.byref(err)):
            _raise(err)
        return rep.as_dict()

    def execute_group_h2d(self, bounds, srcs, dsts, **options):
        """srcs/dsts: lists of (pointer, nbytes). Returns (reports, total)."""
        n = len(bounds)
        bh = (ctypes.c_void_p * n)(*[b._h.value for b in bounds])
        sp = (ctypes.c_void_p * n)(*[s[0] for s in srcs])
        sb = (ctypes.c_size_t * n)(*[s[1] for s in srcs])
        dp = (ctypes.c_void_p * n)(*[d[0] for d in dsts])
        db = (ctypes.c_size_t * n)(*[d[1] for d in dsts])
        reps = (N.relx_report * n)()
        total = N.relx_report()
        err = N.relx_err()
        opt = _options(**options)
        if N.lib().relx_execute_group_h2d(self._h, n, bh, sp, sb, dp, db, ctypes.byref(opt), reps,
                                          ctypes.byref(total), ctypes.byref(err)):
            _raise(err)
        return [r.as_dict() for r in reps], total.as_dict()

    def execute_d2h(self, bound, src_ptr, src_nbytes, dst_ptr, dst_nbytes, **options):
        """Run one bound plan device -> host (every stage on the device);
        `source_pinned` describes the host destination here."""
        rep = N.relx_report()
        err = N.relx_err()
        options.setdefault("host_stages", 0)
        opt = _options(**options)
        if N.lib().relx_execute_d2h(self._h, bound._h, src_ptr, src_nbytes, dst_ptr, dst_nbytes,
                                    ctypes.byref(opt), ctypes.byref(rep), ctypes.byref(err)):
            _raise(err)
        return rep.as_dict()

    def submit_group_h2d(self, bounds, srcs, dsts, owners=None, **options):
        """Enqueue a group without waiting; returns a Completion. `owners`
        are kept alive until the completion is waited for or closed."""
        n = len(bounds)
        bh = (ctypes.c_void_p * n)(*[b._h.value for b in bounds])
        sp = (ctypes.c_void_p * n)(*[s[0] for s in srcs])
        sb = (ctypes.c_size_t * n)(*[s[1] for s in srcs])
        dp = (ctypes.c_void_p * n)(*[d[0] for d in dsts])
        db = (ctypes.c_size_t * n)(*[d[1] for d in dsts])
        reps = (N.relx_report * n)()
        total = N.relx_report()
        err = N.relx_err()
        h = ctypes.c_void_p()
        opt = _options(**options)
        if N.lib().relx_submit_group_h2d(self._h, n, bh, sp, sb, dp, db, ctypes.byref(opt), reps,
                                         ctypes.byref(total), ctypes.byref(h), ctypes.byref(err)):
            _raise(err)
        return Completion(h, [r.as_dict() for r in reps], total.as_dict(), (bounds, owners))

    def index_select_device(self, bound, table_ptr, table_nbytes, dst_ptr, dst_nbytes, stream=0):
        """Gather an indexed plan's selected rows from a device-resident
        table into `dst`, cast fused (async on `stream`, a hipStream_t
        handle; 0 is the legacy null stream, torch's default stream)."""
        err = N.relx_err()
        if N.lib().relx_index_select_device(self._h, bound._h, table_ptr, table_nbytes, dst_ptr,
                                            dst_nbytes, int(stream or 0), ctypes.byref(err)):
            _raise(err)

    def relayout_device(self, bound, wire_ptr, dst_ptr, wire_boundary=0, stream=0):
        """Launch the device relayout on a device-resident wire (async on
        `stream`, a hipStream_t handle; 0 is the legacy null stream, torch's
        default stream). A channel outside the parameters is reported by the
        next synchronize()."""
        err = N.relx_err()
        if N.lib().relx_relayout_device(self._h, bound._h, int(wire_boundary), wire_ptr, dst_ptr,
                                        int(stream or 0), ctypes.byref(err)):
            _raise(err)

    def synchronize(self):
        err = N.relx_err()
        if N.lib().relx_ctx_synchronize(self._h, ctypes.byref(err)):
            _raise(err)

    def time_kernels(self, enable=True):
        """Bracket each chunk's relayout launches of later blocking uploads
        with timing events (resets the sums)."""
        err = N.relx_err()
        if N.lib().relx_ctx_time_kernels(self._h, 1 if enable else 0, ctypes.byref(err)):
            _raise(err)

    def kernel_times(self):
        """{calls, chunks, launches, ms} summed over the timed uploads."""
        t = N.relx_kernel_times()
        err = N.relx_err()
        if N.lib().relx_ctx_kernel_times(self._h, ctypes.byref(t), ctypes.byref(err)):
            _raise(err)
        return {f: getattr(t, f) for f, _ in t._fields_}

    def stats(self):
        s = N.relx_ctx_stats()
        N.lib().relx_ctx_stats_get(self._h, ctypes.byref(s))
        return {f: getattr(s, f) for f, _ in s._fields_}

    def close(self):
        h = getattr(self, "_h", None)
        if h:
            err = N.relx_err()
            self._h = None
            if N.lib().relx_ctx_close(h, ctypes.byref(err)):
                _raise(err)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
        return False

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Completion:
    """An enqueued call (reference dispatch::Completion): wait(), query(),
    wait_stream(stream); closing or dropping it waits for the work first.
    Holds the plans and buffers it was given until then."""

    def __init__(self, handle, reports, total, keep):
        self._h = handle
        self._free = N.lib().relx_completion_free  # kept: module globals may be gone at exit
        self.reports = reports
        self.total = total
        self._keep = keep

    def _call(self, name, *args):
        if not self._h:
            raise TransferError("resources_closed", "completion is closed")
        err = N.relx_err()
        if getattr(N.lib(), name)(self._h, *args, ctypes.byref(err)):
            _raise(err)

    def wait(self):
        self._call("relx_completion_wait")

    def query(self):
        done = ctypes.c_int(0)
        self._call("relx_completion_query", ctypes.byref(done))
        return bool(done.value)

    def wait_stream(self, stream):
        self._call("relx_completion_wait_stream", int(stream))

    def close(self):
        h = getattr(self, "_h", None)
        if h:
            self._free(h)
            self._h = None
            self._keep = None

    def __del__(self):
        self.close()


def verify_launches(bound, wire_boundary=0, chunk_bytes=0):
    """Check on the host every kernel launch the executor would make for
    `bound` (wire at `wire_boundary`, chunks of `chunk_bytes`); returns the
    number of launches checked, raises TransferError on a violation."""
    err = N.relx_err()
    n = ctypes.c_int64(0)
    if N.lib().relx_verify_launches(bound._h, int(wire_boundary), int(chunk_bytes),
                                    ctypes.byref(n), ctypes.byref(err)):
        _raise(err)
    return n.value


def host_stage(bound, host_stages, src_ptr, wire_ptr, threads=8):
    err = N.relx_err()
    if N.lib().relx_host_stage(bound._h, int(host_stages), src_ptr, wire_ptr, int(threads),
                               ctypes.byref(err)):
        _raise(err)


def measure_h2d(device=0, nbytes=256 << 20, iters=20, rounds=3):
    """Pinned H2D ceiling in GB/s (bench/rtrack/multigpu_h2d.cu:46-91 restated)."""
    return N.lib().relx_measure_h2d(int(device), int(nbytes), int(iters), int(rounds))


def measure_copy(device=0, nbytes=256 << 20, iters=20, rounds=3):
    """HBM copy ceiling in GB/s (read + written bytes) of a 16-byte vector copy
    of `nbytes`, over buffers rotated past the Infinity Cache."""
    return N.lib().relx_measure_copy(int(device), int(nbytes), int(iters), int(rounds))


def measure_d2h(device=0, nbytes=256 << 20, iters=20, rounds=3):
    """Pinned D2H ceiling in GB/s (the same measurement, device to host)."""
    return N.lib().relx_measure_d2h(int(device), int(nbytes), int(iters), int(rounds))


# The layout transfer API (sym_amd.transfer) and the typed dispatch API
# (prepare_dispatch / execute_dispatch / groups, sym_amd.dispatch) are
# re-exported here under pyreloc's names. They are looked up on first use
# (module __getattr__), so any of the three modules can be imported first:
# transfer and dispatch import this module themselves.
_REEXPORTS = {
    "transfer": ("BufferView", "DispatchResources", "TransferRequest", "TransferResourceCache",
                 "cuda_enabled", "cuda_pointer_device", "execute_transfer", "make_transfer",
                 "validate_transfer_source"),
    "dispatch": ("Calibration", "DispatchCompletion", "DispatchRequest", "DispatchTemplate",
                 "GatherPool", "GroupRequest", "IndexSelectProgram", "Resources",
                 "execute_dispatch", "execute_dispatch_group", "load_calibration",
                 "prepare_dispatch", "prepare_dispatch_from_template", "prepare_dispatch_group",
                 "prepare_dispatch_template", "prepare_index_select_program", "query_capability",
                 "select_dispatch", "submit_dispatch_group"),
}
_REEXPORTED = {name: mod for mod, names in _REEXPORTS.items() for name in names}


def __getattr__(name):
    mod = _REEXPORTED.get(name)
    if mod is None:
        raise AttributeError("module %r has no attribute %r" % (__name__, name))
    import importlib
    value = getattr(importlib.import_module("." + mod, __package__), name)
    globals()[name] = value
    return value


def __dir__():
    return sorted(set(globals()) | set(_REEXPORTED))
