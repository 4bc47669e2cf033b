"""ctypes driver for oracle/_ref/libreloc_ref.so: the reference's own CPU
libreloc built from its sources (TEST INFRASTRUCTURE ONLY; see Makefile).

Used by tests to cross-check the numpy oracle and by bench.py as the
"reference" CPU baseline. Never imported by the product package.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_ref", "libreloc_ref.so")
_lib = None

KINDS = {"float32": (0, 32), "float16": (0, 16), "bfloat16": (1, 16), "int8": (2, 8),
         "int32": (2, 32), "int64": (2, 64)}


def available():
    return os.path.exists(LIB_PATH)


def lib():
    global _lib
    if _lib is None:
        L = ctypes.CDLL(LIB_PATH)
        vp, cp, sz = ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t
        L.ref_typed_prepare.restype = vp
        L.ref_typed_prepare.argtypes = [cp, sz, ctypes.POINTER(cp), ctypes.POINTER(ctypes.c_int64),
                                        ctypes.c_int, ctypes.POINTER(cp), ctypes.POINTER(ctypes.c_int),
                                        ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int64),
                                        ctypes.POINTER(vp), ctypes.POINTER(sz), ctypes.c_int,
                                        ctypes.c_uint, cp, sz]
        L.ref_typed_result_bytes.restype = ctypes.c_int64
        L.ref_typed_result_bytes.argtypes = [vp]
        L.ref_typed_execute.restype = ctypes.c_int
        L.ref_typed_execute.argtypes = [vp, vp, vp, cp, sz]
        L.ref_typed_free.argtypes = [vp]
        L.ref_layout_prepare.restype = vp
        L.ref_layout_prepare.argtypes = [cp, sz, ctypes.POINTER(cp), ctypes.POINTER(ctypes.c_int64),
                                         ctypes.c_int, ctypes.c_uint, cp, sz]
        L.ref_layout_total_bytes.restype = ctypes.c_int64
        L.ref_layout_total_bytes.argtypes = [vp]
        L.ref_layout_execute.restype = ctypes.c_int
        L.ref_layout_execute.argtypes = [vp, vp, vp]
        L.ref_layout_free.argtypes = [vp]
        L.ref_indexed_decode.restype = ctypes.c_int
        L.ref_indexed_decode.argtypes = [cp, sz, ctypes.POINTER(ctypes.c_int64), cp, sz]
        L.ref_indexed_prepare.restype = vp
        L.ref_indexed_prepare.argtypes = [cp, sz, ctypes.POINTER(cp), ctypes.POINTER(ctypes.c_int64),
                                          ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          ctypes.POINTER(ctypes.c_int64), ctypes.c_int, vp, sz,
                                          ctypes.c_uint, cp, sz]
        _lib = L
    return _lib


def _syms(symbols):
    names = list(symbols)
    arr_n = (ctypes.c_char_p * max(1, len(names)))(*[n.encode() for n in names])
    arr_v = (ctypes.c_int64 * max(1, len(names)))(*[int(symbols[n]) for n in names])
    return arr_n, arr_v, len(names)


class TypedRef:
    """prepare once, execute many (executeHost over every stage)."""

    def __init__(self, blob, symbols, params, threads=1):
        """params: {name: (dtype name, shape list, bytes)}."""
        L = lib()
        sn, sv, ns = _syms(symbols)
        names = list(params)
        np_ = max(1, len(names))
        pn = (ctypes.c_char_p * np_)(*[n.encode() for n in names])
        pk = (ctypes.c_int * np_)(*[KINDS[params[n][0]][0] for n in names])
        pb = (ctypes.c_int * np_)(*[KINDS[params[n][0]][1] for n in names])
        pl = (ctypes.c_int64 * np_)(*[(params[n][1][0] if params[n][1] else -1) for n in names])
        self._keep = [ctypes.create_string_buffer(params[n][2], len(params[n][2])) for n in names]
        pd = (ctypes.c_void_p * np_)(*[ctypes.addressof(b) for b in self._keep])
        psz = (ctypes.c_size_t * np_)(*[len(params[n][2]) for n in names])
        err = ctypes.create_string_buffer(512)
        self.h = L.ref_typed_prepare(blob, len(blob), sn, sv, ns, pn, pk, pb, pl, pd, psz,
                                     len(names), threads, err, 512)
        if not self.h:
            raise RuntimeError(err.value.decode())
        self.result_bytes = L.ref_typed_result_bytes(self.h)

    def execute(self, src, out=None):
        src = np.ascontiguousarray(src)
        if out is None:
            out = np.empty(self.result_bytes, np.uint8)
        err = ctypes.create_string_buffer(512)
        if lib().ref_typed_execute(self.h, src.ctypes.data, out.ctypes.data, err, 512):
            raise RuntimeError(err.value.decode())
        return out

    def __del__(self):
        if getattr(self, "h", None):
            lib().ref_typed_free(self.h)
            self.h = None


class LayoutRef:
    def __init__(self, blob, symbols, threads=1):
        sn, sv, ns = _syms(symbols)
        err = ctypes.create_string_buffer(512)
        self.h = lib().ref_layout_prepare(blob, len(blob), sn, sv, ns, threads, err, 512)
        if not self.h:
            raise RuntimeError(err.value.decode())
        self.total_bytes = lib().ref_layout_total_bytes(self.h)

    def execute(self, src, out=None):
        src = np.ascontiguousarray(src)
        if out is None:
            out = np.empty(self.total_bytes, np.uint8)
        lib().ref_layout_execute(self.h, src.ctypes.data, out.ctypes.data)
        return out

    def __del__(self):
        if getattr(self, "h", None):
            lib().ref_layout_free(self.h)
            self.h = None


def indexed_decode(blob):
    """decodeIndexedPlan: None when valid, else (offset, message)."""
    off = ctypes.c_int64(-1)
    err = ctypes.create_string_buffer(512)
    if lib().ref_indexed_decode(blob, len(blob), ctypes.byref(off), err, 512):
        return off.value, err.value.decode()
    return None


class IndexedRef(TypedRef):
    """decodeIndexedPlan + bindIndexed + the indexed program of
    prepareIndexSelect; execute() runs executeHost's indexed rows over the
    whole table."""

    def __init__(self, blob, symbols, index_dtype, index_extents, index_bytes, threads=1):
        L = lib()
        sn, sv, ns = _syms(symbols)
        kind, bits = KINDS[index_dtype]
        ext = (ctypes.c_int64 * max(1, len(index_extents)))(*[int(e) for e in index_extents])
        self._keep = [ctypes.create_string_buffer(bytes(index_bytes), max(1, len(index_bytes)))]
        err = ctypes.create_string_buffer(512)
        self.h = L.ref_indexed_prepare(blob, len(blob), sn, sv, ns, kind, bits, ext,
                                       len(index_extents), ctypes.addressof(self._keep[0]),
                                       len(index_bytes), threads, err, 512)
        if not self.h:
            raise RuntimeError(err.value.decode())
        self.result_bytes = L.ref_typed_result_bytes(self.h)


HIP_LIB_PATH = os.path.join(HERE, "_ref", "libreloc_ref_hip.so")
_hip = None


def hip_available():
    return os.path.exists(HIP_LIB_PATH)


def hip_lib():
    """libreloc_ref_hip.so: the reference's cpu_reference H2D row (CPU
    transform into pinned ring slots, then hipMemcpyAsync of each slot) on a
    HIP CopyBackend. Loads torch first so one HIP runtime serves both."""
    global _hip
    if _hip is None:
        import torch  # noqa: F401
        lib()  # libreloc_ref.so, which the HIP driver links against
        L = ctypes.CDLL(HIP_LIB_PATH)
        vp, cp, sz = ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t
        L.ref_cpu_h2d_prepare.restype = vp
        L.ref_cpu_h2d_prepare.argtypes = [cp, sz, ctypes.POINTER(cp), ctypes.POINTER(ctypes.c_int64),
                                          ctypes.c_int, ctypes.POINTER(cp), ctypes.POINTER(ctypes.c_int),
                                          ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int64),
                                          ctypes.POINTER(vp), ctypes.POINTER(sz), ctypes.c_int,
                                          ctypes.c_uint, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          cp, sz]
        L.ref_cpu_h2d_result_bytes.restype = ctypes.c_int64
        L.ref_cpu_h2d_result_bytes.argtypes = [vp]
        L.ref_cpu_h2d_execute.restype = ctypes.c_int
        L.ref_cpu_h2d_execute.argtypes = [vp, vp, sz, vp, sz, cp, sz]
        L.ref_cpu_h2d_free.argtypes = [vp]
        _hip = L
    return _hip


class CpuH2dRef:
    """The reference's CPU H2D path end to end: a typed plan through the
    cpu_reference dispatch row (transform on `threads` workers into
    `buffers` pinned slots, each slot's H2D on `queues` streams), a layout
    plan through executeTransfer; `execute` blocks until the result is in
    device memory."""

    def __init__(self, blob, symbols, params=None, threads=8, buffers=2, queues=1, device=0):
        L = hip_lib()
        sn, sv, ns = _syms(symbols)
        params = params or {}
        names = list(params)
        np_ = max(1, len(names))
        pn = (ctypes.c_char_p * np_)(*[n.encode() for n in names])
        pk = (ctypes.c_int * np_)(*[KINDS[params[n][0]][0] for n in names])
        pb = (ctypes.c_int * np_)(*[KINDS[params[n][0]][1] for n in names])
        pl = (ctypes.c_int64 * np_)(*[(params[n][1][0] if params[n][1] else -1) for n in names])
        self._keep = [ctypes.create_string_buffer(params[n][2], len(params[n][2])) for n in names]
        pd = (ctypes.c_void_p * np_)(*[ctypes.addressof(b) for b in self._keep])
        psz = (ctypes.c_size_t * np_)(*[len(params[n][2]) for n in names])
        err = ctypes.create_string_buffer(512)
        self.h = L.ref_cpu_h2d_prepare(blob, len(blob), sn, sv, ns, pn, pk, pb, pl, pd, psz,
                                       len(names), threads, buffers, queues, device, err, 512)
        if not self.h:
            raise RuntimeError(err.value.decode())
        self.result_bytes = L.ref_cpu_h2d_result_bytes(self.h)

    def execute(self, src_ptr, src_bytes, dst_ptr, dst_bytes):
        err = ctypes.create_string_buffer(512)
        if hip_lib().ref_cpu_h2d_execute(self.h, src_ptr, src_bytes, dst_ptr, dst_bytes, err, 512):
            raise RuntimeError(err.value.decode())

    def __del__(self):
        if getattr(self, "h", None):
            hip_lib().ref_cpu_h2d_free(self.h)
            self.h = None


def validate_transfer(blob, symbols, src, dst, direction, source_only=False):
    """The reference's validateTransfer / validateTransferSource on a layout
    plan. Views are (base, capacity, offset, extents, strides, element size,
    kind 'host'|'cuda', device) tuples. Returns ('ok', source span),
    ('error', '<code>: <message>') or ('plan', None) when the plan does not
    decode or bind."""
    L = lib()
    if not hasattr(L, "_vt"):
        f = L.ref_validate_transfer
        i64p = ctypes.POINTER(ctypes.c_int64)
        u64p = ctypes.POINTER(ctypes.c_uint64)
        f.restype = ctypes.c_int
        f.argtypes = ([ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_char_p), i64p,
                       ctypes.c_int] +
                      [u64p, ctypes.c_int, i64p, i64p, ctypes.c_uint32, ctypes.c_int, ctypes.c_int] * 2 +
                      [ctypes.c_int, ctypes.c_int, u64p, ctypes.c_char_p, ctypes.c_size_t])
        L._vt = f
    sn, sv, ns = _syms(symbols)

    def parts(v):
        base, cap, off, ext, strides, es, kind, dev = v
        words = (ctypes.c_uint64 * 3)(base, cap, off)
        e = (ctypes.c_int64 * max(1, len(ext)))(*ext)
        s = (ctypes.c_int64 * max(1, len(strides)))(*strides)
        return [words, len(ext), e, s, es, 1 if kind == "cuda" else 0, dev]

    span = ctypes.c_uint64(0)
    err = ctypes.create_string_buffer(512)
    d = dst if dst is not None else src
    rc = L._vt(blob, len(blob), sn, sv, ns, *parts(src), *parts(d), 1 if direction == "d2h" else 0,
               1 if source_only else 0, ctypes.byref(span), err, 512)
    if rc == 0:
        return "ok", span.value
    if rc == 1:
        return "error", err.value.decode()
    return "plan", None
