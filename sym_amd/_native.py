"""ctypes binding of librelx.so (include/relx.h).

The library is built in-tree by sym_amd/build.py. Importing the product path
without it raises: there is no CPU fallback.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("RELX_LIBRARY", os.path.join(HERE, "librelx.so"))

RELX_MAX_RANK = 8
RELX_MAX_STAGES = 8


class NativeLibraryMissing(RuntimeError):
    pass


class relx_err(ctypes.Structure):
    _fields_ = [("code", ctypes.c_char * 48), ("message", ctypes.c_char * 464),
                ("offset", ctypes.c_int64), ("completion", ctypes.c_int)]


class relx_param(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("kind", ctypes.c_int), ("bits", ctypes.c_int),
                ("rank", ctypes.c_int), ("length", ctypes.c_int64), ("data", ctypes.c_void_p),
                ("nbytes", ctypes.c_size_t)]


_I64R = ctypes.c_int64 * RELX_MAX_RANK


class relx_plan_stage_info(ctypes.Structure):
    _fields_ = [("transform", ctypes.c_int), ("policy", ctypes.c_int), ("in_kind", ctypes.c_int),
                ("in_bits", ctypes.c_int), ("in_signedness", ctypes.c_int),
                ("out_kind", ctypes.c_int), ("out_bits", ctypes.c_int),
                ("out_signedness", ctypes.c_int), ("rank", ctypes.c_int),
                ("axis", ctypes.c_int64), ("has_channel", ctypes.c_int),
                ("scale_kind", ctypes.c_int), ("zero_point_kind", ctypes.c_int)]


class relx_bound_info(ctypes.Structure):
    _fields_ = [("typed", ctypes.c_int), ("rank", ctypes.c_int), ("extents", _I64R),
                ("src_strides", _I64R), ("dst_strides", _I64R), ("pad_lo", _I64R),
                ("pad_hi", _I64R), ("element_size", ctypes.c_int),
                ("total_bytes", ctypes.c_int64), ("source_bytes", ctypes.c_int64),
                ("destination_bytes", ctypes.c_int64), ("parameter_bytes", ctypes.c_int64),
                ("stages", ctypes.c_int), ("bytes_at", ctypes.c_int64 * (RELX_MAX_STAGES + 1)),
                ("source_width", ctypes.c_int), ("result_width", ctypes.c_int),
                ("source_rank", ctypes.c_int), ("source_extents", _I64R),
                ("result_rank", ctypes.c_int), ("result_extents", _I64R),
                ("kernel", ctypes.c_char * 32), ("host_stages_max", ctypes.c_int),
                ("host_stages_auto", ctypes.c_int),
                ("wire_bytes_at", ctypes.c_int64 * (RELX_MAX_STAGES + 1)),
                ("indexed", ctypes.c_int), ("table_rows", ctypes.c_int64),
                ("row_elements", ctypes.c_int64), ("table_bytes", ctypes.c_int64),
                ("index_count", ctypes.c_int64), ("permute_direct", ctypes.c_int),
                ("transpose_tile_q", ctypes.c_int), ("transpose_tile_c", ctypes.c_int),
                ("transpose_row_params", ctypes.c_int)]


class relx_ctx_stats(ctypes.Structure):
    _fields_ = [("pinned_bytes", ctypes.c_int64), ("device_bytes", ctypes.c_int64),
                ("calls", ctypes.c_int64), ("failures", ctypes.c_int64),
                ("quarantined", ctypes.c_int)]


class relx_options(ctypes.Structure):
    _fields_ = [("n_buffers", ctypes.c_int), ("chunk_bytes", ctypes.c_int64),
                ("host_stages", ctypes.c_int), ("gather_threads", ctypes.c_int),
                ("source_pinned", ctypes.c_int), ("caller_stream", ctypes.c_uint64),
                ("no_wait", ctypes.c_int), ("has_caller_stream", ctypes.c_int),
                ("n_streams", ctypes.c_int)]


class relx_report(ctypes.Structure):
    _fields_ = [("implementation", ctypes.c_char * 40), ("source_bytes", ctypes.c_int64),
                ("wire_bytes", ctypes.c_int64), ("destination_bytes", ctypes.c_int64),
                ("parameter_bytes", ctypes.c_int64),
                ("payload_bytes_transferred", ctypes.c_int64), ("chunks", ctypes.c_int64),
                ("kernel_launches", ctypes.c_int64), ("wire_boundary", ctypes.c_int),
                ("direct_dma", ctypes.c_int), ("host_chunk_bytes", ctypes.c_int64),
                ("host_buffers", ctypes.c_int64), ("staging_bytes", ctypes.c_int64),
                ("staging_slots", ctypes.c_int64), ("staging_reused", ctypes.c_int),
                ("copy_streams", ctypes.c_int)]

    def as_dict(self):
        return {f: (getattr(self, f).decode() if f == "implementation" else getattr(self, f))
                for f, _ in self._fields_}


RELX_MAX_VIEW_RANK = 16
_I64V = ctypes.c_int64 * RELX_MAX_VIEW_RANK


class relx_view(ctypes.Structure):
    _fields_ = [("base", ctypes.c_uint64), ("capacity_bytes", ctypes.c_uint64),
                ("offset_bytes", ctypes.c_uint64), ("rank", ctypes.c_int),
                ("extents", _I64V), ("strides", _I64V), ("element_size", ctypes.c_uint32),
                ("kind", ctypes.c_int), ("device", ctypes.c_int)]


class relx_kernel_times(ctypes.Structure):
    _fields_ = [("calls", ctypes.c_int64), ("chunks", ctypes.c_int64),
                ("launches", ctypes.c_int64), ("ms", ctypes.c_double)]


# every entry point include/relx.h declares, with its ctypes signature
_VP, _SZ, _I, _I64, _U64 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int64, ctypes.c_uint64
_E = ctypes.POINTER(relx_err)
SIGNATURES = {
    "relx_version": (ctypes.c_char_p, []),
    "relx_wire_version": (_I, [ctypes.c_char_p, _SZ]),
    "relx_plan_load": (_I, [ctypes.c_char_p, _SZ, ctypes.POINTER(_VP), _E]),
    "relx_plan_is_typed": (_I, [_VP]),
    "relx_plan_version": (_I, [_VP]),
    "relx_plan_symbol_count": (_I, [_VP]),
    "relx_plan_symbol": (ctypes.c_char_p, [_VP, _I]),
    "relx_plan_free": (None, [_VP]),
    "relx_plan_stage_count": (_I, [_VP]),
    "relx_plan_stage": (_I, [_VP, _I, ctypes.POINTER(relx_plan_stage_info)]),
    "relx_plan_fill_count": (_I, [_VP]),
    "relx_plan_parameter": (_I, [_VP, _I, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_I),
                                 ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_I),
                                 ctypes.POINTER(_I)]),
    "relx_bind": (_I, [_VP, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_I64), _I,
                       ctypes.POINTER(relx_param), _I, ctypes.POINTER(_VP), _E]),
    "relx_bind_indexed": (_I, [_VP, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_I64), _I,
                               _I, _I, ctypes.POINTER(_I64), _I, _VP, _SZ, ctypes.POINTER(_VP),
                               _E]),
    "relx_bound_free": (None, [_VP]),
    "relx_bound_query": (_I, [_VP, ctypes.POINTER(relx_bound_info)]),
    "relx_ctx_create": (_I, [_I, _I64, ctypes.POINTER(_VP), _E]),
    "relx_ctx_close": (_I, [_VP, _E]),
    "relx_ctx_stats_get": (_I, [_VP, ctypes.POINTER(relx_ctx_stats)]),
    "relx_execute_h2d": (_I, [_VP, _VP, _VP, _SZ, _VP, _SZ, ctypes.POINTER(relx_options),
                              ctypes.POINTER(relx_report), _E]),
    "relx_execute_h2d_static": (_I, [_VP, _VP, _VP, _SZ, _VP, _SZ, ctypes.POINTER(relx_options),
                                     ctypes.POINTER(relx_report), _E]),
    "relx_view_span_bytes": (_I, [ctypes.POINTER(relx_view), ctypes.c_char_p,
                                  ctypes.POINTER(_U64), _E]),
    "relx_validate_transfer_source": (_I, [_VP, ctypes.POINTER(relx_view), _I,
                                           ctypes.POINTER(_U64), _E]),
    "relx_validate_transfer": (_I, [_VP, ctypes.POINTER(relx_view), ctypes.POINTER(relx_view), _I,
                                    ctypes.POINTER(_U64), ctypes.POINTER(_U64), _E]),
    "relx_execute_transfer": (_I, [_VP, _VP, ctypes.POINTER(relx_view), ctypes.POINTER(relx_view),
                                   _I, ctypes.POINTER(relx_options), ctypes.POINTER(relx_report),
                                   _E]),
    "relx_pointer_device": (_I, [_VP, ctypes.POINTER(_I), _E]),
    "relx_execute_group_h2d": (_I, [_VP, _I, ctypes.POINTER(_VP), ctypes.POINTER(_VP),
                                    ctypes.POINTER(_SZ), ctypes.POINTER(_VP), ctypes.POINTER(_SZ),
                                    ctypes.POINTER(relx_options), ctypes.POINTER(relx_report),
                                    ctypes.POINTER(relx_report), _E]),
    "relx_relayout_device": (_I, [_VP, _VP, _I, _VP, _VP, _U64, _E]),
    "relx_submit_group_h2d": (_I, [_VP, _I, ctypes.POINTER(_VP), ctypes.POINTER(_VP),
                                   ctypes.POINTER(_SZ), ctypes.POINTER(_VP), ctypes.POINTER(_SZ),
                                   ctypes.POINTER(relx_options), ctypes.POINTER(relx_report),
                                   ctypes.POINTER(relx_report), ctypes.POINTER(_VP), _E]),
    "relx_completion_query": (_I, [_VP, ctypes.POINTER(_I), _E]),
    "relx_completion_wait": (_I, [_VP, _E]),
    "relx_completion_wait_stream": (_I, [_VP, _U64, _E]),
    "relx_completion_free": (None, [_VP]),
    "relx_execute_d2h": (_I, [_VP, _VP, _VP, _SZ, _VP, _SZ, ctypes.POINTER(relx_options),
                              ctypes.POINTER(relx_report), _E]),
    "relx_index_select_device": (_I, [_VP, _VP, _VP, _SZ, _VP, _SZ, _U64, _E]),
    "relx_host_stage": (_I, [_VP, _I, _VP, _VP, _I, _E]),
    "relx_verify_launches": (_I, [_VP, _I, ctypes.c_int64, ctypes.POINTER(ctypes.c_int64), _E]),
    "relx_ctx_synchronize": (_I, [_VP, _E]),
    "relx_ctx_time_kernels": (_I, [_VP, _I, _E]),
    "relx_ctx_kernel_times": (_I, [_VP, ctypes.POINTER(relx_kernel_times), _E]),
    "relx_host_alloc": (_I, [_SZ, ctypes.POINTER(_VP), _E]),
    "relx_host_free": (_I, [_VP]),
    "relx_measure_h2d": (ctypes.c_double, [_I, _SZ, _I, _I]),
    "relx_measure_d2h": (ctypes.c_double, [_I, _SZ, _I, _I]),
    "relx_measure_copy": (ctypes.c_double, [_I, _SZ, _I, _I]),
}

_lib = None


def lib():
    """The loaded library; raises NativeLibraryMissing when it is not built."""
    global _lib
    if _lib is None:
        # One HIP runtime per process: when torch is present its bundled
        # libamdhip64.so.7 is loaded first and satisfies librelx's dependency.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        if not os.path.exists(LIB_PATH):
            raise NativeLibraryMissing(
                "librelx.so is not built (%s); run `python -m sym_amd.build`" % LIB_PATH)
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


class RelxError(RuntimeError):
    """A librelx failure: `code` is the stable reason code."""

    def __init__(self, code, message, offset=-1, completion=0):
        super().__init__("%s: %s" % (code, message))
        self.code = code
        self.detail = message
        self.offset = offset
        self.completion = {0: "not_launched", 1: "complete", 2: "unknown"}.get(completion, "unknown")


def check(rc, err):
    if rc != 0:
        raise RelxError(err.code.decode(errors="replace"), err.message.decode(errors="replace"),
                        err.offset, err.completion)
