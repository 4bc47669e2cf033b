"""The layout-transfer surface on the CPU: BufferView's checked span,
validate_transfer_source and make_transfer give the reference's reason
codes (its TransferTest cases, libreloc/test/TransferTest.cpp:106-425), agree
with the reference's own validateTransfer (oracle/_ref) on random views,
and the resource caches behave as the reference's (construction touches no
GPU, stats, close, context manager, no pickling, process check). Nothing
here launches GPU work."""
import pickle

import numpy as np
import pytest

from oracle import ref
from sym_amd import encoder as EN
from sym_amd import pyreloc as P
from sym_amd import workloads as W

HOST, CUDA = "host", "cuda"


def transpose_plan():
    """[4,6] f32 -> transpose -> [6,4] (the reference test's transposePlan)."""
    return EN.encode([4, 6], "float32", [EN.Transpose((1, 0))]).blob


def bound(blob, syms=None):
    return P.bind(P.load_plan(blob), syms or {})


def view(base, cap, off, ext, strides, es, kind=HOST, dev=-1):
    return P.BufferView(base, cap, off, ext, strides, es, kind, dev)


SRC_BASE, DST_BASE = 1 << 20, 1 << 30  # addresses only: nothing is dereferenced


def code_of(fn):
    with pytest.raises(P.TransferError) as e:
        fn()
    return e.value.code


def test_transpose_plan_validates_and_reports_spans():
    b = bound(transpose_plan())
    src = view(SRC_BASE, 96, 0, [4, 6], [6, 1], 4)
    dst = view(DST_BASE, 96, 0, [6, 4], [4, 1], 4, CUDA, 0)
    assert P.validate_transfer_source(b, src, "h2d") == 96
    req = P.make_transfer(b, src, dst, "h2d")
    assert (req.direction, req.source_span_bytes, req.destination_bytes) == ("h2d", 96, 96)
    assert not req.consumed and req.staging == []
    assert req.source is src and req.destination is dst


def test_unsupported_views_are_rejected_with_stable_codes():
    """TransferTest.cpp:168-219, case by case."""
    b = bound(transpose_plan())
    dst = view(DST_BASE, 96, 0, [6, 4], [4, 1], 4)

    def run(src, d=dst, direction="h2d"):
        return code_of(lambda: P.make_transfer(b, src, d, direction))

    assert run(view(SRC_BASE, 96, 0, [4, 6], [-6, 1], 4)) == "unsupported_layout"
    assert run(view(SRC_BASE, 96, 0, [4, 6], [0, 1], 4)) == "unsupported_layout"
    assert run(view(SRC_BASE, 96, 0, [4, 6], [1, 1], 4)) == "unsupported_layout"
    assert run(view(SRC_BASE, 96, 0, [], [], 4)) == "invalid_view"
    assert run(view(SRC_BASE, 96, 0, [0, 6], [6, 1], 4)) == "invalid_view"
    assert run(view(0, 96, 0, [4, 6], [6, 1], 4)) == "invalid_view"
    assert run(view(SRC_BASE, 96, 0, [4, 6], [6, 1], 2)) == "plan_mismatch"
    assert run(view(SRC_BASE, 96, 0, [2, 6], [6, 1], 4)) == "plan_mismatch"
    assert run(view(SRC_BASE, 96, 0, [4, 6], [6, 1], 4, CUDA, 0)) == "direction_mismatch"
    assert run(view(SRC_BASE, 96, 0, [4, 6], [6, 1], 4),
               view(DST_BASE, 96, 0, [6, 4], [4, 1], 4, CUDA, 0), "d2h") == "direction_mismatch"
    assert run(view(SRC_BASE, 96, 0, [4, 6], [6, 1], 4),
               view(DST_BASE, 96, 0, [4, 6], [1, 4], 4)) == "unsupported_layout"
    assert run(view(SRC_BASE, 96, 0, [4, 6], [6, 1], 4),
               view(DST_BASE, 48, 0, [3, 4], [4, 1], 4)) == "plan_mismatch"
    # a CUDA view without an ordinal, a host view with one
    assert run(view(SRC_BASE, 96, 0, [4, 6], [6, 1], 4),
               view(DST_BASE, 96, 0, [6, 4], [4, 1], 4, CUDA, -1)) == "invalid_view"
    assert run(view(SRC_BASE, 96, 0, [4, 6], [6, 1], 4, HOST, 0)) == "invalid_view"


def test_one_byte_short_source_or_destination():
    """TransferTest.cpp:106-135: capacity one byte short fails before any copy."""
    b = bound(transpose_plan())
    good_src = view(SRC_BASE, 96, 0, [4, 6], [6, 1], 4)
    good_dst = view(DST_BASE, 96, 0, [6, 4], [4, 1], 4, CUDA, 0)
    assert code_of(lambda: P.make_transfer(b, view(SRC_BASE, 95, 0, [4, 6], [6, 1], 4), good_dst,
                                           "h2d")) == "insufficient_capacity"
    assert code_of(lambda: P.make_transfer(b, view(SRC_BASE, 96, 1, [4, 6], [6, 1], 4), good_dst,
                                           "h2d")) == "insufficient_capacity"
    assert code_of(lambda: P.make_transfer(b, good_src, view(DST_BASE, 95, 0, [6, 4], [4, 1], 4,
                                                             CUDA, 0), "h2d")) == "insufficient_capacity"


def test_large_checked_products_report_overflow():
    """TransferTest.cpp:137-166: spans past 2^64 are integer_overflow."""
    big = 1 << 62
    v = view(SRC_BASE, (1 << 64) - 1, 0, [4, 3], [big, 1], 4)
    assert code_of(lambda: v.span_bytes) == "integer_overflow"
    v = view(SRC_BASE, (1 << 64) - 1, (1 << 64) - 8, [4, 6], [6, 1], 4)
    assert code_of(lambda: v.span_bytes) == "integer_overflow"


def test_strided_source_views_and_the_plan_reach():
    """A view whose storage holds more than the plan reads (a transposed
    torch tensor, an offset into a larger allocation) is admitted when the
    plan's reach fits the span."""
    b = bound(transpose_plan())
    # column-major storage of the same 24 elements
    assert P.validate_transfer_source(b, view(SRC_BASE, 96, 0, [4, 6], [1, 4], 4), "h2d") == 96
    # an offset element 0 inside a larger allocation
    assert P.validate_transfer_source(b, view(SRC_BASE, 4096, 400, [4, 6], [6, 1], 4), "h2d") == 96
    # a view spanning fewer bytes than the plan reads
    assert code_of(lambda: P.validate_transfer_source(
        b, view(SRC_BASE, 4096, 0, [24], [1], 2), "h2d")) == "plan_mismatch"


def test_typed_plans_take_the_dispatch_path():
    b = P.Bound(P.Plan(W.c4_plan().blob), {"s0": 4, "s1": 8},
                W.param("scale", np.ones(4, np.float32)))
    assert code_of(lambda: P.validate_transfer_source(
        b, view(SRC_BASE, 32, 0, [4, 8], [8, 1], 1), "h2d")) == "typed_unsupported"


def test_source_only_validation_matches_full_validation():
    """TransferTest.cpp:410-423."""
    b = bound(transpose_plan())
    dst = view(DST_BASE, 96, 0, [6, 4], [4, 1], 4, CUDA, 0)
    for src in (view(SRC_BASE, 96, 0, [4, 6], [6, 1], 4), view(SRC_BASE, 95, 0, [4, 6], [6, 1], 4),
                view(SRC_BASE, 96, 0, [4, 6], [6, 0], 4), view(SRC_BASE, 96, 0, [4, 6], [6, 1], 8)):
        try:
            span = P.validate_transfer_source(b, src, "h2d")
        except P.TransferError as e:
            assert code_of(lambda: P.make_transfer(b, src, dst, "h2d")) == e.code
        else:
            assert P.make_transfer(b, src, dst, "h2d").source_span_bytes == span


# ------------------------------------------- against the reference build

def _random_view(rng, n_elem, es, kind):
    rank = int(rng.integers(1, 4))
    # factor n_elem over `rank` axes when possible, else a random shape
    ext = [1] * rank
    rem = n_elem
    for i in range(rank - 1):
        divs = [d for d in range(1, rem + 1) if rem % d == 0]
        ext[i] = int(rng.choice(divs))
        rem //= ext[i]
    ext[-1] = rem
    if rng.random() < 0.1:
        ext[int(rng.integers(rank))] = int(rng.integers(0, 4))
    order = rng.permutation(rank)
    strides = [0] * rank
    run = 1
    for a in reversed(order):
        strides[a] = run
        run *= max(ext[a], 1) + (int(rng.integers(0, 3)) if rng.random() < 0.3 else 0)
    r = rng.random()
    if r < 0.05:
        strides[int(rng.integers(rank))] = -1
    elif r < 0.1:
        strides[int(rng.integers(rank))] = 0
    elif r < 0.15 and rank > 1:
        strides[0] = strides[-1]
    span = (sum((max(e, 1) - 1) * s for e, s in zip(ext, strides)) + 1) * es
    off = int(rng.integers(0, 3)) * es if rng.random() < 0.3 else 0
    cap = max(0, span + off + int(rng.integers(-2, 3)) * (rng.random() < 0.3))
    if rng.random() < 0.05:
        es = int(rng.choice([1, 2, 8]))
    base = SRC_BASE if rng.random() > 0.02 else 0
    dev = 0 if kind == CUDA else -1
    if rng.random() < 0.03:
        dev = -1 if kind == CUDA else 0
    return (base, cap, off, ext, strides, es, kind, dev)


PLANS = [
    (transpose_plan(), {}, 24, 4),
    (EN.encode([3, 5, 4], "float16", [EN.Transpose((2, 0, 1))]).blob, {}, 60, 2),
    (EN.encode([6, 4], "int8", [EN.Pad(1, 1, 2, 0)]).blob, {}, 24, 1),
    (W.c1_plan().blob, {"s0": 256}, 256, 4),
]


@pytest.mark.skipif(not ref.available(), reason="reference CPU build (oracle/_ref) not built")
@pytest.mark.parametrize("pi", range(len(PLANS)))
def test_validation_agrees_with_the_reference_build(pi):
    blob, syms, n_elem, es = PLANS[pi]
    b = bound(blob, syms)
    rng = np.random.default_rng(1000 + pi)
    total = b.total_bytes
    agree = ok = 0
    for _ in range(400):
        direction = "h2d" if rng.random() < 0.7 else "d2h"
        skind = HOST if direction == "h2d" else CUDA
        dkind = CUDA if direction == "h2d" else HOST
        if rng.random() < 0.05:
            skind, dkind = dkind, skind
        s = _random_view(rng, n_elem, es, skind)
        if rng.random() < 0.7:
            d = (DST_BASE, total + (int(rng.integers(-1, 2)) if rng.random() < 0.2 else 0), 0,
                 [total // es], [1], es, dkind, 0 if dkind == CUDA else -1)
        else:
            d = _random_view(rng, total // es, es, dkind)
        want = ref.validate_transfer(blob, syms, s, d, direction)
        try:
            req = P.make_transfer(b, view(*s), view(*d), direction)
            got = ("ok", req.source_span_bytes)
        except P.TransferError as e:
            got = ("error", "%s: %s" % (e.code, e.detail))
        assert got[0] == want[0], (s, d, direction, got, want)
        if got[0] == "ok":
            assert got == want
            ok += 1
        else:
            assert got[1].split(":")[0] == want[1].split(":")[0], (s, d, direction, got, want)
        agree += 1
        src_only = ref.validate_transfer(blob, syms, s, None, direction, source_only=True)
        try:
            got_s = ("ok", P.validate_transfer_source(b, view(*s), direction))
        except P.TransferError as e:
            got_s = ("error", e.code)
        assert got_s[0] == src_only[0] and (got_s[0] != "ok" or got_s == src_only)
        if got_s[0] == "error":
            assert got_s[1] == src_only[1].split(":")[0]
    assert agree == 400 and ok > 20


# ------------------------------------------------------- resource caches

def test_resource_caches_touch_no_gpu_until_used():
    c = P.TransferResourceCache(max_retained_bytes=1 << 20, max_contexts=2)
    st = c.stats()
    assert st["contexts"] == 0 and not st["closed"] and st["process_valid"]
    assert st["limits"]["retained_bytes"] == 1 << 20 and st["limits"]["contexts"] == 2
    with c as same:
        assert same is c
    assert c.closed
    with pytest.raises(P.TransferError, match="resources_closed"):
        c.context(0)
    with pytest.raises(P.TransferError, match="resources_closed"):
        with c:
            pass
    d = P.DispatchResources(max_retained_bytes=1 << 22, max_streams=4)
    assert d.stats()["context_creations"] == 0 and d.stats()["limits"]["streams"] == 4
    d.clear()
    d.close()
    assert d.closed


@pytest.mark.parametrize("options", [
    {"max_contexts": -1}, {"max_retained_bytes": -1}, {"max_contexts_per_device": -1},
    {"max_background_workers": -1}, {"max_live_staging_bytes": -1},
    {"acquire_timeout_ms": -1}, {"max_contexts": 1.5}, {"max_contexts": 2**100},
])
def test_resource_limits_reject_invalid_values(options):
    """The reference's invalid-limit cases
    (libreloc/python/tests/test_transfer_resources.py:87-94)."""
    with pytest.raises((TypeError, ValueError, OverflowError)):
        P.TransferResourceCache(**options)


@pytest.mark.parametrize("options", [{"max_retained_bytes": -1}, {"max_live_bytes": -2},
                                     {"max_streams": 0.5}, {"acquire_timeout_ms": -1}])
def test_dispatch_resource_limits_reject_invalid_values(options):
    with pytest.raises((TypeError, ValueError, OverflowError)):
        P.DispatchResources(**options)


_VIEW = dict(base=1 << 20, capacity_bytes=4 << 20, offset_bytes=0, extents=[1024],
             strides=[1], element_size=4, kind="host", device=-1)


@pytest.mark.parametrize("field,value", [
    ("base", -1), ("base", 1 << 64), ("capacity_bytes", -1), ("capacity_bytes", 1 << 64),
    ("offset_bytes", -1), ("offset_bytes", 1 << 64), ("extents", [1 << 63]),
    ("strides", [-(1 << 63) - 1]), ("element_size", -4), ("element_size", 1 << 32),
    ("device", 1 << 31), ("base", 1.5), ("capacity_bytes", "4096"), ("offset_bytes", None)])
def test_buffer_view_refuses_values_its_types_cannot_hold(field, value):
    """The reference binds base as uintptr_t, capacity and offset as size_t,
    extents and strides as int64, element size as uint32 and device as int
    (PyTransfer.cpp:62-65,312-319): a negative capacity is refused there, not
    wrapped into a 64-bit size that would turn the capacity checks off."""
    with pytest.raises(TypeError):
        P.BufferView(**dict(_VIEW, **{field: value}))


def test_buffer_view_accepts_the_edges_of_its_types():
    v = P.BufferView(**dict(_VIEW, base=(1 << 64) - 1, capacity_bytes=(1 << 64) - 1,
                            offset_bytes=0, extents=[(1 << 63) - 1], strides=[-(1 << 63)],
                            element_size=(1 << 32) - 1, device=-(1 << 31)))
    assert v.base == (1 << 64) - 1 and v.extents == [(1 << 63) - 1]
    v = P.BufferView(**dict(_VIEW, base=np.uint64(4096), capacity_bytes=np.int64(64)))
    assert v.base == 4096 and v.capacity_bytes == 64 and type(v.base) is int


def test_resource_limits_accept_zero_and_none():
    assert P.TransferResourceCache(max_retained_bytes=0, max_live_staging_bytes=None,
                                   acquire_timeout_ms=None).stats()["limits"]["retained_bytes"] == 0
    assert P.DispatchResources(max_retained_bytes=0, acquire_timeout_ms=5).stats()["limits"][
        "acquire_timeout_ms"] == 5


def test_resource_caches_refuse_pickling_and_foreign_processes():
    c = P.TransferResourceCache()
    with pytest.raises(TypeError):
        pickle.dumps(c)
    c._pid = -1  # as if inherited by a forked child
    with pytest.raises(P.TransferError, match="process_mismatch"):
        c.stats()


def test_execute_transfer_argument_checks():
    b = bound(transpose_plan())
    req = P.make_transfer(b, view(SRC_BASE, 96, 0, [4, 6], [6, 1], 4),
                          view(DST_BASE, 96, 0, [6, 4], [4, 1], 4, CUDA, 0), "h2d")
    for kw in ({"n_buffers": 0}, {"n_streams": 0}, {"gather_threads": -1}, {"pinning": "x"},
               {"resources": P.TransferResourceCache()}, {"owners": (None, 1)}):
        with pytest.raises(ValueError):
            P.execute_transfer(req, **kw)
    assert not req.consumed  # argument errors leave the request usable
    assert P.cuda_enabled is True
