"""The reference-shaped typed dispatch API (sym_amd.dispatch, re-exported by
sym_amd.pyreloc): capability rows, selection, view validation and error
codes, on the CPU (nothing here launches). The GPU execution of the same
requests is in test_gpu_parity.py."""
import numpy as np
import pytest

from sym_amd import pyreloc as P
from sym_amd import workloads as W
from tests import golden_io as G


def host_view(a):
    return P.BufferView(a.ctypes.data, a.nbytes, 0, list(a.shape),
                        [s // a.dtype.itemsize for s in a.strides], a.dtype.itemsize, "host")


def fake_device_view(shape, itemsize, capacity=None):
    n = int(np.prod(shape)) * itemsize
    strides, run = [], 1
    for e in reversed(shape):
        strides.insert(0, run)
        run *= e
    return P.BufferView(1 << 40, n if capacity is None else capacity, 0, list(shape), strides,
                        itemsize, "cuda", 0)


def c2_bound():
    return P.Bound(P.Plan(W.c2_plan(n=2).blob), {}, {})


def test_buffer_view_geometry():
    a = np.zeros((3, 4), np.float32)
    v = host_view(a)
    assert v.is_dense() and v.span_bytes == 48 and v.address == a.ctypes.data
    t = host_view(a.T)
    assert not t.is_dense() and t.span_bytes == 48
    with pytest.raises(ValueError):
        P.BufferView(0, 0, 0, [1], [1], 1, "disk")


def test_capability_rows_per_boundary():
    b = c2_bound()  # pad -> transpose -> cast f32->f16 (per tensor)
    cap = P.query_capability(b, "h2d", "cuda")
    assert [r["implementation"] for r in cap["eligible"]] == ["hip_relayout", "hip_relayout@1"]
    n = 2 * 3 * 224 * 224  # the source layout's elements, f32 then f16
    assert [r["wire_bytes"] for r in cap["eligible"]] == [4 * n, 2 * n]
    d2h = P.query_capability(b, "d2h", "cuda")["eligible"]
    assert [r["implementation"] for r in d2h] == ["hip_relayout"]
    assert d2h[0]["wire_bytes"] == b.destination_bytes and d2h[0]["wire_result_layout"]
    assert P.query_capability(b, "h2d", "host")["eligible"] == []
    c3 = P.Bound(P.Plan(W.c3_plan().blob), {"s0": 64, "s1": 128},
                 W.param("scale", np.ones(128, np.float32)))
    cap = P.query_capability(c3, "h2d", "cuda")
    # dequantize is per channel: no row may apply it on the host
    assert [r["implementation"] for r in cap["eligible"]] == ["hip_relayout"]
    assert [r["implementation"] for r in cap["excluded"]] == ["hip_relayout@1", "hip_relayout@2"]


@pytest.mark.parametrize("meta,blob", G.typed_fixtures(), ids=[m["name"] for m, _ in G.typed_fixtures()])
def test_corpus_capability_is_consistent(meta, blob):
    for binding in meta["bindings"]:
        b = P.bind_typed(P.load_typed_plan(blob), binding["symbols"], G.fixture_params(meta))
        rows = P.query_capability(b, "h2d", "cuda")["eligible"]
        assert rows[0]["implementation"] == "hip_relayout"
        assert len(rows) == b.info.host_stages_max + 1
        assert b.info.host_stages_auto <= b.info.host_stages_max
        # the boundary-0 wire is the source itself
        assert rows[0]["wire_bytes"] == binding["footprints"]["h2d"]["source_bytes"]


def test_selection_and_forced_rows():
    b = c2_bound()
    t = P.prepare_dispatch_template(b, "h2d", "cuda")
    assert t.selection["implementation"] == "hip_relayout@1"  # the narrowing cast is staged
    assert t.selection["placement_reason"] == "device_relayout"
    t0 = P.prepare_dispatch_template(b, "h2d", "cuda", implementation="hip_relayout")
    assert t0.selection["host_stages"] == 0 and t0.selection["placement_reason"] == "forced"
    with pytest.raises(P.TransferError) as e:
        P.prepare_dispatch_template(b, "h2d", "cuda", implementation="cpu_reference")
    assert e.value.code == "implementation_unavailable"
    with pytest.raises(P.TransferError) as e:
        P.prepare_dispatch_template(b, "h2d", "cuda", policy="original_cpu")
    assert e.value.code == "implementation_unavailable"
    t = P.prepare_dispatch_template(b, "d2h", "cuda")
    assert t.selection["implementation"] == "hip_relayout" and t.selection["host_stages"] == 0
    with pytest.raises(ValueError):
        P.prepare_dispatch_template(b, "h2d", "cuda", policy="fastest")
    with pytest.raises(ValueError):
        P.prepare_dispatch_template(b, "h2d", "cuda", threads=0)


def test_view_validation_codes():
    b = c2_bound()
    src = np.zeros((2, 3, 224, 224), np.float32)
    good = fake_device_view([2, 224, 224, 4], 2)
    req = P.prepare_dispatch(b, host_view(src), good, "h2d")
    assert req.selected["implementation"] == "hip_relayout@1" and not req.consumed

    def code(s, d):
        with pytest.raises(P.TransferError) as e:
            P.prepare_dispatch(b, s, d, "h2d")
        return e.value.code

    assert code(host_view(src), fake_device_view([2, 224, 224, 4], 4)) == "plan_mismatch"
    assert code(host_view(src[:1]), good) == "plan_mismatch"
    assert code(host_view(np.zeros((2, 3, 224, 224), np.float16)), good) == "plan_mismatch"
    assert code(host_view(np.asfortranarray(src)), good) == "unsupported_layout"
    assert code(host_view(src), fake_device_view([2, 224, 224, 4], 2, capacity=100)) == \
        "insufficient_capacity"
    host_dst = host_view(np.zeros((2, 224, 224, 4), np.float16))
    # host views are admitted on either end (reference checkView); this
    # library's rows need the device end in device memory
    assert code(host_view(src), host_dst) == "backend_mismatch"
    # device-to-host: a cuda source into a host destination
    dev_src = fake_device_view([2, 3, 224, 224], 4)
    req = P.prepare_dispatch(b, dev_src, host_dst, "d2h")
    assert req.template.direction == "d2h"
    with pytest.raises(P.TransferError) as e:
        P.prepare_dispatch(b, host_view(src), host_dst, "d2h")
    assert e.value.code == "backend_mismatch"
    with pytest.raises(P.TransferError) as e:
        P.prepare_dispatch(b, host_view(src), fake_device_view([2, 224, 224, 4], 2), "d2h")
    assert e.value.code == "direction_mismatch"


def test_group_preparation():
    b = c2_bound()
    src = np.zeros((2, 3, 224, 224), np.float32)
    g = P.prepare_dispatch_group([(b, host_view(src), fake_device_view([2, 224, 224, 4], 2), "h2d")] * 3)
    assert len(g.items) == 3 and not g.consumed
    with pytest.raises(P.TransferError):
        P.prepare_dispatch_group([])
