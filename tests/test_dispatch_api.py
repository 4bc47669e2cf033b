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


# ------------------------------------------------- calibration, pools, selection

CAL = """# costmodel calibration v0
# machine: testbox
pcie.h2d_gbps 10
cpu.t8.contiguous.contig_read_gbps 20
hbm.bw_gbps 100
overhead.a_ms 0.5  # a trailing comment
"""


def test_calibration_files_load(tmp_path):
    """The reference's calibration format (libreloc/src/CostModel.cpp:29-76):
    its test file, its two committed machine files (tests/golden/calibration,
    copied from calibration/), and the parser's diagnostics."""
    p = tmp_path / "test.cal"
    p.write_text(CAL)
    cal = P.load_calibration(str(p))
    assert cal.machine == "testbox" and cal.value("overhead.a_ms") == 0.5
    gen3 = P.load_calibration(G.path("calibration", "epyc7351-2080ti.cal"))
    gen4 = P.load_calibration(G.path("calibration", "7800x3d-4070tis.cal"))
    assert (gen3.machine, gen4.machine) == ("epyc7351-2080ti", "7800x3d-4070tis")
    assert gen3.value("pcie.h2d_gbps") == 13.07
    bad = {"no header\n": "first non-blank line must be the v0 version header (line 1)",
           "": "empty file",
           "# costmodel calibration v0\nkey\n": "expected 'key value' at line 2",
           "# costmodel calibration v0\n\nk 1 2\n": "trailing junk at line 3",
           "# costmodel calibration v0\nk one\n": "non-numeric value at line 2",
           "# costmodel calibration v0\nk inf\n": "non-numeric value at line 2",
           "# costmodel calibration v0\nk 1_0\n": "non-numeric value at line 2",
           "# costmodel calibration v0\nk 1\nk 2\n": "duplicate key 'k' at line 3"}
    for text, msg in bad.items():
        p.write_text(text)
        with pytest.raises(ValueError, match=msg.replace("(", r"\(").replace(")", r"\)")):
            P.load_calibration(str(p))
    p.write_text("# costmodel calibration v0\nk 0x10\n")
    assert P.load_calibration(str(p)).value("k") == 16.0  # strtod reads hex floats
    with pytest.raises(ValueError, match="cannot read"):
        P.load_calibration(str(tmp_path / "missing.cal"))


def test_calibration_is_accepted_and_changes_no_row(tmp_path):
    p = tmp_path / "test.cal"
    p.write_text(CAL)
    cal = P.load_calibration(str(p))
    b = c2_bound()
    t = P.prepare_dispatch_template(b, "h2d", "cuda", calibration=cal)
    assert t.selection == P.prepare_dispatch_template(b, "h2d", "cuda").selection
    with pytest.raises(TypeError):
        P.prepare_dispatch_template(b, "h2d", "cuda", calibration="gen3")


def test_select_dispatch_rows():
    """select_dispatch (PyDispatch.cpp:438-462): the selected row's fields
    plus policy and placement reason, without buffers."""
    b = c2_bound()
    s = P.select_dispatch(b, "h2d", "cuda", threads=8)
    assert s["implementation"] == "hip_relayout@1" and s["wire_boundary"] == 1
    assert s["policy"] == "auto" and s["placement_reason"] == "device_relayout"
    f = P.select_dispatch(b, "h2d", "cuda", implementation="hip_relayout")
    assert f["wire_boundary"] == 0 and f["placement_reason"] == "forced"
    assert P.select_dispatch(b, "d2h", "cuda")["implementation"] == "hip_relayout"
    with pytest.raises(P.TransferError) as e:
        P.select_dispatch(b, "h2d")  # the host device end: no CPU rows here
    assert e.value.code == "implementation_unavailable"
    with pytest.raises(ValueError):
        P.select_dispatch(b, "h2d", "gpu")
    with pytest.raises(ValueError):
        P.select_dispatch(b, "h2d", "cuda", threads=0)


def test_gather_pool_handle():
    pool = P.GatherPool(3)
    assert pool.threads == 3 and not pool.closed
    assert P.GatherPool().threads >= 1  # 0: every core
    with pytest.raises(ValueError):
        P.GatherPool(-1)
    with pool:
        pass
    assert pool.closed
    pool.close()  # idempotent
    b = c2_bound()
    x = np.zeros((2, 3, 224, 224), np.float32)
    req = P.prepare_dispatch(b, host_view(x), fake_device_view([2, 224, 224, 4], 2), "h2d")
    with pytest.raises(ValueError, match="gather_pool is closed"):
        P.execute_dispatch(req, gather_pool=pool)
    with pytest.raises(TypeError):
        P.execute_dispatch(req, gather_pool=4)
    assert not req.consumed and not req.executing


# How the in-scope callers call pyreloc: reloc_torch's dispatch, transport,
# group, resources and index_select modules and the WeightFetcher workload
# (libreloc/python/examples/workloads/common.py), as (positional arguments,
# keyword names) per name, read from their call sites.
CALLER_SURFACE = {
    "BufferView": (0, ["base", "capacity_bytes", "device", "element_size", "extents", "kind",
                       "offset_bytes", "strides"]),
    "DispatchResources": (0, ["acquire_timeout_ms", "max_background_workers", "max_contexts",
                              "max_contexts_per_device", "max_live_bytes", "max_retained_bytes",
                              "max_streams"]),
    "TransferResourceCache": (0, ["acquire_timeout_ms", "max_background_workers", "max_contexts",
                                  "max_contexts_per_device", "max_live_staging_bytes",
                                  "max_retained_bytes"]),
    "bind_indexed": (3, []), "bind_typed": (3, []), "cuda_pointer_device": (1, []),
    "execute_dispatch": (1, ["caller_stream", "chunk_size", "direct_dense_upload", "gather_pool",
                             "gather_threads", "min_pinned_bytes", "n_buffers", "n_streams",
                             "owners", "pinning", "pipeline", "resources"]),
    "execute_transfer": (1, ["caller_stream", "gather_pool", "gather_threads", "min_pinned_bytes",
                             "n_buffers", "n_streams", "owners", "pinning", "resources"]),
    "load_calibration": (1, []), "make_transfer": (4, []),
    "prepare_dispatch": (4, ["calibration", "implementation", "policy", "threads"]),
    "prepare_dispatch_from_template": (3, []), "prepare_dispatch_group": (1, []),
    "prepare_dispatch_template": (3, ["calibration", "implementation", "policy", "threads"]),
    "prepare_index_select_program": (2, []), "query_capability": (3, []),
    "select_dispatch": (3, ["threads"]), "validate_transfer_source": (3, []),
    "execute_dispatch_group": (1, []), "submit_dispatch_group": (1, []),
    "GatherPool": (1, []), "Calibration": None, "BindError": None, "DecodeError": None,
    "TransferError": None, "cuda_enabled": None,
}


@pytest.mark.parametrize("name", sorted(CALLER_SURFACE))
def test_callers_find_every_name_they_use(name):
    import inspect
    assert hasattr(P, name), name
    shape = CALLER_SURFACE[name]
    if shape is None:
        return
    n, kws = shape
    obj = getattr(P, name)
    sig = inspect.signature(obj.__init__ if inspect.isclass(obj) else obj)
    args = [None] * (n + (1 if inspect.isclass(obj) else 0))  # self
    sig.bind_partial(*args, **{k: None for k in kws})


def test_group_scratch_limit_refused_before_launch():
    """A group whose wire exceeds max_scratch_bytes is refused before any
    work (no GPU is touched), and its requests are spent, as the reference's
    owner refuses scratch past its live-byte limit
    (libreloc/python/tests/torch_frontend/test_group.py:176-179)."""
    b = c2_bound()
    src = np.zeros((2, 3, 224, 224), np.float32)
    entries = [(b, host_view(src), fake_device_view([2, 224, 224, 4], 2), "h2d") for _ in range(3)]
    g = P.prepare_dispatch_group(entries)
    wire = 3 * 2 * 3 * 224 * 224 * 2  # three f16 wires after the staged cast
    with pytest.raises(P.TransferError, match="live-byte limit") as e:
        P.execute_dispatch_group(g, max_scratch_bytes=wire // 2)
    assert e.value.code == "insufficient_capacity"
    assert g.consumed and all(r.consumed for r in g.items)
    with pytest.raises(P.TransferError, match="already_executed"):
        P.execute_dispatch_group(g, max_scratch_bytes=1 << 40)
    g2 = P.prepare_dispatch_group(entries)
    with pytest.raises(P.TransferError, match="live-byte limit"):
        P.submit_dispatch_group(g2, max_scratch_bytes=1000, owners=((), ()))
    assert g2.consumed


def test_live_byte_limit_of_the_owner_refused_before_launch():
    """DispatchResources(max_live_bytes=...) caps the scratch of one call
    (reference DispatchResources.h:57-61: maxLiveBytes also caps scratch
    during a call): a request whose wire exceeds it is refused before any
    work, with no GPU touched; 0 means no cap."""
    b = c2_bound()
    src = np.zeros((2, 3, 224, 224), np.float32)
    wire = 2 * 3 * 224 * 224 * 2  # the f16 wire after the staged cast
    owner = P.DispatchResources(max_live_bytes=wire - 1)
    req = P.prepare_dispatch(b, host_view(src), fake_device_view([2, 224, 224, 4], 2), "h2d")
    with pytest.raises(P.TransferError, match="live-byte limit") as e:
        P.execute_dispatch(req, resources=owner)
    assert e.value.code == "insufficient_capacity" and req.consumed
    g = P.prepare_dispatch_group([(b, host_view(src), fake_device_view([2, 224, 224, 4], 2), "h2d")])
    with pytest.raises(P.TransferError, match="live-byte limit"):
        P.execute_dispatch_group(g, resources=owner, max_scratch_bytes=1 << 40)
    assert owner.stats()["context_creations"] == 0
    owner.close()
