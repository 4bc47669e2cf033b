"""Indexed plans (wire v2) on the MI355X: host-table uploads through the
dispatch API and the C-ABI, and the device row gather (relx_index_select_device),
bit-exact against the CPU oracle (oracle/relx_oracle.py: execute_indexed,
pinned in tests/test_indexed.py). Cases follow the reference's
libreloc/python/tests/test_indexed_plan.py and
libreloc/python/tests/torch_frontend/test_index_select.py."""
import sys

import numpy as np
import pytest

from oracle import relx_oracle as O
from sym_amd import pyreloc as P
from sym_amd.encoder import encode_index_select

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

PAIRS = [("float32", "float16"), ("float16", "float32"), ("float32", "float32"),
         ("float16", "float16"), ("int8", "int8")]
NP = {"float32": np.float32, "float16": np.float16, "int8": np.int8}
TORCH_BITS = {1: torch.uint8, 2: torch.int16, 4: torch.int32}


def say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def resources():
    assert torch.cuda.is_available(), "a GPU test needs the MI355X"
    r = P.Resources(0)
    yield r
    r.close()


def host_view(a):
    return P.BufferView(a.ctypes.data, a.nbytes, 0, list(a.shape),
                        [s // a.dtype.itemsize for s in a.strides], a.dtype.itemsize, "host")


def device_view(t):
    return P.BufferView(t.data_ptr(), t.numel() * t.element_size(), 0, list(t.shape),
                        list(t.stride()), t.element_size(), "cuda", t.device.index)


def table(rng, dtype, shape):
    n = int(np.prod(shape))
    if dtype == "float32":
        x = rng.standard_normal(n).astype(np.float32)
        if n >= 12:
            x[:7] = [np.nan, np.inf, -np.inf, 65520.0, 2.0 ** -25, -0.0, 65504.0]
            xb = x.view(np.uint32)
            xb[7], xb[8], xb[9] = 0x7F800001, 0xFFC12345, 0x33000001
    elif dtype == "float16":
        x = rng.integers(0, 1 << 16, n, dtype=np.uint16).view(np.float16)
    else:
        x = rng.integers(-128, 128, n, dtype=np.int8)
    return x.reshape(shape)


def bind(shape, sd, rd, idt, idx, symbolic=False):
    if symbolic:
        blob = encode_index_select(["N", "D"], sd, "M", idt, rd)
        syms = {"N": shape[0], "D": shape[1], "M": len(idx)}
    else:
        blob = encode_index_select(list(shape), sd, len(idx), idt, rd)
        syms = {}
    b = P.bind_indexed(P.load_indexed_plan(blob), syms,
                       (idt, [len(idx)], np.asarray(idx, dtype=idt).tobytes()))
    ob = O.bind_indexed(O.decode_indexed_plan(blob), syms, O.DTYPE_TYPES[idt], [len(idx)],
                        np.asarray(idx, dtype=idt).tobytes())
    return b, ob


def empty_out(b, rd):
    w = np.dtype(NP[rd]).itemsize
    return torch.empty(b.result_extents, dtype=TORCH_BITS[w], device="cuda")


@pytest.mark.parametrize("sd,rd", PAIRS)
@pytest.mark.parametrize("idt", ["int32", "int64"])
@pytest.mark.parametrize("shape", [(7,), (7, 129), (7, 3, 5)])
def test_dispatch_row_order_repeats_and_casts(resources, rng, sd, rd, idt, shape):
    """test_index_select.py:63-85 through prepare_index_select_program /
    prepare_dispatch / execute_dispatch, on every eligible row."""
    idx = np.array([6, 0, 3, 6, 1, 5, 0, 4, 2], dtype=idt)
    x = table(rng, sd, shape)
    b, ob = bind(shape, sd, rd, idt, idx)
    want = O.execute_indexed(ob, x)
    prog = P.prepare_index_select_program(b, host_view(x))
    rows = [r["implementation"] for r in P.query_capability(prog, "h2d", "cuda")["eligible"]]
    for impl in [""] + rows:
        say("dispatch", sd, rd, idt, shape, impl or "auto")
        out = empty_out(b, rd)
        req = P.prepare_dispatch(prog, host_view(x), device_view(out), "h2d", implementation=impl)
        rep = P.execute_dispatch(req, resources=resources, gather_threads=3)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint8).reshape(-1), want), impl
        assert rep["artifact_version"] == 2
        assert rep["source_bytes"] == x.nbytes
        assert rep["parameter_bytes"] == len(idx) * np.dtype(idt).itemsize
        assert rep["destination_bytes"] == want.size
        with pytest.raises(P.TransferError, match="already_executed"):
            P.execute_dispatch(req, resources=resources)


@pytest.mark.parametrize("rows,width,count", [(8, 5, 3), (3, 129, 11), (19, 1, 7)])
def test_symbolic_execution_and_accounting(resources, rows, width, count):
    """test_indexed_plan.py:32-51: the default row narrows on the host, so
    the payload is the f16 output."""
    say("symbolic", rows, width, count)
    x = np.arange(rows * width, dtype=np.float32).reshape(rows, width)
    indices = (np.arange(count) * 7 + 2) % rows
    b, _ = bind((rows, width), "float32", "float16", "int64", indices, symbolic=True)
    assert b.source_extents == [rows, width] and b.result_extents == [count, width]
    out = torch.empty((count, width), dtype=torch.float16, device="cuda")
    prog = P.prepare_index_select_program(b, host_view(x))
    rep = P.execute_dispatch(P.prepare_dispatch(prog, host_view(x), device_view(out), "h2d"),
                             resources=resources, gather_threads=2)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), x[indices].astype(np.float16))
    assert rep["artifact_version"] == 2 and rep["source_bytes"] == x.nbytes
    assert rep["parameter_bytes"] == count * 8
    assert rep["payload_bytes_transferred"] == out.numel() * 2


def test_binding_owns_index_values(resources):
    """test_indexed_plan.py:112-120."""
    say("ownership")
    indices = np.array([7, 0, 7], dtype=np.int64)
    b, _ = bind((8, 5), "float32", "float16", "int64", indices, symbolic=True)
    indices[:] = 1
    x = np.arange(40, dtype=np.float32).reshape(8, 5)
    out = torch.empty((3, 5), dtype=torch.float16, device="cuda")
    prog = P.prepare_index_select_program(b, host_view(x))
    P.execute_dispatch(P.prepare_dispatch(prog, host_view(x), device_view(out), "h2d"),
                       resources=resources)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), x[[7, 0, 7]].astype(np.float16))


def test_cast_rounding_edges(resources):
    """test_index_select.py:88-98."""
    say("rounding edges")
    x = np.array([0., -0., 1., 1.00048828125, 65504., 65520., 2 ** -24, 2 ** -25, np.inf, -np.inf,
                  np.nan], dtype=np.float32).reshape(1, -1)
    idx = np.array([0, 0], dtype=np.int64)
    b, ob = bind(x.shape, "float32", "float16", "int64", idx)
    want = O.execute_indexed(ob, x)
    for k in (0, 1):
        out = torch.empty((2, 11), dtype=torch.int16, device="cuda")
        resources.execute_h2d(b, x.ctypes.data, x.nbytes, out.data_ptr(), out.numel() * 2,
                              host_stages=k)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint8).reshape(-1), want), k
    t = torch.from_numpy(x).cuda()
    out = torch.empty((2, 11), dtype=torch.int16, device="cuda")
    resources.index_select_device(b, t.data_ptr(), x.nbytes, out.data_ptr(), 44)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint8).reshape(-1), want)


@pytest.mark.parametrize("sd,rd", PAIRS)
@pytest.mark.parametrize("pinned", [False, True])
def test_long_selection_from_a_small_table_sends_the_table(resources, rng, sd, rd, pinned):
    """A selection of at least 2^16 rows from a table no larger than the
    gathered rows: the table crosses PCIe as it is (byte chunks, 256-byte
    multiples) and the device gathers the rows with the cast fused. Explicit
    host stages keep the host gather."""
    shape, count = (1500, 7), 70000
    idx = rng.integers(0, shape[0], count)
    x = table(rng, sd, shape)
    b, ob = bind(shape, sd, rd, "int64", idx)
    want = O.execute_indexed(ob, x)
    src, keep = x, None
    if pinned:
        keep = torch.from_numpy(x.view(np.uint8).reshape(-1).copy()).pin_memory()
        src = keep.numpy().view(x.dtype).reshape(shape)
    for chunk in (0, 4096, 4000):
        say("table upload", sd, rd, "pinned" if pinned else "pageable", "chunk", chunk)
        out = empty_out(b, rd)
        rep = resources.execute_h2d(b, src.ctypes.data, src.nbytes, out.data_ptr(),
                                    out.numel() * out.element_size(), chunk_bytes=chunk)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint8).reshape(-1), want), chunk
        assert rep["implementation"] == "hip_table_gather"
        assert rep["wire_bytes"] == rep["payload_bytes_transferred"] == x.nbytes
        assert rep["direct_dma"] == (1 if pinned else 0)
        assert rep["chunks"] == (1 if chunk == 0 else -(-x.nbytes // (chunk // 256 * 256)))
    say("host gather kept", sd, rd)
    out = empty_out(b, rd)
    rep = resources.execute_h2d(b, src.ctypes.data, src.nbytes, out.data_ptr(),
                                out.numel() * out.element_size(), host_stages=0)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint8).reshape(-1), want)
    assert rep["implementation"] == "hip_relayout"


@pytest.mark.parametrize("sd,rd", PAIRS)
@pytest.mark.parametrize("pinned", [False, True])
def test_chunked_uploads_split_rows(resources, rng, sd, rd, pinned):
    """Chunks of a few KiB cut selected rows at arbitrary elements; every
    host boundary, pinned and pageable tables."""
    shape, count = (3000, 129), 5000
    idx = rng.integers(0, shape[0], count)
    x = table(rng, sd, shape)
    b, ob = bind(shape, sd, rd, "int64", idx)
    want = O.execute_indexed(ob, x)
    src, keep = x, None
    if pinned:
        keep = torch.from_numpy(x.view(np.uint8).reshape(-1).copy()).pin_memory()
        src = keep.numpy().view(x.dtype).reshape(shape)
    for k in range(b.info.host_stages_max + 1):
        for chunk in (4096, 1 << 20, 0):
            say("chunked", sd, rd, "pinned" if pinned else "pageable", "k", k, "chunk", chunk)
            out = empty_out(b, rd)
            rep = resources.execute_h2d(b, src.ctypes.data, src.nbytes, out.data_ptr(),
                                        out.numel() * out.element_size(), host_stages=k,
                                        chunk_bytes=chunk, gather_threads=4, n_buffers=3)
            torch.cuda.synchronize()
            assert np.array_equal(out.cpu().numpy().view(np.uint8).reshape(-1), want), (k, chunk)
            assert rep["direct_dma"] == 0 and rep["source_bytes"] == x.nbytes


@pytest.mark.parametrize("sd,rd", PAIRS)
@pytest.mark.parametrize("idt", ["int32", "int64"])
@pytest.mark.parametrize("shape,count", [((7, 129), 9), ((1000, 256), 3000), ((4096, 5), 777),
                                         ((64, 3, 5), 17), ((50,), 200)])
def test_device_gather_matches_oracle(resources, rng, sd, rd, idt, shape, count):
    idx = rng.integers(0, shape[0], count).astype(idt)
    x = table(rng, sd, shape)
    b, ob = bind(shape, sd, rd, idt, idx)
    want = O.execute_indexed(ob, x)
    sw, rw = np.dtype(NP[sd]).itemsize, np.dtype(NP[rd]).itemsize
    # aligned, then table and destination one element off 16-byte alignment
    for shift in (0, 1):
        say("device gather", sd, rd, idt, shape, count, "shift", shift)
        t = torch.zeros(x.nbytes + 64, dtype=torch.uint8, device="cuda")
        t[shift * sw:shift * sw + x.nbytes].copy_(torch.from_numpy(x.view(np.uint8).reshape(-1)))
        o = torch.full((want.size + 64,), 0xAB, dtype=torch.uint8, device="cuda")
        resources.index_select_device(b, t.data_ptr() + shift * sw, x.nbytes,
                                      o.data_ptr() + shift * rw, want.size)
        torch.cuda.synchronize()
        got = o.cpu().numpy()
        assert np.array_equal(got[shift * rw:shift * rw + want.size], want)
        assert (got[:shift * rw] == 0xAB).all() and (got[shift * rw + want.size:] == 0xAB).all()


def test_device_gather_on_a_caller_stream(resources, rng):
    say("device gather stream")
    shape, count = (20000, 512), 60000
    idx = rng.integers(0, shape[0], count)
    x = rng.standard_normal(shape).astype(np.float32)
    b, ob = bind(shape, "float32", "float16", "int64", idx)
    t = torch.from_numpy(x).cuda()
    out = torch.empty((count, 512), dtype=torch.float16, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    resources.index_select_device(b, t.data_ptr(), x.nbytes, out.data_ptr(), out.numel() * 2,
                                  stream=s.cuda_stream)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    assert torch.equal(out, t[torch.from_numpy(idx).cuda()].half())


def test_device_gather_with_wide_indices(resources):
    """A table of 2^31 + 16 one-byte rows: row indices past 2^31 take the
    64-bit index kernel."""
    say("wide indices")
    n = (1 << 31) + 16
    t = torch.empty(n, dtype=torch.uint8, device="cuda")
    full = n // 256 * 256
    t[:full].view(-1, 256).copy_(torch.arange(256, dtype=torch.uint8, device="cuda").expand(full // 256, 256))
    t[full:].copy_(torch.arange(n - full, dtype=torch.uint8, device="cuda"))
    idx = np.array([n - 1, 0, n - 2, (1 << 31) + 5, (1 << 31) - 1, 12345678901 % n], dtype=np.int64)
    b, _ = bind((n, 1), "int8", "int8", "int64", idx)
    out = torch.empty(len(idx), dtype=torch.uint8, device="cuda")
    resources.index_select_device(b, t.data_ptr(), n, out.data_ptr(), len(idx))
    torch.cuda.synchronize()
    assert out.cpu().numpy().tolist() == [int(v % 256) for v in idx]
    del t


def test_device_gather_rejects_bad_buffers(resources):
    idx = np.array([1, 0], dtype=np.int64)
    b, _ = bind((4, 8), "float32", "float16", "int64", idx)
    t = torch.zeros(32, dtype=torch.float32, device="cuda")
    out = torch.empty(16, dtype=torch.float16, device="cuda")
    with pytest.raises(P.TransferError, match="insufficient_capacity"):
        resources.index_select_device(b, t.data_ptr(), 64, out.data_ptr(), 32)
    with pytest.raises(P.TransferError, match="insufficient_capacity"):
        resources.index_select_device(b, t.data_ptr(), 128, out.data_ptr(), 16)
    with pytest.raises(P.TransferError, match="invalid_view"):
        resources.index_select_device(b, t.data_ptr() + 2, 128, out.data_ptr(), 32)
    with pytest.raises(P.TransferError, match="plan_mismatch"):
        resources.execute_d2h(b, t.data_ptr(), 128, np.zeros(16, np.float16).ctypes.data, 32)


@pytest.mark.parametrize("table_first", [True, False])
def test_table_upload_member_in_a_group(resources, rng, table_first):
    """A long selection from a small table (sent whole, gathered on the
    device) next to an ordinary typed member, in either order, through the
    dispatch API: the two members' chunks go to different copy streams."""
    say("group with a table upload", "first" if table_first else "second")
    shape, count = (700, 9), 80000
    idx = rng.integers(0, shape[0], count)
    x = rng.standard_normal(shape).astype(np.float32)
    b, ob = bind(shape, "float32", "float16", "int64", idx)
    from sym_amd.encoder import Cast, encode
    y = rng.standard_normal((129, 65)).astype(np.float32)
    tb = P.bind_typed(P.load_typed_plan(encode([129, 65], "float32", [Cast("float16")]).blob), {}, {})
    o1 = torch.empty((count, 9), dtype=torch.float16, device="cuda")
    o2 = torch.empty((129, 65), dtype=torch.float16, device="cuda")
    prog = P.prepare_index_select_program(b, host_view(x))
    items = [(prog, host_view(x), device_view(o1), "h2d"), (tb, host_view(y), device_view(o2), "h2d")]
    if not table_first:
        items.reverse()
    g = P.prepare_dispatch_group(items)
    rep = P.execute_dispatch_group(g, resources=resources, gather_threads=3)
    torch.cuda.synchronize()
    assert np.array_equal(o1.cpu().numpy().view(np.uint8).reshape(-1), O.execute_indexed(ob, x))
    assert np.array_equal(o2.cpu().numpy(), y.astype(np.float16))
    it = rep["items"][0 if table_first else 1]
    assert it["implementation"] == "hip_table_gather" and it["host_kernel"] == "copy"
    assert it["payload_bytes_transferred"] == x.nbytes and it["artifact_version"] == 2


def test_indexed_member_in_a_group(resources, rng):
    """An indexed upload and a typed cast in one group schedule."""
    say("group")
    shape, count = (512, 64), 300
    idx = rng.integers(0, shape[0], count)
    x = rng.standard_normal(shape).astype(np.float32)
    b, ob = bind(shape, "float32", "float16", "int64", idx)
    from sym_amd.encoder import Cast, encode
    y = rng.standard_normal((33, 65)).astype(np.float32)
    tb = P.bind_typed(P.load_typed_plan(encode([33, 65], "float32", [Cast("float16")]).blob), {}, {})
    o1 = torch.empty((count, 64), dtype=torch.float16, device="cuda")
    o2 = torch.empty((33, 65), dtype=torch.float16, device="cuda")
    prog = P.prepare_index_select_program(b, host_view(x))
    g = P.prepare_dispatch_group([(prog, host_view(x), device_view(o1), "h2d"),
                                  (tb, host_view(y), device_view(o2), "h2d")])
    rep = P.execute_dispatch_group(g, resources=resources, gather_threads=3)
    torch.cuda.synchronize()
    assert np.array_equal(o1.cpu().numpy().view(np.uint8).reshape(-1), O.execute_indexed(ob, x))
    assert np.array_equal(o2.cpu().numpy(), y.astype(np.float16))
    assert rep["items"][0]["artifact_version"] == 2 and rep["items"][1]["artifact_version"] == 1
