"""Layout transfers through the reference-shaped transfer API on the MI355X:
make_transfer + execute_transfer move the README plan (C1) at every N,
including N = 2^24, and other layout plans in both directions, bit-exact
against numpy's transpose/pad of the same bytes; requests are single-use;
resource caches retain one context per device; the call is ordered after
the caller's stream; host-to-host requests and foreign pointers are
refused."""
import sys

import numpy as np
import pytest

from sym_amd import encoder as EN
from sym_amd import pyreloc as P
from sym_amd import workloads as W

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


def storage_view(t, kind):
    """The view reloc_torch builds from a tensor's storage
    (reloc_torch/transport.py: _storage_view)."""
    es = t.element_size()
    st = t.untyped_storage()
    return P.BufferView(st.data_ptr(), st.nbytes(), t.storage_offset() * es, list(t.shape),
                        list(t.stride()), es, kind, t.device.index if kind == "cuda" else -1)


@pytest.fixture(scope="module")
def cache():
    assert torch.cuda.is_available(), "a GPU test needs the MI355X"
    c = P.TransferResourceCache()
    yield c
    c.close()


@pytest.mark.parametrize("n", W.C1_SIZES)
def test_c1_readme_plan_through_execute_transfer(cache, n):
    say("c1 execute_transfer N=%d" % n)
    x = torch.from_numpy(W.c1_input(n))
    b = P.bind(P.load_plan(W.c1_plan().blob), {"s0": n})
    out = torch.empty((64, n // 64), dtype=torch.float32, device="cuda")
    req = P.make_transfer(b, storage_view(x, "host"), storage_view(out, "cuda"), "h2d")
    assert req.source_span_bytes == 4 * n and req.destination_bytes == 4 * n
    P.execute_transfer(req, resources=cache, owners=(x, out), n_buffers=4,
                       caller_stream=torch.cuda.current_stream().cuda_stream)
    assert req.consumed
    assert req.staging[0]["wire_bytes"] == 4 * n
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), x.numpy().reshape(n // 64, 64).T)
    with pytest.raises(P.TransferError, match="already_executed"):
        P.execute_transfer(req, resources=cache, owners=(x, out))
    assert cache.stats()["contexts"] == 1


def test_pinned_and_offset_sources(cache):
    """A page-locked source (direct DMA) and a source view at an offset into
    a larger allocation: the plan reads from the view's element 0."""
    n = 1 << 20
    b = P.bind(P.load_plan(W.c1_plan().blob), {"s0": n})
    big = torch.from_numpy(np.random.default_rng(5).uniform(-1, 1, n + 1000).astype(np.float32))
    for pinned in (False, True):
        say("offset source, pinned", pinned)
        base = big.pin_memory() if pinned else big
        x = base[1000:]
        out = torch.empty((64, n // 64), dtype=torch.float32, device="cuda")
        req = P.make_transfer(b, storage_view(x, "host"), storage_view(out, "cuda"), "h2d")
        P.execute_transfer(req, resources=cache, owners=(x, out))
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), x.numpy().reshape(n // 64, 64).T)


@pytest.mark.parametrize("case", ["transpose3d_f16", "pad_i8", "transpose_f32"])
def test_layout_plans_both_directions(cache, case):
    rng = np.random.default_rng(17)
    if case == "transpose3d_f16":
        shape, dt, ops = [48, 40, 33], "float16", [EN.Transpose((2, 0, 1))]
        x = rng.standard_normal(shape).astype(np.float16)
        want = np.ascontiguousarray(x.transpose(2, 0, 1))
    elif case == "pad_i8":
        shape, dt, ops = [300, 70], "int8", [EN.Pad(1, 3, 5, 7)]
        x = rng.integers(-128, 128, shape).astype(np.int8)
        want = np.pad(x, ((0, 0), (3, 5)), constant_values=7)
    else:
        shape, dt, ops = [2048, 1536], "float32", [EN.Transpose((1, 0))]
        x = rng.standard_normal(shape).astype(np.float32)
        want = np.ascontiguousarray(x.T)
    b = P.bind(P.load_plan(EN.encode(shape, dt, ops).blob), {})
    tx = torch.from_numpy(x.copy())
    out = torch.empty(want.shape, dtype=getattr(torch, dt), device="cuda")
    say("layout", case, "h2d")
    P.execute_transfer(P.make_transfer(b, storage_view(tx, "host"), storage_view(out, "cuda"), "h2d"),
                       resources=cache, owners=(tx, out))
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), want)
    say("layout", case, "d2h")
    dev_src = tx.cuda()
    host_out = torch.empty(want.shape, dtype=getattr(torch, dt))
    P.execute_transfer(P.make_transfer(b, storage_view(dev_src, "cuda"), storage_view(host_out, "host"),
                                       "d2h"), resources=cache, owners=(dev_src, host_out),
                       caller_stream=torch.cuda.current_stream().cuda_stream)
    assert np.array_equal(host_out.numpy(), want)


def test_transfer_is_ordered_after_the_caller_stream(cache):
    n = 1 << 22
    b = P.bind(P.load_plan(W.c1_plan().blob), {"s0": n})
    x = torch.from_numpy(W.c1_input(n))
    out = torch.empty((64, n // 64), dtype=torch.float32, device="cuda")
    ballast = torch.ones(32 << 20, device="cuda")
    for _ in range(3):
        for _ in range(20):
            ballast.mul_(1.0)
        out.fill_(-5.0)  # queued behind the busy work on torch's stream
        req = P.make_transfer(b, storage_view(x, "host"), storage_view(out, "cuda"), "h2d")
        P.execute_transfer(req, resources=cache, owners=(x, out),
                           caller_stream=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), x.numpy().reshape(n // 64, 64).T)


def test_refusals():
    b = P.bind(P.load_plan(W.c1_plan().blob), {"s0": 256})
    x = torch.from_numpy(W.c1_input(256))
    host_out = torch.empty((64, 4), dtype=torch.float32)
    req = P.make_transfer(b, storage_view(x, "host"), storage_view(host_out, "host"), "h2d")
    with pytest.raises(P.TransferError, match="backend_mismatch"):
        P.execute_transfer(req)
    t = torch.empty(16, device="cuda")
    assert P.cuda_pointer_device(t.data_ptr()) == 0
    with pytest.raises(P.TransferError, match="invalid_view"):
        P.cuda_pointer_device(x.data_ptr())
