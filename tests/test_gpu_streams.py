"""Ordering against the caller's stream on the MI355X.

The reference orders every private stream after the caller's stream whenever
a caller stream is given, the legacy null stream (handle 0) included
(libreloc/python/PyDispatch.cpp:199-202, libreloc/src/Dispatch.cpp:1995,
libreloc/cuda/CudaBackend.cu:190-208), and its kernel wrappers launch on the
stream they are handed, null meaning the legacy default stream
(libreloc/include/reloc/CudaKernels.h:28-122). Each test here keeps torch's
stream busy for milliseconds before it enqueues a producer (a fill or a
copy), so a call that is not ordered after that stream would observe the
buffer before the producer ran, or have its result overwritten by it."""
import sys

import numpy as np
import pytest

from oracle import relx_oracle as O
from sym_amd import pyreloc as P
from sym_amd import workloads as W

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    assert torch.cuda.is_available(), "a GPU test needs the MI355X"
    c = P.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def ballast():
    return torch.ones(64 << 20, dtype=torch.float32, device="cuda")  # 256 MiB


def busy(ballast, rounds=24):
    """About 5 ms of element-wise work on torch's current stream."""
    for _ in range(rounds):
        ballast.mul_(1.0)


def c2_case(n=2, h=32, w=32):
    x = W.c2_input(n, 3, h, w)
    plan = P.Plan(W.c2_plan(n, 3, h, w).blob)
    b = P.Bound(plan, {})
    want = np.frombuffer(O.run_typed(plan.blob, {}, {}, x).tobytes(), np.uint8)
    return x, b, want


def host_view(a):
    return P.BufferView(a.ctypes.data, a.nbytes, 0, list(a.shape),
                        [s // a.dtype.itemsize for s in a.strides], a.dtype.itemsize, "host")


def device_view(t):
    return P.BufferView(t.data_ptr(), t.numel() * t.element_size(), 0, list(t.shape),
                        list(t.stride()), t.element_size(), "cuda", t.device.index)


@pytest.mark.parametrize("pinned", [False, True])
def test_upload_is_ordered_after_a_fill_on_torchs_stream(ctx, ballast, pinned):
    x, b, want = c2_case()
    src = torch.from_numpy(x.copy())
    if pinned:
        src = src.pin_memory()
    out = torch.empty(want.size, dtype=torch.uint8, device="cuda")
    for round_ in range(3):
        say("ordered upload, pinned", pinned, "round", round_)
        busy(ballast)
        out.fill_(0xA5)  # queued behind the busy work
        ctx.execute_h2d(b, src.data_ptr(), x.nbytes, out.data_ptr(), out.numel(),
                        caller_stream=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), want)


def test_dispatch_orders_after_the_null_stream(ballast):
    """execute_dispatch with torch's default stream handle (0) as caller."""
    x, b, want = c2_case()
    r = P.Resources(0)
    try:
        out = torch.empty(want.size // 2, dtype=torch.float16, device="cuda").view(2, 32, 32, 4)
        t = P.prepare_dispatch_template(b, "h2d")
        assert torch.cuda.current_stream().cuda_stream == 0
        for round_ in range(3):
            say("ordered dispatch round", round_)
            busy(ballast)
            out.fill_(7.0)
            req = P.prepare_dispatch_from_template(t, host_view(x), device_view(out))
            P.execute_dispatch(req, caller_stream=torch.cuda.current_stream().cuda_stream,
                               resources=r)
            torch.cuda.synchronize()
            assert np.array_equal(out.cpu().numpy().view(np.uint8).reshape(-1), want)
    finally:
        r.close()


def test_caller_stream_waits_for_a_no_wait_call(ctx, ballast):
    """A consumer enqueued on the caller's stream after a call that returned
    early sees the call's result."""
    x, b, want = c2_case(4, 64, 64)
    src = torch.from_numpy(x.copy()).pin_memory()
    out = torch.empty(want.size, dtype=torch.uint8, device="cuda")
    side = torch.cuda.Stream()
    for round_ in range(3):
        say("no_wait consumer round", round_)
        out.fill_(0)
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            ctx.execute_h2d(b, src.data_ptr(), x.nbytes, out.data_ptr(), out.numel(),
                            caller_stream=side.cuda_stream, no_wait=True, source_pinned=1)
            copy = out.clone()  # ordered after the call by the caller stream
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        assert np.array_equal(copy.cpu().numpy(), want)
    ctx.synchronize()


def test_relayout_device_on_the_null_stream(ctx, ballast):
    """stream=0 is the legacy null stream: the launch follows a copy queued
    there behind busy work."""
    x, b, want = c2_case()
    host = torch.from_numpy(x.view(np.uint8).reshape(-1).copy()).pin_memory()
    d_src = torch.zeros(x.nbytes, dtype=torch.uint8, device="cuda")
    out = torch.empty(want.size, dtype=torch.uint8, device="cuda")
    for round_ in range(3):
        say("null-stream relayout round", round_)
        d_src.zero_()
        out.fill_(0xA5)
        busy(ballast)
        d_src.copy_(host, non_blocking=True)
        ctx.relayout_device(b, d_src.data_ptr(), out.data_ptr(), stream=0)
        torch.cuda.synchronize()
        ctx.synchronize()
        assert np.array_equal(out.cpu().numpy(), want)


@pytest.mark.parametrize("pinned", [False, True])
def test_download_reads_a_source_written_on_torchs_stream(ctx, ballast, pinned):
    """The device-to-host source is produced by a copy queued behind busy work
    on torch's stream; the call is ordered after it."""
    rng = np.random.default_rng(7)
    x = rng.standard_normal((2, 256, 32, 128)).astype(np.float16)
    s = rng.uniform(0.02, 0.05, 32).astype(np.float32)
    plan = P.Plan(W.c5_plan().blob)
    syms = {"B": 2, "S": 256}
    b = P.Bound(plan, syms, W.param("scale", s))
    want = O.run_typed(plan.blob, syms, {"scale": (O.DTYPE_TYPES["float32"], [32], s.tobytes())}, x)
    want = np.frombuffer(want.tobytes(), np.uint8)
    staged = torch.from_numpy(x.view(np.uint8).reshape(-1).copy()).pin_memory()
    d_src = torch.zeros(x.nbytes, dtype=torch.uint8, device="cuda")
    for round_ in range(3):
        say("ordered download, pinned", pinned, "round", round_)
        d_src.zero_()
        host = torch.full((want.size,), 0x5A, dtype=torch.uint8)
        if pinned:
            host = host.pin_memory()
        busy(ballast)
        d_src.copy_(staged, non_blocking=True)
        ctx.execute_d2h(b, d_src.data_ptr(), d_src.numel(), host.data_ptr(), want.size,
                        source_pinned=1 if pinned else 0,
                        caller_stream=torch.cuda.current_stream().cuda_stream)
        assert np.array_equal(host.numpy(), want)
    torch.cuda.synchronize()


def test_index_select_on_the_null_stream(ctx, ballast):
    from tests.test_gpu_indexed import bind
    rng = np.random.default_rng(11)
    shape, count = (4096, 256), 5000
    idx = rng.integers(0, shape[0], count).astype(np.int64)
    x = rng.standard_normal(shape).astype(np.float32)
    b, ob = bind(shape, "float32", "float16", "int64", idx)
    want = O.execute_indexed(ob, x)
    staged = torch.from_numpy(x.view(np.uint8).reshape(-1).copy()).pin_memory()
    t = torch.zeros(x.nbytes, dtype=torch.uint8, device="cuda")
    out = torch.empty(want.size, dtype=torch.uint8, device="cuda")
    say("null-stream index_select")
    busy(ballast)
    t.copy_(staged, non_blocking=True)
    ctx.index_select_device(b, t.data_ptr(), x.nbytes, out.data_ptr(), want.size, stream=0)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), want.view(np.uint8).reshape(-1))


@pytest.mark.parametrize("pinned", [False, True])
def test_no_wait_calls_back_to_back(ctx, pinned):
    """Uploads in flight together: each call's copies overwrite the wire
    arena the call before may still be reading. Different sources into
    different destinations, one synchronization at the end."""
    n = 6
    cases = [c2_case(2, 32, 32 + 16 * i) for i in range(n)]
    outs = [torch.empty(w.size, dtype=torch.uint8, device="cuda") for _, _, w in cases]
    torch.cuda.synchronize()
    srcs = [torch.from_numpy(x.copy()).pin_memory() if pinned else x for x, _, _ in cases]
    for i, ((x, b, _), out, s) in enumerate(zip(cases, outs, srcs)):
        say("no_wait burst", i, "pinned" if pinned else "pageable")
        ptr = s.data_ptr() if pinned else s.ctypes.data
        ctx.execute_h2d(b, ptr, x.nbytes, out.data_ptr(), out.numel(), no_wait=True,
                        chunk_bytes=16384, source_pinned=1 if pinned else 0)
    ctx.synchronize()
    for (_, _, want), out in zip(cases, outs):
        assert np.array_equal(out.cpu().numpy(), want)


@pytest.mark.parametrize("no_wait", [False, True])
def test_small_uploads_read_their_slot(ctx, no_wait):
    """Uploads of one small chunk from pageable sources: the kernel reads the
    ring slot in page-locked host memory (zero-copy). Back-to-back calls with
    different data reuse the three slots; blocking calls record no slot
    events, no_wait calls do and are synchronized once at the end."""
    n = 8
    cases = [c2_case(2, 32, 32 + 16 * i) for i in range(n)]
    outs = [torch.empty(w.size, dtype=torch.uint8, device="cuda") for _, _, w in cases]
    torch.cuda.synchronize()
    for i, ((x, b, want), out) in enumerate(zip(cases, outs)):
        say("small upload", i, "no_wait" if no_wait else "blocking")
        rep = ctx.execute_h2d(b, x.ctypes.data, x.nbytes, out.data_ptr(), out.numel(),
                              no_wait=no_wait, source_pinned=0)
        assert rep["chunks"] == 1 and not rep["direct_dma"], rep
        if not no_wait:
            assert np.array_equal(out.cpu().numpy(), want), i
    ctx.synchronize()
    for i, ((_, _, want), out) in enumerate(zip(cases, outs)):
        assert np.array_equal(out.cpu().numpy(), want), i


@pytest.mark.parametrize("chunk", [32768, 0], ids=["chunked", "one_chunk"])
@pytest.mark.parametrize("shared", [True, False])
def test_threads_upload_at_once(shared, chunk):
    """Host threads upload at once through one context (its calls are
    serialized) or one context each, sharing the bound plan and its device
    caches; each thread's result equals the oracle's. One chunk: each call's
    kernel reads its ring slot (zero-copy), calls from different threads
    taking turns on one context's slots."""
    import threading
    x, b, want = c2_case(4, 64, 64)
    n, rounds = 4, 5
    ctxs = [P.Context(0)] * n if shared else [P.Context(0) for _ in range(n)]
    outs = [torch.empty(want.size, dtype=torch.uint8, device="cuda") for _ in range(n)]
    torch.cuda.synchronize()
    errors = []

    def work(i):
        try:
            for _ in range(rounds):
                ctxs[i].execute_h2d(b, x.ctypes.data, x.nbytes, outs[i].data_ptr(), outs[i].numel(),
                                    chunk_bytes=chunk, gather_threads=2)
                got = outs[i].cpu().numpy()
                if not np.array_equal(got, want):
                    errors.append((i, int(np.argmax(got != want))))
        except Exception as e:  # reported by the main thread
            errors.append((i, repr(e)))

    say("threads", n, "shared" if shared else "one context each", "chunk", chunk)
    ts = [threading.Thread(target=work, args=(i,)) for i in range(n)]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=60)
    assert not any(t.is_alive() for t in ts)
    for c in set(ctxs):
        c.close()
    assert not errors, errors
