"""The allocation-free upload (relx_execute_h2d_static) on the MI355X,
called through the C-ABI: its output equals relx_execute_h2d's bit for bit,
on two calls in a row, the second with a smaller input (the scratch keeps
the first call's contents), for a typed plan with parameter tables and a
layout plan; a context that only made such calls holds no wire arena and
no staging ring; sizes beyond the scratch and pageable sources are
rejected before anything runs."""
import ctypes
import sys

import numpy as np
import pytest

from sym_amd import _native as N
from sym_amd import pyreloc as P
from sym_amd import workloads as W

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


def static_call(ctx, bound, src, dst, nbytes):
    """relx_execute_h2d_static through the C-ABI: returns (rc, err, report)."""
    opt = P._options(source_pinned=1)
    rep = N.relx_report()
    err = N.relx_err()
    rc = N.lib().relx_execute_h2d_static(ctx._h, bound._h, src.data_ptr(),
                                         src.numel() * src.element_size(), dst.data_ptr(), nbytes,
                                         ctypes.byref(opt), ctypes.byref(rep), ctypes.byref(err))
    return rc, err, rep


def reference_call(ctx, bound, src, dst, nbytes):
    opt = P._options(source_pinned=1)
    rep = N.relx_report()
    err = N.relx_err()
    rc = N.lib().relx_execute_h2d(ctx._h, bound._h, src.data_ptr(),
                                  src.numel() * src.element_size(), dst.data_ptr(), nbytes,
                                  ctypes.byref(opt), ctypes.byref(rep), ctypes.byref(err))
    N.check(rc, err)
    return rep


def c5_case(B, S, seed):
    x, sc = W.c5_input(B, S, seed=seed)
    b = P.Bound(P.Plan(W.c5_plan().blob), {"B": B, "S": S}, W.param("scale", sc))
    return torch.from_numpy(x.view(np.uint8).reshape(-1).copy()).pin_memory(), b, x.size


def c1_case(n, seed):
    x = W.c1_input(n, seed=seed)
    b = P.Bound(P.Plan(W.c1_plan().blob), {"s0": n})
    return torch.from_numpy(x.view(np.uint8).copy()).pin_memory(), b, x.nbytes


@pytest.mark.parametrize("kind", ["c5", "c1"])
def test_static_upload_matches_the_allocating_upload(kind):
    ctx = P.Context(0)  # a fresh context: the static calls must allocate nothing in it
    ref_ctx = P.Context(0)
    try:
        # two calls in a row, the second smaller: 32 MiB then 1 MiB of wire
        shapes = [(4, 1024), (1, 128)] if kind == "c5" else [(1 << 23,), (1 << 18,)]
        for i, shape in enumerate(shapes):
            src, b, out_bytes = c5_case(*shape, seed=11 + i) if kind == "c5" else c1_case(*shape, 11 + i)
            say("no-alloc", kind, shape)
            got = torch.full((out_bytes + 256,), 0x5A, dtype=torch.uint8, device="cuda")
            want = torch.full((out_bytes + 256,), 0x5A, dtype=torch.uint8, device="cuda")
            torch.cuda.synchronize()
            rc, err, rep = static_call(ctx, b, src, got, out_bytes)
            N.check(rc, err)
            ref = reference_call(ref_ctx, b, src, want, out_bytes)
            torch.cuda.synchronize()
            assert torch.equal(got, want), (kind, shape)
            assert (got[out_bytes:] == 0x5A).all()  # nothing past the destination
            assert rep.destination_bytes == ref.destination_bytes == out_bytes
            assert rep.direct_dma == 1 and rep.wire_boundary == 0
            st = ctx.stats()
            assert st["device_bytes"] == 0 and st["pinned_bytes"] == 0, st
    finally:
        ctx.close()
        ref_ctx.close()


def test_static_upload_rejects_what_it_cannot_hold():
    ctx = P.Context(0)
    try:
        # a wire of 64 MiB exceeds the 63 MiB the scratch stages
        src, b, out_bytes = c5_case(8, 1024, 3)
        dst = torch.empty(out_bytes, dtype=torch.uint8, device="cuda")
        rc, err, _ = static_call(ctx, b, src, dst, out_bytes)
        assert rc != 0 and err.code.decode() == "insufficient_capacity", err.message
        # a pageable source would need the staging ring
        x = np.zeros(1 << 20, np.float32)
        b1 = P.Bound(P.Plan(W.c1_plan().blob), {"s0": x.size})
        dst1 = torch.empty(x.nbytes, dtype=torch.uint8, device="cuda")
        opt = P._options(source_pinned=0)
        err = N.relx_err()
        rep = N.relx_report()
        rc = N.lib().relx_execute_h2d_static(ctx._h, b1._h, x.ctypes.data, x.nbytes,
                                             dst1.data_ptr(), x.nbytes, ctypes.byref(opt),
                                             ctypes.byref(rep), ctypes.byref(err))
        assert rc != 0 and err.code.decode() == "invalid_options", err.message
        assert err.completion != 2  # rejected before anything was enqueued: completion known
        assert ctx.stats()["device_bytes"] == 0
    finally:
        ctx.close()
