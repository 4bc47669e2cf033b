"""Random plans on the MI355X (tests/fuzz_plans.py; the CPU side of the same
draws is tests/test_fuzz.py): each plan the oracle accepts runs host ->
device at every host boundary (pageable and pinned sources, default and
4 KiB chunks), device-resident, and device -> host (pageable and pinned
destinations), and every result equals the oracle's bit for bit."""
import sys
import warnings

import numpy as np
import pytest

from oracle import relx_oracle as O
from sym_amd import encoder as EN
from sym_amd import pyreloc as P
from tests import fuzz_plans as F

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

# RELX_FUZZ_SEEDS=lo:hi widens the draw (the suite runs 0:400)
import os  # noqa: E402
_lo, _hi = (int(v) for v in os.environ.get("RELX_FUZZ_SEEDS", "0:400").split(":"))
SEEDS = range(_lo, _hi)


def say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    assert torch.cuda.is_available(), "a GPU test needs the MI355X"
    c = P.Context(0)
    yield c
    c.close()


def oracle_bytes(plan, src):
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        try:
            if plan.typed:
                return O.run_typed(plan.blob, {}, {}, src).tobytes()
            return O.execute_layout(O.bind(O.decode_plan(plan.blob), {}), src.tobytes())
        except (O.DecodeError, O.BindError, O.ExecutionError):
            return None


@pytest.mark.parametrize("block", range(8))
def test_random_plans_on_the_gpu(ctx, block):
    n_run = 0
    for seed in SEEDS[block::8]:
        r = F.make_plan(seed)
        if r is None:
            continue
        plan, src, ops = r
        want = oracle_bytes(plan, src)
        if want is None:
            continue
        b = P.Bound(P.Plan(plan.blob), {}, {} if plan.typed else None)
        out_bytes = b.destination_bytes if plan.typed else b.total_bytes
        assert out_bytes == len(want)
        src_u8 = src.view(np.uint8).reshape(-1)
        out = torch.empty(max(out_bytes, 1), dtype=torch.uint8, device="cuda")
        for k in range(b.info.host_stages_max + 1):
            for pinned, chunk in ((False, 0), (True, 4096 if seed % 3 == 0 else 0)):
                say("fuzz seed", seed, "kernel", b.kernel, "h2d k", k, "pinned", pinned, "chunk", chunk)
                s = torch.from_numpy(src_u8.copy()).pin_memory() if pinned else None
                ptr, nb = (s.data_ptr(), s.numel()) if pinned else (src.ctypes.data, src.nbytes)
                # the fill runs on torch's stream: the call is ordered after it
                out.fill_(0xA5)
                ctx.execute_h2d(b, ptr, nb, out.data_ptr(), out_bytes, host_stages=k,
                                chunk_bytes=chunk, source_pinned=1 if pinned else 0,
                                caller_stream=torch.cuda.current_stream().cuda_stream)
                torch.cuda.synchronize()
                assert out[:out_bytes].cpu().numpy().tobytes() == want, (seed, ops, k, pinned, chunk)
        d_src = torch.from_numpy(src_u8.copy()).cuda()
        say("fuzz seed", seed, "device-resident")
        out.fill_(0xA5)
        ctx.relayout_device(b, d_src.data_ptr(), out.data_ptr(),
                            stream=torch.cuda.current_stream().cuda_stream)
        ctx.synchronize()
        torch.cuda.synchronize()
        assert out[:out_bytes].cpu().numpy().tobytes() == want, (seed, ops, "device")
        for pinned in (False, True):
            say("fuzz seed", seed, "d2h pinned", pinned)
            host = torch.full((max(out_bytes, 1),), 0xA5, dtype=torch.uint8)
            if pinned:
                host = host.pin_memory()
            ctx.execute_d2h(b, d_src.data_ptr(), d_src.numel(), host.data_ptr(), out_bytes,
                            chunk_bytes=4096 if seed % 2 else 0, source_pinned=1 if pinned else 0,
                            caller_stream=torch.cuda.current_stream().cuda_stream)
            assert host[:out_bytes].numpy().tobytes() == want, (seed, ops, "d2h", pinned)
        n_run += 1
    assert n_run > min(30, len(SEEDS) // 16)


# Plans of the encoder's pad rules (a same-fill pad widened, a padded axis
# kept through a reshape that merges the axes before it, then transposed),
# at sizes that take several kernel tiles; the truth is numpy's.
RULE_CASES = [
    ([64, 96, 48], [EN.Pad(2, 3, 5, 1.5), EN.Pad(2, 1, 0, 1.5), EN.Reshape((64 * 96, 57)),
                    EN.Transpose((1, 0))]),
    ([40, 3, 130], [EN.Pad(0, 2, 6), EN.Reshape((48, 390))]),
    ([6, 4, 256], [EN.Pad(2, 0, 64), EN.Reshape((24, 320)), EN.Transpose((1, 0))]),
]


def _numpy_rule(shape, ops):
    x = np.arange(int(np.prod(shape)), dtype=np.float32).reshape(shape)
    for op in ops:
        if isinstance(op, EN.Pad):
            w = [(0, 0)] * x.ndim
            w[op.axis] = (op.lo, op.hi)
            x = np.pad(x, w, constant_values=op.value)
        elif isinstance(op, EN.Reshape):
            x = x.reshape(op.to)
        else:
            x = x.transpose(op.perm)
    return np.ascontiguousarray(x).tobytes()


@pytest.mark.parametrize("case", range(len(RULE_CASES)))
def test_encoder_rule_plans_on_the_gpu(ctx, case):
    shape, ops = RULE_CASES[case]
    plan = EN.encode(shape, "float32", ops)
    src = np.arange(int(np.prod(shape)), dtype=np.float32).reshape(shape)
    want = _numpy_rule(shape, ops)
    assert oracle_bytes(plan, src) == want
    b = P.Bound(P.Plan(plan.blob), {}, None)
    assert b.total_bytes == len(want)
    out = torch.empty(len(want), dtype=torch.uint8, device="cuda")
    for chunk in (0, 4096):
        say("encoder rule case", case, "kernel", b.kernel, "h2d chunk", chunk)
        out.fill_(0xA5)
        ctx.execute_h2d(b, src.ctypes.data, src.nbytes, out.data_ptr(), len(want),
                        chunk_bytes=chunk, caller_stream=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert out.cpu().numpy().tobytes() == want, (case, chunk)
    say("encoder rule case", case, "device-resident")
    d_src = torch.from_numpy(src.view(np.uint8).reshape(-1).copy()).cuda()
    out.fill_(0xA5)
    ctx.relayout_device(b, d_src.data_ptr(), out.data_ptr(),
                        stream=torch.cuda.current_stream().cuda_stream)
    ctx.synchronize()
    torch.cuda.synchronize()
    assert out.cpu().numpy().tobytes() == want, (case, "device")
