"""Random plans on the CPU (tests/fuzz_plans.py): transposes, reshapes, pads,
casts, quantize and dequantize over random shapes, encoded by
sym_amd.encoder.

For every draw: the oracle's result equals the reference's compiled CPU
executor's (oracle/_ref), bit for bit, or both reject the plan; the
library binds exactly the plans they accept; and every kernel launch the
library would make, at every host boundary, chunked and whole, in both
directions, passes the host-side launch verifier. The same draws run on the
GPU in tests/test_gpu_fuzz.py."""
import warnings

import numpy as np
import pytest

from oracle import ref
from oracle import relx_oracle as O
from sym_amd import pyreloc as P
from tests import fuzz_plans as F

SEEDS = range(0, 400)


def oracle_result(plan, src):
    """The oracle's result bytes, or the exception it raised."""
    try:
        with warnings.catch_warnings():
            warnings.simplefilter("ignore")
            if plan.typed:
                return O.run_typed(plan.blob, {}, {}, src).tobytes()
            return O.execute_layout(O.bind(O.decode_plan(plan.blob), {}), src.tobytes())
    except (O.DecodeError, O.BindError, O.ExecutionError) as e:
        return e


@pytest.mark.parametrize("block", range(8))
def test_random_plans(block):
    n_run = 0
    for seed in SEEDS[block::8]:
        r = F.make_plan(seed)
        if r is None:
            continue
        plan, src, ops = r
        want = oracle_result(plan, src)
        if ref.available():
            try:
                if plan.typed:
                    got = ref.TypedRef(plan.blob, {}, {}).execute(src).tobytes()
                else:
                    got = ref.LayoutRef(plan.blob, {}).execute(src).tobytes()
            except RuntimeError:
                got = None
            if isinstance(want, Exception):
                assert got is None, (seed, ops, want)
            else:
                assert got == want, (seed, ops)
        try:
            b = P.Bound(P.Plan(plan.blob), {}, {} if plan.typed else None)
        except (P.BindError, P.TransferError) as e:
            assert isinstance(want, Exception), (seed, ops, e)
            continue
        assert not isinstance(want, Exception), (seed, ops, want)
        for k in range(b.info.host_stages_max + 1):
            for chunk in (0, 4096):
                assert P.verify_launches(b, k, chunk) > 0
        n_run += 1
    assert n_run > 30
