"""Artifacts written by sym_amd.artifact run on the MI355X: each recipe is
compiled to a `.reloc`, serialized, admitted again, bound through its own
symbol and parameter declarations, executed through execute_dispatch, and
compared bit for bit with the oracle run on the same plan bytes."""
import sys

import numpy as np
import pytest

from oracle import relx_oracle as O
from sym_amd import artifact as A
from sym_amd import pyreloc as P

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


def _c(v):
    return ["const", v]


def _s(n):
    return ["symbol", n]


def recipes():
    scale_rows = {"dtype": "float32", "extents": [_s("s1")], "kind": "binding", "name": "scale"}
    c3 = {"direction": "h2d",
          "source": {"dtype": "int8", "offset": _c(0), "shape": [_s("s0"), _s("s1")],
                     "strides": [_s("s1"), _c(1)]},
          "operations": [{"axis": 1, "dtype": "float32", "kind": "dequantize", "policy": "affine",
                          "scale": scale_rows, "zero_point": None},
                         {"dtype": "float16", "kind": "cast", "policy": "ieee_rne"},
                         {"kind": "transpose", "perm": [1, 0]}],
          "destination": {"dtype": "float16", "offset": _c(0), "shape": [_s("s1"), _s("s0")],
                          "strides": [_s("s0"), _c(1)]}}
    heads = {"dtype": "float32", "extents": [_c(32)], "kind": "binding", "name": "scale"}
    c5 = {"direction": "h2d",
          "source": {"dtype": "float16", "offset": _c(0),
                     "shape": [_s("B"), _s("S"), _c(32), _c(128)],
                     "strides": [["mul", _c(4096), _s("S")], _c(4096), _c(128), _c(1)]},
          "operations": [{"kind": "transpose", "perm": [0, 2, 1, 3]},
                         {"dtype": "float32", "kind": "cast", "policy": "exact"},
                         {"axis": 1, "dtype": "int8", "kind": "quantize",
                          "policy": "symmetric_rne", "scale": heads, "zero_point": None}],
          "destination": {"dtype": "int8", "offset": _c(0),
                          "shape": [_s("B"), _c(32), _s("S"), _c(128)],
                          "strides": [["mul", _c(4096), _s("S")], ["mul", _c(128), _s("S")],
                                      _c(128), _c(1)]}}
    return {"c3": (c3, (1024, 1536), "int8"), "c5": (c5, (2, 1024, 32, 128), "float16")}


@pytest.mark.parametrize("name", ["c3", "c5"])
def test_written_artifact_runs_against_the_oracle(name):
    rec, shape, dtype = recipes()[name]
    art = A.CompiledArtifact.from_bytes(A.compile_recipe(rec).to_bytes())
    rng = np.random.default_rng(29)
    if dtype == "int8":
        x = rng.integers(-127, 128, shape, dtype=np.int8)
    else:
        x = rng.standard_normal(shape).astype(np.float16)
    syms = art.bind_symbols(list(shape))
    params = {}
    for pname, (pdt, ext) in art.parameter_extents(syms).items():
        params[pname] = (pdt, list(ext), rng.uniform(0.02, 0.05, ext).astype(np.float32).tobytes())
    plan = art.load_plan()
    bound = P.bind_typed(plan, syms, params)
    out = torch.empty(bound.destination_bytes, dtype=torch.uint8, device="cuda")
    say("artifact", name, shape)
    res = P.Resources(0)
    try:
        view = P.BufferView(x.ctypes.data, x.nbytes, 0, list(x.shape),
                            [s // x.itemsize for s in x.strides], x.itemsize, "host")
        rext = list(bound.info.result_extents[:bound.info.result_rank])
        strides, run = [], 1
        for e in reversed(rext):
            strides.append(run)
            run *= e
        dst = P.BufferView(out.data_ptr(), out.numel(), 0, rext, list(reversed(strides)),
                           bound.info.result_width, "cuda", 0)
        P.execute_dispatch(P.prepare_dispatch(bound, view, dst, "h2d"), resources=res,
                           caller_stream=torch.cuda.current_stream().cuda_stream, gather_threads=8)
        torch.cuda.synchronize()
    finally:
        res.close()
    want = O.run_typed(art.plan_bytes, syms,
                       {k: (O.DTYPE_TYPES[v[0]], v[1], v[2]) for k, v in params.items()}, x)
    assert out.cpu().numpy().tobytes() == want.tobytes()
