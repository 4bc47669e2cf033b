"""The recipe encoder against the reference compiler's own outputs.

* every corpus plan (17 layout, 16 typed) re-encoded from its recipe is
  byte-identical to the committed compiler output;
* the two exported example plans match the digests the reference recorded
  (docs/runtime-evidence/cuda.json: split_transpose = config C1's plan);
* the five config plans, executed by the reference's own compiled CPU
  executor (oracle/_ref) and by the numpy oracle, equal a direct numpy
  replay of the recipe.
"""
import hashlib

import numpy as np
import pytest

from oracle import ref, relx_oracle as O
from sym_amd import encoder as EN
from sym_amd import recipe_json as RJ
from sym_amd import workloads as W
from tests import golden_io as G


def _layout_ops(meta):
    out = []
    for op in meta["ops"]:
        if op["kind"] == "transpose":
            out.append(EN.Transpose(tuple(op["perm"])))
        elif op["kind"] == "reshape":
            out.append(EN.Reshape(tuple(op["to"])))
        else:
            out.append(EN.Pad(op["axis"], op["lo"], op["hi"], op["value"]))
    return out


DT = {"f32": "float32", "f16": "float16", "i8": "int8"}


@pytest.mark.parametrize("meta,blob", G.layout_fixtures(), ids=[m["name"] for m, _ in G.layout_fixtures()])
def test_layout_corpus_bytes(meta, blob):
    assert EN.encode(meta["src_shape"], DT[meta["dtype"]], _layout_ops(meta)).blob == blob


@pytest.mark.parametrize("meta,blob", G.typed_fixtures(), ids=[m["name"] for m, _ in G.typed_fixtures()])
def test_typed_corpus_bytes(meta, blob):
    assert RJ.encode_recipe(meta["recipe"]).blob == blob


def test_exported_plan_digests():
    digests = {d["recipe"]: d for d in G.goldens()["exported_plan_digests"]}
    c1 = W.c1_plan()
    assert len(c1.blob) == digests["split_transpose"]["plan_bytes"]
    assert hashlib.sha256(c1.blob).hexdigest() == digests["split_transpose"]["plan_sha256"]
    tp = EN.encode([2, 3, 4], "float32", [EN.Transpose((1, 2, 0)), EN.Pad(0, 1, 2, 1.5)])
    assert hashlib.sha256(tp.blob).hexdigest() == digests["transpose_pad"]["plan_sha256"]


def _f16_bits_of(x32):
    return O.narrow_f32_f16_bits(np.ascontiguousarray(x32, np.float32).view(np.uint32))


def small_cases(rng):
    """(name, plan, symbols, params, source, expected result bytes) at sizes
    the CPU checks finish quickly; expected values come from numpy replays
    of each recipe built on the oracle's pinned scalar arithmetic."""
    out = []
    x = W.c1_input(4096)
    out.append(("c1", W.c1_plan(), {"s0": 4096}, {}, x, x.reshape(64, 64).T.copy().tobytes()))
    x = W.c2_input(2, 3, 16, 24)
    padded = np.pad(x, [(0, 0), (0, 1), (0, 0), (0, 0)])
    out.append(("c2", W.c2_plan(2, 3, 16, 24), {}, {}, x,
                _f16_bits_of(padded.transpose(0, 2, 3, 1)).tobytes()))
    q, s = W.c3_input(96, 128)
    deq = O.dequantize_s8_f32(q, s[None, :], np.int32(0))
    out.append(("c3", W.c3_plan(), {"s0": 96, "s1": 128}, W.param("scale", s), q,
                _f16_bits_of(deq.T).tobytes()))
    q = rng.integers(-127, 128, (64, 80), dtype=np.int8)
    s = W.scales(64, rng)
    out.append(("c4", W.c4_plan(), {"s0": 64, "s1": 80}, W.param("scale", s), q,
                _f16_bits_of(O.dequantize_s8_f32(q, s[:, None], np.int32(0))).tobytes()))
    x, s = W.c5_input(2, 16, 32, 128)
    inv = (np.float32(1) / s).astype(np.float32)
    wid = x.transpose(0, 2, 1, 3).astype(np.float32)
    out.append(("c5", W.c5_plan(), {"B": 2, "S": 16}, W.param("scale", s), x,
                O.quantize_f32_s8(wid, inv[None, :, None, None]).tobytes()))
    return out


@pytest.mark.skipif(not ref.available(), reason="oracle/_ref not built (needs /root/reference)")
def test_config_plans_through_the_reference_executor(rng):
    for name, plan, syms, params, src, expected in small_cases(rng):
        if plan.typed:
            got = ref.TypedRef(plan.blob, syms, params).execute(src)
        else:
            got = ref.LayoutRef(plan.blob, syms).execute(src)
        assert got.tobytes() == expected, name


def test_config_plans_through_the_oracle(rng):
    for name, plan, syms, params, src, expected in small_cases(rng):
        if plan.typed:
            p = {k: (O.DTYPE_TYPES[d], s, b) for k, (d, s, b) in params.items()}
            got = O.run_typed(plan.blob, syms, p, src).tobytes()
        else:
            got = O.execute_layout(O.bind(O.decode_plan(plan.blob), syms), src.tobytes())
        assert got == expected, name


def test_encoder_rejections():
    with pytest.raises(EN.EncodeError):
        EN.encode([4, 6], "float32", [EN.Reshape((5, 5))])
    with pytest.raises(EN.EncodeError):  # a pad cannot fold through a per-channel stage
        EN.encode([4, 6], "float32", [EN.Pad(0, 1, 1, 0.0),
                                       EN.Quantize(EN.BindingParam("s", "float32", (6,)), axis=1)])
    with pytest.raises(EN.EncodeError):
        EN.encode([4], "int8", [EN.Cast("float16")])
