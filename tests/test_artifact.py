"""`.reloc` artifacts without the MLIR compiler (sym_amd/artifact.py), on
the CPU:

* every typed corpus artifact the reference's exporter wrote
  (tests/golden/corpus/typed/*.reloc) is admitted and serializes back to
  the same bytes;
* the writer regenerates each of them byte for byte from its recipe alone
  (plan bytes, manifest, both digests; the MLIR text hashes to the
  exporter's recorded input_sha256);
* the recorded export of the README plan (C1) pins the constraints,
  symbols and plan digest of a symbolic layout artifact;
* tampered artifacts are refused with the reference's messages;
* artifacts for the five workloads and an indexed recipe are written,
  admitted, and bind."""
import base64
import glob
import hashlib
import json
import os

import pytest

from sym_amd import artifact as A
from sym_amd import pyreloc as P
from tests import golden_io as G

CORPUS = sorted(glob.glob(os.path.join(G.CORPUS, "typed", "*.reloc")))


def _c(v):
    return ["const", v]


def _s(n):
    return ["symbol", n]


def descriptor(shape, dtype):
    strides, run = [], 1
    for d in reversed(shape):
        strides.append(run)
        run *= d
    return {"dtype": dtype, "offset": _c(0), "shape": [_c(d) for d in shape],
            "strides": [_c(s) for s in reversed(strides)]}


@pytest.mark.parametrize("path", CORPUS, ids=[os.path.basename(p) for p in CORPUS])
def test_corpus_artifact_round_trips_byte_for_byte(path):
    data = open(path, "rb").read()
    art = A.CompiledArtifact.from_bytes(data)
    assert art.to_bytes() == data
    assert art.format_version == 2 and art.typed and not art.indexed


@pytest.mark.parametrize("path", CORPUS, ids=[os.path.basename(p) for p in CORPUS])
def test_writer_regenerates_the_exporters_artifact(path):
    data = open(path, "rb").read()
    payload = json.loads(data)
    recipe = A.Recipe(payload["recipe"])
    mlir = A.emit_mlir(recipe).encode()
    assert hashlib.sha256(mlir).hexdigest() == payload["manifest"]["input_sha256"]
    art = A.compile_recipe(payload["recipe"], compiler=payload["manifest"]["compiler"])
    assert art.plan_bytes == base64.b64decode(payload["plan_base64"])
    assert art.manifest == payload["manifest"]
    assert art.to_bytes() == data


def c1_recipe():
    n64 = ["floordiv", _s("s0"), 64]
    return {"direction": "h2d",
            "source": {"dtype": "float32", "offset": _c(0), "shape": [_s("s0")], "strides": [_c(1)]},
            "operations": [{"kind": "reshape", "shape": [n64, _c(64)]},
                           {"kind": "transpose", "perm": [1, 0]}],
            "destination": {"dtype": "float32", "offset": _c(0), "shape": [_c(64), n64],
                            "strides": [n64, _c(1)]}}


def test_readme_plan_artifact_matches_the_recorded_export():
    rec = {d["recipe"]: d for d in G.goldens()["exported_plan_digests"]}["split_transpose"]
    art = A.compile_recipe(c1_recipe())
    assert art.format_version == 1 and not art.typed
    assert art.manifest["plan_sha256"] == rec["plan_sha256"]
    assert len(art.plan_bytes) == rec["plan_bytes"]
    assert art.manifest["constraints"] == rec["constraints"]
    assert art.manifest["symbols"] == rec["symbols"]
    again = A.CompiledArtifact.from_bytes(art.to_bytes())
    assert again.to_bytes() == art.to_bytes()
    assert again.bind_symbols([16777216]) == {"s0": 16777216}
    with pytest.raises(A.ArtifactError, match="divisibility"):
        again.bind_symbols([100])
    b = P.bind(again.load_plan(), again.bind_symbols([256]))
    assert b.extents and b.total_bytes == 1024


def _tamper(data, fn):
    payload = json.loads(data)
    fn(payload)
    return json.dumps(payload, sort_keys=True, separators=(",", ":")).encode() + b"\n"


def test_tampered_artifacts_are_refused():
    data = open(os.path.join(G.CORPUS, "typed", "quantize_channel_transpose_sym.reloc"), "rb").read()

    def refuse(fn, match):
        with pytest.raises(A.ArtifactError, match=match):
            A.CompiledArtifact.from_bytes(_tamper(data, fn))

    def flip_plan(p):
        b = bytearray(base64.b64decode(p["plan_base64"]))
        b[-1] ^= 1
        p["plan_base64"] = base64.b64encode(bytes(b)).decode()

    refuse(flip_plan, "plan digest mismatch|invalid plan|does not match")
    refuse(lambda p: p.update(format_version=1), "format version does not match")
    refuse(lambda p: p.update(format_version=7), "format version mismatch")
    refuse(lambda p: p.pop("recipe"), "invalid artifact fields")
    refuse(lambda p: p["manifest"].update(input_sha256="0" * 64), "input digest mismatch")
    refuse(lambda p: p["manifest"]["compiler"].update(name="other"), "unsupported compiler")
    refuse(lambda p: p["manifest"].update(symbols=[]), "symbol order")
    refuse(lambda p: p["manifest"].update(extra=1), "invalid success fields")
    refuse(lambda p: p["manifest"]["stages"][0].update(axis=0), "channel axis mismatch")
    refuse(lambda p: p["manifest"]["stages"][0].update(policy="exact"), "does not match the recipe")
    refuse(lambda p: p["manifest"]["parameters"][0].update(name="t"), "parameters do not match")
    refuse(lambda p: p["manifest"]["logical_source"].update(dtype="float16"), "logical source")
    refuse(lambda p: p["recipe"]["operations"][0].update(policy="affine"),
           "does not match the recipe transform|input digest")
    with pytest.raises(A.ArtifactError, match="malformed"):
        A.CompiledArtifact.from_bytes(b"{not json")


def test_workload_artifacts_are_written_and_admitted(tmp_path):
    c2 = {"direction": "h2d", "source": descriptor([32, 3, 224, 224], "float32"),
          "operations": [{"axis": 1, "fill": {"bits": 0, "dtype": "float32"}, "hi": _c(1),
                          "kind": "pad", "lo": _c(0)},
                         {"kind": "transpose", "perm": [0, 2, 3, 1]},
                         {"dtype": "float16", "kind": "cast", "policy": "ieee_rne"}],
          "destination": descriptor([32, 224, 224, 4], "float16")}
    scale = {"dtype": "float32", "extents": [_c(32)], "kind": "binding", "name": "scale"}
    c5 = {"direction": "h2d",
          "source": {"dtype": "float16", "offset": _c(0),
                     "shape": [_s("B"), _s("S"), _c(32), _c(128)],
                     "strides": [["mul", _c(4096), _s("S")], _c(4096), _c(128), _c(1)]},
          "operations": [{"kind": "transpose", "perm": [0, 2, 1, 3]},
                         {"dtype": "float32", "kind": "cast", "policy": "exact"},
                         {"axis": 1, "dtype": "int8", "kind": "quantize", "policy": "symmetric_rne",
                          "scale": scale, "zero_point": None}],
          "destination": {"dtype": "int8", "offset": _c(0),
                          "shape": [_s("B"), _c(32), _s("S"), _c(128)],
                          "strides": [["mul", _c(4096), _s("S")], ["mul", _c(128), _s("S")],
                                      _c(128), _c(1)]}}
    from sym_amd import workloads as W
    for name, rec, plan in (("c2", c2, W.c2_plan()), ("c5", c5, W.c5_plan())):
        art = A.compile_recipe(rec)
        assert art.plan_bytes == plan.blob, name  # the workloads' own plans
        path = tmp_path / (name + ".reloc")
        art.save(path)
        back = A.CompiledArtifact.load(path)
        assert back.to_bytes() == art.to_bytes()
    c5a = A.CompiledArtifact.from_bytes(A.compile_recipe(c5).to_bytes())
    syms = c5a.bind_symbols([8, 1024, 32, 128])
    assert syms == {"B": 8, "S": 1024}
    assert c5a.parameter_extents(syms) == {"scale": ("float32", (32,))}


def test_indexed_artifact():
    rec = {"direction": "h2d", "source": {"dtype": "float32", "offset": _c(0),
                                           "shape": [_s("N"), _c(16)], "strides": [_c(16), _c(1)]},
           "operations": [{"axis": 0, "indices": {"dtype": "int64", "offset": _c(0),
                                                  "shape": [_s("M")], "strides": [_c(1)]},
                           "kind": "index_select"},
                          {"dtype": "float16", "kind": "cast", "policy": "ieee_rne"}],
           "destination": {"dtype": "float16", "offset": _c(0), "shape": [_s("M"), _c(16)],
                           "strides": [_c(16), _c(1)]}}
    art = A.compile_recipe(rec)
    assert art.format_version == 3 and art.indexed and art.manifest["schema_version"] == 3
    assert A.CompiledArtifact.from_bytes(art.to_bytes()).to_bytes() == art.to_bytes()
    plan = art.load_plan()
    assert plan.metadata["policy"] == "ieee_rne" and plan.symbols == ["N", "M"]


def test_decoded_typed_plan_metadata():
    """The plan handle's stage/parameter view the admission reads (reference
    TypedPlanHandle.stages / .parameters / .fills)."""
    data = open(os.path.join(G.CORPUS, "typed", "dequant_channel_runtime_transpose.reloc"), "rb").read()
    plan = A.CompiledArtifact.from_bytes(data).load_plan()
    assert plan.num_stages == 1 and plan.fills == 0
    st = plan.stages[0]
    assert (st["transform"], st["policy"], st["input"], st["output"], st["axis"],
            st["has_channel"]) == ("dequantize", "affine", "int8", "float32", 1, True)
    assert st["input_signedness"] == "signed" and st["scale"] == "binding"
    assert [(p["name"], p["dtype"], p["rank"], p["role"]) for p in plan.parameters] == [
        ("scales", "float32", 1, "scale"), ("zero_points", "int32", 1, "zero_point")]
