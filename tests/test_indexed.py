"""Indexed plans (wire v2) on the CPU: decoder, binder, encoder, host gather
and launch plans, pinned before any GPU run.

The oracle's indexed restatement (oracle/relx_oracle.py: decode_indexed_plan,
bind_indexed, execute_indexed) is pinned by
  * the reference exporter's frozen v2 bytes (indexed_export_check.py:50-57),
  * the reference's own compiled decoder/binder/executor (oracle/_ref), on
    every dtype pair, both index widths, NaN payloads and repeated rows,
  * numpy's fancy indexing + IEEE float16 conversion for finite values,
and a planted mistake in the oracle must fail the _ref comparison. The
product's decoder, binder and host gather (through the C-ABI, no GPU) are
then compared with the oracle. Cases follow the reference's
libreloc/python/tests/test_indexed_plan.py and
libreloc/python/tests/torch_frontend/test_index_select.py.
"""
import struct

import numpy as np
import pytest

from oracle import ref
from oracle import relx_oracle as O
from sym_amd import pyreloc as P
from sym_amd.encoder import EncodeError, encode_index_select
from tests import golden_io as G

FROZEN = G.goldens()["indexed_v2"]["static_f32_8x5_i64_3_exact"]
PAIRS = [("float32", "float16"), ("float16", "float32"), ("float32", "float32"),
         ("float16", "float16"), ("int8", "int8")]
NEEDS_REF = pytest.mark.skipif(not ref.available(), reason="oracle/_ref not built")


def symbolic(sd="float32", rd="float16", idt="int64"):
    return encode_index_select(["N", "D"], sd, "M", idt, rd)


def table(rng, dtype, shape, specials=True):
    n = int(np.prod(shape))
    if dtype == "float32":
        x = rng.standard_normal(n).astype(np.float32)
        if specials and n >= 12:
            x[:7] = [np.nan, np.inf, -np.inf, 65520.0, 2.0 ** -25, -0.0, 65504.0]
            xb = x.view(np.uint32)
            xb[7], xb[8], xb[9] = 0x7F800001, 0xFFC12345, 0x33000001  # sNaN, payload, just above half ulp
    elif dtype == "float16":
        x = rng.integers(0, 1 << 16, n, dtype=np.uint16).view(np.float16)  # NaNs included
    else:
        x = rng.integers(-128, 128, n, dtype=np.int8)
    return x.reshape(shape)


def oracle_run(blob, syms, idt, idx, x):
    p = O.decode_indexed_plan(blob)
    b = O.bind_indexed(p, syms, O.DTYPE_TYPES[idt], [len(idx)], np.asarray(idx, idt).tobytes())
    return O.execute_indexed(b, x)


# ------------------------------------------------------------ format pins

def test_encoder_reproduces_the_frozen_static_plan():
    assert encode_index_select([8, 5], "float32", 3, "int64").hex() == FROZEN


def test_frozen_plan_decodes_everywhere():
    blob = bytes.fromhex(FROZEN)
    p = O.decode_indexed_plan(blob)
    assert p.symbols == [] and p.axis == 0 and p.policy == O.P_EXACT
    plan = P.load_indexed_plan(blob)
    assert plan.metadata == {
        "source": {"shape": [["const", 8], ["const", 5]], "dtype": "float32"},
        "indices": {"shape": [["const", 3]], "dtype": "int64"},
        "result": {"shape": [["const", 3], ["const", 5]], "dtype": "float32"},
        "axis": 0, "policy": "exact"}
    assert blob[-5:] == struct.pack("<IB", 0, 1)


def test_symbolic_plan_contract():
    """indexed_export_check.py:37-46: symbols by first use, shapes, dtype,
    policy and axis of the select -> cast chain."""
    blob = symbolic()
    assert blob[:8] == b"RPLN\x02\x00\x00\x00"
    plan = P.load_indexed_plan(blob)
    assert plan.symbols == ["N", "D", "M"]
    md = plan.metadata
    assert md["source"]["shape"] == [["symbol", "N"], ["symbol", "D"]]
    assert md["result"]["shape"] == [["symbol", "M"], ["symbol", "D"]]
    assert md["indices"]["dtype"] == "int64"
    assert (md["policy"], md["axis"]) == ("ieee_rne", 0)


@NEEDS_REF
@pytest.mark.parametrize("sd,rd", PAIRS)
@pytest.mark.parametrize("idt", ["int32", "int64"])
def test_reference_accepts_encoder_output(sd, rd, idt):
    assert ref.indexed_decode(symbolic(sd, rd, idt)) is None
    assert ref.indexed_decode(bytes.fromhex(FROZEN)) is None


@pytest.mark.parametrize("sd,rd", [("float32", "bfloat16"), ("int8", "float16"),
                                   ("float16", "int8"), ("bfloat16", "bfloat16")])
def test_encoder_rejects_unsupported_pairs(sd, rd):
    with pytest.raises(EncodeError):
        encode_index_select([8, 5], sd, 3, "int64", rd)


def test_encoder_rejects_bad_indices_and_extents():
    with pytest.raises(EncodeError):
        encode_index_select([8, 5], "float32", 3, "float32")
    with pytest.raises(EncodeError):
        encode_index_select([8, 5], "float32", 0, "int64")


# ------------------------------------------------------------ oracle pins

@NEEDS_REF
@pytest.mark.parametrize("sd,rd", PAIRS)
@pytest.mark.parametrize("idt", ["int32", "int64"])
@pytest.mark.parametrize("shape", [(7,), (7, 129), (7, 3, 5)])
def test_oracle_equals_reference_executor(rng, sd, rd, idt, shape):
    """Row order, repeats and more output rows than source rows
    (test_index_select.py:63-85), NaN payloads included."""
    blob = encode_index_select(list(shape), sd, 9, idt, rd)
    idx = np.array([6, 0, 3, 6, 1, 5, 0, 4, 2], dtype=idt)
    x = table(rng, sd, shape)
    r = ref.IndexedRef(blob, {}, idt, [9], idx.tobytes())
    assert np.array_equal(oracle_run(blob, {}, idt, idx, x), r.execute(x))


@pytest.mark.parametrize("sd,rd", PAIRS)
def test_oracle_equals_numpy_fancy_indexing(rng, sd, rd):
    x = table(rng, sd, (50, 33), specials=False)
    if sd == "float16":
        x = rng.standard_normal((50, 33)).astype(np.float16)
    idx = rng.integers(0, 50, 200)
    got = oracle_run(symbolic(sd, rd), {"N": 50, "D": 33, "M": 200}, "int64", idx, x)
    want = x[idx].astype(np.dtype(rd))
    assert np.array_equal(got, want.reshape(-1).view(np.uint8))


@NEEDS_REF
def test_oracle_cast_rounding_edges_match_reference():
    """test_index_select.py:88-98: ties, overflow to inf, subnormals, NaN."""
    x = np.array([0., -0., 1., 1.00048828125, 65504., 65520., 2 ** -24, 2 ** -25, np.inf, -np.inf,
                  np.nan], dtype=np.float32).reshape(1, -1)
    blob = encode_index_select([1, 11], "float32", 2, "int64", "float16")
    idx = np.array([0, 0], dtype=np.int64)
    got = oracle_run(blob, {}, "int64", idx, x)
    assert np.array_equal(got, ref.IndexedRef(blob, {}, "int64", [2], idx.tobytes()).execute(x))
    fin = np.isfinite(x[0]) | np.isinf(x[0])
    with np.errstate(over="ignore"):
        half = x[[0, 0]].astype(np.float16)
    assert np.array_equal(got.view(np.uint16).reshape(2, -1)[:, fin], half.view(np.uint16)[:, fin])


@NEEDS_REF
def test_planted_index_mistake_fails_against_reference(rng, monkeypatch):
    real = O.execute_indexed

    def off_by_one(b, t):
        b.indices = [min(v + 1, b.source_extents[0] - 1) for v in b.indices]
        return real(b, t)
    monkeypatch.setattr(O, "execute_indexed", off_by_one)
    blob = encode_index_select([7, 5], "float32", 9, "int64", "float16")
    idx = np.array([6, 0, 3, 6, 1, 5, 0, 4, 2], dtype=np.int64)
    x = table(rng, "float32", (7, 5))
    assert not np.array_equal(oracle_run(blob, {}, "int64", idx, x),
                              ref.IndexedRef(blob, {}, "int64", [9], idx.tobytes()).execute(x))


# ------------------------------------------------------------ decoder parity

def _our_decode(blob):
    try:
        P.load_indexed_plan(blob)
        return None
    except P.DecodeError as e:
        return e.offset, str(e).rsplit(" (at byte", 1)[0]


def _oracle_decode(blob):
    try:
        O.decode_indexed_plan(blob)
        return None
    except O.DecodeError as e:
        return e.offset, e.message


def _corruptions(blob):
    out = [blob[:end] for end in range(len(blob))]
    out += [blob + b"\x00", b"FAIL" + blob[4:], blob[:4] + struct.pack("<I", 1) + blob[8:],
            blob[:-5] + struct.pack("<IB", 1, 0), blob[:-1] + b"\xff", blob[:-1] + b"\x01"]
    return [b for b in out if b != blob]


@pytest.mark.parametrize("which", ["symbolic", "frozen"])
def test_decoder_rejects_corruption_like_oracle_and_reference(which):
    """test_indexed_plan.py:68-80, with each error's offset and message."""
    blob = symbolic() if which == "symbolic" else bytes.fromhex(FROZEN)
    for bad in _corruptions(blob):
        ours, want = _our_decode(bad), _oracle_decode(bad)
        assert ours is not None and ours == want, (bad.hex(), ours, want)
        if ref.available():
            assert ref.indexed_decode(bad) == want


def test_decoder_matches_oracle_on_bit_flips(rng):
    blob = symbolic()
    for _ in range(400):
        b = bytearray(blob)
        i = int(rng.integers(0, len(b)))
        b[i] ^= 1 << int(rng.integers(0, 8))
        b = bytes(b)
        assert _our_decode(b) == _oracle_decode(b)
        if ref.available():
            assert ref.indexed_decode(b) == _oracle_decode(b)


def test_wrong_loaders_reject_v2_and_v2_loader_rejects_others():
    blob = symbolic()
    for load in (P.load_plan, P.load_typed_plan):
        with pytest.raises(P.DecodeError):
            load(blob)
    v1 = bytes.fromhex(G.goldens()["typed_v1"]["kCastF32F16Hex"]) \
        if "kCastF32F16Hex" in G.goldens()["typed_v1"] else None
    for other in [bytes.fromhex(next(iter(G.goldens()["typed_v1"].values()))),
                  bytes.fromhex(next(iter(G.goldens()["layout_v0"].values())))] + ([v1] if v1 else []):
        with pytest.raises(P.DecodeError):
            P.load_indexed_plan(other)


# ------------------------------------------------------------ binder parity

BAD_BINDINGS = [([-1], {}), ([8], {}), ([], {}), ([0], {"N": 0}), ([0], {"D": 0}),
                ([0], {"D": 2 ** 62}), ([0], {"M": 2}), ([0], {"extra": 1})]


def _bind_ours(blob, syms, op):
    try:
        P.bind_indexed(P.load_indexed_plan(blob), syms, op)
        return None
    except P.BindError as e:
        return str(e)


def _bind_oracle(blob, syms, op):
    try:
        O.bind_indexed(O.decode_indexed_plan(blob), syms, O.DTYPE_TYPES[op[0]], op[1], op[2])
        return None
    except O.BindError as e:
        return str(e)


@pytest.mark.parametrize("values,symbols", BAD_BINDINGS)
def test_binder_rejects_invalid_values_and_shapes(values, symbols):
    """test_indexed_plan.py:83-87 with each message compared."""
    v = np.asarray(values, dtype="<i8")
    syms = {"N": 8, "D": 5, "M": len(values), **symbols}
    op = ("int64", [len(values)], v.tobytes())
    ours = _bind_ours(symbolic(), syms, op)
    assert ours is not None and ours == _bind_oracle(symbolic(), syms, op)
    if ref.available():
        with pytest.raises(RuntimeError) as e:
            ref.IndexedRef(symbolic(), syms, "int64", [len(values)], v.tobytes())
        assert str(e.value) == "bind: " + ours


@pytest.mark.parametrize("operand", [("int32", [3], bytes(12)), ("int64", [3, 1], bytes(24)),
                                     ("int64", [2], bytes(16)), ("int64", [3], bytes(23))])
def test_binder_rejects_index_descriptor_and_bytes(operand):
    """test_indexed_plan.py:90-98."""
    for syms in ({"N": 8, "D": 5, "M": 3}, {"N": 8, "M": 3}):
        ours = _bind_ours(symbolic(), syms, operand)
        assert ours is not None and ours == _bind_oracle(symbolic(), syms, operand)


def test_symbolic_result_must_agree_with_both_operands():
    """test_indexed_plan.py:101-109: the result's last extent names N, not D."""
    blob = symbolic()
    sym_d = struct.pack("<IBI", 1, 0, 1)
    at = blob.rfind(sym_d)
    bad = blob[:at] + struct.pack("<IBI", 1, 0, 0) + blob[at + 9:]
    op = ("int64", [3], np.array([7, 0, 7], "<i8").tobytes())
    msg = _bind_ours(bad, {"N": 8, "D": 5, "M": 3}, op)
    assert msg is not None and "result shape" in msg
    assert msg == _bind_oracle(bad, {"N": 8, "D": 5, "M": 3}, op)


def test_output_size_overflow_is_checked():
    """test_index_select.py:131-135."""
    blob = encode_index_select([1, 2 ** 60], "float32", 3, "int64")
    with pytest.raises(P.BindError, match="overflow"):
        P.bind_indexed(P.load_indexed_plan(blob), {}, ("int64", [3], bytes(24)))


def test_bind_facts_and_ownership():
    plan = P.load_indexed_plan(symbolic())
    idx = np.array([7, 0, 7], dtype="<i8")
    b = P.bind_indexed(plan, {"N": 8, "D": 5, "M": 3}, ("int64", [3], idx.tobytes()))
    idx[:] = 1
    assert b.indices == [7, 0, 7]
    assert b.source_extents == [8, 5] and b.result_extents == [3, 5]
    assert (b.table_bytes, b.source_bytes, b.destination_bytes, b.parameter_bytes) == (160, 60, 30, 24)
    assert b.indexed and b.typed and b.stage_count == 1
    i32 = np.array([1, 2], dtype="<i4")
    b2 = P.bind_indexed_from_pointer(P.load_indexed_plan(symbolic(idt="int32")),
                                     {"N": 8, "D": 5, "M": 2}, "int32", [2], i32.ctypes.data, 8)
    assert b2.indices == [1, 2] and b2.parameter_bytes == 8
    with pytest.raises(ValueError):
        P.bind_indexed(plan, {"N": 8, "D": 5, "M": 3}, ("int64", [3]))
    with pytest.raises(ValueError):
        P.bind_indexed_from_pointer(plan, {"N": 8, "D": 5, "M": 3}, "int64", [3], 0, 24)


def test_indexed_plans_do_not_bind_as_typed():
    with pytest.raises(P.BindError):
        P.bind_typed(P.Plan(symbolic()), {"N": 8, "D": 5, "M": 3}, {})


# ------------------------------------------------------------ product host gather

def _host_stage(b, k, x):
    out = np.empty(b.info.wire_bytes_at[k], np.uint8)
    P.host_stage(b, k, x.ctypes.data, out.ctypes.data, threads=3)
    return out


@pytest.mark.parametrize("sd,rd", PAIRS)
@pytest.mark.parametrize("idt", ["int32", "int64"])
@pytest.mark.parametrize("shape", [(7,), (7, 129), (7, 3, 5), (300, 1000)])
def test_host_gather_matches_oracle(rng, sd, rd, idt, shape):
    """The staging-side gather the H2D path runs (relx_host_stage), at every
    host boundary the plan allows."""
    count = 9 if shape[0] == 7 else 700
    idx = np.array([6, 0, 3, 6, 1, 5, 0, 4, 2], dtype=idt) if count == 9 else \
        rng.integers(0, shape[0], count).astype(idt)
    blob = encode_index_select(list(shape), sd, count, idt, rd)
    x = table(rng, sd, shape)
    b = P.bind_indexed(P.load_indexed_plan(blob), {}, (idt, [count], idx.tobytes()))
    want = oracle_run(blob, {}, idt, idx, x)
    for k in range(b.info.host_stages_max + 1):
        got = _host_stage(b, k, x)
        if k == b.stage_count:
            assert np.array_equal(got, want)
        else:  # boundary 0: the selected rows, bit for bit
            assert np.array_equal(got, x.reshape(shape[0], -1)[idx.astype(np.int64)].reshape(-1).view(np.uint8))


# ------------------------------------------------------------ launch plans

@pytest.mark.parametrize("sd,rd", PAIRS)
@pytest.mark.parametrize("shape,count", [((8, 5), 3), ((7, 129), 9), ((1000, 4096), 512),
                                         ((1 << 20, 64), 4096), ((100, 7), 64), ((5,), 11),
                                         ((64, 3, 5), 17)])
def test_launch_plans_verify(sd, rd, shape, count):
    blob = encode_index_select(list(shape), sd, count, "int64", rd)
    idx = (np.arange(count) * 7 + 2) % shape[0]
    b = P.bind_indexed(P.load_indexed_plan(blob), {}, ("int64", [count], idx.astype("<i8").tobytes()))
    for k in range(b.info.host_stages_max + 1):
        for chunk in (0, 4096, 1 << 20):
            assert P.verify_launches(b, k, chunk) >= 3


# ------------------------------------------------------------ dispatch API (no launch)

def _view(a, kind="host", offset=0, capacity=None):
    return P.BufferView(a.ctypes.data, a.nbytes if capacity is None else capacity, offset,
                        list(a.shape), [s // a.itemsize for s in a.strides], a.itemsize, kind)


def test_index_select_program_checks_the_table_view():
    """test_index_select.py:115-128 and checkView's indexed branch."""
    plan = P.load_indexed_plan(encode_index_select([8, 4], "float32", 2, "int64"))
    b = P.bind_indexed(plan, {}, ("int64", [2], np.array([7, 0], "<i8").tobytes()))
    x = np.zeros((8, 4), np.float32)
    prog = P.prepare_index_select_program(b, _view(x))
    cap = P.query_capability(prog, "h2d", "cuda")
    assert [r["implementation"] for r in cap["eligible"]] == ["hip_relayout"]
    with pytest.raises(P.TransferError, match="plan_mismatch"):
        P.prepare_index_select_program(b, _view(x.reshape(4, 8)))
    with pytest.raises(P.TransferError, match="insufficient_capacity"):
        P.prepare_index_select_program(b, _view(x, capacity=4))
    with pytest.raises(P.TransferError, match="direction_mismatch"):
        P.prepare_index_select_program(b, _view(x, kind="cuda"))
    with pytest.raises(P.TransferError, match="plan_mismatch"):
        P.prepare_index_select_program(b, _view(x.view(np.float16)))
    with pytest.raises(P.TransferError, match="unsupported_layout"):
        P.prepare_index_select_program(b, P.BufferView(x.ctypes.data, x.nbytes, 0, [8, 4], [1, 8],
                                                       4, "host"))
    with pytest.raises(TypeError):
        P.prepare_index_select_program(object(), _view(x))


def test_index_select_has_no_device_to_host_row():
    plan = P.load_indexed_plan(symbolic())
    b = P.bind_indexed(plan, {"N": 8, "D": 5, "M": 3}, ("int64", [3], np.array([7, 0, 7], "<i8").tobytes()))
    x = np.zeros((8, 5), np.float32)
    prog = P.prepare_index_select_program(b, _view(x))
    cap = P.query_capability(prog, "d2h", "cuda")
    assert cap["eligible"] == [] and cap["excluded"][0]["reason"] == "host_index_select"
    out = np.zeros((3, 5), np.float16)
    with pytest.raises(P.TransferError):
        P.prepare_dispatch(prog, _view(x), _view(out), "d2h")
    rows = [r["implementation"] for r in P.query_capability(prog, "h2d", "cuda")["eligible"]]
    assert rows == ["hip_relayout", "hip_relayout@1"]
