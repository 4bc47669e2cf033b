"""Pin the CPU oracle (oracle/relx_oracle.py) before trusting it.

Each check is chosen so that a plausible mistake in the oracle (a dropped
term, a wrong rounding, a swapped operand, a wrong stride) fails it:

* the reference's golden corpus (libreloc/test/corpus): expected bits and
  sha256 per binding, produced by the reference's own exporter + executor;
* the layout corpus replayed with numpy transpose/reshape/pad (the reference's
  own oracle method, libreloc/python/tests/oracle.py:57-75);
* the typed witness vectors of docs/reloc-typed-semantics.md section 6;
* library routines: numpy's IEEE float16 conversion, exact float64 products;
* exhaustive enumeration (all 65536 binary16 patterns);
* the reference's structural decode expectations (DecodeTest.cpp,
  TypedDecodeTest.cpp) and bind/chunk closed forms (BindTest.cpp:158-178,
  ChunkScheduleTest.cpp:56-146).
"""
import hashlib
import struct

import numpy as np
import pytest

from oracle import relx_oracle as O
from tests import golden_io as G


def _params(meta):
    return {k: (O.DTYPE_TYPES[d], shape, data) for k, (d, shape, data) in G.fixture_params(meta).items()}


# --------------------------------------------------------------- typed corpus

TYPED = G.typed_fixtures()


@pytest.mark.parametrize("meta,blob", TYPED, ids=[m["name"] for m, _ in TYPED])
def test_typed_corpus_expected_bits_and_sha(meta, blob):
    for b in meta["bindings"]:
        src = G.bits_array(b["source"])
        out = O.run_typed(blob, b["symbols"], _params(meta), src)
        exp = G.bits_array(b["expected"])
        got = out.view(exp.dtype)
        assert np.array_equal(got, exp), (meta["name"], b["symbols"])
        assert hashlib.sha256(got.tobytes()).hexdigest() == b["expected"]["sha256"]


@pytest.mark.parametrize("meta,blob", TYPED, ids=[m["name"] for m, _ in TYPED])
def test_typed_corpus_footprints(meta, blob):
    plan = O.decode_typed_plan(blob)
    for b in meta["bindings"]:
        bound = O.bind_typed(plan, b["symbols"], _params(meta))
        fp = b["footprints"]["h2d"]
        assert bound.source_bytes == fp["source_bytes"]
        assert bound.destination_bytes == fp["destination_bytes"]
        assert bound.parameter_bytes == fp["parameter_bytes"]
        # the reference's cpu_reference H2D wire is the last boundary's bytes
        assert bound.cuts[fp["wire_boundary"]].bytes == fp["wire_bytes"]


def test_typed_corpus_plan_sha_matches_manifest():
    for meta, blob in TYPED:
        assert hashlib.sha256(blob).hexdigest() == meta["plan_sha256"]


# -------------------------------------------------------------- layout corpus

def _eval_dim(d, binding):
    if isinstance(d, int):
        return d
    parts = d.split()
    if len(parts) == 3 and parts[1] == "floordiv":
        return binding[parts[0]] // int(parts[2])
    return binding[d]


def _numpy_replay(meta, binding, src):
    a = src
    for op in meta["ops"]:
        if op["kind"] == "transpose":
            a = np.transpose(a, op["perm"])
        elif op["kind"] == "reshape":
            a = a.reshape([_eval_dim(d, binding) for d in op["to"]])
        else:
            w = [(0, 0)] * a.ndim
            w[op["axis"]] = (op["lo"], op["hi"])
            a = np.pad(a, w, constant_values=a.dtype.type(op["value"]))
    return np.ascontiguousarray(a)


LAYOUT = G.layout_fixtures()
NPD = {"f32": np.float32, "f16": np.float16, "i8": np.int8}


@pytest.mark.parametrize("meta,blob", LAYOUT, ids=[m["name"] for m, _ in LAYOUT])
def test_layout_corpus_numpy_replay(meta, blob, rng):
    plan = O.decode_plan(blob)
    bindings = [{}]
    if meta["symbols"]:
        bindings = [{n: c["multiple_of"] * f for n, c in meta["symbols"].items()}
                    for f in range(1, 4)]
    for binding in bindings:
        shape = [_eval_dim(d, binding) for d in meta["src_shape"]]
        dt = NPD[meta["dtype"]]
        n = int(np.prod(shape)) * np.dtype(dt).itemsize
        src = rng.integers(0, 256, n, dtype=np.uint8).view(dt).reshape(shape)
        bound = O.bind(plan, binding)
        got = O.execute_layout(bound, src.tobytes())
        assert got == _numpy_replay(meta, binding, src).tobytes(), (meta["name"], binding)


# -------------------------------------------------------------- wire goldens

def test_worked_example_181_bytes():
    blob = bytes.fromhex(G.goldens()["layout_v0"]["kIdentityHex"])
    assert len(blob) == 181  # docs/reloc-plan-format.md:108-151
    p = O.decode_plan(blob)
    assert p.symbols == [] and p.perm == [0] and [a.name for a in p.axes] == ["x"]
    assert p.src.element_type.kind == O.KIND_INT and p.src.element_type.bitwidth == 32
    assert p.inverse == [[(O.OP_PUSH_DIM, 0)]]
    b = O.bind(p, {})
    assert (b.extents, b.src_strides, b.dst_strides, b.element_size, b.total_bytes) == \
        ([8], [1], [1], 4, 32)


def test_reference_plan_coalesces_to_three_axes():
    # BindTest.cpp:158-178
    p = O.decode_plan(bytes.fromhex(G.goldens()["layout_v0"]["kReferenceHex"]))
    b = O.bind(p, {"N": 32768})
    assert b.extents == [512, 4096, 512]
    assert b.src_strides == [64, 32768, 1]
    assert b.dst_strides == [2097152, 512, 1]
    assert b.L == 512 and b.element_size == 4
    assert b.total_bytes == 512 * 64 * 64 * 512 * 4


def test_typed_goldens_decode_structurally():
    g = G.goldens()["typed_v1"]
    for name, hx in g.items():
        p = O.decode_typed_plan(bytes.fromhex(hx))
        assert p.stages, name
    # TypedDecodeTest.cpp:171-191 (pad_quantize): one inline scale 0.5, fill 1.0 -> code 2
    p = O.decode_typed_plan(bytes.fromhex(g["kPadQuantizeHex"]))
    s = p.stages[0]
    assert s.transform == O.T_QUANTIZE and s.policy == O.P_SYMMETRIC_RNE
    assert s.scale.kind == O.PARAM_INLINE and s.scale.inline_bits == [0x3f000000]
    assert p.fills[0].bits == 0x3f800000 and p.layout.pad_fill[0].fill_bits == 2


def test_decoder_rejections():
    blob = bytes.fromhex(G.goldens()["layout_v0"]["kIdentityHex"])
    with pytest.raises(O.DecodeError) as e:
        O.decode_plan(b"XPLN" + blob[4:])
    assert e.value.offset == 0
    with pytest.raises(O.DecodeError) as e:
        O.decode_typed_plan(blob)  # v0 blob under the v1 decoder
    assert e.value.offset == 4
    with pytest.raises(O.DecodeError):
        O.decode_plan(blob + b"\0")  # trailing bytes
    for n in range(len(blob)):
        with pytest.raises(O.DecodeError):
            O.decode_plan(blob[:n])
    typed = bytes.fromhex(G.goldens()["typed_v1"]["kPadQuantizeHex"])
    assert len(typed) == 393
    bad = bytearray(typed)
    bad[308] = 7  # unknown transform (TypedDecodeTest.cpp:254-260)
    with pytest.raises(O.DecodeError):
        O.decode_typed_plan(bytes(bad))
    bad = bytearray(typed)
    bad[264] = 3  # fused fill no longer matches the folded original
    with pytest.raises(O.DecodeError, match="fill fold mismatch"):
        O.decode_typed_plan(bytes(bad))


def test_decoder_fuzz_bit_flips_never_crash(rng):
    typed = bytes.fromhex(G.goldens()["typed_v1"]["kDequantCastHex"])
    for _ in range(400):
        b = bytearray(typed)
        i = int(rng.integers(0, len(b)))
        b[i] ^= 1 << int(rng.integers(0, 8))
        try:
            O.decode_typed_plan(bytes(b))
        except O.DecodeError:
            pass


# ------------------------------------------------------ stage arithmetic pins

def _f32(xs):
    return np.array(xs, np.float32).view(np.uint32)


def test_f16_narrowing_witness_vectors():
    xs = [0.0, -0.0, 2.0 ** -24, 2.0 ** -25, 1.5 * 2.0 ** -25, 2.0 ** -14, 65504.0,
          65519.99, 65520.0, 1e5, 1 + 2.0 ** -11, 1 + 3 * 2.0 ** -12]
    exp = [0x0000, 0x8000, 0x0001, 0x0000, 0x0001, 0x0400, 0x7BFF, 0x7BFF, 0x7C00, 0x7C00,
           0x3C00, 0x3C01]
    assert O.narrow_f32_f16_bits(_f32(xs)).tolist() == exp
    specials = O.narrow_f32_f16_bits(_f32([np.inf, -np.inf]))
    assert specials.tolist() == [0x7C00, 0xFC00]
    # observed reference NaN behaviour (truncated payload, quiet bit)
    assert O.narrow_f32_f16_bits(np.array([0x7fc12345, 0xffe00000], np.uint32)).tolist() == \
        [0x7e09, 0xff00]


def test_f16_narrowing_equals_numpy_ieee_on_random_bits(rng):
    bits = rng.integers(0, 2 ** 32, 1 << 20, dtype=np.uint64).astype(np.uint32)
    # add every exponent boundary with tie patterns
    e = np.arange(256, dtype=np.uint32) << 23
    ties = np.concatenate([e | m for m in (0, 0x1000, 0x0fff, 0x1fff, 0x2000, 0x7fffff, 0x3000)])
    bits = np.concatenate([bits, ties, ties | 0x80000000])
    x = bits.view(np.float32)
    keep = ~np.isnan(x)
    got = O.narrow_f32_f16_bits(bits[keep])
    with np.errstate(over="ignore"):
        ref = x[keep].astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_f16_widening_exhaustive():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.widen_f16_f32_bits(h)
    f = h.view(np.float16)
    keep = ~np.isnan(f)
    assert np.array_equal(got[keep], f[keep].astype(np.float32).view(np.uint32))
    wit = O.widen_f16_f32_bits(np.array([0x0001, 0x0400, 0x7BFF, 0x7C00, 0xFC00, 0x8000], np.uint16))
    assert wit.tolist() == [0x33800000, 0x38800000, 0x477FE000, 0x7F800000, 0xFF800000, 0x80000000]
    # NaN payload shifts left by 13 (Quant.cpp:206)
    assert O.widen_f16_f32_bits(np.array([0x7d01], np.uint16)).tolist() == [0x7fa02000]


def test_bf16_witness_and_nearest_even(rng):
    xs = [0.0, -0.0, 1 + 2.0 ** -8, 1 + 3 * 2.0 ** -9, 2.0 ** -133, 2.0 ** -134,
          1.5 * 2.0 ** -134, 2.0 ** -126]
    exp = [0x0000, 0x8000, 0x3F80, 0x3F81, 0x0001, 0x0000, 0x0001, 0x0080]
    assert O.narrow_f32_bf16_bits(_f32(xs)).tolist() == exp
    assert O.narrow_f32_bf16_bits(np.array([0x7F7F0000, 0x7F7F8000, f32b(3.4e38)], np.uint32)).tolist() \
        == [0x7F7F, 0x7F80, 0x7F80]
    assert O.widen_bf16_f32_bits(np.array([0x0001, 0x0080, 0x7F7F, 0x7F80, 0xFF80, 0x8000, 0x3F81],
                                          np.uint16)).tolist() == \
        [0x00010000, 0x00800000, 0x7F7F0000, 0x7F800000, 0xFF800000, 0x80000000, 0x3F810000]
    # independent nearest-even oracle in exact integer arithmetic on |bits|
    bits = rng.integers(0, 2 ** 32, 200000, dtype=np.uint64).astype(np.uint32)
    bits = bits[~np.isnan(bits.view(np.float32))]
    mag = (bits & 0x7fffffff).astype(np.int64)
    lo = mag >> 16
    rem = mag & 0xffff
    up = (rem > 0x8000) | ((rem == 0x8000) & (lo & 1 == 1))
    ref = ((lo + up) | ((bits >> 16) & 0x8000)).astype(np.uint16)
    assert np.array_equal(O.narrow_f32_bf16_bits(bits), ref)


def f32b(x):
    return O.f32_bits(x)


def test_quantize_witness_vectors():
    inv1 = np.float32(1.0)
    assert O.quantize_f32_s8(np.array([-2.5, -1.5, -0.5, 0.5, 1.5, 2.5], np.float32), inv1).tolist() \
        == [-2, -2, 0, 0, 2, 2]
    assert O.quantize_f32_s8(np.array([-129, -128, -127, 126, 127, 128], np.float32), inv1).tolist() \
        == [-128, -128, -127, 126, 127, 127]
    assert O.quantize_f32_s8(np.array([np.nan, np.inf, -np.inf, -0.0, 1e-40], np.float32),
                             inv1).tolist() == [-128, 127, -128, 0, 0]


def test_reciprocal_formation_differs_in_three_of_eight():
    xs = np.array([0.1, 0.3, 0.7, 1.1, 2.9, 10.1, 100.3, 1000.7], np.float32)
    s = np.float32(0.3)
    inv = np.float32(1.0) / s
    a = (xs * inv).astype(np.float32).view(np.uint32)
    b = (xs / s).astype(np.float32).view(np.uint32)
    assert int(np.sum(a != b)) == 3


def test_dequantize_witness_and_exact_product(rng):
    q = np.array([-128, -1, 0, 1, 127], np.int8)
    got = O.dequantize_s8_f32(q, np.float32(0.3), np.int32(0)).view(np.uint32)
    assert got.tolist() == [0xC219999A, 0xBE99999A, 0x00000000, 0x3E99999A, 0x42186667]
    assert O.dequantize_s8_f32(np.array([-128], np.int8), np.float32(0.3), np.int32(127)) \
        .view(np.uint32).tolist() == [0xC2990000]
    # one rounding: float64 product of (|d| <= 255) and a binary32 scale is exact
    q = rng.integers(-128, 128, 100000).astype(np.int8)
    zp = rng.integers(-128, 128, 100000).astype(np.int32)
    sc = rng.uniform(1e-3, 2e-2, 100000).astype(np.float32)
    ref = ((q.astype(np.float64) - zp) * sc.astype(np.float64)).astype(np.float32)
    assert np.array_equal(O.dequantize_s8_f32(q, sc, zp).view(np.uint32), ref.view(np.uint32))


def test_quantize_equals_clamp_then_round_for_finite(rng):
    x = rng.normal(0, 100, 100000).astype(np.float32)
    inv = np.float32(1.0) / np.float32(0.37)
    ref = np.clip(np.rint((x * inv).astype(np.float32)), -128, 127).astype(np.int8)
    assert np.array_equal(O.quantize_f32_s8(x, inv), ref)


def test_channel_witness_slice():
    # docs/reloc-typed-semantics.md section 4.3 witness: [2,3,4], axis 1
    x = (np.arange(24, dtype=np.float32) - np.float32(11.5)).reshape(2, 3, 4)
    inv = (np.float32(1.0) / np.array([0.5, 1.0, 2.0], np.float32)).astype(np.float32)
    q = O.quantize_f32_s8(x, inv[None, :, None])
    assert q[0].tolist() == [[-23, -21, -19, -17], [-8, -6, -6, -4], [-2, -1, -1, 0]]


# ------------------------------------------------------- chunk schedule pins

def _bound(ext, ss, ds, es, pads=()):
    padded = list(ext)
    for p in pads:
        padded[p.axis] += p.lo + p.hi
    return O.BoundPlan(list(ext), list(ss), list(ds), list(range(len(ext))), list(pads), es,
                       int(np.prod(padded)) * es, False, 1, [])


def _cover(chunks, row_bytes, padded_outer, total):
    pos, covered = 0, 0
    for c in chunks:
        assert c.padded_begin == pos and c.byte_offset == pos * row_bytes
        pos = c.padded_end
        covered += c.bytes
    assert pos == padded_outer and covered == total


def test_plan_chunks_reference_expectations():
    b = _bound([64, 16], [16, 1], [16, 1], 4)
    ch, mx, lo, rb, ser = O.plan_chunks(b, 2, 64)
    assert not ser and rb == 64 and len(ch) == 64
    b = _bound([8, 128], [128, 1], [128, 1], 4)
    assert len(O.plan_chunks(b, 4)[0]) == 1
    b = _bound([1024, 16384], [16384, 1], [16384, 1], 4)
    ch = O.plan_chunks(b, 2)[0]
    assert len(ch) == 16
    _cover(ch, 16384 * 4, 1024, b.total_bytes)
    b = _bound([65536, 16384], [16384, 1], [16384, 1], 4)
    ch, mx, *_ = O.plan_chunks(b, 2)
    assert len(ch) >= 16 and mx * 2 <= 128 << 20
    b = _bound([128, 16384], [16384, 1], [16384, 1], 4)
    assert len(O.plan_chunks(b, 4)[0]) == 2
    b = _bound([6, 4], [4, 1], [4, 1], 4, [O.PadRegion(0, 1, 1, 0xDEADBEEF)])
    ch, mx, lo, rb, ser = O.plan_chunks(b, 2, 16)
    assert lo == 1 and ch[0].valid_begin == ch[0].valid_end
    assert (ch[1].valid_begin, ch[1].valid_end) == (0, 1)
    assert ch[-1].valid_begin == ch[-1].valid_end
    b = _bound([8, 3], [3, 1], [1, 1], 4)
    ch, mx, lo, rb, ser = O.plan_chunks(b, 4, 4)
    assert ser and len(ch) == 1 and ch[0].bytes == b.total_bytes


# ---------------------------------------------- planted mistakes are caught

def test_planted_rounding_mistake_fails_the_corpus(monkeypatch):
    """A truncating (round-toward-zero) f16 narrowing in the oracle must fail
    the corpus: proves the corpus check has teeth for the cast stage."""
    meta, blob = next((m, b) for m, b in TYPED if m["name"] == "cast_transpose_f16")

    def truncating(x):
        x = np.asarray(x, np.uint32)
        return (((x >> 16) & 0x8000) | (((x & 0x7fffffff) - 0x38000000) >> 13)).astype(np.uint16)

    monkeypatch.setattr(O, "narrow_f32_f16_bits", truncating)
    b = meta["bindings"][0]
    out = O.run_typed(blob, b["symbols"], {}, G.bits_array(b["source"]))
    assert not np.array_equal(out.view(np.uint16), G.bits_array(b["expected"]))


def test_planted_stride_mistake_fails_the_layout_corpus(monkeypatch, rng):
    meta, blob = next((m, b) for m, b in LAYOUT if m["name"] == "transpose_2d_f32")
    plan = O.decode_plan(blob)
    bound = O.bind(plan, {})
    bound.src_strides = list(reversed(bound.src_strides))  # transposed operand
    shape = meta["src_shape"]
    src = rng.standard_normal(int(np.prod(shape))).astype(np.float32).reshape(shape)
    try:
        got = O.execute_layout(bound, src.tobytes())
    except IndexError:
        return  # the wrong strides leave the source bounds: caught
    assert got != _numpy_replay(meta, {}, src).tobytes()
