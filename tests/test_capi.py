"""The C-ABI library: loads, exports every symbol include/relx.h declares,
and its host-side decode/bind agrees with the oracle (no GPU calls)."""
import ctypes
import os
import re

import numpy as np
import pytest

from oracle import relx_oracle as O
from sym_amd import _native as N
from sym_amd import pyreloc as P
from tests import golden_io as G

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    text = open(os.path.join(ROOT, "include", "relx.h")).read()
    return sorted(set(re.findall(r"\b(relx_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_header_symbol():
    L = N.lib()
    declared = header_symbols()
    assert len(declared) >= 20
    for name in declared:
        assert hasattr(L, name), name
    assert set(declared) == set(N.SIGNATURES), "ctypes table and header disagree"


def test_struct_layouts_match_the_header(tmp_path):
    """Every ctypes mirror of a relx_* struct has the size and field offsets
    that the C compiler gives include/relx.h."""
    import subprocess
    structs = [(n, c) for n, c in sorted(vars(N).items())
               if isinstance(c, type) and issubclass(c, ctypes.Structure) and n.startswith("relx_")]
    assert len(structs) >= 8
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "relx.h"', "int main(void) {"]
    for n, c in structs:
        lines.append('  printf("%s %%zu\\n", sizeof(%s));' % (n, n))
        for f in c._fields_:
            lines.append('  printf("%s.%s %%zu\\n", offsetof(%s, %s));' % (n, f[0], n, f[0]))
    lines.append("  return 0;\n}")
    (tmp_path / "layout.c").write_text("\n".join(lines) + "\n")
    exe = str(tmp_path / "layout")
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), "-o", exe, str(tmp_path / "layout.c")],
                   check=True, capture_output=True)
    got = dict(line.split() for line in subprocess.run([exe], check=True, capture_output=True,
                                                       text=True).stdout.splitlines())
    for n, c in structs:
        assert int(got[n]) == ctypes.sizeof(c), n
        for f in c._fields_:
            assert int(got[n + "." + f[0]]) == getattr(c, f[0]).offset, (n, f[0])


def test_version_and_wire_version():
    assert "librelx" in P.version()
    blob = bytes.fromhex(G.goldens()["layout_v0"]["kIdentityHex"])
    assert P.wire_version(blob) == 0
    assert P.wire_version(b"nope") is None


def _params(meta):
    return {k: (O.DTYPE_TYPES[d], s, x) for k, (d, s, x) in G.fixture_params(meta).items()}


@pytest.mark.parametrize("meta,blob", G.typed_fixtures(), ids=[m["name"] for m, _ in G.typed_fixtures()])
def test_typed_bind_matches_oracle(meta, blob):
    plan = P.load_typed_plan(blob)
    assert plan.typed
    for b in meta["bindings"]:
        bd = P.bind_typed(plan, b["symbols"], G.fixture_params(meta))
        ob = O.bind_typed(O.decode_typed_plan(blob), b["symbols"], _params(meta))
        assert bd.extents == ob.layout.extents
        assert bd.src_strides == ob.layout.src_strides
        assert bd.dst_strides == ob.layout.dst_strides
        assert bd.footprints() == [c.bytes for c in ob.cuts]
        assert bd.parameter_bytes == ob.parameter_bytes
        assert bd.destination_bytes == b["footprints"]["h2d"]["destination_bytes"]


@pytest.mark.parametrize("meta,blob", G.layout_fixtures(), ids=[m["name"] for m, _ in G.layout_fixtures()])
def test_layout_bind_matches_oracle(meta, blob):
    plan = P.load_plan(blob)
    bindings = [{}] if not meta["symbols"] else \
        [{n: c["multiple_of"] * f for n, c in meta["symbols"].items()} for f in (1, 2, 3)]
    for binding in bindings:
        bd = P.bind(plan, binding)
        ob = O.bind(O.decode_plan(blob), binding)
        assert (bd.extents, bd.src_strides, bd.dst_strides, bd.total_bytes) == \
            (ob.extents, ob.src_strides, ob.dst_strides, ob.total_bytes)


def test_reference_plan_coalescing():
    # BindTest.cpp:158-178 through the C-ABI
    bd = P.bind(P.load_plan(bytes.fromhex(G.goldens()["layout_v0"]["kReferenceHex"])), {"N": 32768})
    assert bd.extents == [512, 4096, 512]
    assert bd.src_strides == [64, 32768, 1]
    assert bd.dst_strides == [2097152, 512, 1]


def test_decode_errors_carry_offsets():
    blob = bytes.fromhex(G.goldens()["layout_v0"]["kIdentityHex"])
    with pytest.raises(P.DecodeError) as e:
        P.load_plan(b"XPLN" + blob[4:])
    assert e.value.offset == 0
    with pytest.raises(P.DecodeError):
        P.load_plan(blob + b"\0")
    for n in (0, 3, 8, 100, 180):
        with pytest.raises(P.DecodeError):
            P.Plan(blob[:n])
    typed = bytearray(bytes.fromhex(G.goldens()["typed_v1"]["kPadQuantizeHex"]))
    typed[264] = 3
    with pytest.raises(P.DecodeError, match="fill fold mismatch"):
        P.load_typed_plan(bytes(typed))
    with pytest.raises(P.DecodeError) as e:
        P.load_typed_plan(blob)
    assert e.value.offset == 4


def test_decode_rejections_match_oracle_on_bit_flips(rng):
    typed = bytes.fromhex(G.goldens()["typed_v1"]["kDequantCastHex"])
    for _ in range(300):
        b = bytearray(typed)
        b[int(rng.integers(0, len(b)))] ^= 1 << int(rng.integers(0, 8))
        try:
            O.decode_typed_plan(bytes(b))
            ok_oracle = True
        except O.DecodeError as e:
            ok_oracle, off = False, e.offset
        try:
            P.Plan(bytes(b))
            ok_lib = True
        except P.DecodeError as e:
            ok_lib = False
            assert not ok_oracle and e.offset == off, bytes(b).hex()
        assert ok_lib == ok_oracle


def test_bind_errors():
    blob = next(b for m, b in G.layout_fixtures() if m["name"] == "reshape_split_sym")
    plan = P.load_plan(blob)
    with pytest.raises(P.BindError, match="unbound symbol"):
        P.bind(plan, {})
    with pytest.raises(P.BindError, match="unknown symbol"):
        P.bind(plan, {"N": 64, "M": 1})
    with pytest.raises(P.BindError, match="divisibility"):
        P.bind(plan, {"N": 65})
    meta, tblob = next((m, b) for m, b in G.typed_fixtures() if m["name"] == "dequant_then_f16")
    tplan = P.load_typed_plan(tblob)
    good = G.fixture_params(meta)
    with pytest.raises(P.BindError, match="unbound parameter"):
        P.bind_typed(tplan, {"s0": 5}, {})
    bad = {"s": ("float32", [3], np.array([1.0, -1.0, 2.0], np.float32).tobytes())}
    with pytest.raises(P.BindError, match="finite and strictly positive"):
        P.bind_typed(tplan, {"s0": 5}, bad)
    short = {"s": ("float32", [2], np.array([1.0, 2.0], np.float32).tobytes())}
    with pytest.raises(P.BindError, match="length"):
        P.bind_typed(tplan, {"s0": 5}, short)
    P.bind_typed(tplan, {"s0": 5}, good)


def test_fastdiv_is_exact_on_the_host():
    """The 32-bit division-by-constant the kernels use (program.cpp make_div)
    restated on the CPU: exact for every numerator class that matters."""
    def make(d):
        s = 0
        while (1 << s) < d:
            s += 1
        m = ((1 << 32) * ((1 << s) - d)) // d + 1
        return m & 0xffffffff, s

    rng = np.random.default_rng(3)
    for d in [1, 2, 3, 7, 64, 100, 128, 224, 4096, 11008, 50176, 14336, 2**31 - 1, 2**32 - 1]:
        m, s = make(d)
        ns = np.concatenate([rng.integers(0, 2**32, 20000, dtype=np.uint64),
                             np.array([0, 1, d - 1, d, d + 1, 2**32 - 1], np.uint64)])
        ns = ns[ns < 2**32]
        hi = (ns * np.uint64(m)) >> np.uint64(32)
        q = (hi + ns) >> np.uint64(s)
        assert np.array_equal(q, ns // np.uint64(d)), d


def test_caller_stream_option_mapping():
    """None means no producer stream; any handle, 0 (the legacy null stream,
    torch's default) included, orders the call after that stream
    (reference hasCallerStream, libreloc/python/PyDispatch.cpp:199-202)."""
    none = P._options()
    assert none.has_caller_stream == 0 and none.caller_stream == 0
    null = P._options(caller_stream=0)
    assert null.has_caller_stream == 1 and null.caller_stream == 0
    other = P._options(caller_stream=0x1234)
    assert other.has_caller_stream == 1 and other.caller_stream == 0x1234
    # the ctypes layout matches the header's field order
    text = open(os.path.join(ROOT, "include", "relx.h")).read()
    body = text[text.index("typedef struct relx_options"):text.index("} relx_options;")]
    fields = re.findall(r"^\s+(?:int|int64_t|uint64_t)\s+(\w+);", body, re.M)
    assert fields == [f for f, _ in N.relx_options._fields_]
