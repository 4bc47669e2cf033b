"""Every kernel launch the executor would make stays inside its buffers.

relx_verify_launches walks each launch of the chunk schedule (and the
device-resident whole-box launch) with the kernels' own index arithmetic
and checks every access against the wire and result extents, 16-byte
alignment of vector accesses and parameter-table bounds. Runs on the CPU:
corpus plans at every wire boundary, every configuration at full size, and
several chunk sizes."""
import numpy as np
import pytest

from sym_amd import encoder as EN
from sym_amd import pyreloc as P
from sym_amd import workloads as W
from tests import golden_io as G
from tests import permute_cases as PC
from tests import transpose_cases as TC

CHUNKS = [0, 1 << 16, 3 << 20]


def _check(bound, boundaries, chunks=CHUNKS):
    total = 0
    for k in boundaries:
        for c in chunks:
            total += P.verify_launches(bound, k, c)
    assert total > 0


@pytest.mark.parametrize("meta,blob", G.typed_fixtures(), ids=[m["name"] for m, _ in G.typed_fixtures()])
def test_typed_corpus_launches(meta, blob):
    plan = P.load_typed_plan(blob)
    for b in meta["bindings"]:
        bd = P.bind_typed(plan, b["symbols"], G.fixture_params(meta))
        _check(bd, range(len(bd.footprints())))


@pytest.mark.parametrize("meta,blob", G.layout_fixtures(), ids=[m["name"] for m, _ in G.layout_fixtures()])
def test_layout_corpus_launches(meta, blob):
    plan = P.load_plan(blob)
    bindings = [{}] if not meta["symbols"] else \
        [{n: c["multiple_of"] * f for n, c in meta["symbols"].items()} for f in (1, 2, 3)]
    for binding in bindings:
        _check(P.bind(plan, binding), [0])


@pytest.mark.parametrize("n", W.C1_SIZES)
def test_c1_launches(n):
    b = P.Bound(P.Plan(W.c1_plan().blob), {"s0": n})
    assert b.kernel == ("transpose" if n % 4096 == 0 else "generic") or n < 4096
    _check(b, [0])


@pytest.mark.parametrize("n", [32, 1, 3])
def test_c2_launches(n):
    b = P.Bound(P.Plan(W.c2_plan(n=n).blob), {}, {})
    assert b.kernel == "interleave"
    _check(b, [0, 1])


def test_c3_launches():
    b = P.Bound(P.Plan(W.c3_plan().blob), {"s0": 4096, "s1": 11008},
                W.param("scale", np.ones(11008, np.float32)))
    # 11008 = 86 x 128 and 4096 = 32 x 128: 128 x 128 byte tiles, whose
    # tile rows read whole 128-byte lines
    assert b.kernel == "transpose" and (b.transpose_tile_q, b.transpose_tile_c) == (128, 128)
    # the per-row scale of the dequantize stage: one channel per result row
    assert b.transpose_row_params
    _check(b, [0])


@pytest.mark.parametrize("f32", [False, True])
@pytest.mark.parametrize("rows,cols,tile_q,tile_c", [(4096, 11008, 128, 128), (256, 4032, 64, 64),
                                                     (192, 4160, 64, 64), (4000, 11008, 128, 64),
                                                     (128, 128, 128, 128), (64, 64, 64, 64),
                                                     (192, 256, 128, 64), (100, 300, 128, 64)])
def test_transpose_tile_width(rows, cols, tile_q, tile_c, f32):
    """One-byte transposes take tiles 128 q wide when the source-contiguous
    extent is a multiple of 128 (edge strips element-wise), else 64, and
    with f16 and f32 results 128 c wide byte tiles when the c extent is a
    multiple of 128 too; the
    verifier walks the rotated tile order of the wide tiles (a bijection onto
    the plane) at several chunk sizes, so chunk boundaries along c and q
    keep the tile alignment."""
    scale = EN.BindingParam("scale", "float32", ("s1",))
    ops = [EN.Dequantize(scale, axis=1)] + ([] if f32 else [EN.Cast("float16")])
    plan = EN.encode(["s0", "s1"], "int8", ops + [EN.Transpose((1, 0))])
    b = P.Bound(P.Plan(plan.blob), {"s0": rows, "s1": cols}, W.param("scale", np.ones(cols, np.float32)))
    if cols % 16:
        assert b.kernel != "transpose"
        return
    want_c = tile_c
    assert b.kernel == "transpose" and (b.transpose_tile_q, b.transpose_tile_c) == (tile_q, want_c)
    # the scale runs along the result rows: f16 byte tiles index it by row
    assert b.transpose_row_params == (want_c == 128 and not f32)
    _check(b, range(len(b.footprints())), chunks=[0, 1 << 12, 1 << 16, 3 << 20])


def test_random_one_byte_transposes():
    """120 random one-byte transposes (layout, dequantize, dequantize + f16;
    batched or not; edge strips): each transpose program takes the tile
    width its q extent allows, and every launch is verified at several
    chunk sizes."""
    kinds, rows = set(), 0
    for name, blob, x, width in TC.random_cases(120):
        b = P.Bound(P.Plan(blob), {}, {})
        if b.kernel == "transpose":
            assert (b.transpose_tile_q, b.transpose_tile_c) == width, name
        rows += b.transpose_row_params
        kinds.add((b.kernel, b.transpose_tile_q, b.transpose_tile_c))
        _check(b, [0], chunks=[0, 4096, 1 << 16])
    assert kinds == {("transpose", 128, 128), ("transpose", 128, 64), ("transpose", 64, 64),
                     ("generic", 0, 0)}
    assert rows > 0


def test_transpose_tile_width_wider_elements():
    """Sources of two and four bytes keep 64-wide tiles."""
    b = P.Bound(P.Plan(W.c1_plan().blob), {"s0": 64 * 4096})
    assert b.kernel == "transpose" and (b.transpose_tile_q, b.transpose_tile_c) == (64, 64)
    b = P.Bound(P.Plan(W.c4_plan().blob), {"s0": 512, "s1": 256},
                W.param("scale", np.ones(512, np.float32)))
    assert b.transpose_tile_q == 0


@pytest.mark.parametrize("rows,cols", [(14336, 4096), (4096, 14336)])
def test_c4_launches(rows, cols):
    b = P.Bound(P.Plan(W.c4_plan().blob), {"s0": rows, "s1": cols},
                W.param("scale", np.ones(rows, np.float32)))
    assert b.kernel == "stream"
    _check(b, [0])


@pytest.mark.parametrize("bs,seq", W.C5_SHAPES)
def test_c5_launches(bs, seq):
    b = P.Bound(P.Plan(W.c5_plan().blob), {"B": bs, "S": seq},
                W.param("scale", np.ones(32, np.float32)))
    # per-head scales along c, C*E = 4096 and E = 128: the direct body, whose
    # parameter entries the verifier compares with the stage's channel map
    # on every vector
    assert b.kernel == "permute" and b.permute_direct
    big = bs * seq >= 64 * 1024
    _check(b, [0, 1], chunks=[0] if big else CHUNKS)


@pytest.mark.parametrize("bs,seq", [(1, 4096), (1, 65536), (64, 4096)])
def test_permute_direct_chunked(bs, seq):
    """C5 uploads in chunks: one batch entry splits along its sequence axis,
    so launches start inside a plane of the result; every launch verified,
    direct ones against the stage's channel map on every vector."""
    b = P.Bound(P.Plan(W.c5_plan().blob), {"B": bs, "S": seq},
                W.param("scale", np.ones(32, np.float32)))
    assert b.permute_direct
    assert P.verify_launches(b, 0, 1 << 20 if bs == 1 else 64 << 20) > 2


@pytest.mark.parametrize("case", PC.cases(), ids=[c[0] for c in PC.cases()])
def test_permute_bodies(case):
    """Which permute body each plan gets, and every launch of either body
    verified (a direct launch's parameter entry against the stage's channel
    map on every vector)."""
    name, blob, x, direct = case
    b = P.Bound(P.Plan(blob), {}, {})
    assert b.kernel == "permute", name
    assert b.permute_direct == direct, name
    _check(b, range(len(b.footprints())))


def test_random_permutes():
    """200 random block permutes (tests/permute_cases.random_cases: shapes
    with and without power-of-two heads and head dims, every chain the
    permute runs, parameters per tensor or along any axis): both kernels
    taken, every launch verified at every wire boundary and three chunk
    sizes."""
    kinds = set()
    for name, blob, x in PC.random_cases(200):
        b = P.Bound(P.Plan(blob), {}, {})
        assert b.kernel == "permute", name
        kinds.add(b.permute_direct)
        _check(b, range(len(b.footprints())), chunks=[0, 4096, 1 << 16])
    assert kinds == {True, False}
