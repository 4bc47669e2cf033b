"""HIP path parity: librelx on an MI355X against the pinned oracle.

Bit-exact for every config (the reference contract is bit-exact for dequant
too, inside the <= 1 ULP allowance). Small cases compare whole outputs with
the oracle / numpy replays; full-size configs compare whole outputs where
numpy finishes in seconds and otherwise every element of randomly sampled
rows, plus size-independent checks (checksums of the whole buffer against
the sampled oracle where exact).
"""
import hashlib
import os
import sys

import numpy as np
import pytest

from oracle import relx_oracle as O
from sym_amd import encoder as EN
from sym_amd import pyreloc as P
from sym_amd import workloads as W
from tests import golden_io as G
from tests import permute_cases as PC
from tests import transpose_cases as TC
from tests.test_encoder import small_cases

# RELX_TRANSPOSE_DRAW=n:seed widens the random transposes (the suite runs 120:11)
_TN, _TS = (int(v) for v in os.environ.get("RELX_TRANSPOSE_DRAW", "120:11").split(":"))

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    assert torch.cuda.is_available(), "a GPU test needs the MI355X"
    c = P.Context(0)
    yield c
    c.close()


def run_h2d(ctx, blob, syms, params, src, name="", **opts):
    plan = P.Plan(blob)
    b = P.Bound(plan, syms, params if plan.typed else None)
    nbytes = b.destination_bytes if plan.typed else b.total_bytes
    out = torch.empty(max(1, nbytes), dtype=torch.uint8, device="cuda")
    src = np.ascontiguousarray(src)
    say(name, "kernel=%s" % b.kernel, "src=%d B dst=%d B" % (src.nbytes, nbytes), opts)
    rep = ctx.execute_h2d(b, src.ctypes.data, src.nbytes, out.data_ptr(), nbytes, **opts)
    torch.cuda.synchronize()
    return out[:nbytes].cpu().numpy(), rep, b


def f16_bits(x32):
    return O.narrow_f32_f16_bits(np.ascontiguousarray(x32, np.float32).view(np.uint32))


# ------------------------------------------------------------- corpus

TYPED = G.typed_fixtures()


@pytest.mark.parametrize("meta,blob", TYPED, ids=[m["name"] for m, _ in TYPED])
@pytest.mark.parametrize("host_stages", [0, -1])
def test_typed_corpus(ctx, meta, blob, host_stages):
    for b in meta["bindings"]:
        src = G.bits_array(b["source"])
        out, rep, _ = run_h2d(ctx, blob, b["symbols"], G.fixture_params(meta), src,
                              meta["name"], host_stages=host_stages)
        exp = G.bits_array(b["expected"])
        assert np.array_equal(out.view(exp.dtype), exp), (meta["name"], b["symbols"])
        assert hashlib.sha256(out.tobytes()).hexdigest() == b["expected"]["sha256"]
        assert rep["destination_bytes"] == b["footprints"]["h2d"]["destination_bytes"]


LAYOUT = G.layout_fixtures()
NPD = {"f32": np.float32, "f16": np.float16, "i8": np.int8}


def _eval_dim(d, binding):
    if isinstance(d, int):
        return d
    p = d.split()
    return binding[p[0]] // int(p[2]) if len(p) == 3 else binding[d]


@pytest.mark.parametrize("meta,blob", LAYOUT, ids=[m["name"] for m, _ in LAYOUT])
def test_layout_corpus(ctx, meta, blob, rng):
    bindings = [{}] if not meta["symbols"] else \
        [{n: c["multiple_of"] * f for n, c in meta["symbols"].items()} for f in (1, 2, 3)]
    for binding in bindings:
        shape = [_eval_dim(d, binding) for d in meta["src_shape"]]
        dt = NPD[meta["dtype"]]
        src = rng.integers(0, 256, int(np.prod(shape)) * np.dtype(dt).itemsize,
                           dtype=np.uint8).view(dt).reshape(shape)
        out, _, b = run_h2d(ctx, blob, binding, None, src, meta["name"])
        want = O.execute_layout(O.bind(O.decode_plan(blob), binding), src.tobytes())
        assert out.tobytes() == want, (meta["name"], binding)


# ---------------------------------------------------------- configs small

def test_configs_small(ctx, rng):
    for name, plan, syms, params, src, expected in small_cases(rng):
        for hs in (0, -1):
            out, rep, _ = run_h2d(ctx, plan.blob, syms, params, src, name, host_stages=hs)
            assert out.tobytes() == expected, (name, hs)


# ------------------------------------------------------------ C1 (all N)

@pytest.mark.parametrize("n", W.C1_SIZES)
def test_c1_readme_plan(ctx, n):
    x = W.c1_input(n)
    out, rep, b = run_h2d(ctx, W.c1_plan().blob, {"s0": n}, None, x, "c1 N=%d" % n)
    assert out.view(np.float32).reshape(64, n // 64).tobytes() == x.reshape(n // 64, 64).T.tobytes()
    assert rep["wire_bytes"] == 4 * n and rep["destination_bytes"] == 4 * n


def test_c1_one_plan_rebinds(ctx):
    plan = P.Plan(W.c1_plan().blob)
    for n in (128, 192, 256, 4096, 64 * 1000):
        b = P.Bound(plan, {"s0": n})
        x = W.c1_input(n, seed=n)
        out = torch.empty(4 * n, dtype=torch.uint8, device="cuda")
        say("c1 rebind N=%d" % n)
        ctx.execute_h2d(b, x.ctypes.data, x.nbytes, out.data_ptr(), 4 * n)
        assert out.cpu().numpy().tobytes() == x.reshape(n // 64, 64).T.tobytes()
    with pytest.raises(P.BindError, match="divisibility"):
        P.Bound(plan, {"s0": 100})


# ------------------------------------------------------------------ C2

@pytest.mark.parametrize("host_stages", [0, 1])
def test_c2_image_batch_full(ctx, host_stages):
    x = W.c2_input()
    out, rep, b = run_h2d(ctx, W.c2_plan().blob, {}, None, x, "c2", host_stages=host_stages)
    want = f16_bits(np.pad(x, [(0, 0), (0, 1), (0, 0), (0, 0)]).transpose(0, 2, 3, 1))
    assert np.array_equal(out.view(np.uint16).reshape(want.shape), want)
    assert b.kernel == "interleave"
    assert rep["wire_bytes"] == (19267584 if host_stages == 0 else 9633792)
    assert rep["destination_bytes"] == 12845056


@pytest.mark.parametrize("shape,lo,hi", [((3, 3, 20, 24), 0, 1), ((1, 1, 16, 8), 1, 0),
                                          ((2, 5, 12, 16), 1, 2), ((2, 3, 3, 10, 8), 0, 1)])
@pytest.mark.parametrize("dtype,cast", [("float32", "float16"), ("float32", None),
                                        ("float16", None), ("int8", None), ("float16", "float32")])
def test_planar_to_interleaved_with_channel_pad(ctx, shape, lo, hi, dtype, cast):
    """C2's pattern over channel counts, pads, batch ranks and element
    types: NC...HW -> N...HWC with the channel axis padded (the fill folds
    through the cast); contiguous batch axes merge into one level, which
    takes the preloaded-argument variant for per-tensor chains."""
    from sym_amd import encoder as EN
    rng = np.random.default_rng(sum(shape) * 31 + lo + 7 * hi)
    caxis = len(shape) - 3
    n = int(np.prod(shape))
    if dtype == "int8":
        x = rng.integers(-128, 128, n, dtype=np.int8).reshape(shape)
        fill = -5
    else:
        x = (rng.standard_normal(n) * 10).astype(dtype).reshape(shape)
        fill = 1.5
    perm = tuple(range(caxis)) + (caxis + 1, caxis + 2, caxis)
    ops = [EN.Pad(caxis, lo, hi, fill), EN.Transpose(perm)] + ([EN.Cast(cast)] if cast else [])
    try:
        plan = EN.encode(list(shape), dtype, ops)
    except EN.EncodeError as e:
        pytest.skip("not encodable: %s" % e)
    want = (O.run_typed(plan.blob, {}, {}, x).tobytes() if plan.typed else
            O.execute_layout(O.bind(O.decode_plan(plan.blob), {}), x.tobytes()))
    for hs in (0, -1):
        out, rep, b = run_h2d(ctx, plan.blob, {}, {}, x, "interleave %s %s %s->%s" % (shape, (lo, hi), dtype, cast),
                              host_stages=hs)
        assert out.tobytes() == want, hs
    xd = torch.from_numpy(x.view(np.uint8).reshape(-1).copy()).cuda()
    dev = torch.empty(len(want), dtype=torch.uint8, device="cuda")
    ctx.relayout_device(b, xd.data_ptr(), dev.data_ptr())
    torch.cuda.synchronize()
    assert dev.cpu().numpy().tobytes() == want


@pytest.mark.parametrize("host_stages", [-1, 0])
def test_c2_pinned_source(ctx, host_stages):
    """Automatic: the f32 -> f16 cast is staged from the pinned source too;
    with no host stages the f32 source crosses by direct DMA."""
    x = torch.from_numpy(W.c2_input()).pin_memory()
    plan = P.Plan(W.c2_plan().blob)
    b = P.Bound(plan, {})
    out = torch.empty(b.destination_bytes, dtype=torch.uint8, device="cuda")
    say("c2 pinned, host_stages", host_stages)
    rep = ctx.execute_h2d(b, x.data_ptr(), x.numel() * 4, out.data_ptr(), out.numel(),
                          host_stages=host_stages)
    if host_stages == 0:
        assert rep["direct_dma"] == 1 and rep["wire_boundary"] == 0
    else:
        assert rep["direct_dma"] == 0 and rep["wire_boundary"] == 1
    want = f16_bits(np.pad(x.numpy(), [(0, 0), (0, 1), (0, 0), (0, 0)]).transpose(0, 2, 3, 1))
    assert np.array_equal(out.cpu().numpy().view(np.uint16).reshape(want.shape), want)


# ------------------------------------------------------------------ C3

@pytest.mark.parametrize("opts", [{}, {"chunk_bytes": 1 << 20, "n_buffers": 2}, {"source_pinned": 0, "gather_threads": 1}])
def test_c3_weight_full(ctx, opts):
    q, s = W.c3_input()
    out, rep, b = run_h2d(ctx, W.c3_plan().blob, {"s0": 4096, "s1": 11008}, W.param("scale", s), q,
                          "c3", **opts)
    assert b.kernel == "transpose"
    want = f16_bits(O.dequantize_s8_f32(q, s[None, :], np.int32(0)).T)
    assert np.array_equal(out.view(np.uint16).reshape(11008, 4096), want)
    assert rep["wire_bytes"] == 45088768 and rep["destination_bytes"] == 90177536
    if "chunk_bytes" in opts:
        assert rep["chunks"] > 10


@pytest.mark.parametrize("rows,cols", [(4000, 1104), (200, 336), (64 * 3, 80)])
@pytest.mark.parametrize("opts", [{}, {"chunk_bytes": 256 << 10}, {"source_pinned": 1}])
def test_transpose_with_partial_tiles(ctx, rows, cols, opts):
    """C3's dequantizing transpose at extents that are not multiples of the
    64x64 tile (rows still 16-byte aligned on both sides): whole tiles in the
    tile kernel, the q and c edge strips in the element-wise kernel;
    chunked, pinned, and from HBM."""
    rng = np.random.default_rng(rows * 7919 + cols)
    q = W.int8_weight(rows, cols, rng)
    s = W.scales(cols, rng)
    src = q
    if opts.get("source_pinned"):
        src = torch.from_numpy(q.view(np.uint8).copy()).pin_memory().numpy().view(np.int8).reshape(q.shape)
    out, rep, b = run_h2d(ctx, W.c3_plan().blob, {"s0": rows, "s1": cols}, W.param("scale", s), src,
                          "c3 %dx%d %s" % (rows, cols, opts), **opts)
    assert b.kernel == "transpose"
    want = f16_bits(O.dequantize_s8_f32(q, s[None, :], np.int32(0)).T)
    assert np.array_equal(out.view(np.uint16).reshape(cols, rows), want)
    # the same launches over a device-resident wire
    qd = torch.from_numpy(q.view(np.uint8).copy()).cuda()
    dev = torch.empty(rows * cols * 2, dtype=torch.uint8, device="cuda")
    ctx.relayout_device(b, qd.data_ptr(), dev.data_ptr())
    torch.cuda.synchronize()
    assert np.array_equal(dev.cpu().numpy().view(np.uint16).reshape(cols, rows), want)


@pytest.mark.parametrize("n", [1000003, 4099, 13, 5])
@pytest.mark.parametrize("dtype", ["float32", "int8"])
def test_flat_stream_with_a_tail(ctx, n, dtype):
    """A flat tensor whose length is not a multiple of the 16-byte vector:
    the vector kernel takes the whole vectors, the tail runs element-wise;
    staged, chunked (4 KiB), pinned and from HBM."""
    from sym_amd import encoder as EN
    rng = np.random.default_rng(n)
    if dtype == "float32":
        x = (rng.standard_normal(n) * 100).astype(np.float32)
        ops = [EN.Cast("float16")]
    else:
        x = rng.integers(-128, 128, n, dtype=np.int8)
        ops = [EN.Dequantize(EN.InlineParam((0.0625,), "float32", 0))]
    plan = EN.encode([n], dtype, ops)
    want = O.run_typed(plan.blob, {}, {}, x).tobytes()
    pin = torch.from_numpy(x.view(np.uint8).copy()).pin_memory().numpy().view(x.dtype)
    for src, opts in ((x, {}), (x, {"chunk_bytes": 4096}), (pin, {"source_pinned": 1})):
        out, rep, b = run_h2d(ctx, plan.blob, {}, {}, src, "flat %s n=%d" % (dtype, n), **opts)
        assert b.kernel == "stream"
        assert out.tobytes() == want, opts
    xd = torch.from_numpy(x.view(np.uint8).copy()).cuda()
    dev = torch.empty(len(want), dtype=torch.uint8, device="cuda")
    ctx.relayout_device(b, xd.data_ptr(), dev.data_ptr())
    torch.cuda.synchronize()
    assert dev.cpu().numpy().tobytes() == want


# ------------------------------------------------------------------ C4

def _c4_expected_rows(q, s, rows):
    return f16_bits(O.dequantize_s8_f32(q[rows], s[rows, None], np.int32(0)))


def test_c4_expert_group(ctx):
    """Two experts (6 matrices) as one grouped transfer at full size; every
    element of every matrix checked against the oracle (gate/up [14336, 4096]
    and down [4096, 14336]), in blocks of 2048 rows to bound the oracle's
    memory."""
    pool = W.c4_pool(experts=2)
    plan = P.Plan(W.c4_plan().blob)
    bounds, srcs, dsts, outs = [], [], [], []
    for e in range(2):
        for q, s in pool[e]:
            b = P.Bound(plan, {"s0": q.shape[0], "s1": q.shape[1]}, W.param("scale", s))
            out = torch.empty(b.destination_bytes, dtype=torch.uint8, device="cuda")
            bounds.append(b)
            srcs.append((q.ctypes.data, q.nbytes))
            dsts.append((out.data_ptr(), out.numel()))
            outs.append(out)
    say("c4 group of", len(bounds))
    reps, total = ctx.execute_group_h2d(bounds, srcs, dsts)
    torch.cuda.synchronize()
    assert total["wire_bytes"] == 352321536 and total["destination_bytes"] == 704643072
    i = 0
    for e in range(2):
        for q, s in pool[e]:
            got = outs[i].cpu().numpy().view(np.uint16).reshape(q.shape)
            for r0 in range(0, q.shape[0], 2048):
                rows = np.arange(r0, min(q.shape[0], r0 + 2048))
                assert np.array_equal(got[rows], _c4_expected_rows(q, s, rows)), (e, q.shape, r0)
            i += 1


def test_c4_device_relayout_matches_h2d(ctx):
    """relx_relayout_device on a device-resident wire equals the H2D path."""
    rng = np.random.default_rng(7)
    q = W.int8_weight(1024, 4096, rng)
    s = W.scales(1024, rng)
    plan = P.Plan(W.c4_plan().blob)
    b = P.Bound(plan, {"s0": 1024, "s1": 4096}, W.param("scale", s))
    wire = torch.from_numpy(q).cuda()
    out = torch.empty(b.destination_bytes, dtype=torch.uint8, device="cuda")
    say("c4 device relayout")
    ctx.relayout_device(b, wire.data_ptr(), out.data_ptr())
    ctx.synchronize()
    want = _c4_expected_rows(q, s, np.arange(1024))
    assert np.array_equal(out.cpu().numpy().view(np.uint16).reshape(q.shape), want)


# ------------------------------------------------------------------ C5

def _c5_expected(x, s, b_idx=None):
    inv = (np.float32(1) / s).astype(np.float32)
    sub = x if b_idx is None else x[b_idx]
    wid = np.ascontiguousarray(sub.transpose(0, 2, 1, 3)).astype(np.float32)
    return O.quantize_f32_s8(wid, inv[None, :, None, None])


@pytest.mark.parametrize("B,S", W.C5_SHAPES)
def test_c5_activation_quant(ctx, B, S):
    """One plan bound per (B, S); every output element is checked against the
    oracle (by groups of batch entries past E = 32M elements, to bound the
    oracle's memory)."""
    plan = W.c5_plan()
    x, s = W.c5_input(B, S, seed=B * 10007 + S)
    out, rep, b = run_h2d(ctx, plan.blob, {"B": B, "S": S}, W.param("scale", s), x,
                          "c5 B=%d S=%d" % (B, S))
    E = B * S * 4096
    assert rep["wire_bytes"] == 2 * E and rep["destination_bytes"] == E
    got = out.view(np.int8).reshape(B, 32, S, 128)
    if E <= 33554432:
        assert np.array_equal(got, _c5_expected(x, s))
    else:
        step = max(1, 33554432 // (S * 4096))
        for b0 in range(0, B, step):
            picks = list(range(b0, min(B, b0 + step)))
            assert np.array_equal(got[picks], _c5_expected(x, s, picks)), picks


@pytest.mark.parametrize("case", PC.cases(), ids=[c[0] for c in PC.cases()])
def test_permute_bodies(ctx, case):
    """Block permutes through the direct body (shift indexing, parameters by
    head) and the general one, each against the oracle: uploaded with every
    stage on the device, with a 64 KiB chunk schedule, and device-resident."""
    name, blob, x, direct = case
    want = (O.run_typed(blob, {}, {}, x).tobytes() if P.Plan(blob).typed else
            O.execute_layout(O.bind(O.decode_plan(blob), {}), x.tobytes()))
    for opts in ({"host_stages": 0}, {"host_stages": 0, "chunk_bytes": 1 << 16}):
        out, rep, b = run_h2d(ctx, blob, {}, {}, x, "permute " + name, **opts)
        assert b.kernel == "permute" and b.permute_direct == direct
        assert out.tobytes() == want, opts
    xd = torch.from_numpy(x.view(np.uint8).reshape(-1).copy()).cuda()
    dev = torch.empty(len(want), dtype=torch.uint8, device="cuda")
    ctx.relayout_device(b, xd.data_ptr(), dev.data_ptr())
    torch.cuda.synchronize()
    assert dev.cpu().numpy().tobytes() == want


def test_random_permutes(ctx):
    """The 200 random block permutes of the launch tests against the oracle:
    uploaded with every stage on the device (default and 4 KiB chunks),
    device-resident, and device -> host into pageable memory (default and
    4 KiB chunks, alternately)."""
    direct = 0
    for i, (name, blob, x) in enumerate(PC.random_cases(200)):
        want = (O.run_typed(blob, {}, {}, x).tobytes() if P.Plan(blob).typed else
                O.execute_layout(O.bind(O.decode_plan(blob), {}), x.tobytes()))
        for chunk in (0, 4096):
            out, rep, b = run_h2d(ctx, blob, {}, {}, x, "random permute %d %s" % (i, name),
                                  host_stages=0, chunk_bytes=chunk)
            assert out.tobytes() == want, (i, name, chunk)
        direct += b.permute_direct
        xd = torch.from_numpy(np.ascontiguousarray(x).view(np.uint8).reshape(-1).copy()).cuda()
        dev = torch.empty(len(want), dtype=torch.uint8, device="cuda")
        ctx.relayout_device(b, xd.data_ptr(), dev.data_ptr())
        torch.cuda.synchronize()
        assert dev.cpu().numpy().tobytes() == want, (i, name, "device")
        # device -> host: the permute into the device result, copied out in chunks
        host = np.full(len(want), 0xA5, np.uint8)
        ctx.execute_d2h(b, xd.data_ptr(), xd.numel(), host.ctypes.data, len(want),
                        chunk_bytes=4096 if i % 2 else 0, source_pinned=0)
        assert host.tobytes() == want, (i, name, "d2h")
    assert 0 < direct < 200


def test_random_one_byte_transposes(ctx):
    """The 120 random one-byte transposes of the launch tests (128 x 128 byte
    tiles and 64 c x 128 q tiles in the rotated order, 64-wide tiles, edge
    strips, element-wise ones)
    against the oracle: uploaded with every stage on the device (default and
    4 KiB chunks), device-resident, and device -> host into pageable memory
    (default and 4 KiB chunks, alternately)."""
    wide = byte_tiles = 0
    for i, (name, blob, x, width) in enumerate(TC.random_cases(_TN, seed=_TS)):
        want = (O.run_typed(blob, {}, {}, x).tobytes() if P.Plan(blob).typed else
                O.execute_layout(O.bind(O.decode_plan(blob), {}), x.tobytes()))
        for chunk in (0, 4096):
            out, rep, b = run_h2d(ctx, blob, {}, {}, x, "random transpose %d %s" % (i, name),
                                  host_stages=0, chunk_bytes=chunk)
            assert out.tobytes() == want, (i, name, chunk)
        wide += b.transpose_tile_q == 128
        byte_tiles += b.transpose_tile_c == 128
        xd = torch.from_numpy(np.ascontiguousarray(x).view(np.uint8).reshape(-1).copy()).cuda()
        dev = torch.empty(len(want), dtype=torch.uint8, device="cuda")
        ctx.relayout_device(b, xd.data_ptr(), dev.data_ptr())
        torch.cuda.synchronize()
        assert dev.cpu().numpy().tobytes() == want, (i, name, "device")
        host = np.full(len(want), 0xA5, np.uint8)
        ctx.execute_d2h(b, xd.data_ptr(), xd.numel(), host.ctypes.data, len(want),
                        chunk_bytes=4096 if i % 2 else 0, source_pinned=0)
        assert host.tobytes() == want, (i, name, "d2h")
    assert wide > 40 and byte_tiles >= 5


@pytest.mark.parametrize("B,S", [(1, 65536), (64, 4096)])
def test_c5_device_resident(ctx, B, S):
    """Device-resident C5 boxes of 256 MiB and 1 GiB of result, one direct
    launch each (relx_relayout_device), checked against the oracle in
    sequence slices."""
    x, sc = W.c5_input(B, S, seed=B * 7919 + S)
    b = P.Bound(P.Plan(W.c5_plan().blob), {"B": B, "S": S}, W.param("scale", sc))
    assert b.permute_direct
    say("c5 device-resident B=%d S=%d" % (B, S))
    xd = torch.from_numpy(x.view(np.uint8).reshape(-1)).cuda()
    dev = torch.empty(B * S * 4096, dtype=torch.int8, device="cuda")
    ctx.relayout_device(b, xd.data_ptr(), dev.data_ptr())
    torch.cuda.synchronize()
    del xd
    got = dev.cpu().numpy().reshape(B, 32, S, 128)
    step = max(1, 8388608 // (B * 4096))
    for s0 in range(0, S, step):
        assert np.array_equal(got[:, :, s0:s0 + step], _c5_expected(x[:, s0:s0 + step], sc)), s0


# -------------------------------------------------------- value sweeps

def _cast_plan(src_dtype, dst_dtype, n):
    return EN.encode([n], src_dtype, [EN.Cast(dst_dtype)]).blob


def test_f16_widening_exhaustive(ctx):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    out, _, _ = run_h2d(ctx, _cast_plan("float16", "float32", 65536), {}, {}, h, "widen all f16")
    assert np.array_equal(out.view(np.uint32), O.widen_f16_f32_bits(h))  # NaN payloads included


def test_f32_narrowing_sweep(ctx):
    rng = np.random.default_rng(11)
    e = np.arange(256, dtype=np.uint32) << 23
    edges = np.concatenate([e | m for m in (0, 1, 0x1000, 0x0fff, 0x1fff, 0x2000, 0x3000,
                                            0x7fffff, 0x400000, 0x7fe000, 0x7ff000)])
    bits = np.concatenate([rng.integers(0, 2**32, 1 << 24, dtype=np.uint64).astype(np.uint32),
                           edges, edges | 0x80000000]).astype(np.uint32)
    n = bits.size
    out, _, _ = run_h2d(ctx, _cast_plan("float32", "float16", n), {}, {}, bits, "narrow sweep")
    assert np.array_equal(out.view(np.uint16), O.narrow_f32_f16_bits(bits))  # NaNs included
    out, _, _ = run_h2d(ctx, _cast_plan("float32", "bfloat16", n), {}, {}, bits, "bf16 sweep")
    assert np.array_equal(out.view(np.uint16), O.narrow_f32_bf16_bits(bits))


def test_quantize_dequantize_sweep(ctx):
    rng = np.random.default_rng(12)
    bits = np.concatenate([rng.integers(0, 2**32, 1 << 22, dtype=np.uint64).astype(np.uint32),
                           np.array([0x7fc00000, 0xffc00000, 0x7f800000, 0xff800000, 0x80000000,
                                     0x00000001, 0x3f000000, 0xbfc00000], np.uint32)])
    x = bits.view(np.float32)
    for scale in (0.3, 1.0, 1e-3, 2.0 ** -130):
        sc = EN.InlineParam((scale,))
        plan = EN.encode([x.size], "float32", [EN.Quantize(sc)]).blob
        out, _, _ = run_h2d(ctx, plan, {}, {}, x, "quant scale=%g" % scale)
        inv = (np.float32(1) / np.float32(scale)).astype(np.float32)
        assert np.array_equal(out.view(np.int8), O.quantize_f32_s8(x, inv))
    q = np.arange(-128, 128, dtype=np.int8).repeat(4096)
    for scale, zp in ((0.3, 0), (0.3, 127), (2.0 ** -140, -128), (1e30, 5)):
        plan = EN.encode([q.size], "int8", [EN.Dequantize(EN.InlineParam((scale,)),
                                                          EN.InlineParam((zp,), "int32"))]).blob
        out, _, _ = run_h2d(ctx, plan, {}, {}, q, "dequant scale=%g zp=%d" % (scale, zp))
        want = O.dequantize_s8_f32(q, np.float32(scale), np.int32(zp))
        assert np.array_equal(out.view(np.uint32), want.view(np.uint32))


def test_context_stats_and_reuse(ctx):
    st = ctx.stats()
    assert st["calls"] > 0 and st["failures"] == 0 and not st["quarantined"]
    assert st["device_bytes"] > 0


# ------------------------------------------------ double rounding regression

def _double_rounding_rows(rng, want_rows=256):
    """(q, scale) rows where f16(fl32(q*s)) differs from a single rounding of
    the exact product to f16: a fused multiply+narrow would flip them."""
    rows, scales = [], []
    q_all = np.arange(-128, 128, dtype=np.int32)
    while len(rows) < want_rows:
        s = rng.uniform(1e-3, 2e-2, 4096).astype(np.float32)
        exact = q_all[None, :].astype(np.float64) * s[:, None].astype(np.float64)
        two = O.narrow_f32_f16_bits(exact.astype(np.float32).view(np.uint32))
        one = exact.astype(np.float16).view(np.uint16)  # single rounding of the exact product
        hit = np.argwhere(two != one)
        for r, c in hit:
            row = np.full(256, q_all[c], np.int8)
            row[:] = rng.integers(-127, 128, 256)
            row[0] = q_all[c]
            rows.append(row)
            scales.append(s[r])
            if len(rows) >= want_rows:
                break
    return np.stack(rows), np.array(scales, np.float32)


def test_dequant_f16_keeps_both_roundings(ctx):
    rng = np.random.default_rng(99)
    q, s = _double_rounding_rows(rng)
    want = f16_bits(O.dequantize_s8_f32(q, s[:, None], np.int32(0)))
    # stream family (C4 layout)
    out, _, b = run_h2d(ctx, W.c4_plan().blob, {"s0": q.shape[0], "s1": q.shape[1]},
                        W.param("scale", s), q, "double rounding, stream")
    assert b.kernel == "stream"
    assert np.array_equal(out.view(np.uint16).reshape(q.shape), want)
    # transpose family (C3 layout): source [256 cols x rows] with per-column scales
    qt = np.ascontiguousarray(q.T)
    out, _, b = run_h2d(ctx, W.c3_plan().blob, {"s0": qt.shape[0], "s1": qt.shape[1]},
                        W.param("scale", s), qt, "double rounding, transpose")
    assert b.kernel == "transpose"
    assert np.array_equal(out.view(np.uint16).reshape(q.shape), want)
