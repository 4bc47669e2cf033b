"""The reference-shaped dispatch API on the MI355X: the typed corpus and a
grouped C4-like step through prepare_dispatch / execute_dispatch (and the
template and group forms), bit-exact against the corpus expectations and
the oracle, with the reference's report fields and single-use rules."""
import hashlib
import sys

import numpy as np
import pytest

from oracle import relx_oracle as O
from sym_amd import pyreloc as P
from sym_amd import workloads as W
from tests import golden_io as G

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


def host_view(a):
    return P.BufferView(a.ctypes.data, a.nbytes, 0, list(a.shape),
                        [s // a.dtype.itemsize for s in a.strides], a.dtype.itemsize, "host")


def device_view(t):
    return P.BufferView(t.data_ptr(), t.numel() * t.element_size(), 0, list(t.shape),
                        list(t.stride()), t.element_size(), "cuda", t.device.index)


TORCH = {"f16": torch.float16, "f32": torch.float32, "i8": torch.int8, "bf16": torch.bfloat16,
         "u8": torch.uint8, "i32": torch.int32}


@pytest.fixture(scope="module")
def resources():
    assert torch.cuda.is_available(), "a GPU test needs the MI355X"
    r = P.Resources(0)
    yield r
    r.close()


TYPED = G.typed_fixtures()


@pytest.mark.parametrize("meta,blob", TYPED, ids=[m["name"] for m, _ in TYPED])
def test_corpus_through_dispatch(resources, meta, blob):
    plan = P.load_typed_plan(blob)
    for binding in meta["bindings"]:
        src = np.ascontiguousarray(G.bits_array(binding["source"]).reshape(binding["source"]["shape"]))
        exp = G.bits_array(binding["expected"]).reshape(binding["expected"]["shape"])
        b = P.bind_typed(plan, binding["symbols"], G.fixture_params(meta))
        rows = [r["implementation"] for r in P.query_capability(b, "h2d", "cuda")["eligible"]]
        for impl in [""] + rows:
            say(meta["name"], binding["symbols"], "row", impl or "auto")
            out = torch.empty(list(exp.shape), dtype=torch.uint8 if exp.dtype.itemsize == 1
                              else {2: torch.int16, 4: torch.int32, 8: torch.int64}[exp.dtype.itemsize],
                              device="cuda")
            req = P.prepare_dispatch(b, host_view(src), device_view(out), "h2d", implementation=impl)
            rep = P.execute_dispatch(req, resources=resources)
            torch.cuda.synchronize()
            got = out.cpu().numpy().view(exp.dtype)
            assert np.array_equal(got, exp), (meta["name"], impl)
            assert hashlib.sha256(got.tobytes()).hexdigest() == binding["expected"]["sha256"]
            fp = binding["footprints"]["h2d"]
            for key in ("source_bytes", "destination_bytes", "parameter_bytes"):
                assert rep[key] == fp[key], (meta["name"], key)
            assert rep["executed"] is True and rep["payload_bytes_transferred"] == rep["wire_bytes"]
            if impl:
                assert rep["implementation"] == impl and rep["placement_reason"] == "forced"
            with pytest.raises(P.TransferError) as e:
                P.execute_dispatch(req, resources=resources)
            assert e.value.code == "already_executed"


def test_template_reuse_over_many_views(resources, rng):
    plan = P.Plan(W.c2_plan(n=2).blob)
    b = P.Bound(plan, {}, {})
    t = P.prepare_dispatch_template(b, "h2d", "cuda")
    for seed in range(3):
        x = np.random.default_rng(seed).standard_normal((2, 3, 224, 224), dtype=np.float32)
        out = torch.empty((2, 224, 224, 4), dtype=torch.float16, device="cuda")
        say("template reuse", seed)
        rep = P.execute_dispatch(P.prepare_dispatch_from_template(t, host_view(x), device_view(out)),
                                 resources=resources)
        torch.cuda.synchronize()
        want = np.zeros((2, 224, 224, 4), np.float16)
        want[..., :3] = np.transpose(x, (0, 2, 3, 1)).astype(np.float16)
        assert np.array_equal(out.cpu().numpy().view(np.uint16), want.view(np.uint16))
        assert rep["implementation"] == "hip_relayout@1"  # pageable source: the cast is staged


def _c5_want(x, s):
    inv = (np.float32(1) / s).astype(np.float32)
    wid = np.ascontiguousarray(x.transpose(0, 2, 1, 3)).astype(np.float32)
    return O.quantize_f32_s8(wid, inv[None, :, None, None])


def test_fresh_bindings_find_their_own_parameters(resources, rng):
    """Each call binds C5 afresh (the headline step's pattern), alternating
    three scale tables and a binding kept from the first call: the context
    keeps parameter tables by content, so every call must still quantize
    with its own scales (oracle, bit-exact)."""
    B, S = 2, 256
    plan = P.load_typed_plan(W.c5_plan().blob)
    x, _ = W.c5_input(B, S, seed=5)
    scales = [rng.uniform(0.02, 0.05, 32).astype(np.float32) for _ in range(3)]
    kept = P.bind_typed(plan, {"B": B, "S": S}, W.param("scale", scales[0]))
    for i, k in enumerate([0, 1, 2, 1, 0, 2, -1, 2]):
        bound = kept if k < 0 else P.bind_typed(plan, {"B": B, "S": S}, W.param("scale", scales[k]))
        s = scales[0] if k < 0 else scales[k]
        out = torch.empty((B, 32, S, 128), dtype=torch.int8, device="cuda")
        say("fresh binding", i, "scales", k)
        req = P.prepare_dispatch(bound, host_view(x), device_view(out), "h2d")
        P.execute_dispatch(req, caller_stream=torch.cuda.current_stream().cuda_stream,
                           resources=resources)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), _c5_want(x, s)), (i, k)


@pytest.mark.parametrize("opts,pipeline_kind,chunks", [
    ({}, "direct_dma", None),
    ({"direct_dense_upload": False}, "pinned_ring", None),
    ({"pipeline": False, "direct_dense_upload": False}, "pinned_ring", 1),
    ({"pipeline": False}, "direct_dma", 1)])
def test_dispatch_upload_options(resources, opts, pipeline_kind, chunks):
    """direct_dense_upload=False stages a dense pinned source through the
    ring; pipeline=False sends the whole buffer as one chunk (reference
    TransferOptions, Transfer.h:129-134). Results bit-exact either way."""
    B, S = 4, 1024
    plan = P.load_typed_plan(W.c5_plan().blob)
    x, s = W.c5_input(B, S, seed=9)
    xp = torch.from_numpy(x).pin_memory()
    b = P.bind_typed(plan, {"B": B, "S": S}, W.param("scale", s))
    out = torch.empty((B, 32, S, 128), dtype=torch.int8, device="cuda")
    view = P.BufferView(xp.data_ptr(), x.nbytes, 0, list(x.shape),
                        [st // 2 for st in x.strides], 2, "host")
    say("dispatch options", opts)
    rep = P.execute_dispatch(P.prepare_dispatch(b, view, device_view(out), "h2d"),
                             chunk_size=4 << 20, resources=resources, **opts)
    torch.cuda.synchronize()
    assert rep["host_pipeline"] == pipeline_kind, rep
    if chunks is not None:
        assert rep["host_chunks"] == chunks, rep
    else:
        assert rep["host_chunks"] > 1, rep
    assert np.array_equal(out.cpu().numpy(), _c5_want(x, s))


def test_headline_schedule_end_to_end():
    """C5 at B=64, S=4096 through execute_dispatch with the options of the
    bench's steps (ordered after torch's stream, 8 staging threads, retained
    resources), from a page-locked source (32 direct DMA chunks of 64 MiB,
    kernel batches of 16, 16, 16, 14 and 2 batch entries) with 3 and with 2
    ring slots, and from the pageable source with 3 slots and with
    reloc_torch's 2 (64 chunks of 32 MiB; with the chunks left to the
    library a ring has at least three slots); every output byte equals the
    oracle (the reference checks every eligible H2D row end to end,
    DispatchTest.cpp:883)."""
    B, S = 64, 4096
    plan = P.load_typed_plan(W.c5_plan().blob)
    x, s = W.c5_input(B, S)
    want = np.empty((B, 32, S, 128), np.int8)
    for b0 in range(0, B, 2):
        want[b0:b0 + 2] = _c5_want(x[b0:b0 + 2], s)
    xp = torch.from_numpy(x).pin_memory()
    pinned = P.BufferView(xp.data_ptr(), x.nbytes, 0, list(x.shape),
                          [st // 2 for st in x.strides], 2, "host")
    stream = torch.cuda.current_stream().cuda_stream
    res = P.Resources(0)
    try:
        M = 1 << 20
        for view, slots, pipeline, chunks, chunk_bytes in ((pinned, 3, "direct_dma", 32, 0),
                                                           (pinned, 2, "direct_dma", 32, 0),
                                                           (host_view(x), 3, "pinned_ring", 64, 32 * M),
                                                           (host_view(x), 2, "pinned_ring", 64, 32 * M)):
            out = torch.empty((B, 32, S, 128), dtype=torch.int8, device="cuda")
            b = P.bind_typed(plan, {"B": B, "S": S}, W.param("scale", s))
            say("headline schedule", pipeline, "slots", slots)
            rep = P.execute_dispatch(P.prepare_dispatch(b, view, device_view(out), "h2d"),
                                     caller_stream=stream, resources=res, gather_threads=8,
                                     n_buffers=slots)
            torch.cuda.synchronize()
            assert rep["host_pipeline"] == pipeline and rep["host_chunks"] == chunks, rep
            assert rep["kernel_launches"] == 5, rep
            if chunk_bytes:
                assert rep["host_chunk_bytes"] == chunk_bytes, rep
                assert rep["host_buffers"] == 3, rep
            got = out.cpu().numpy()
            for b0 in range(0, B, 8):
                assert np.array_equal(got[b0:b0 + 8], want[b0:b0 + 8]), (pipeline, slots, b0)
            del out, got
    finally:
        res.close()


@pytest.mark.parametrize("limit", [0, 3 << 20])
def test_retained_scratch_is_bounded(rng, limit):
    """max_retained_bytes of a resource cache: after each call the ring and
    the wire arena are released until what is kept fits, and the next call
    allocates them again with the same results."""
    B, S = 2, 1024  # 16 MiB of f16 source, 8 MiB of int8 output
    plan = P.load_typed_plan(W.c5_plan().blob)
    x, s = W.c5_input(B, S, seed=6)
    want = _c5_want(x, s)
    cache = P.DispatchResources(max_retained_bytes=limit)
    try:
        for i in range(3):
            out = torch.empty((B, 32, S, 128), dtype=torch.int8, device="cuda")
            say("retained limit", limit, "call", i)
            b = P.bind_typed(plan, {"B": B, "S": S}, W.param("scale", s))
            P.execute_dispatch(P.prepare_dispatch(b, host_view(x), device_view(out), "h2d"),
                               caller_stream=torch.cuda.current_stream().cuda_stream,
                               resources=cache, chunk_size=1 << 20)
            torch.cuda.synchronize()
            assert np.array_equal(out.cpu().numpy(), want), i
            st = cache.stats()
            assert st["retained_bytes"] <= limit, st
    finally:
        cache.close()


def test_group_dispatch_c4_like(resources, rng):
    rows, cols = 512, 256
    plan = P.Plan(W.c4_plan().blob)
    entries, outs, wants, keep = [], [], [], []
    for j in range(6):
        q = W.int8_weight(rows, cols, rng)
        s = W.scales(rows, rng)
        keep.append(q)  # views borrow the memory: the arrays must outlive the call
        b = P.Bound(plan, {"s0": rows, "s1": cols}, W.param("scale", s))
        out = torch.empty((rows, cols), dtype=torch.float16, device="cuda")
        entries.append((b, host_view(q), device_view(out), "h2d"))
        outs.append(out)
        deq = np.ascontiguousarray(O.dequantize_s8_f32(q, s[:, None], np.int32(0)), np.float32)
        wants.append(O.narrow_f32_f16_bits(deq.view(np.uint32)).astype(np.uint16).tobytes())
    say("group of 6", rows, cols)
    g = P.prepare_dispatch_group(entries)
    rep = P.execute_dispatch_group(g, resources=resources, owners=(tuple(keep), tuple(outs)))
    torch.cuda.synchronize()
    assert rep["logical_transfers"] == 6 and rep["completion_granularity"] == "group"
    for out, want in zip(outs, wants):
        assert out.cpu().numpy().tobytes() == want
    with pytest.raises(P.TransferError):
        P.execute_dispatch_group(g, resources=resources)


# ------------------------------------------------------------- D2H

def test_corpus_device_to_host(resources):
    for meta, blob in TYPED:
        plan = P.load_typed_plan(blob)
        for binding in meta["bindings"]:
            src = np.ascontiguousarray(G.bits_array(binding["source"]).reshape(binding["source"]["shape"]))
            exp = G.bits_array(binding["expected"]).reshape(binding["expected"]["shape"])
            b = P.bind_typed(plan, binding["symbols"], G.fixture_params(meta))
            src_t = torch.from_numpy(src.view(np.uint8).copy()).cuda()
            dsrc = P.BufferView(src_t.data_ptr(), src.nbytes, 0, list(src.shape),
                                [s // src.itemsize for s in src.strides], src.itemsize, "cuda", 0)
            out = np.full(exp.shape, 0xCD, dtype=np.uint8).view(exp.dtype) if exp.itemsize == 1 \
                else np.zeros(exp.shape, exp.dtype)
            say(meta["name"], binding["symbols"], "d2h")
            req = P.prepare_dispatch(b, dsrc, host_view(out), "d2h")
            rep = P.execute_dispatch(req, resources=resources)
            assert np.array_equal(out, exp), meta["name"]
            fp = binding["footprints"]["d2h"]
            for key in ("source_bytes", "destination_bytes", "parameter_bytes"):
                assert rep[key] == fp[key], (meta["name"], key)
            assert rep["implementation"] == "hip_relayout_d2h" and rep["executed"]


def _c5_expected(x, s):
    x32 = O.widen_f16_f32_bits(x.view(np.uint16)).view(np.float32)      # [B,S,32,128]
    q = O.quantize_f32_s8(x32, (np.float32(1.0) / s.astype(np.float32))[None, None, :, None])
    return np.ascontiguousarray(np.transpose(q, (0, 2, 1, 3)))             # [B,32,S,128]


@pytest.mark.parametrize("pinned", [False, True])
@pytest.mark.parametrize("chunk,S", [(0, 1024), (64 << 10, 1024), (0, 4096)])
def test_c5_kv_evict_device_to_host(resources, pinned, chunk, S):
    """C5's quantizing permute in the other direction (KV eviction): a device
    f16 [B,S,32,128] tensor to a host int8 [B,32,S,128] buffer, chunked
    (ring reuse with two slots at 64 KiB) into pageable or pinned memory.
    S = 4096: the permute stores its result through the caches (planes
    512 KiB apart), and the copies that follow read it."""
    B = 2
    x, s = W.c5_input(B, S, seed=77)
    b = P.Bound(P.Plan(W.c5_plan().blob), {"B": B, "S": S}, W.param("scale", s))
    xs = torch.from_numpy(x.view(np.uint16).view(np.int16).copy()).cuda()
    if pinned:
        out_t = torch.empty(B * 32 * S * 128, dtype=torch.int8).pin_memory()
        out = out_t.numpy()
    else:
        out = np.empty(B * 32 * S * 128, np.int8)
    say("c5 d2h", B, S, "pinned" if pinned else "pageable", "chunk", chunk)
    rep = resources.execute_d2h(b, xs.data_ptr(), x.nbytes, out.ctypes.data, out.nbytes,
                                chunk_bytes=chunk, n_buffers=2, source_pinned=1 if pinned else 0)
    assert rep["direct_dma"] == (1 if pinned else 0)
    if chunk:
        assert rep["chunks"] > 4  # byte-chunked copies after one permute launch
    assert np.array_equal(out.reshape(B, 32, S, 128), _c5_expected(x, s))


def test_c3_device_to_host_matches_h2d(resources, rng):
    """The same bound plan in both directions gives the same bytes."""
    rows, cols = 256, 512
    q, s = W.int8_weight(rows, cols, rng), W.scales(cols, rng)
    b = P.Bound(P.Plan(W.c3_plan().blob), {"s0": rows, "s1": cols}, W.param("scale", s))
    dev = torch.empty(rows * cols * 2, dtype=torch.uint8, device="cuda")
    say("c3 h2d then d2h")
    resources.execute_h2d(b, q.ctypes.data, q.nbytes, dev.data_ptr(), dev.numel())
    torch.cuda.synchronize()
    via_h2d = dev.cpu().numpy()
    qd = torch.from_numpy(q.view(np.uint8).copy()).cuda()
    out = np.empty(rows * cols * 2, np.uint8)
    resources.execute_d2h(b, qd.data_ptr(), q.nbytes, out.ctypes.data, out.nbytes, chunk_bytes=16 << 10)
    assert np.array_equal(out, via_h2d)


# ------------------------------------------------------------ asynchronous

def _expert_group(rng, rows, cols, n, pinned):
    plan = P.Plan(W.c4_plan().blob)
    entries, outs, wants, keep = [], [], [], []
    for _ in range(n):
        q, s = W.int8_weight(rows, cols, rng), W.scales(rows, rng)
        if pinned:
            qt = torch.from_numpy(q).pin_memory()
            q = qt.numpy()
            keep.append(qt)
        keep.append(q)
        b = P.Bound(plan, {"s0": rows, "s1": cols}, W.param("scale", s))
        out = torch.empty((rows, cols), dtype=torch.float16, device="cuda")
        entries.append((b, host_view(q), device_view(out), "h2d"))
        outs.append(out)
        deq = np.ascontiguousarray(O.dequantize_s8_f32(q, s[:, None], np.int32(0)), np.float32)
        wants.append(O.narrow_f32_f16_bits(deq.view(np.uint32)).astype(np.uint16))
    return entries, outs, wants, keep


@pytest.mark.parametrize("pinned", [False, True])
def test_submitted_groups_overlap_and_order_a_stream(resources, rng, pinned):
    """Two groups in flight at once; the second is consumed on a torch stream
    through wait_stream (no host wait) and the first through wait()."""
    ea, oa, wa, ka = _expert_group(rng, 1024, 512, 3, pinned)
    eb, ob, wb, kb = _expert_group(rng, 512, 1024, 3, pinned)
    say("submit two groups", "pinned" if pinned else "pageable")
    ca = P.submit_dispatch_group(P.prepare_dispatch_group(ea), resources=resources,
                                 owners=(tuple(ka), tuple(oa)))
    cb = P.submit_dispatch_group(P.prepare_dispatch_group(eb), resources=resources,
                                 owners=(tuple(kb), tuple(ob)))
    consumer = torch.cuda.Stream()
    cb.wait_stream(consumer.cuda_stream)
    with torch.cuda.stream(consumer):
        sums = [o.view(torch.int16).to(torch.int64).sum() for o in ob]
    rep = ca.wait()
    assert rep["logical_transfers"] == 3 and ca.query()
    for out, want in zip(oa, wa):
        assert np.array_equal(out.cpu().numpy().view(np.uint16), want)
    consumer.synchronize()
    for sm, want in zip(sums, wb):
        assert int(sm.item()) == int(want.view(np.int16).astype(np.int64).sum())
    cb.wait()
    for out, want in zip(ob, wb):
        assert np.array_equal(out.cpu().numpy().view(np.uint16), want)
    with pytest.raises(P.TransferError):
        P.submit_dispatch_group(ca.group, resources=resources, owners=((), ()))
    ca.close()
    cb.close()


@pytest.mark.parametrize("pinned", [False, True])
def test_call_after_submitted_group_waits_for_its_wire(resources, rng, pinned):
    """A blocking group right after a submitted one reuses the context's wire
    arena: it must not overwrite wire bytes the first group's kernels have
    yet to read."""
    ea, oa, wa, ka = _expert_group(rng, 2048, 2048, 3, pinned)
    eb, ob, wb, kb = _expert_group(rng, 256, 512, 2, pinned)
    say("submit, then a blocking group on the same resources", "pinned" if pinned else "pageable")
    ca = P.submit_dispatch_group(P.prepare_dispatch_group(ea), resources=resources,
                                 owners=(tuple(ka), tuple(oa)))
    P.execute_dispatch_group(P.prepare_dispatch_group(eb), resources=resources)
    for out, want in zip(ob, wb):
        assert np.array_equal(out.cpu().numpy().view(np.uint16), want)
    ca.wait()
    for out, want in zip(oa, wa):
        assert np.array_equal(out.cpu().numpy().view(np.uint16), want)
    ca.close()


def test_device_to_host_after_a_submitted_group(resources, rng):
    """A device-to-host call writes the wire arena that a submitted upload
    may still be reading: it is ordered after that upload."""
    ea, oa, wa, ka = _expert_group(rng, 2048, 2048, 3, True)
    rows, cols = 256, 512
    q, s = W.int8_weight(rows, cols, rng), W.scales(cols, rng)
    b = P.Bound(P.Plan(W.c3_plan().blob), {"s0": rows, "s1": cols}, W.param("scale", s))
    qd = torch.from_numpy(q.view(np.uint8).copy()).cuda()
    dev = torch.empty(rows * cols * 2, dtype=torch.uint8, device="cuda")
    resources.execute_h2d(b, q.ctypes.data, q.nbytes, dev.data_ptr(), dev.numel())
    torch.cuda.synchronize()
    want = dev.cpu().numpy()
    say("submit, then a device-to-host call on the same resources")
    ca = P.submit_dispatch_group(P.prepare_dispatch_group(ea), resources=resources,
                                 owners=(tuple(ka), tuple(oa)))
    out = np.empty(rows * cols * 2, np.uint8)
    resources.execute_d2h(b, qd.data_ptr(), q.nbytes, out.ctypes.data, out.nbytes)
    assert np.array_equal(out, want)
    ca.wait()
    for o, w in zip(oa, wa):
        assert np.array_equal(o.cpu().numpy().view(np.uint16), w)
    ca.close()


def test_abandoned_completion_drains(resources, rng):
    e, o, w, k = _expert_group(rng, 256, 256, 2, True)
    c = P.submit_dispatch_group(P.prepare_dispatch_group(e), resources=resources,
                                owners=(tuple(k), tuple(o)))
    c.close()  # waits for the work before releasing the handle
    for out, want in zip(o, w):
        assert np.array_equal(out.cpu().numpy().view(np.uint16), want)


# ------------------------------------------------------------ error flag

def _shifted_channel_plan(monkeypatch):
    """A per-row dequantize whose channel expression is `row + 1`: the last
    row selects a channel one past its scale table (the element-wise kernel's
    range check, reported through the call's status flag)."""
    from sym_amd import encoder as EN
    orig = EN._stage

    def shifted(op, dtype, shape, rank):
        st = orig(op, dtype, shape, rank)
        if st.channel is not None:
            st.channel = EN.E("add", st.channel, EN.E.c(1))
        return st

    monkeypatch.setattr(EN, "_stage", shifted)
    scales = EN.InlineParam((0.5, 0.25, 0.125, 2.0), "float32", 1)
    return EN.encode([4, 6], "int8", [EN.Dequantize(scales, axis=0)])


def test_channel_outside_the_table_is_reported(resources, rng, monkeypatch):
    plan = _shifted_channel_plan(monkeypatch)
    monkeypatch.undo()  # the plans below come from the ordinary encoder
    q = rng.integers(-128, 128, (4, 6), dtype=np.int8)
    with pytest.raises(O.ExecutionError, match="channel_out_of_range"):
        O.run_typed(plan.blob, {}, {}, q)
    b = P.bind_typed(P.load_typed_plan(plan.blob), {}, {})
    out = torch.empty((4, 6), dtype=torch.float32, device="cuda")
    say("channel out of range, h2d then d2h")
    with pytest.raises(P.TransferError, match="channel_out_of_range"):
        resources.execute_h2d(b, q.ctypes.data, q.nbytes, out.data_ptr(), out.numel() * 4)
    qd = torch.from_numpy(q.view(np.uint8).copy()).cuda()
    host = np.empty(24, np.float32)
    with pytest.raises(P.TransferError, match="channel_out_of_range"):
        resources.execute_d2h(b, qd.data_ptr(), q.nbytes, host.ctypes.data, host.nbytes)
    say("channel out of range, device-resident")
    resources.relayout_device(b, qd.data_ptr(), out.data_ptr(), stream=0)
    with pytest.raises(P.TransferError, match="channel_out_of_range"):
        resources.synchronize()
    resources.synchronize()  # reported once
    # the flag belongs to its call: a good call on the same resources is clean
    rows, cols = 64, 128
    q2, s2 = W.int8_weight(rows, cols, rng), W.scales(cols, rng)
    b2 = P.Bound(P.Plan(W.c3_plan().blob), {"s0": rows, "s1": cols}, W.param("scale", s2))
    dev = torch.empty(rows * cols * 2, dtype=torch.uint8, device="cuda")
    resources.execute_h2d(b2, q2.ctypes.data, q2.nbytes, dev.data_ptr(), dev.numel())
    torch.cuda.synchronize()
