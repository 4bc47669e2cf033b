"""CPU oracle for the libreloc plan-execution path (TEST INFRASTRUCTURE ONLY).

This module is the checker the parity tests compare the HIP path against. It
restates, in numpy, the reference runtime's algorithm for the hot path:

* wire decode v0/v1      -- libreloc/src/Decode.cpp:115-948
* wire decode v2         -- libreloc/src/Decode.cpp:950-1012 (indexed plans)
* expression evaluation  -- libreloc/src/Bind.cpp:84-161
* bind (layout)          -- libreloc/src/Bind.cpp:176-384
* bindTyped              -- libreloc/src/Bind.cpp:494-699
* prepareProgram         -- libreloc/src/TypedExecute.cpp:292-403
* stage arithmetic       -- libreloc/quant/Quant.cpp:107-214,
                            libreloc/quant/QuantKernels.h:23-28,
                            libreloc/src/TypedExecute.cpp:472-499
* fillAt                 -- libreloc/src/TypedExecute.cpp:422-464
* executeHost            -- libreloc/src/TypedExecute.cpp:726-922 (the walker
                            semantics of walk()/element(), 202-290)
* layout gather          -- libreloc/src/Execute.cpp:94-134
* planChunks             -- libreloc/src/ChunkSchedule.cpp:9-90
* bindIndexed + the indexed host rows
                         -- libreloc/src/Bind.cpp:701-819,
                            libreloc/src/TypedExecute.cpp:741-790

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import it, and only as the checker; the product (sym_amd) never does.

Pinning (what each function is checked against) is listed in the module's
test file tests/test_oracle.py. Every function here has at least one check
beyond restating its own formula: the reference's golden corpus
(expected bits + sha256 per binding), the typed witness vectors, numpy's own
IEEE conversions, exhaustive enumeration where the domain allows it, and the
reference's own compiled CPU executor (oracle/_ref) where it builds.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

I64_MIN = -(1 << 63)
I64_MAX = (1 << 63) - 1

# ---------------------------------------------------------------------------
# Wire model (libreloc/include/reloc/Plan.h:20-189)
# ---------------------------------------------------------------------------

OP_PUSH_SYM, OP_PUSH_CONST, OP_ADD, OP_SUB, OP_MUL, OP_FLOORDIV, OP_MOD, OP_PUSH_DIM = range(8)
KIND_FLOAT, KIND_BFLOAT, KIND_INT, KIND_INDEX = range(4)
T_CAST, T_QUANTIZE, T_DEQUANTIZE = range(3)
P_IEEE_RNE, P_EXACT, P_SYMMETRIC_RNE, P_AFFINE = range(4)
PARAM_NONE, PARAM_INLINE, PARAM_BINDING = range(3)


class DecodeError(Exception):
    def __init__(self, offset: int, message: str):
        super().__init__(f"{message} (at byte {offset})")
        self.offset = offset
        self.message = message


class BindError(Exception):
    pass


class ExecutionError(Exception):
    def __init__(self, code: str, message: str):
        super().__init__(f"{code}: {message}")
        self.code = code


@dataclass
class ElementType:
    kind: int
    bitwidth: int

    def same(self, other: "ElementType") -> bool:
        return self.kind == other.kind and self.bitwidth == other.bitwidth

    @property
    def width(self) -> int:
        # typed::byteWidth, libreloc/src/TypedValue.cpp:12-16
        if self.bitwidth == 0 or self.bitwidth % 8:
            return 0
        return self.bitwidth // 8


@dataclass
class TensorDesc:
    extents: List[list]
    strides: List[list]
    offset: list
    element_type: ElementType


@dataclass
class Axis:
    name: str
    extent: list
    src_stride: list
    dst_stride: list


@dataclass
class PadFill:
    dst_axis: int
    lo: list
    hi: list
    fill_type: ElementType
    fill_bits: int


@dataclass
class Plan:
    symbols: List[str]
    src: TensorDesc
    dst: TensorDesc
    perm: List[int]
    axes: List[Axis]
    pad_fill: List[PadFill]
    divisibility: List[Tuple[list, int]]
    alignment: List[Tuple[int, int]]
    contiguity: List[int]
    no_copy: bool
    runtime_pad_check: bool
    inverse: List[list]


@dataclass
class StageType:
    type: ElementType
    signedness: int = 0


@dataclass
class StageParam:
    kind: int = PARAM_NONE
    rank: int = 0
    element_type: Optional[ElementType] = None
    inline_bits: List[int] = field(default_factory=list)
    binding_name: str = ""
    binding_extents: List[list] = field(default_factory=list)


@dataclass
class ValueStage:
    transform: int
    policy: int
    input: StageType
    output: StageType
    shape: List[list]
    scale: StageParam
    zero_point: StageParam
    axis: int
    has_channel: bool
    channel: list


@dataclass
class TypedFill:
    dst_axis: int
    stage: int
    type: ElementType
    bits: int


@dataclass
class TypedPlan:
    symbols: List[str]
    source: TensorDesc
    result: TensorDesc
    layout: Plan
    stages: List[ValueStage]
    fills: List[TypedFill]


# ---------------------------------------------------------------------------
# Decoder (libreloc/src/Decode.cpp)
# ---------------------------------------------------------------------------

CTX_PLAN, CTX_INVERSE, CTX_CHANNEL = range(3)


class _Reader:
    """Little-endian bounds-checked reader (Decode.cpp:17-108)."""

    def __init__(self, data: bytes):
        self.data = bytes(data)
        self.off = 0

    def remaining(self) -> int:
        return len(self.data) - self.off

    def fail(self, at: int, msg: str):
        raise DecodeError(at, msg)

    def u8(self) -> int:
        if self.remaining() < 1:
            self.fail(self.off, "truncated: expected u8")
        v = self.data[self.off]
        self.off += 1
        return v

    def u32(self) -> int:
        if self.remaining() < 4:
            self.fail(self.off, "truncated: expected u32")
        v = struct.unpack_from("<I", self.data, self.off)[0]
        self.off += 4
        return v

    def u64(self) -> int:
        if self.remaining() < 8:
            self.fail(self.off, "truncated: expected u64")
        v = struct.unpack_from("<Q", self.data, self.off)[0]
        self.off += 8
        return v

    def i64(self) -> int:
        if self.remaining() < 8:
            self.fail(self.off, "truncated: expected u64")
        v = struct.unpack_from("<q", self.data, self.off)[0]
        self.off += 8
        return v

    def count(self, what: str) -> int:
        at = self.off
        v = self.u32()
        if v > self.remaining():
            self.fail(at, "count exceeds remaining bytes: " + what)
        return v

    def string(self) -> str:
        n = self.count("string length")
        s = self.data[self.off:self.off + n].decode("utf-8", errors="surrogateescape")
        self.off += n
        return s


def _parse_expr(r: _Reader, ctx: int, nsym: int, ndim: int) -> list:
    """Decode.cpp:115-189."""
    start = r.off
    n = r.count("expression op_count")
    if n == 0:
        r.fail(start, "empty expression stream")
    out = []
    depth = 0
    for _ in range(n):
        at = r.off
        op = r.u8()
        if op == OP_PUSH_SYM:
            if ctx == CTX_INVERSE:
                r.fail(at, "PUSH_SYM is not allowed in inverse expressions")
            idx = r.u32()
            if idx >= nsym:
                r.fail(at, "PUSH_SYM symbol index out of range")
            out.append((op, idx))
            depth += 1
        elif op == OP_PUSH_CONST:
            out.append((op, r.i64()))
            depth += 1
        elif op == OP_PUSH_DIM:
            if ctx == CTX_PLAN:
                r.fail(at, "PUSH_DIM is only allowed in inverse and channel expressions")
            idx = r.u32()
            if idx >= ndim:
                r.fail(at, "PUSH_DIM dim index out of range")
            out.append((op, idx))
            depth += 1
        elif op in (OP_ADD, OP_SUB, OP_MUL, OP_FLOORDIV, OP_MOD):
            if depth < 2:
                r.fail(at, "expression stack underflow")
            depth -= 1
            out.append((op, 0))
        else:
            r.fail(at, "unknown expression opcode")
    if depth != 1:
        r.fail(start, "expression stream must leave exactly one value")
    return out


def _parse_type(r: _Reader) -> ElementType:
    """Decode.cpp:191-218."""
    at = r.off
    kind = r.u8()
    bw = r.u32()
    ok = ((kind == 0 and bw in (16, 32, 64)) or (kind == 1 and bw == 16)
          or (kind == 2 and 1 <= bw <= 64) or (kind == 3 and bw == 64))
    if not ok:
        r.fail(at, "invalid element type kind/bitwidth")
    return ElementType(kind, bw)


def _parse_desc(r: _Reader, nsym: int) -> TensorDesc:
    """Decode.cpp:220-248."""
    rank = r.count("tensor_desc rank")
    extents = [_parse_expr(r, CTX_PLAN, nsym, 0) for _ in range(rank)]
    at = r.off
    sc = r.count("tensor_desc stride_count")
    if sc != 0 and sc != rank:
        r.fail(at, "tensor_desc stride_count must be 0 or the rank")
    strides = [_parse_expr(r, CTX_PLAN, nsym, 0) for _ in range(sc)]
    offset = _parse_expr(r, CTX_PLAN, nsym, 0)
    et = _parse_type(r)
    return TensorDesc(extents, strides, offset, et)


def _parse_layout_body(r: _Reader, symbols: List[str]) -> Plan:
    """Decode.cpp:253-430 (sections 3..12)."""
    nsym = len(symbols)
    src = _parse_desc(r, nsym)
    dst_at = r.off
    dst = _parse_desc(r, nsym)
    perm_at = r.off
    pc = r.count("perm count")
    perm = [r.u32() for _ in range(pc)]
    axes_at = r.off
    ac = r.count("axes count")
    if ac < 1:
        r.fail(axes_at, "axis count must be >= 1")
    axes = []
    for _ in range(ac):
        name = r.string()
        e = _parse_expr(r, CTX_PLAN, nsym, 0)
        s = _parse_expr(r, CTX_PLAN, nsym, 0)
        d = _parse_expr(r, CTX_PLAN, nsym, 0)
        axes.append(Axis(name, e, s, d))
    if len(perm) != len(axes):
        r.fail(perm_at, "perm size must equal the axis count")
    seen = [False] * len(axes)
    for v in perm:
        if v >= len(axes) or seen[v]:
            r.fail(perm_at, "perm is not a permutation of [0, axis count)")
        seen[v] = True
    if len(dst.extents) != len(axes):
        r.fail(dst_at, "dst rank must equal the axis count")
    pads = []
    for _ in range(r.count("pad_fill count")):
        at = r.off
        ax = r.u32()
        if ax >= len(axes):
            r.fail(at, "pad_fill dst_axis out of range")
        lo = _parse_expr(r, CTX_PLAN, nsym, 0)
        hi = _parse_expr(r, CTX_PLAN, nsym, 0)
        ft = _parse_type(r)
        fb = r.u64()
        pads.append(PadFill(ax, lo, hi, ft, fb))
    divs = []
    for _ in range(r.count("divisibility count")):
        e = _parse_expr(r, CTX_PLAN, nsym, 0)
        divs.append((e, r.i64()))
    aligns = []
    for _ in range(r.count("alignment count")):
        at = r.off
        ax = r.u32()
        if ax >= len(axes):
            r.fail(at, "alignment axis out of range")
        aligns.append((ax, r.i64()))
    cat = r.off
    cc = r.count("contiguity count")
    if cc != 0 and cc != len(axes):
        r.fail(cat, "contiguity count must be 0 or the axis count")
    contig = []
    for _ in range(cc):
        at = r.off
        f = r.u8()
        if f > 1:
            r.fail(at, "contiguity flag must be 0 or 1")
        contig.append(f)
    at = r.off
    no_copy = r.u8()
    if no_copy > 1:
        r.fail(at, "no_copy flag must be 0 or 1")
    at = r.off
    rpc = r.u8()
    if rpc > 1:
        r.fail(at, "runtime_pad_check flag must be 0 or 1")
    nd_at = r.off
    nd = r.u32()
    nr_at = r.off
    nr = r.u32()
    if nd != len(axes):
        r.fail(nd_at, "inverse num_dims must equal the axis count")
    if nr != len(axes):
        r.fail(nr_at, "inverse num_results must equal the axis count")
    inverse = [_parse_expr(r, CTX_INVERSE, nsym, nd) for _ in range(nr)]
    return Plan(list(symbols), src, dst, perm, axes, pads, divs, aligns, contig,
                bool(no_copy), bool(rpc), inverse)


def _parse_header(r: _Reader, expected: int) -> List[str]:
    """Decode.cpp:433-458."""
    if r.remaining() < 4:
        r.fail(r.off, "truncated: expected magic")
    if r.data[:4] != b"RPLN":
        r.fail(0, "bad magic (expected RPLN)")
    r.off = 4
    at = r.off
    v = r.u32()
    if v != expected:
        r.fail(at, "unsupported wire format version")
    n = r.count("symbol table count")
    return [r.string() for _ in range(n)]


def peek_wire_version(data: bytes) -> Optional[int]:
    """Decode.cpp:868-874."""
    if len(data) < 8 or data[:4] != b"RPLN":
        return None
    return struct.unpack_from("<I", data, 4)[0]


def decode_plan(data: bytes) -> Plan:
    """decodePlan, Decode.cpp:876-888."""
    r = _Reader(data)
    symbols = _parse_header(r, 0)
    plan = _parse_layout_body(r, symbols)
    if r.remaining():
        r.fail(r.off, "trailing bytes after inverse section")
    return plan


def _parse_param(r: _Reader, nsym: int) -> StageParam:
    """Decode.cpp:478-535."""
    at = r.off
    kind = r.u8()
    if kind > 2:
        r.fail(at, "invalid parameter kind")
    p = StageParam(kind=kind)
    if kind == PARAM_NONE:
        return p
    if kind == PARAM_INLINE:
        rat = r.off
        rank = r.u8()
        if rank > 1:
            r.fail(rat, "parameter rank must be 0 or 1")
        p.rank = rank
        p.element_type = _parse_type(r)
        cat = r.off
        cnt = r.count("inline parameter count")
        if cnt == 0:
            r.fail(cat, "inline parameter must hold a value")
        if rank == 0 and cnt != 1:
            r.fail(cat, "rank-0 inline parameter must hold exactly one value")
        if cnt > r.remaining() // 8:
            r.fail(cat, "count exceeds remaining bytes: inline parameter")
        p.inline_bits = [r.u64() for _ in range(cnt)]
        return p
    nat = r.off
    p.binding_name = r.string()
    if not p.binding_name:
        r.fail(nat, "binding name must not be empty")
    rat = r.off
    rank = r.u8()
    if rank > 1:
        r.fail(rat, "parameter rank must be 0 or 1")
    p.rank = rank
    p.binding_extents = [_parse_expr(r, CTX_PLAN, nsym, 0) for _ in range(rank)]
    p.element_type = _parse_type(r)
    return p


def _parse_stage(r: _Reader, nsym: int, result_rank: int) -> ValueStage:
    """Decode.cpp:537-590."""
    at = r.off
    tr = r.u8()
    if tr > 2:
        r.fail(at, "unknown stage transform")
    pat = r.off
    pol = r.u8()
    if pol > 3:
        r.fail(pat, "unknown numerical policy")

    def stage_type():
        t = _parse_type(r)
        sat = r.off
        s = r.u8()
        if s > 2:
            r.fail(sat, "invalid stage type signedness")
        return StageType(t, s)

    inp = stage_type()
    out = stage_type()
    rat = r.off
    rank = r.count("stage shape rank")
    if rank == 0:
        r.fail(rat, "stage shape must have rank >= 1")
    shape = [_parse_expr(r, CTX_PLAN, nsym, 0) for _ in range(rank)]
    scale = _parse_param(r, nsym)
    zp = _parse_param(r, nsym)
    axis = r.i64()
    cat = r.off
    hc = r.u8()
    if hc > 1:
        r.fail(cat, "has_channel flag must be 0 or 1")
    channel: list = []
    if hc:
        dat = r.off
        nd = r.u32()
        if nd != result_rank:
            r.fail(dat, "channel map num_dims must equal the result rank")
        channel = _parse_expr(r, CTX_CHANNEL, nsym, nd)
    return ValueStage(tr, pol, inp, out, shape, scale, zp, axis, bool(hc), channel)


def _const_of(stream: list) -> Optional[int]:
    if len(stream) == 1 and stream[0][0] == OP_PUSH_CONST:
        return stream[0][1]
    return None


def _sign_extend(bits: int, bw: int) -> int:
    if bw >= 64:
        bits &= (1 << 64) - 1
        return bits - (1 << 64) if bits >> 63 else bits
    mask = (1 << bw) - 1
    v = bits & mask
    if v & (1 << (bw - 1)):
        v -= 1 << bw
    return v


def _is_nan_bits(bits: int, t: ElementType) -> bool:
    """Decode.cpp:614-624."""
    if t.kind == KIND_BFLOAT and t.bitwidth == 16:
        return ((bits >> 7) & 0xff) == 0xff and (bits & 0x7f) != 0
    if t.kind != KIND_FLOAT:
        return False
    if t.bitwidth == 32:
        return ((bits >> 23) & 0xff) == 0xff and (bits & 0x7fffff) != 0
    if t.bitwidth == 16:
        return ((bits >> 10) & 0x1f) == 0x1f and (bits & 0x3ff) != 0
    return False


def _isf(t: ElementType, w: int) -> bool:
    return t.kind == KIND_FLOAT and t.bitwidth == w


def _isbf16(t: ElementType) -> bool:
    return t.kind == KIND_BFLOAT and t.bitwidth == 16


def _isi8(t: ElementType) -> bool:
    return t.kind == KIND_INT and t.bitwidth == 8


def _validate_typed(r: _Reader, p: TypedPlan, layout_at, stages_at, stage_at, fills_at, fill_at):
    """validateTyped, Decode.cpp:628-866."""
    st, rt = p.source.element_type, p.result.element_type
    if not p.layout.src.element_type.same(st):
        r.fail(layout_at, "layout src element type must equal the source type")
    if not p.layout.dst.element_type.same(rt):
        r.fail(layout_at, "layout dst element type must equal the result type")
    if len(p.layout.src.extents) != len(p.source.extents):
        r.fail(layout_at, "layout src rank must equal the source rank")
    if not p.stages:
        r.fail(stages_at, "typed plan needs at least one stage")
    if not p.stages[0].input.type.same(st):
        r.fail(stage_at[0], "stage 0 input type must equal the source type")
    for k in range(1, len(p.stages)):
        if not p.stages[k].input.type.same(p.stages[k - 1].output.type):
            r.fail(stage_at[k], "stage input type must equal the previous stage's output type")
    if not p.stages[-1].output.type.same(rt):
        r.fail(stage_at[-1], "last stage output type must equal the result type")
    declared: List[StageParam] = []
    for k, s in enumerate(p.stages):
        at = stage_at[k]
        signless = s.input.signedness == 0 and s.output.signedness == 0
        if s.transform == T_CAST:
            half16 = _isf(s.output.type, 16) or _isbf16(s.output.type)
            from16 = _isf(s.input.type, 16) or _isbf16(s.input.type)
            narrow = _isf(s.input.type, 32) and half16 and s.policy == P_IEEE_RNE
            widen = from16 and _isf(s.output.type, 32) and s.policy == P_EXACT
            if not (narrow or widen) or not signless:
                r.fail(at, "invalid cast signature (f32 -> f16/bf16 ieee_rne or f16/bf16 -> f32 exact, signless)")
            if (s.scale.kind != PARAM_NONE or s.zero_point.kind != PARAM_NONE or s.axis != -1
                    or s.has_channel):
                r.fail(at, "cast stages carry no parameters")
            continue
        if s.transform == T_QUANTIZE:
            if not (_isf(s.input.type, 32) and s.input.signedness == 0 and _isi8(s.output.type)
                    and s.output.signedness == 1 and s.policy == P_SYMMETRIC_RNE):
                r.fail(at, "invalid quantize signature (f32 -> signed int 8, symmetric_rne)")
        else:
            if not (_isi8(s.input.type) and s.input.signedness == 1 and _isf(s.output.type, 32)
                    and s.output.signedness == 0 and s.policy == P_AFFINE):
                r.fail(at, "invalid dequantize signature (signed int 8 -> f32, affine)")
        if s.scale.kind == PARAM_NONE:
            r.fail(at, "quantize/dequantize stages require a scale")
        if not _isf(s.scale.element_type, 32):
            r.fail(at, "scale element type must be f32")
        if s.zero_point.kind != PARAM_NONE:
            if s.zero_point.element_type.kind != KIND_INT:
                r.fail(at, "zero_point element type must be an integer")
            if s.zero_point.kind == PARAM_BINDING and s.zero_point.element_type.bitwidth != 32:
                r.fail(at, "zero_point bindings must declare int 32")
        if s.axis == -1:
            if s.scale.rank != 0 or (s.zero_point.kind != PARAM_NONE and s.zero_point.rank != 0) \
                    or s.has_channel:
                r.fail(at, "per-tensor stage requires rank-0 parameters and no channel map")
        else:
            if s.axis < 0 or s.axis >= len(s.shape):
                r.fail(at, "axis out of range for the stage shape")
            if s.scale.rank != 1:
                r.fail(at, "per-channel stage requires a rank-1 scale")
            if not s.has_channel:
                r.fail(at, "per-channel stage requires a channel map")
            ext = _const_of(s.shape[s.axis])
            for prm in (s.scale, s.zero_point):
                if prm.kind == PARAM_INLINE and prm.rank == 1 and ext is not None \
                        and len(prm.inline_bits) != ext:
                    r.fail(at, "inline parameter length must equal the channel extent")
        if s.scale.kind == PARAM_INLINE:
            for b in s.scale.inline_bits:
                v = float(np.uint32(b & 0xffffffff).view(np.float32))
                if not np.isfinite(v) or not v > 0.0:
                    r.fail(at, "inline scale must be finite and strictly positive")
        if s.zero_point.kind == PARAM_INLINE:
            for b in s.zero_point.inline_bits:
                v = _sign_extend(b, s.zero_point.element_type.bitwidth)
                if v < -128 or v > 127:
                    r.fail(at, "inline zero point out of [-128, 127]")
                if s.policy == P_SYMMETRIC_RNE and v != 0:
                    r.fail(at, "symmetric_rne admits only the constant zero point 0")
        if s.policy == P_SYMMETRIC_RNE and s.zero_point.kind == PARAM_BINDING:
            r.fail(at, "symmetric_rne rejects a zero-point binding")
        if (s.scale.kind == PARAM_BINDING and s.zero_point.kind == PARAM_BINDING
                and s.scale.binding_name == s.zero_point.binding_name):
            r.fail(at, "runtime parameters must use distinct binding names")
        for prm in (s.scale, s.zero_point):
            if prm.kind != PARAM_BINDING:
                continue
            for seen in declared:
                if seen.binding_name != prm.binding_name:
                    continue
                same = (seen.rank == prm.rank and seen.element_type.same(prm.element_type)
                        and seen.binding_extents == prm.binding_extents)
                if not same:
                    r.fail(at, "conflicting parameter declaration for binding '%s'" % prm.binding_name)
            declared.append(prm)
    has_fill = [False] * len(p.layout.pad_fill)
    for i, f in enumerate(p.fills):
        at = fill_at[i]
        pad = None
        for j, pf in enumerate(p.layout.pad_fill):
            if pf.dst_axis == f.dst_axis:
                if has_fill[j]:
                    r.fail(at, "duplicate fill for a layout pad")
                has_fill[j] = True
                pad = pf
        if pad is None:
            r.fail(at, "fill dst_axis has no layout pad")
        if f.stage > len(p.stages):
            r.fail(at, "fill stage out of range")
        entry = st if f.stage == 0 else p.stages[f.stage - 1].output.type
        if not f.type.same(entry):
            r.fail(at, "fill type must equal the type entering its stage")
        if not pad.fill_type.same(rt):
            r.fail(at, "layout pad fill type must equal the result type")
        bits, t = f.bits, f.type
        for k in range(f.stage, len(p.stages)):
            folded = fold_fill(bits, t, p.stages[k])
            if folded is None:
                r.fail(at, "fill cannot fold through a per-channel or runtime-parameter stage")
            bits, t = folded, p.stages[k].output.type
        both_nan = _is_nan_bits(bits, rt) and _is_nan_bits(pad.fill_bits, rt)
        if bits != pad.fill_bits and not both_nan:
            r.fail(at, "fill fold mismatch with the layout's fused fill")
    for j, h in enumerate(has_fill):
        if not h:
            r.fail(fills_at, "layout pad without a typed fill")


def decode_typed_plan(data: bytes) -> TypedPlan:
    """decodeTypedPlan, Decode.cpp:890-948."""
    r = _Reader(data)
    symbols = _parse_header(r, 1)
    nsym = len(symbols)
    source = _parse_desc(r, nsym)
    result = _parse_desc(r, nsym)
    layout_at = r.off
    layout = _parse_layout_body(r, symbols)
    stages_at = r.off
    sc = r.count("stage count")
    stage_at, stages = [], []
    for _ in range(sc):
        stage_at.append(r.off)
        stages.append(_parse_stage(r, nsym, len(result.extents)))
    fills_at = r.off
    fc = r.count("fill count")
    fill_at, fills = [], []
    for _ in range(fc):
        fill_at.append(r.off)
        da = r.u32()
        stg = r.u32()
        t = _parse_type(r)
        b = r.u64()
        fills.append(TypedFill(da, stg, t, b))
    if r.remaining():
        r.fail(r.off, "trailing bytes after fills section")
    p = TypedPlan(symbols, source, result, layout, stages, fills)
    _validate_typed(r, p, layout_at, stages_at, stage_at, fills_at, fill_at)
    return p


# ---------------------------------------------------------------------------
# Stage arithmetic: scalar forms (Quant.cpp) and vectorized numpy forms
# ---------------------------------------------------------------------------

def f32_bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def bits_f32(b: int) -> float:
    return struct.unpack("<f", struct.pack("<I", b & 0xffffffff))[0]


def narrow_f32_f16_bits(x: np.ndarray) -> np.ndarray:
    """f32ToF16Scalar, libreloc/quant/Quant.cpp:107-133, over uint32 bit arrays."""
    x = np.asarray(x, dtype=np.uint32)
    sign = ((x >> 16) & 0x8000).astype(np.uint32)
    a = x & np.uint32(0x7fffffff)
    out = np.zeros(a.shape, dtype=np.uint32)
    nan = a > 0x7f800000
    inf = (~nan) & (a >= 0x477ff000)
    norm = (~nan) & (~inf) & (a >= 0x38800000)
    zero = (~nan) & (~inf) & (~norm) & (a <= 0x33000000)
    sub = ~(nan | inf | norm | zero)
    out[nan] = 0x7e00 | ((a[nan] >> 13) & 0x3ff)
    out[inf] = 0x7c00
    an = a[norm]
    r = an + np.uint32(0xfff) + ((an >> 13) & 1)
    out[norm] = (r - np.uint32(0x38000000)) >> 13
    asub = a[sub]
    shift = np.uint32(126) - (asub >> 23)
    mant = (asub & 0x7fffff) | 0x800000
    rr = mant >> shift
    rem = mant & ((np.uint32(1) << shift) - 1)
    half = np.uint32(1) << (shift - 1)
    rr = rr + ((rem > half) | ((rem == half) & ((rr & 1) == 1))).astype(np.uint32)
    out[sub] = rr
    return (out | sign).astype(np.uint16)


def widen_f16_f32_bits(h: np.ndarray) -> np.ndarray:
    """widenF16F32, Quant.cpp:183-214, over uint16 bit arrays (exact)."""
    h = np.asarray(h, dtype=np.uint16).astype(np.uint32)
    sign = (h & 0x8000) << 16
    e = (h >> 10) & 0x1f
    m = h & 0x3ff
    out = np.zeros(h.shape, dtype=np.uint32)
    normal = (e != 0) & (e != 31)
    out[normal] = ((e[normal] + 112) << 23) | (m[normal] << 13)
    special = e == 31
    out[special] = 0x7f800000 | (m[special] << 13)
    sub = (e == 0) & (m != 0)
    ms = m[sub]
    # renormalize: count shifts until bit 10 is set
    shifts = np.zeros(ms.shape, dtype=np.uint32)
    mm = ms.copy()
    for _ in range(10):
        need = (mm & 0x400) == 0
        mm = np.where(need, mm << 1, mm)
        shifts = shifts + need.astype(np.uint32)
    out[sub] = ((np.uint32(127 - 14) - shifts) << 23) | ((mm & 0x3ff) << 13)
    return (out | sign).astype(np.uint32)


def narrow_f32_bf16_bits(x: np.ndarray) -> np.ndarray:
    """narrowF32BF16, Quant.cpp:164-174."""
    x = np.asarray(x, dtype=np.uint32)
    nan = (x & 0x7fffffff) > 0x7f800000
    lsb = (x >> 16) & 1
    rne = ((x.astype(np.uint64) + 0x7fff + lsb) >> 16).astype(np.uint32)
    out = np.where(nan, (x >> 16) | 0x0040, rne)
    return (out & 0xffff).astype(np.uint16)


def widen_bf16_f32_bits(b: np.ndarray) -> np.ndarray:
    """widenBF16F32, Quant.cpp:176-181."""
    return np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16


def quantize_f32_s8(x: np.ndarray, inv: np.ndarray) -> np.ndarray:
    """quantOne, libreloc/quant/QuantKernels.h:23-28: fmax first so NaN -> -128,
    then fmin, nearbyint (ties to even). x, inv are float32 arrays (broadcast)."""
    y = np.multiply(np.asarray(x, np.float32), np.asarray(inv, np.float32), dtype=np.float32)
    y = np.fmax(y, np.float32(-128.0))
    y = np.fmin(y, np.float32(127.0))
    return np.rint(y).astype(np.int8)


def dequantize_s8_f32(q: np.ndarray, scale: np.ndarray, zp: np.ndarray) -> np.ndarray:
    """applyStage Dequantize, TypedExecute.cpp:489-496: d = q - zp exactly,
    then one binary32 multiply."""
    d = (np.asarray(q, np.int8).astype(np.int32) - np.asarray(zp, np.int32)).astype(np.float32)
    return np.multiply(d, np.asarray(scale, np.float32), dtype=np.float32)


def fold_fill(bits: int, t: ElementType, s: ValueStage) -> Optional[int]:
    """typed::foldFill, libreloc/src/TypedValue.cpp:74-120."""
    if not t.same(s.input.type):
        return None
    if s.transform == T_CAST:
        if _isf(t, 32) and _isf(s.output.type, 16):
            return int(narrow_f32_f16_bits(np.array([bits], np.uint32))[0])
        if _isf(t, 16) and _isf(s.output.type, 32):
            return int(widen_f16_f32_bits(np.array([bits], np.uint16))[0])
        if _isf(t, 32) and _isbf16(s.output.type):
            return int(narrow_f32_bf16_bits(np.array([bits], np.uint32))[0])
        if _isbf16(t) and _isf(s.output.type, 32):
            return int(widen_bf16_f32_bits(np.array([bits], np.uint16))[0])
        return None
    if s.transform == T_QUANTIZE:
        if (not _isf(t, 32) or not _isi8(s.output.type) or s.axis >= 0
                or s.scale.kind != PARAM_INLINE or s.scale.rank != 0 or not s.scale.inline_bits):
            return None
        inv = np.float32(1.0) / np.uint32(s.scale.inline_bits[0] & 0xffffffff).view(np.float32)
        x = np.uint32(bits & 0xffffffff).view(np.float32)
        q = quantize_f32_s8(np.array([x]), np.array([inv]))[0]
        return int(np.uint8(q.view(np.uint8)))
    if (not _isi8(t) or not _isf(s.output.type, 32) or s.axis >= 0
            or s.scale.kind != PARAM_INLINE or s.scale.rank != 0 or not s.scale.inline_bits):
        return None
    zp = 0
    if s.zero_point.kind == PARAM_INLINE:
        if s.zero_point.rank != 0 or not s.zero_point.inline_bits:
            return None
        zp = _sign_extend(s.zero_point.inline_bits[0], s.zero_point.element_type.bitwidth)
    elif s.zero_point.kind != PARAM_NONE:
        return None
    q = _sign_extend(bits, 8)
    scale = np.uint32(s.scale.inline_bits[0] & 0xffffffff).view(np.float32)
    y = np.float32(np.float32(q - zp) * scale)
    return int(np.float32(y).view(np.uint32))


# ---------------------------------------------------------------------------
# Expression evaluation and binding (libreloc/src/Bind.cpp)
# ---------------------------------------------------------------------------

def _floordiv(a: int, b: int) -> int:
    """Bind.cpp:19-29 (checked floor division)."""
    if b == 0:
        raise BindError("division by zero")
    if a == I64_MIN and b == -1:
        raise BindError("integer overflow in floordiv")
    return a // b  # Python // is floor division


def _chk(v: int, what: str) -> int:
    if v < I64_MIN or v > I64_MAX:
        raise BindError("integer overflow in " + what)
    return v


def eval_expr(stream: list, symbols: Sequence[int], dims: Optional[Sequence[int]] = None) -> int:
    """evalStream, Bind.cpp:84-161. `dims` is None in the plan context."""
    st: List[int] = []
    for op, v in stream:
        if op == OP_PUSH_SYM:
            if v < 0 or v >= len(symbols):
                raise BindError("symbol index out of range")
            st.append(symbols[v])
        elif op == OP_PUSH_CONST:
            st.append(v)
        elif op == OP_PUSH_DIM:
            if dims is None:
                raise BindError("PUSH_DIM is not valid in a plan expression")
            if v < 0 or v >= len(dims):
                raise BindError("dimension index out of range")
            st.append(dims[v])
        else:
            if len(st) < 2:
                raise BindError("expression stack underflow")
            b = st.pop()
            a = st.pop()
            if op == OP_ADD:
                r = _chk(a + b, "add")
            elif op == OP_SUB:
                r = _chk(a - b, "sub")
            elif op == OP_MUL:
                r = _chk(a * b, "mul")
            elif op == OP_FLOORDIV:
                r = _floordiv(a, b)
            else:
                q = _floordiv(a, b)
                r = _chk(a - _chk(q * b, "mod"), "mod")
            st.append(r)
    if len(st) != 1:
        raise BindError("expression did not evaluate to a single value")
    return st[0]


def eval_channel_vec(stream: list, symbols: Sequence[int], coords: Sequence[np.ndarray]) -> np.ndarray:
    """Vectorized evalChannel (Bind.cpp:168-172) over arrays of result
    coordinates. Overflow is impossible at the sizes the oracle runs."""
    st: List[np.ndarray] = []
    for op, v in stream:
        if op == OP_PUSH_SYM:
            st.append(np.int64(symbols[v]))
        elif op == OP_PUSH_CONST:
            st.append(np.int64(v))
        elif op == OP_PUSH_DIM:
            st.append(np.asarray(coords[v], np.int64))
        else:
            b = st.pop()
            a = st.pop()
            if op == OP_ADD:
                st.append(a + b)
            elif op == OP_SUB:
                st.append(a - b)
            elif op == OP_MUL:
                st.append(a * b)
            elif op in (OP_FLOORDIV, OP_MOD):
                if np.any(np.asarray(b) == 0):
                    raise ExecutionError("channel_evaluation_failed", "division by zero")
                st.append(np.floor_divide(a, b) if op == OP_FLOORDIV else np.mod(a, b))
    return np.asarray(st[0], np.int64)


def _resolve(symbols: List[str], sym_map: Dict[str, int]) -> List[int]:
    """resolveSymbols, Bind.cpp:37-51."""
    for k in sym_map:
        if k not in symbols:
            raise BindError("unknown symbol in binding: " + k)
    out = []
    for s in symbols:
        if s not in sym_map:
            raise BindError("unbound symbol: " + s)
        out.append(int(sym_map[s]))
    return out


@dataclass
class PadRegion:
    axis: int
    lo: int
    hi: int
    fill_bits: int


@dataclass
class BoundPlan:
    extents: List[int]
    src_strides: List[int]
    dst_strides: List[int]
    perm: List[int]
    pad_regions: List[PadRegion]
    element_size: int
    total_bytes: int
    no_copy: bool
    L: int
    required_alignments: List[Tuple[int, int]]
    typed: bool = False


def _mul_ok(a: int, b: int) -> Optional[int]:
    r = a * b
    return r if I64_MIN <= r <= I64_MAX else None


def bind(plan: Plan, sym_map: Dict[str, int]) -> BoundPlan:
    """bind, Bind.cpp:176-384 (strategy and cost model omitted: they choose a
    CPU executor, never the bytes)."""
    syms = _resolve(plan.symbols, sym_map)

    def ev(stream, what):
        try:
            return eval_expr(stream, syms)
        except BindError as e:
            raise BindError(f"{what}: {e}")

    for expr, divisor in plan.divisibility:
        if divisor <= 0:
            raise BindError("divisibility divisor must be positive")
        v = ev(expr, "divisibility expr")
        if v % divisor != 0:  # zero-ness agrees for floor and truncating remainders
            raise BindError(f"divisibility violated: value {v} not divisible by {divisor}")
    axes = []
    for a in plan.axes:
        e = ev(a.extent, "axis extent")
        s = ev(a.src_stride, "axis src_stride")
        d = ev(a.dst_stride, "axis dst_stride")
        if e < 1:
            raise BindError("axis extent must be >= 1 (v0 rejects zero/negative)")
        if s < 0 or d < 0:
            raise BindError("strides must be non-negative in v0")
        axes.append([e, s, d, False, 0, 0, 0])
    for pad in plan.pad_fill:
        lo = ev(pad.lo, "pad lo")
        hi = ev(pad.hi, "pad hi")
        if pad.dst_axis >= len(plan.axes):
            raise BindError("pad dst_axis out of range")
        ax = axes[pad.dst_axis]
        ax[3], ax[4], ax[5], ax[6] = True, lo, hi, pad.fill_bits
        if lo < 0 or hi < 0:
            raise BindError("pad width negative")
        if plan.runtime_pad_check:
            if pad.dst_axis >= len(plan.dst.extents):
                raise BindError("pad dst_axis out of range for dst extents")
            de = ev(plan.dst.extents[pad.dst_axis], "dst extent")
            if ax[0] + lo + hi != de:
                raise BindError(f"pad range inconsistent: extent + lo + hi ({ax[0] + lo + hi}) "
                                f"!= dst extent ({de})")
    absorbed = [1] * len(axes)
    changed = True
    while changed:
        changed = False
        for k in range(len(axes) - 1):
            o, i = axes[k], axes[k + 1]
            if o[3] or i[3]:
                continue
            sp, dp, ep = _mul_ok(i[1], i[0]), _mul_ok(i[2], i[0]), _mul_ok(o[0], i[0])
            if sp is None or dp is None or ep is None:
                continue
            if o[1] != sp or o[2] != dp:
                continue
            axes[k] = [ep, i[1], i[2], False, 0, 0, 0]
            del axes[k + 1]
            absorbed[k] += absorbed[k + 1]
            del absorbed[k + 1]
            changed = True
            break
    orig_to_c = []
    for c, n in enumerate(absorbed):
        orig_to_c += [c] * n
    bw = plan.dst.element_type.bitwidth
    if bw == 0 or bw % 8:
        raise BindError("element type bitwidth must be a positive multiple of 8 in v0")
    es = bw // 8
    aligns = []
    for ax, b in plan.alignment:
        if ax >= len(plan.axes):
            raise BindError("alignment axis out of range")
        aligns.append((orig_to_c[ax], b))
    total = 1
    pads = []
    for k, a in enumerate(axes):
        padded = a[0]
        if a[3]:
            pads.append(PadRegion(k, a[4], a[5], a[6]))
            padded += a[4] + a[5]
        total = _mul_ok(total, padded)
        if total is None:
            raise BindError("overflow computing total element count")
    tb = _mul_ok(total, es)
    if tb is None:
        raise BindError("overflow computing total bytes")
    inner = axes[-1]
    L = inner[0] if (inner[1] == 1 and inner[2] == 1) else 1
    return BoundPlan([a[0] for a in axes], [a[1] for a in axes], [a[2] for a in axes],
                     list(plan.perm), pads, es, tb, plan.no_copy, L, aligns)


@dataclass
class BoundParameter:
    present: bool = False
    element_type: Optional[ElementType] = None
    length: int = 0
    data: bytes = b""
    binding_name: str = ""


@dataclass
class BoundStage:
    transform: int
    policy: int
    input: StageType
    output: StageType
    shape: List[int]
    axis: int
    has_channel: bool
    channel: list
    scale: BoundParameter
    zero_point: BoundParameter


@dataclass
class Footprint:
    boundary: int
    element_type: ElementType
    elements: int
    bytes: int


@dataclass
class TypedBoundPlan:
    layout: BoundPlan
    source_extents: List[int]
    result_extents: List[int]
    source_type: ElementType
    result_type: ElementType
    symbols: List[int]
    stages: List[BoundStage]
    fills: List[TypedFill]
    cuts: List[Footprint]
    source_bytes: int
    destination_bytes: int
    parameter_bytes: int


def _dense_desc(desc: TensorDesc, syms: List[int], what: str) -> List[int]:
    """concreteDenseDescriptor, Bind.cpp:401-440."""
    def ev(s):
        try:
            return eval_expr(s, syms)
        except BindError as e:
            raise BindError(f"{what}: {e}")
    ext = [ev(e) for e in desc.extents]
    if not ext:
        raise BindError(f"{what}: rank must be >= 1")
    if any(e < 1 for e in ext):
        raise BindError(f"{what}: extents must be >= 1")
    if ev(desc.offset) != 0:
        raise BindError(f"{what}: only zero offsets are supported")
    if desc.strides:
        strides = [ev(s) for s in desc.strides]
        running = 1
        for k in range(len(ext) - 1, -1, -1):
            if strides[k] != running:
                raise BindError(f"{what}: only dense row-major strides are supported")
            running = _mul_ok(running, ext[k])
            if running is None:
                raise BindError(f"{what}: stride product overflows")
    return ext


def _param_values_ok(p: BoundParameter, is_scale: bool, policy: int):
    """checkParameterValues, Bind.cpp:453-476."""
    w = p.element_type.width
    for i in range(p.length):
        el = p.data[i * w:(i + 1) * w]
        if is_scale:
            v = np.frombuffer(el, np.float32)[0]
            if not np.isfinite(v) or not v > 0.0:
                raise BindError("scale: scale must be finite and strictly positive")
            continue
        zp = _sign_extend(int.from_bytes(el, "little"), p.element_type.bitwidth)
        if zp < -128 or zp > 127:
            raise BindError("zero_point: zero point must lie in [-128, 127]")
        if policy == P_SYMMETRIC_RNE and zp != 0:
            raise BindError("zero_point: symmetric_rne admits only the zero point 0")


ParameterMap = Dict[str, Tuple[ElementType, List[int], bytes]]


def bind_typed(plan: TypedPlan, sym_map: Dict[str, int], params: ParameterMap) -> TypedBoundPlan:
    """bindTyped, Bind.cpp:494-699."""
    try:
        layout = bind(plan.layout, sym_map)
    except BindError as e:
        raise BindError("layout: " + str(e))
    layout.typed = True
    syms = _resolve(plan.layout.symbols, sym_map)
    src_ext = _dense_desc(plan.source, syms, "source")
    res_ext = _dense_desc(plan.result, syms, "result")
    st, rt = plan.source.element_type, plan.result.element_type
    if st.width == 0 or rt.width == 0:
        raise BindError("element type bitwidth must be a positive multiple of 8")
    used = set()
    stages = []
    param_bytes = 0
    for s in plan.stages:
        shape = []
        for e in s.shape:
            try:
                shape.append(eval_expr(e, syms))
            except BindError as err:
                raise BindError("stage shape: " + str(err))
        if any(e < 1 for e in shape):
            raise BindError("stage shape extents must be >= 1")
        if s.axis >= 0 and s.axis >= len(shape):
            raise BindError("stage channel axis out of range")
        bs = BoundStage(s.transform, s.policy, s.input, s.output, shape, s.axis, s.has_channel,
                        s.channel, BoundParameter(), BoundParameter())
        for declared, is_scale in ((s.scale, True), (s.zero_point, False)):
            if declared.kind == PARAM_NONE:
                continue
            expected = 1 if declared.rank == 0 else shape[s.axis]
            w = declared.element_type.width
            if w == 0:
                raise BindError("parameter element type bitwidth must be a positive multiple of 8")
            if declared.kind == PARAM_INLINE:
                data = b"".join(int(b & ((1 << 64) - 1)).to_bytes(8, "little")[:w]
                                for b in declared.inline_bits)
                tgt = BoundParameter(True, declared.element_type, len(declared.inline_bits), data)
                if tgt.length != expected:
                    raise BindError(f"inline parameter holds {tgt.length} values but the channel "
                                    f"extent is {expected}")
            else:
                name = declared.binding_name
                if name not in params:
                    raise BindError("unbound parameter: " + name)
                used.add(name)
                vt, vext, vbytes = params[name]
                if not vt.same(declared.element_type):
                    raise BindError(f"parameter '{name}' element type differs from its declaration")
                if len(vext) != declared.rank:
                    raise BindError(f"parameter '{name}' rank differs from its declaration")
                dl = 1
                if declared.rank == 1:
                    try:
                        dl = eval_expr(declared.binding_extents[0], syms)
                    except BindError as err:
                        raise BindError("parameter extent: " + str(err))
                if dl != expected:
                    raise BindError(f"parameter '{name}' declares length {dl} but the channel "
                                    f"extent is {expected}")
                vl = 1 if declared.rank == 0 else vext[0]
                if vl != expected:
                    raise BindError(f"parameter '{name}' has length {vl} but the channel extent "
                                    f"is {expected}")
                if len(vbytes) != expected * w:
                    raise BindError(f"parameter '{name}' has {len(vbytes)} bytes, expected "
                                    f"{expected * w}")
                tgt = BoundParameter(True, declared.element_type, expected, bytes(vbytes), name)
            _param_values_ok(tgt, is_scale, s.policy)
            param_bytes += len(tgt.data)
            if is_scale:
                bs.scale = tgt
            else:
                bs.zero_point = tgt
        stages.append(bs)
    for k in params:
        if k not in used:
            raise BindError("unknown parameter in binding: " + k)
    src_elems = int(np.prod(src_ext, dtype=object))
    src_bytes = src_elems * st.width
    ax_ext = [eval_expr(a.extent, syms) for a in plan.layout.axes]
    pad_w = [0] * len(ax_ext)
    pad_stage = [0] * len(ax_ext)
    for pad in plan.layout.pad_fill:
        lo, hi = eval_expr(pad.lo, syms), eval_expr(pad.hi, syms)
        if lo < 0 or hi < 0:
            raise BindError("pad widths must be non-negative")
        pad_w[pad.dst_axis] = lo + hi
        for f in plan.fills:
            if f.dst_axis == pad.dst_axis:
                pad_stage[pad.dst_axis] = f.stage
    cuts = []
    for b in range(len(plan.stages) + 1):
        et = st if b == 0 else plan.stages[b - 1].output.type
        n = 1
        for a, e in enumerate(ax_ext):
            if pad_w[a] and pad_stage[a] <= b:
                e += pad_w[a]
            n *= e
        if et.width == 0:
            raise BindError("stage element type bitwidth must be a positive multiple of 8")
        cuts.append(Footprint(b, et, n, n * et.width))
    dest_bytes = cuts[-1].bytes
    if dest_bytes != layout.total_bytes:
        raise BindError(f"layout footprint ({layout.total_bytes} bytes) disagrees with the result "
                        f"descriptor ({dest_bytes} bytes)")
    if int(np.prod(res_ext, dtype=object)) != cuts[-1].elements:
        raise BindError("result descriptor element count disagrees with the layout")
    return TypedBoundPlan(layout, src_ext, res_ext, st, rt, syms, stages, list(plan.fills), cuts,
                          src_bytes, dest_bytes, param_bytes)


# ---------------------------------------------------------------------------
# Program preparation and host execution (libreloc/src/TypedExecute.cpp)
# ---------------------------------------------------------------------------

@dataclass
class StageArith:
    transform: int
    policy: int
    input: ElementType
    output: ElementType
    scale: np.ndarray
    inv_scale: np.ndarray
    zero_point: np.ndarray
    per_channel: bool
    channel_is_dim: bool
    channel_dim: int
    channel_length: int
    channel: list


@dataclass
class Program:
    plan: TypedBoundPlan
    stages: List[StageArith]
    result_strides: List[int]
    source_elements: int
    result_elements: int


def prepare_program(plan: TypedBoundPlan) -> Program:
    """prepareProgram, TypedExecute.cpp:292-403."""
    rank = len(plan.result_extents)
    rs = [1] * rank
    for j in range(rank - 1, 0, -1):
        rs[j - 1] = rs[j] * plan.result_extents[j]
    out = []
    for k, b in enumerate(plan.stages):
        where = f"stage {k}: "
        it, ot = b.input.type, b.output.type
        scale = np.zeros(0, np.float32)
        inv = np.zeros(0, np.float32)
        zp = np.zeros(1, np.int32)
        if b.transform == T_CAST:
            narrow = _isf(it, 32) and (_isf(ot, 16) or _isbf16(ot)) and b.policy == P_IEEE_RNE
            widen = (_isf(it, 16) or _isbf16(it)) and _isf(ot, 32) and b.policy == P_EXACT
            if not (narrow or widen):
                raise ExecutionError("unsupported_stage", where + "only cast f32->f16/bf16 ieee_rne "
                                     "and f16/bf16->f32 exact have a reference implementation")
        else:
            if b.transform == T_QUANTIZE and not (_isf(it, 32) and _isi8(ot)
                                                  and b.policy == P_SYMMETRIC_RNE):
                raise ExecutionError("unsupported_stage", where + "only quantize f32->s8")
            if b.transform == T_DEQUANTIZE and not (_isi8(it) and _isf(ot, 32)
                                                    and b.policy == P_AFFINE):
                raise ExecutionError("unsupported_stage", where + "only dequantize s8->f32")
            if not b.scale.present:
                raise ExecutionError("invalid_parameter", where + "scale is absent")
            scale = np.frombuffer(b.scale.data, np.float32).copy()
            if not np.all(np.isfinite(scale)) or np.any(scale <= 0):
                raise ExecutionError("invalid_parameter",
                                     where + "scale is not finite and strictly positive")
            if b.zero_point.present:
                w = b.zero_point.element_type.width
                zp = np.array([_sign_extend(int.from_bytes(b.zero_point.data[i * w:(i + 1) * w],
                                                           "little"),
                                            b.zero_point.element_type.bitwidth)
                               for i in range(b.zero_point.length)], np.int32)
            if b.transform == T_QUANTIZE:
                if np.any(zp != 0):
                    raise ExecutionError("invalid_parameter",
                                         where + "symmetric_rne admits only zero point 0")
                inv = (np.float32(1.0) / scale).astype(np.float32)  # fl32(1/scale), once
        ch_is_dim, ch_dim, ch_len = False, 0, 1
        if b.has_channel:
            if scale.size == 0:
                raise ExecutionError("invalid_parameter", where + "per-channel stage without scales")
            ch_len = scale.size
            if zp.size > 1 and zp.size != scale.size:
                raise ExecutionError("invalid_parameter",
                                     where + "zero point length disagrees with the scale")
            c = b.channel
            if c and c[0][0] == OP_PUSH_DIM and 0 <= c[0][1] < rank:
                ch_dim = c[0][1]
                ch_is_dim = len(c) == 1
                if len(c) == 3 and c[2][0] == OP_MOD and c[1][0] in (OP_PUSH_CONST, OP_PUSH_SYM):
                    try:
                        mod = eval_expr([c[1]], plan.symbols)
                    except BindError:
                        mod = 0
                    if mod > 0 and plan.result_extents[ch_dim] <= mod:
                        ch_is_dim = True
        else:
            if scale.size > 1 or zp.size > 1:
                raise ExecutionError("invalid_parameter",
                                     where + "per-tensor stage with more than one parameter")
        out.append(StageArith(b.transform, b.policy, it, ot, scale, inv, zp, b.has_channel,
                              ch_is_dim, ch_dim, ch_len, b.channel))
    return Program(plan, out, rs, int(np.prod(plan.source_extents, dtype=object)),
                   int(np.prod(plan.result_extents, dtype=object)))


def type_at(p: Program, boundary: int) -> ElementType:
    return p.plan.source_type if boundary == 0 else p.stages[boundary - 1].output


_NP_BITS = {1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}


def apply_stage(s: StageArith, bits: np.ndarray, channel: Optional[np.ndarray]) -> np.ndarray:
    """applyStage, TypedExecute.cpp:472-499, vectorized. `bits` holds the
    input bit patterns in their natural unsigned width; `channel` the
    per-element parameter index (None for per-tensor stages)."""
    c = channel if s.per_channel else 0
    if s.transform == T_CAST:
        if _isf(s.input, 32):
            if _isbf16(s.output):
                return narrow_f32_bf16_bits(bits)
            return narrow_f32_f16_bits(bits)
        if _isbf16(s.input):
            return widen_bf16_f32_bits(bits)
        return widen_f16_f32_bits(bits)
    if s.transform == T_QUANTIZE:
        x = np.asarray(bits, np.uint32).view(np.float32)
        inv = s.inv_scale[c] if s.per_channel else s.inv_scale[0]
        return quantize_f32_s8(x, inv).view(np.uint8)
    q = np.asarray(bits, np.uint8).view(np.int8)
    scale = s.scale[c] if s.per_channel else s.scale[0]
    zp = s.zero_point[0] if s.zero_point.size == 1 else s.zero_point[c]
    return dequantize_s8_f32(q, scale, zp).view(np.uint32)


def pads_settled_by(p: Program, boundary: int) -> bool:
    return all(f.stage <= boundary for f in p.plan.fills)


def fill_at(p: Program, boundary: int) -> Optional[int]:
    """fillAt, TypedExecute.cpp:422-464."""
    if boundary > len(p.stages):
        raise ExecutionError("invalid_boundary", "boundary beyond the last stage")
    if not p.plan.fills:
        return None
    agreed = None
    for f in p.plan.fills:
        if f.stage > boundary:
            raise ExecutionError("pad_not_entered", f"a pad enters at stage {f.stage}, after "
                                 f"boundary {boundary}")
        bits, t = f.bits, f.type
        for k in range(f.stage, boundary):
            s = p.stages[k]
            if s.per_channel:
                raise ExecutionError("fill_crosses_channel_stage",
                                     f"a pad fill would cross per-channel stage {k}")
            if not t.same(s.input):
                raise ExecutionError("fill_type_mismatch", f"pad fill type disagrees with stage {k}")
            arr = np.array([bits], dtype=_NP_BITS[t.width])
            bits = int(apply_stage(s, arr, None)[0])
            t = s.output
        if not t.same(type_at(p, boundary)):
            raise ExecutionError("fill_type_mismatch",
                                 f"pad fill type disagrees with boundary {boundary}")
        if agreed is not None and agreed != bits:
            raise ExecutionError("mixed_fills_unsupported",
                                 f"pads carry different values at boundary {boundary}")
        agreed = bits
    if (boundary == len(p.stages) and p.plan.layout.pad_regions
            and p.plan.layout.pad_regions[0].fill_bits != agreed):
        raise ExecutionError("fill_mismatch", "folded fill disagrees with the layout's fused fill")
    return agreed


def _offsets(extents: Sequence[int], strides: Sequence[int], shifts: Sequence[int]) -> np.ndarray:
    """All Σ (c_k + shift_k) * stride_k over the box, in row-major order of c."""
    off = np.zeros((), np.int64)
    for e, s, sh in zip(extents, strides, shifts):
        off = np.add.outer(off, (np.arange(e, dtype=np.int64) + sh) * s)
    return off.reshape(-1)


def execute_host(p: Program, frm: int, to: int, src: np.ndarray) -> np.ndarray:
    """executeHost, TypedExecute.cpp:726-939: `src` holds the dense
    SOURCE-layout values at boundary `frm` (any dtype of that width); returns
    the dense RESULT-layout bytes at boundary `to` as a uint8 array.
    Elements the walker never reaches keep fillAt(to)."""
    n_st = len(p.stages)
    if frm > to or to > n_st:
        raise ExecutionError("invalid_boundary", f"stage range [{frm}, {to}) is not inside the program")
    if not pads_settled_by(p, to):
        raise ExecutionError("pads_not_settled", f"a pad enters after boundary {to}")
    fill = fill_at(p, to)
    wf, wt = type_at(p, frm).width, type_at(p, to).width
    lay = p.plan.layout
    out = np.zeros(p.result_elements, dtype=_NP_BITS[wt])
    if fill is not None:
        out[:] = fill
    lo = [0] * len(lay.extents)
    for pr in lay.pad_regions:
        lo[pr.axis] = pr.lo
    src_bits = np.frombuffer(np.ascontiguousarray(src).tobytes(), dtype=_NP_BITS[wf])
    so = _offsets(lay.extents, lay.src_strides, [0] * len(lay.extents))
    do = _offsets(lay.extents, lay.dst_strides, lo)
    vals = src_bits[so]
    coords = None
    for k in range(frm, to):
        s = p.stages[k]
        ch = None
        if s.per_channel:
            if coords is None:
                coords = []
                rest = do.copy()
                for j, stride in enumerate(p.result_strides):
                    cj = rest // stride
                    rest = rest - cj * stride
                    coords.append(cj)
            if s.channel_is_dim:
                ch = coords[s.channel_dim]
            else:
                ch = eval_channel_vec(s.channel, p.plan.symbols, coords)
            bad = (ch < 0) | (ch >= s.channel_length)
            if np.any(bad):
                first = int(ch[np.argmax(bad)])
                raise ExecutionError("channel_out_of_range", f"stage {k} selected channel {first} "
                                     f"of {s.channel_length}")
        vals = apply_stage(s, vals, ch)
    out[do] = vals.astype(out.dtype, copy=False)
    return out.view(np.uint8)


def execute_layout(b: BoundPlan, src: bytes) -> bytes:
    """executeH2D's byte-exact gather semantics (Execute.cpp:94-134 gatherChunk
    + fill): dst[Σ(c+lo)d] = src[Σ c s] for element-size-wide units; pad
    positions hold the low elementSize bytes of each pad's fill."""
    es = b.element_size
    n = b.total_bytes // es
    dt = np.dtype([("b", np.uint8, es)])
    out = np.zeros(n, dtype=dt)
    if b.pad_regions:
        pattern = b.pad_regions[0].fill_bits.to_bytes(8, "little")[:es]
        out[:] = np.frombuffer(pattern, dtype=dt)[0]
    lo = [0] * len(b.extents)
    for pr in b.pad_regions:
        lo[pr.axis] = pr.lo
    s = np.frombuffer(bytes(src), dtype=dt)
    out[_offsets(b.extents, b.dst_strides, lo)] = s[_offsets(b.extents, b.src_strides,
                                                             [0] * len(b.extents))]
    return out.tobytes()


# ---------------------------------------------------------------------------
# Chunk schedule (libreloc/src/ChunkSchedule.cpp:9-90)
# ---------------------------------------------------------------------------

K_MIN_CHUNK = 4 << 20
K_MAX_CHUNK = 64 << 20
K_CHUNKS_PER_BUFFER = 8


@dataclass
class Chunk:
    padded_begin: int
    padded_end: int
    valid_begin: int
    valid_end: int
    byte_offset: int
    bytes: int


def plan_chunks(b: BoundPlan, n_buffers: int, override: int = 0):
    """planChunks: returns (chunks, max_chunk_bytes, outer_lo, row_bytes, serialized)."""
    n_buffers = max(1, n_buffers)
    es = b.element_size
    outer_lo = outer_hi = 0
    padded = list(b.extents)
    for pr in b.pad_regions:
        padded[pr.axis] += pr.lo + pr.hi
        if pr.axis == 0:
            outer_lo, outer_hi = pr.lo, pr.hi
    row_bytes = b.dst_strides[0] * es
    valid = b.extents[0]
    padded_outer = valid + outer_lo + outer_hi
    span = sum((padded[k] - 1) * b.dst_strides[k] for k in range(1, len(b.extents)))
    disjoint = b.dst_strides[0] >= span + 1
    if not disjoint or padded_outer <= 0:
        return ([Chunk(0, padded_outer, 0, valid, 0, b.total_bytes)], b.total_bytes, outer_lo,
                row_bytes, True)
    target = override if override else min(max(b.total_bytes // (K_CHUNKS_PER_BUFFER * n_buffers),
                                               K_MIN_CHUNK), K_MAX_CHUNK)
    rows = min(padded_outer, max(1, target // row_bytes)) if row_bytes > 0 else padded_outer
    chunks = []
    pb = 0
    while pb < padded_outer:
        pe = pb + min(rows, padded_outer - pb)
        vb = min(max(pb - outer_lo, 0), valid)
        ve = min(pe - outer_lo, valid)
        ve = max(ve, vb)
        chunks.append(Chunk(pb, pe, vb, ve, pb * row_bytes, (pe - pb) * row_bytes))
        pb = pe
    return chunks, rows * row_bytes, outer_lo, row_bytes, False


# ---------------------------------------------------------------------------
# Convenience: one call from wire bytes to result bytes
# ---------------------------------------------------------------------------

def run_typed(blob: bytes, symbols: Dict[str, int], params: ParameterMap, src: np.ndarray,
              frm: int = 0, to: Optional[int] = None) -> np.ndarray:
    plan = decode_typed_plan(blob)
    bound = bind_typed(plan, symbols, params)
    prog = prepare_program(bound)
    return execute_host(prog, frm, len(prog.stages) if to is None else to, src)


DTYPE_TYPES = {
    "float32": ElementType(KIND_FLOAT, 32), "float16": ElementType(KIND_FLOAT, 16),
    "bfloat16": ElementType(KIND_BFLOAT, 16), "int8": ElementType(KIND_INT, 8),
    "int32": ElementType(KIND_INT, 32), "int64": ElementType(KIND_INT, 64),
}


# ---------------------------------------------------------------------------
# Indexed plans (wire v2): index_select along axis 0, then at most one cast
# ---------------------------------------------------------------------------

@dataclass
class IndexedPlan:
    symbols: List[str]
    source: TensorDesc
    indices: TensorDesc
    result: TensorDesc
    axis: int
    policy: int


def validate_indexed_plan(p: IndexedPlan) -> Optional[str]:
    """validateIndexedPlan, Decode.cpp:950-991."""
    def const(e):
        return e[0][1] if len(e) == 1 and e[0][0] == OP_PUSH_CONST else None

    for d in (p.source, p.indices, p.result):
        if not d.extents or d.strides or const(d.offset) != 0:
            return "indexed plan requires dense zero-offset positive-rank descriptors"
        for e in d.extents:
            c = const(e)
            if c is not None and c <= 0:
                return "indexed plan extents must be positive"
    it = p.indices.element_type
    if p.axis != 0 or len(p.indices.extents) != 1 or it.kind != KIND_INT or \
            it.bitwidth not in (32, 64):
        return "indexed plan requires axis 0 and rank-one i32/i64 indices"
    if len(p.source.extents) != len(p.result.extents):
        return "indexed plan source/result rank mismatch"
    for i, a in enumerate(p.result.extents):
        b = p.indices.extents[0] if i == 0 else p.source.extents[i]
        ca, cb = const(a), const(b)
        if ca is not None and cb is not None and ca != cb:
            return "indexed plan result extent mismatch"
    a, b = p.source.element_type, p.result.element_type
    supported = _isf(a, 32) or _isf(a, 16) or _isi8(a)
    if (a.same(b) and supported and p.policy == P_EXACT) or \
            (_isf(a, 32) and _isf(b, 16) and p.policy == P_IEEE_RNE) or \
            (_isf(a, 16) and _isf(b, 32) and p.policy == P_EXACT):
        return None
    return "indexed plan has an unsupported type/policy pair"


def decode_indexed_plan(data: bytes) -> IndexedPlan:
    """decodeIndexedPlan, Decode.cpp:993-1012."""
    r = _Reader(data)
    symbols = _parse_header(r, 2)
    n = len(symbols)
    source = _parse_desc(r, n)
    indices = _parse_desc(r, n)
    result = _parse_desc(r, n)
    axis = r.u32()
    policy = r.u8()
    if r.remaining():
        r.fail(r.off, "trailing bytes after indexed plan")
    p = IndexedPlan(symbols, source, indices, result, axis, policy)
    why = validate_indexed_plan(p)
    if why:
        r.fail(r.off, why)
    return p


@dataclass
class IndexedBoundPlan:
    source_extents: List[int]  # the table
    result_extents: List[int]
    indices: List[int]
    row_elements: int
    source_type: ElementType
    result_type: ElementType
    policy: int
    source_bytes: int          # selected rows, source type
    destination_bytes: int
    parameter_bytes: int       # index bytes


def bind_indexed(plan: IndexedPlan, sym_map: Dict[str, int], index_dtype: ElementType,
                 index_extents: Sequence[int], index_bytes: bytes) -> IndexedBoundPlan:
    """bindIndexed, Bind.cpp:708-819 (error messages as there)."""
    why = validate_indexed_plan(plan)
    if why:
        raise BindError(why)
    syms = _resolve(plan.symbols, sym_map)
    table = _dense_desc(plan.source, syms, "source")
    ind = _dense_desc(plan.indices, syms, "indices")
    result = _dense_desc(plan.result, syms, "result")
    if list(index_extents) != ind or not index_dtype.same(plan.indices.element_type):
        raise BindError("index operand dtype/extents do not match the plan")
    selected = [ind[0]] + table[1:]
    if selected != result:
        raise BindError("indexed result shape does not match source and indices")
    iw = index_dtype.width
    ib = _mul_ok(ind[0], iw)
    if ib is None or ib != len(index_bytes):
        raise BindError("index operand byte size mismatch or overflow")
    row = 1
    for e in table[1:]:
        row = _mul_ok(row, e)
        if row is None:
            raise BindError("indexed row size overflow")
    sw, rw = plan.source.element_type.width, plan.result.element_type.width
    sizes = []
    for a, b in ((table[0], row), (ind[0], row)):
        n = _mul_ok(a, b)
        sizes.append(n)
    ok = sizes[0] is not None and _mul_ok(sizes[0], sw) is not None and sizes[1] is not None \
        and _mul_ok(sizes[1], sw) is not None and _mul_ok(sizes[1], rw) is not None
    if not ok:
        raise BindError("indexed tensor size overflow")
    vals = [_sign_extend(int.from_bytes(index_bytes[i * iw:(i + 1) * iw], "little"),
                         index_dtype.bitwidth) for i in range(ind[0])]
    if any(v < 0 or v >= table[0] for v in vals):
        raise BindError("index_out_of_range: index_select row is outside the source")
    return IndexedBoundPlan(table, result, vals, row, plan.source.element_type,
                            plan.result.element_type, plan.policy, sizes[1] * sw, sizes[1] * rw, ib)


def execute_indexed(b: IndexedBoundPlan, table: np.ndarray) -> np.ndarray:
    """The indexed branch of executeHost (TypedExecute.cpp:741-790): each
    selected row copied, or cast element by element with the stage
    arithmetic of applyStage. Returns the dense selected rows as bytes."""
    sw, rw = b.source_type.width, b.result_type.width
    raw = np.ascontiguousarray(table).view(np.uint8).reshape(-1)
    rows = raw[:b.source_extents[0] * b.row_elements * sw].reshape(b.source_extents[0], -1)
    sel = rows[np.asarray(b.indices, dtype=np.int64)]
    if b.source_type.same(b.result_type):
        return sel.reshape(-1).copy()
    bits = sel.reshape(-1).view(_NP_BITS[sw])
    if _isf(b.source_type, 32):
        out = narrow_f32_f16_bits(bits).astype(np.uint16)
    else:
        out = widen_f16_f32_bits(bits).astype(np.uint32)
    return out.view(np.uint8)
