"""Recipe -> relocation plan encoder (wire v0 layout, wire v1 typed, wire v2
indexed).

The reference produces plans with its MLIR exporter (`sym-reloc-export`,
sym/dialect/reloc/Transforms/PlanBuilder.h:27-172 and
sym/dialect/reloc/IR/RelocSerialization.cpp), which cannot exist on this
machine. This module folds the same op vocabulary -- reshape, transpose, pad,
cast, quantize, dequantize -- into one plan in the wire format of
docs/reloc-plan-format.md:

  * the view starts as the identity over the source (axis k has the source's
    row-major stride); transposes permute axes, reshapes split/merge them
    (symbolic splits emit divisibility constraints), pads attach to an axis
    (a second same-fill pad of the axis widens it; a reshape keeps a padded
    axis only 1:1);
  * value stages record their logical operand shape and a channel map over
    the logical result coordinates; pending pad fills fold through later
    per-tensor stages (a per-channel stage after a pad is rejected);
  * finalisation merges neighbouring axes that are contiguous in the source
    (never padded ones), derives row-major destination strides, `perm`
    (source-view rank of each destination axis), the inverse map and
    contiguity flags, and assigns symbol indices by first use.

Plans it writes decode and bind under the reference runtime; semantic parity
with the recipe is tested by executing them (tests/test_encoder.py).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple, Union

# ------------------------------------------------------------------ exprs

PUSH_SYM, PUSH_CONST, ADD, SUB, MUL, FLOORDIV, MOD, PUSH_DIM = range(8)


class E:
    """A small symbolic integer expression: const, sym, dim or binary op."""

    __slots__ = ("kind", "a", "b", "value")

    def __init__(self, kind, a=None, b=None, value=None):
        self.kind, self.a, self.b, self.value = kind, a, b, value

    # constructors -------------------------------------------------------
    @staticmethod
    def c(v):
        return E("const", value=int(v))

    @staticmethod
    def s(name):
        return E("sym", value=str(name))

    @staticmethod
    def d(i):
        return E("dim", value=int(i))

    def is_const(self, v=None):
        return self.kind == "const" and (v is None or self.value == v)

    def key(self):
        if self.kind in ("const", "sym", "dim"):
            return (self.kind, self.value)
        return (self.kind, self.a.key(), self.b.key())

    def __eq__(self, other):
        return isinstance(other, E) and self.key() == other.key()

    def __hash__(self):
        return hash(self.key())

    def __repr__(self):
        if self.kind == "const":
            return str(self.value)
        if self.kind == "sym":
            return self.value
        if self.kind == "dim":
            return "d%d" % self.value
        op = {"add": "+", "sub": "-", "mul": "*", "floordiv": "//", "mod": "%"}[self.kind]
        return "(%r %s %r)" % (self.a, op, self.b)

    def eval(self, syms: Dict[str, int], dims: Sequence[int] = ()):
        k = self.kind
        if k == "const":
            return self.value
        if k == "sym":
            return syms[self.value]
        if k == "dim":
            return dims[self.value]
        a, b = self.a.eval(syms, dims), self.b.eval(syms, dims)
        return {"add": a + b, "sub": a - b, "mul": a * b,
                "floordiv": a // b, "mod": a % b}[k]


def add(a: E, b: E) -> E:
    if a.is_const() and b.is_const():
        return E.c(a.value + b.value)
    if a.is_const(0):
        return b
    if b.is_const(0):
        return a
    if b.is_const() and a.kind == "add" and a.b.is_const():
        return add(a.a, E.c(a.b.value + b.value))  # (x + c1) + c2 -> x + (c1 + c2)
    return E("add", a, b)


def mul(a: E, b: E) -> E:
    if a.is_const() and b.is_const():
        return E.c(a.value * b.value)
    if a.is_const(1):
        return b
    if b.is_const(1):
        return a
    # (x // c) * c stays symbolic; divisibility is carried separately
    return E("mul", a, b)


def floordiv(a: E, b: E) -> E:
    if a.is_const() and b.is_const():
        return E.c(a.value // b.value)
    if b.is_const(1):
        return a
    return E("floordiv", a, b)


def sub(a: E, b: E) -> E:
    if a.is_const() and b.is_const():
        return E.c(a.value - b.value)
    if b.is_const(0):
        return a
    return E("sub", a, b)


def align_up_pad(e, align: int) -> E:
    """The trailing pad width that rounds extent `e` up to a multiple of
    `align`: ((e + align - 1) // align) * align - e."""
    e = expr(e)
    return sub(mul(floordiv(add(e, E.c(align - 1)), E.c(align)), E.c(align)), e)


def mod(a: E, b: E) -> E:
    if a.is_const() and b.is_const():
        return E.c(a.value % b.value)
    return E("mod", a, b)


def expr(v) -> E:
    """int -> const, str -> symbol or `<sym> floordiv <k>` / `<sym> * <k>`."""
    if isinstance(v, E):
        return v
    if isinstance(v, int):
        return E.c(v)
    parts = str(v).split()
    if len(parts) == 1:
        return E.s(parts[0])
    if len(parts) == 3 and parts[1] in ("floordiv", "//"):
        return floordiv(expr(parts[0]), expr(int(parts[2]) if parts[2].lstrip("-").isdigit() else parts[2]))
    if len(parts) == 3 and parts[1] == "*":
        return mul(expr(_num(parts[0])), expr(_num(parts[2])))
    raise ValueError("unsupported dim expression: %r" % (v,))


def _num(t):
    return int(t) if t.lstrip("-").isdigit() else t


def _factors(e: E) -> List[E]:
    """Flatten a product into its factors."""
    if e.kind == "mul":
        return _factors(e.a) + _factors(e.b)
    return [e]


def product(es: Sequence[E]) -> E:
    out = E.c(1)
    for x in es:
        out = mul(out, x)
    return out


# ---------------------------------------------------------------- dtypes

DTYPES = {  # name -> (kind, bitwidth)
    "float32": (0, 32), "float16": (0, 16), "float64": (0, 64), "bfloat16": (1, 16),
    "int8": (2, 8), "int16": (2, 16), "int32": (2, 32), "int64": (2, 64),
}
SIGNLESS, SIGNED = 0, 1
TRANSFORMS = {"cast": 0, "quantize": 1, "dequantize": 2}
POLICIES = {"ieee_rne": 0, "exact": 1, "symmetric_rne": 2, "affine": 3}

# ------------------------------------------------------------------ ops


@dataclass(frozen=True)
class Transpose:
    perm: Tuple[int, ...]


@dataclass(frozen=True)
class Reshape:
    to: Tuple[Union[int, str, E], ...]


@dataclass(frozen=True)
class Pad:
    axis: int
    lo: Union[int, str, E]
    hi: Union[int, str, E]
    value: float = 0.0  # the fill, in the current element type (int for int8)
    bits: Optional[int] = None  # exact fill bit pattern (overrides `value`)


@dataclass(frozen=True)
class InlineParam:
    values: Tuple[float, ...]
    dtype: str = "float32"
    rank: int = 0  # 0 per tensor, 1 per channel
    bits: Optional[Tuple[int, ...]] = None  # exact element bit patterns

    def element_bits(self):
        if self.bits is not None:
            return [int(b) for b in self.bits]
        return [_value_bits(v, self.dtype) for v in self.values]


@dataclass(frozen=True)
class BindingParam:
    name: str
    dtype: str
    extents: Tuple[Union[int, str, E], ...] = ()


@dataclass(frozen=True)
class Cast:
    dtype: str
    policy: str = "ieee_rne"


@dataclass(frozen=True)
class Quantize:
    scale: Union[InlineParam, BindingParam]
    zero_point: Optional[Union[InlineParam, BindingParam]] = None
    axis: Optional[int] = None
    policy: str = "symmetric_rne"
    dtype: str = "int8"


@dataclass(frozen=True)
class Dequantize:
    scale: Union[InlineParam, BindingParam]
    zero_point: Optional[Union[InlineParam, BindingParam]] = None
    axis: Optional[int] = None
    policy: str = "affine"
    dtype: str = "float32"


class EncodeError(ValueError):
    pass


# ----------------------------------------------------------- fill values

def _f32_bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", float(x)))[0]


def _value_bits(value, dtype: str) -> int:
    kind, bits = DTYPES[dtype]
    if kind == 2:
        return int(value) & ((1 << bits) - 1)
    if dtype == "float32":
        return _f32_bits(value)
    if dtype == "float64":
        return struct.unpack("<Q", struct.pack("<d", float(value)))[0]
    if dtype == "float16":
        import numpy as np
        return int(np.array([value], np.float16).view(np.uint16)[0])
    if dtype == "bfloat16":
        from . import _hostmath
        return _hostmath.f32_to_bf16(_f32_bits(value))
    raise EncodeError("unsupported fill dtype " + dtype)


# ---------------------------------------------------------------- builder

@dataclass
class _Axis:
    extent: E
    stride: E
    src_pos: int  # position in source-view order (0 = outermost)


@dataclass
class _PadState:
    axis: int
    lo: E
    hi: E
    bits: int  # fused fill in the current dtype
    original_bits: int
    original_dtype: str
    stage: int


@dataclass
class _Stage:
    transform: str
    policy: str
    input: str
    output: str
    shape: List[E]
    scale: Optional[object]
    zero_point: Optional[object]
    axis: int
    channel: Optional[E]  # over the current view dims


@dataclass
class Plan:
    blob: bytes
    symbols: List[str]
    typed: bool
    source_shape: List[E]
    result_shape: List[E]
    source_dtype: str
    result_dtype: str
    divisibility: List[Tuple[E, int]] = field(default_factory=list)
    parameters: List[Tuple[str, str, List[E]]] = field(default_factory=list)
    # typed plans: the value stages as written (shape, parameters, channel map
    # over result coordinates) and the pad fills (destination axis of the
    # plan, entry stage, dtype, bits), for an artifact's manifest
    stages: List["_Stage"] = field(default_factory=list)
    fills: List[Tuple[int, int, str, int]] = field(default_factory=list)


def encode(source_shape: Sequence, source_dtype: str, ops: Sequence, *, force_typed=False) -> Plan:
    """Fold `ops` over a dense row-major source into one wire plan."""
    shape = [expr(d) for d in source_shape]
    if not shape:
        raise EncodeError("source rank must be >= 1")
    # identity view
    strides = []
    running = E.c(1)
    for e in reversed(shape):
        strides.append(running)
        running = _times(e, running)
    strides.reverse()
    axes = [_Axis(e, s, i) for i, (e, s) in enumerate(zip(shape, strides))]
    pads: List[_PadState] = []
    stages: List[_Stage] = []
    divisibility: List[Tuple[E, int]] = []
    dtype = source_dtype

    def view_shape():
        out = []
        for i, a in enumerate(axes):
            p = next((p for p in pads if p.axis == i), None)
            out.append(add(add(a.extent, p.lo), p.hi) if p else a.extent)
        return out

    for op in ops:
        if isinstance(op, Transpose):
            perm = list(op.perm)
            if sorted(perm) != list(range(len(axes))):
                raise EncodeError("transpose perm is not a permutation of the rank")
            inv = [perm.index(i) for i in range(len(axes))]
            axes = [axes[p] for p in perm]
            for p in pads:
                p.axis = inv[p.axis]
            for s in stages:
                if s.channel is not None:
                    s.channel = _remap_dims(s.channel, inv)
        elif isinstance(op, Reshape):
            for s in stages:
                if s.channel is not None:
                    raise EncodeError("reshape after a per-channel stage is not folded")
            target = [expr(t) for t in op.to]
            if any(t.kind == "const" and t.value <= 0 for t in target):
                raise EncodeError("reshape to a non-positive extent")
            if pads:
                axes, divs = _reshape_padded(axes, pads, target)
            else:
                axes, divs = _reshape(axes, target)
            for d in divs:
                if d not in divisibility:
                    divisibility.append(d)
        elif isinstance(op, Pad):
            if not 0 <= op.axis < len(axes):
                raise EncodeError("pad axis out of range")
            lo, hi = expr(op.lo), expr(op.hi)
            # sym/dialect/reloc/Transforms/PlanBuilder.cpp:497-506: a provably
            # negative width is refused, two zero widths record nothing
            if any(w.kind == "const" and w.value < 0 for w in (lo, hi)):
                raise EncodeError("negative pad width")
            if lo.is_const(0) and hi.is_const(0):
                continue
            bits = op.bits if op.bits is not None else _value_bits(op.value, dtype)
            old = next((p for p in pads if p.axis == op.axis), None)
            if old is not None:
                # PlanBuilder.cpp:534-548: a second pad of the axis with the
                # same fill, entering at the same value stage, wraps the first
                # (widths add); the format keeps one fill per axis
                if old.bits != bits or old.stage != len(stages):
                    raise EncodeError("one pad per axis: a second pad needs the same fill "
                                      "and value stage")
                old.lo, old.hi = add(old.lo, lo), add(old.hi, hi)
            else:
                pads.append(_PadState(op.axis, lo, hi, bits, bits, dtype, len(stages)))
            # earlier stages' channel maps read the padded axis shifted by the
            # leading width (the reference builder does the same,
            # sym/dialect/reloc/Transforms/PlanBuilder.h:44-47)
            if not lo.is_const(0):
                for s in stages:
                    if s.channel is not None:
                        s.channel = _shift_dim(s.channel, op.axis, lo)
        elif isinstance(op, (Cast, Quantize, Dequantize)):
            st = _stage(op, dtype, view_shape(), len(axes))
            for p in pads:
                p.bits = _fold(p.bits, st)
            stages.append(st)
            dtype = st.output
        else:
            raise EncodeError("unsupported op %r" % (op,))
    typed = bool(stages) or force_typed
    if typed and not stages:
        raise EncodeError("a typed plan needs at least one stage")
    result_shape = view_shape()
    return _finalize(shape, source_dtype, axes, pads, stages, divisibility, dtype, result_shape,
                     typed)


def _shift_dim(e: E, axis: int, lo: E) -> E:
    """`e` with view coordinate `axis` replaced by (coordinate - lo)."""
    if e.kind == "dim":
        return E("sub", e, lo) if e.value == axis else e
    if e.kind in ("const", "sym"):
        return e
    return E(e.kind, _shift_dim(e.a, axis, lo), _shift_dim(e.b, axis, lo))


def _remap_dims(e: E, inv: List[int]) -> E:
    if e.kind == "dim":
        return E.d(inv[e.value])
    if e.kind in ("const", "sym"):
        return e
    return E(e.kind, _remap_dims(e.a, inv), _remap_dims(e.b, inv))


def _reshape_padded(axes: List[_Axis], pads: List[_PadState], target: List[E]):
    """Reshape a padded view: each padded axis must be kept 1:1 (a target
    entry equal to its padded extent, the axes before it regrouping onto the
    entries before that one); the unpadded axes between regroup among
    themselves. A split or merge of a padded axis is refused, as the valid
    region would no longer be a per-axis box (the reference builder's rule,
    sym/dialect/reloc/Transforms/PlanBuilder.cpp reshape fold; unittest
    PlanBuilderTest.cpp:631-682). Moves the pads to their new positions."""
    by_axis = {p.axis: p for p in pads}
    out: List[_Axis] = []
    divs: List[Tuple[E, int]] = []
    where = {}
    a0 = t0 = 0
    for i in sorted(by_axis):
        p = by_axis[i]
        ext = add(add(axes[i].extent, p.lo), p.hi)
        for j in range(t0, len(target)):
            if not target[j] == ext:
                continue
            try:
                seg, d = _reshape(axes[a0:i], target[t0:j])
            except EncodeError:
                continue
            break
        else:
            raise EncodeError("reshape splits or merges a padded axis")
        out += seg
        divs += d
        where[i] = len(out)
        out.append(_Axis(axes[i].extent, axes[i].stride, axes[i].src_pos))
        a0, t0 = i + 1, j + 1
    seg, d = _reshape(axes[a0:], target[t0:])
    out += seg
    divs += d
    for p in pads:
        p.axis = where[p.axis]
    return out, divs


def _reshape(axes: List[_Axis], target: List[E]):
    """Split/merge the dense view into `target`; returns (axes, divisibility)."""
    out: List[_Axis] = []
    divs: List[Tuple[E, int]] = []
    i = 0
    j = 0
    while i < len(axes) or j < len(target):
        if i < len(axes) and j < len(target) and axes[i].extent == target[j]:
            out.append(_Axis(axes[i].extent, axes[i].stride, axes[i].src_pos))
            i += 1
            j += 1
            continue
        if i < len(axes) and axes[i].extent.is_const(1):
            i += 1
            continue
        if j < len(target) and target[j].is_const(1):
            out.append(_Axis(E.c(1), E.c(0), -1))
            j += 1
            continue
        if i >= len(axes) or j >= len(target):
            raise EncodeError("reshape element counts disagree")
        a = axes[i]
        t = target[j]
        # constant regroup: the smallest old/new groups with equal products;
        # the old group must be contiguous in the source (one strided block),
        # which is then split into the new dims
        if a.extent.is_const() and t.is_const():
            i2, j2 = i + 1, j + 1
            po, pn = a.extent.value, t.value
            while po != pn:
                if po < pn:
                    if i2 >= len(axes) or not axes[i2].extent.is_const():
                        raise EncodeError("cannot factor constant reshape")
                    po *= axes[i2].extent.value
                    i2 += 1
                else:
                    if j2 >= len(target) or not target[j2].is_const():
                        raise EncodeError("cannot factor constant reshape")
                    pn *= target[j2].value
                    j2 += 1
            group = axes[i:i2]
            for x, y in zip(group, group[1:]):
                if x.stride != _times(y.extent, y.stride):
                    raise EncodeError("reshape merges non-contiguous axes")
            inner = group[-1].stride
            sub = []
            for tv in reversed(target[j:j2]):
                sub.append(_Axis(tv, inner, group[0].src_pos))
                inner = _times(tv, inner)
            out.extend(reversed(sub))
            i, j = i2, j2
            continue
        # symbolic split: s -> [s // c, c] or [c, s // c]
        if j + 1 < len(target):
            t0, t1 = target[j], target[j + 1]
            c = None
            if t0.kind == "floordiv" and t0.a == a.extent and t0.b.is_const() and t1 == t0.b:
                c, outer_first = t0.b.value, True
            elif t1.kind == "floordiv" and t1.a == a.extent and t1.b.is_const() and t0 == t1.b:
                c, outer_first = t1.b.value, False
            if c is not None:
                divs.append((a.extent, c))
                out.append(_Axis(t0, _times(t1, a.stride), a.src_pos))
                out.append(_Axis(t1, a.stride, a.src_pos))
                i += 1
                j += 2
                continue
        # merge several contiguous axes into one target dim
        group = [a]
        ext = a.extent
        k = i + 1
        while ext != t and k < len(axes):
            nxt = axes[k]
            if group[-1].stride != _times(nxt.extent, nxt.stride):
                raise EncodeError("reshape merges non-contiguous axes")
            group.append(nxt)
            ext = mul(ext, nxt.extent)
            k += 1
            if ext.is_const() and t.is_const() and ext.value == t.value:
                ext = t
        if ext != t and not (_const_product(ext) is not None and t.is_const()
                             and _const_product(ext) == t.value):
            raise EncodeError("cannot fold reshape to %r" % (t,))
        out.append(_Axis(t, group[-1].stride, group[0].src_pos))
        i = k
        j += 1
    # renumber source-view positions densely (merges/splits keep order)
    order = sorted(range(len(out)), key=lambda x: (out[x].src_pos, -_rank_hint(out, x)))
    for rank, x in enumerate(order):
        out[x].src_pos = rank
    return out, divs


def _times(extent: E, stride: E) -> E:
    """The stride of the axis just outside one with (extent, stride): the
    compiler writes it stride-first (`stride * extent`)."""
    if stride.is_const(1):
        return extent
    return mul(stride, extent)


def _const_product(e: E):
    fs = _factors(e)
    if all(f.is_const() for f in fs):
        v = 1
        for f in fs:
            v *= f.value
        return v
    return None


def _rank_hint(axes, x):
    # within one source axis split into pieces, the outer piece comes first
    return -x


def _param_dtype(p):
    return p.dtype


def _stage(op, dtype: str, shape: List[E], rank: int) -> _Stage:
    if isinstance(op, Cast):
        pol = op.policy
        if dtype == "float32" and op.dtype in ("float16", "bfloat16"):
            pol = "ieee_rne"
        elif dtype in ("float16", "bfloat16") and op.dtype == "float32":
            pol = "exact"
        else:
            raise EncodeError("unsupported cast %s -> %s" % (dtype, op.dtype))
        return _Stage("cast", pol, dtype, op.dtype, list(shape), None, None, -1, None)
    if isinstance(op, Quantize):
        if dtype != "float32":
            raise EncodeError("quantize consumes float32")
        out = "int8"
    else:
        if dtype != "int8":
            raise EncodeError("dequantize consumes int8")
        out = "float32"
    axis = -1 if op.axis is None else int(op.axis)
    channel = None
    if axis >= 0:
        if axis >= rank:
            raise EncodeError("channel axis out of range")
        channel = E.d(axis)
    return _Stage("quantize" if isinstance(op, Quantize) else "dequantize", op.policy, dtype, out,
                  list(shape), op.scale, op.zero_point, axis, channel)


def _fold(bits: int, st: _Stage) -> int:
    """Fold a pending fill through one stage (typed::foldFill semantics)."""
    from . import _hostmath as H
    if st.transform == "cast":
        return H.cast_bits(bits, st.input, st.output)
    sc = st.scale
    if st.axis >= 0 or not isinstance(sc, InlineParam) or sc.rank != 0:
        raise EncodeError("fill_not_foldable: a pad cannot cross a per-channel or runtime-parameter stage")
    zp = 0
    if st.zero_point is not None:
        if not isinstance(st.zero_point, InlineParam) or st.zero_point.rank != 0:
            raise EncodeError("fill_not_foldable")
        zb = st.zero_point.element_bits()[0]
        zbits = DTYPES[st.zero_point.dtype][1]
        zp = zb - (1 << zbits) if zb >> (zbits - 1) & 1 else zb
    scale_bits = sc.element_bits()[0]
    if st.transform == "quantize":
        return H.quantize_bits(bits, scale_bits)
    return H.dequantize_bits(bits, scale_bits, zp)


# ------------------------------------------------------------- finalise

class _Writer:
    """Little-endian wire writer; expressions name symbols by their index in
    `symbols` (docs/reloc-plan-format.md:74-97)."""

    def __init__(self, symbols=None):
        self.out = bytearray()
        self.symbols = symbols if symbols is not None else []

    def u8(self, v):
        self.out += struct.pack("<B", v)

    def u32(self, v):
        self.out += struct.pack("<I", v)

    def i64(self, v):
        self.out += struct.pack("<q", v)

    def u64(self, v):
        self.out += struct.pack("<Q", v & ((1 << 64) - 1))

    def str(self, s):
        b = s.encode()
        self.u32(len(b))
        self.out += b

    def expr(self, e: E):
        ops = []

        def emit(x):
            if x.kind == "const":
                ops.append((PUSH_CONST, x.value))
            elif x.kind == "sym":
                ops.append((PUSH_SYM, self.symbols.index(x.value)))
            elif x.kind == "dim":
                ops.append((PUSH_DIM, x.value))
            else:
                emit(x.a)
                emit(x.b)
                ops.append(({"add": ADD, "sub": SUB, "mul": MUL, "floordiv": FLOORDIV,
                             "mod": MOD}[x.kind], None))
        emit(e)
        self.u32(len(ops))
        for op, v in ops:
            self.u8(op)
            if op == PUSH_CONST:
                self.i64(v)
            elif op in (PUSH_SYM, PUSH_DIM):
                self.u32(v)

    def dtype(self, dt):
        kind, bits = DTYPES[dt]
        self.u8(kind)
        self.u32(bits)

    def desc(self, shape, dt):
        self.u32(len(shape))
        for e in shape:
            self.expr(e)
        self.u32(0)  # canonical row-major strides
        self.expr(E.c(0))
        self.dtype(dt)


def _finalize(source_shape, source_dtype, axes, pads, stages, divisibility, dtype, result_shape,
              typed) -> Plan:
    # merge neighbours contiguous in the source (unpadded), like the compiler's
    # canonical axis merging; pad axes are renumbered
    merged: List[_Axis] = []
    pad_of = {p.axis: p for p in pads}
    new_pads: Dict[int, _PadState] = {}
    for i, a in enumerate(axes):
        if merged and i - 1 not in pad_of and i not in pad_of and not a.extent.is_const(1) \
                and merged[-1][0].stride == _times(a.extent, a.stride) \
                and merged[-1][1] == i - 1:
            prev = merged[-1][0]
            merged[-1] = (_Axis(mul(prev.extent, a.extent), a.stride, prev.src_pos), i)
        else:
            merged.append((_Axis(a.extent, a.stride, a.src_pos), i))
            if i in pad_of:
                new_pads[len(merged) - 1] = pad_of[i]
    maxes = [m[0] for m in merged]
    # source-view rank of each destination axis
    order = sorted(range(len(maxes)), key=lambda k: maxes[k].src_pos)
    perm = [0] * len(maxes)
    for rank, k in enumerate(order):
        perm[k] = rank
    # padded destination extents and row-major strides
    pext = []
    for k, a in enumerate(maxes):
        p = new_pads.get(k)
        pext.append(add(add(a.extent, p.lo), p.hi) if p else a.extent)
    dstr = [E.c(1)] * len(pext)
    running = E.c(1)
    for k in range(len(pext) - 1, -1, -1):
        dstr[k] = running
        running = _times(pext[k], running)

    symbols: List[str] = []

    def note(e: E):
        if e.kind == "sym":
            if e.value not in symbols:
                symbols.append(e.value)
        elif e.kind not in ("const", "dim"):
            note(e.a)
            note(e.b)

    w = _Writer(symbols)

    # symbol table by first use, in section order
    seq: List[E] = []
    if typed:
        seq += list(source_shape) + list(result_shape)
    seq += list(source_shape) + pext
    for a, s in zip(maxes, dstr):
        seq += [a.extent, a.stride, s]
    for k in sorted(new_pads):
        seq += [new_pads[k].lo, new_pads[k].hi]
    seq += [d[0] for d in divisibility]
    for st in stages:
        seq += st.shape
        for p in (st.scale, st.zero_point):
            if isinstance(p, BindingParam):
                seq += [expr(x) for x in p.extents]
        if st.channel is not None:
            seq.append(st.channel)
    for e in seq:
        note(e)

    w.out += b"RPLN"
    w.u32(1 if typed else 0)
    w.u32(len(symbols))
    for s in symbols:
        w.str(s)
    if typed:
        w.desc(source_shape, source_dtype)
        w.desc(result_shape, dtype)
    # layout body (v0 sections 3..12)
    w.desc(source_shape, source_dtype)
    w.desc(pext, dtype)
    w.u32(len(perm))
    for p in perm:
        w.u32(p)
    w.u32(len(maxes))
    for k, (a, s) in enumerate(zip(maxes, dstr)):
        w.str("d%d" % k)
        w.expr(a.extent)
        w.expr(a.stride)
        w.expr(s)
    w.u32(len(new_pads))
    for k in sorted(new_pads):
        p = new_pads[k]
        w.u32(k)
        w.expr(p.lo)
        w.expr(p.hi)
        w.dtype(dtype)
        w.u64(p.bits)
    w.u32(len(divisibility))
    for e, d in divisibility:
        w.expr(e)
        w.i64(d)
    w.u32(0)  # alignment
    w.u32(len(maxes))
    for a in maxes:
        w.u8(1 if a.stride.is_const(1) else 0)
    # a layout-only plan whose axes move nothing is a pure view
    view = not typed and not new_pads and all(a.stride == s for a, s in zip(maxes, dstr))
    w.u8(1 if view else 0)  # no_copy
    # a symbolic pad width leaves the padded range to be checked at bind time
    # (sym/dialect/reloc/Transforms/PlanBuilder.cpp:74-79)
    w.u8(1 if any(not (p.lo.is_const() and p.hi.is_const()) for p in new_pads.values()) else 0)
    w.u32(len(maxes))
    w.u32(len(maxes))
    inv = [perm.index(i) for i in range(len(perm))]
    for i in range(len(maxes)):
        w.expr(E.d(inv[i]))
    params: List[Tuple[str, str, List[E]]] = []
    if typed:
        w.u32(len(stages))
        for st in stages:
            w.u8(TRANSFORMS[st.transform])
            w.u8(POLICIES[st.policy])
            w.dtype(st.input)
            w.u8(SIGNED if st.transform == "dequantize" else SIGNLESS)
            w.dtype(st.output)
            w.u8(SIGNED if st.transform == "quantize" else SIGNLESS)
            w.u32(len(st.shape))
            for e in st.shape:
                w.expr(e)
            for role, p in (("scale", st.scale), ("zero_point", st.zero_point)):
                if p is None:
                    w.u8(0)
                elif isinstance(p, InlineParam):
                    w.u8(1)
                    w.u8(p.rank)
                    w.dtype(p.dtype)
                    eb = p.element_bits()
                    w.u32(len(eb))
                    for v in eb:
                        w.u64(v)
                else:
                    w.u8(2)
                    w.str(p.name)
                    w.u8(len(p.extents))
                    for x in p.extents:
                        w.expr(expr(x))
                    w.dtype(p.dtype)
                    params.append((p.name, p.dtype, [expr(x) for x in p.extents]))
            w.i64(st.axis)
            if st.channel is not None:
                w.u8(1)
                w.u32(len(result_shape))
                w.expr(st.channel)
            else:
                w.u8(0)
        w.u32(len(new_pads))
        for k in sorted(new_pads):
            p = new_pads[k]
            w.u32(k)
            w.u32(p.stage)
            w.dtype(p.original_dtype)
            w.u64(p.original_bits)
    elif pads and len({p.bits for p in pads}) > 1:
        raise EncodeError("layout plans carry a single fill value")
    fills = [(k, new_pads[k].stage, new_pads[k].original_dtype, new_pads[k].original_bits)
             for k in sorted(new_pads)] if typed else []
    return Plan(bytes(w.out), symbols, typed, list(source_shape), list(result_shape), source_dtype,
                dtype, list(divisibility), params, list(stages) if typed else [], fills)


# ------------------------------------------------------------ indexed (v2)

# Element-type pairs an indexed plan may carry, with the numeric policy the
# cast takes (docs/reloc-plan-format.md:287-345; validateIndexedPlan,
# libreloc/src/Decode.cpp:950-991).
_INDEXED_PAIRS = {("float32", "float32"): "exact", ("float16", "float16"): "exact",
                  ("int8", "int8"): "exact", ("float32", "float16"): "ieee_rne",
                  ("float16", "float32"): "exact"}


def encode_index_select(source_shape: Sequence, source_dtype: str, count, index_dtype: str,
                        result_dtype: Optional[str] = None) -> bytes:
    """Wire v2 plan of `index_select(source, indices, axis 0)` followed by an
    optional cast to `result_dtype` (the reference exporter's
    `reloc.index_select` [+ `reloc.cast`] chain, test/dialect/reloc/
    indexed_export.mlir). Extents are ints or symbol names; `count` is the
    index operand's extent. Symbols are numbered by first use: source, then
    indices, then result."""
    result_dtype = result_dtype or source_dtype
    policy = _INDEXED_PAIRS.get((source_dtype, result_dtype))
    if policy is None:
        raise EncodeError("indexed plans cast only f32 -> f16 and f16 -> f32 "
                          "(or keep f32, f16, i8): %s -> %s" % (source_dtype, result_dtype))
    if index_dtype not in ("int32", "int64"):
        raise EncodeError("indices must be int32 or int64, got %s" % index_dtype)
    src = [expr(x) for x in source_shape]
    if not src:
        raise EncodeError("index_select needs a source of rank >= 1")
    for e in src + [expr(count)]:
        if e.is_const() and e.value <= 0:
            raise EncodeError("indexed plan extents must be positive")
    ind = [expr(count)]
    res = ind + src[1:]
    symbols: List[str] = []

    def note(e: E):
        if e.kind == "sym":
            if e.value not in symbols:
                symbols.append(e.value)
        elif e.kind not in ("const", "dim"):
            note(e.a)
            note(e.b)

    for e in src + ind + res:
        note(e)
    w = _Writer(symbols)
    w.out += b"RPLN"
    w.u32(2)
    w.u32(len(symbols))
    for name in symbols:
        w.str(name)
    w.desc(src, source_dtype)
    w.desc(ind, index_dtype)
    w.desc(res, result_dtype)
    w.u32(0)  # axis
    w.u8(POLICIES[policy])
    return bytes(w.out)
