"""Compiled-plan artifacts (`.reloc` files) without the MLIR compiler.

An artifact is one JSON object (`format_version`, `manifest`, `plan_base64`,
`recipe`), serialized with sorted keys and compact separators plus a
newline, exactly as the reference's `CompiledRecipe.to_bytes` writes it
(libreloc/python/reloc_torch/artifact.py:219-262). Format 1 carries a
layout-only recipe over a wire v0 plan (manifest schema 1), format 2 a typed
recipe over a wire v1 plan (schema 2), format 3 an indexed recipe over a wire
v2 plan (schema 3).

* `compile_recipe(recipe)` is the writer: it folds the recipe into plan bytes
  with this package's encoder (sym_amd/encoder.py, byte-identical to the
  reference exporter on the corpus) and writes the manifest the exporter
  writes: symbols in wire order, the logical descriptors, divisibility
  constraints, typed stages, fills and parameter declarations, the plan's
  SHA-256 and the SHA-256 of the recipe's MLIR text (`emit_mlir`, the text
  the reference's frontend hands its compiler, mlir_emit.py:56-135).
* `CompiledArtifact.from_bytes` admits an artifact as the reference does
  (artifact.py:224-250, 706-762; indexed_artifact.py:46-92): exact keys,
  versions, compiler interface, symbols against the wire, the decoded plan
  and the recipe, descriptors and constraints against the recipe, typed
  sections against the recipe and the plan the native decoder read, and
  both digests.

The manifest names the compiler interface it follows (`sym-reloc-export`,
interface 1), the one the reference's loader admits; `build_identity` says
that this package's encoder wrote it.
"""
import base64
import hashlib
import json
from pathlib import Path

from . import encoder as EN

LAYOUT, TYPED, INDEXED = (1, 0), (2, 1), (3, 2)  # (schema_version, wire_version)
DEFAULT_COMPILER = {"name": "sym-reloc-export", "interface_version": 1, "llvm_version": "none",
                    "build_identity": "librelx encoder (sym_amd.encoder)"}
_TENSOR_DTYPES = ("float32", "float16", "bfloat16", "int8")
_WIDTHS = {"float32": 32, "float16": 16, "bfloat16": 16, "int8": 8, "int32": 32, "int64": 64}
_MLIR = {"float32": "f32", "float16": "f16", "bfloat16": "bf16", "int8": "i8", "int32": "i32",
         "int64": "i64"}
_TYPED_KINDS = ("cast", "quantize", "dequantize")


class ArtifactError(RuntimeError):
    """An artifact or recipe the loader refuses (the reference raises
    RuntimeError with these messages)."""


# ------------------------------------------------------------- expressions
#
# Expressions keep the artifact's JSON form as tuples: ("const", n),
# ("symbol", name), ("add", a, b), ("mul", a, b), ("floordiv", a, n),
# ("mod", a, n); channel maps add ("dim", k) and expression divisors.

def _c(v):
    return ("const", int(v))


def _tuple(v):
    return tuple(_tuple(x) if isinstance(x, list) else x for x in v)


def _list(e):
    return [_list(x) if isinstance(x, tuple) else x for x in e]


def _int(v, where):
    if type(v) is not int:
        raise ArtifactError("compiler manifest %s must be an integer" % where)
    return v


def _str(v, where):
    if type(v) is not str or not v:
        raise ArtifactError("compiler manifest %s must be a nonempty string" % where)
    return v


def _keys(v, expected, where):
    if type(v) is not dict or set(v) != set(expected):
        raise ArtifactError("compiler manifest has invalid %s fields" % where)


def parse_expr(v, where):
    """A shape expression of the artifact grammar (artifact.py:340-361)."""
    if type(v) is not list or not v or type(v[0]) is not str:
        raise ArtifactError("compiler manifest %s has invalid expression" % where)
    tag = v[0]
    if tag == "const" and len(v) == 2:
        return _c(_int(v[1], where))
    if tag == "symbol" and len(v) == 2:
        name = _str(v[1], where)
        if not name.isidentifier() or not name.isascii():
            raise ArtifactError("compiler manifest %s has invalid expression" % where)
        return ("symbol", name)
    if tag in ("add", "mul") and len(v) == 3:
        return (tag, parse_expr(v[1], where), parse_expr(v[2], where))
    if tag in ("floordiv", "mod") and len(v) == 3:
        d = _int(v[2], where)
        if d <= 0:
            raise ArtifactError("compiler manifest %s has nonpositive divisor" % where)
        return (tag, parse_expr(v[1], where), d)
    raise ArtifactError("compiler manifest %s has unsupported expression" % where)


def _repr(e):
    """The reference frontend's dataclass repr of an expression; its
    commutative normal form orders terms by it (symbolic.py:135-160)."""
    tag = e[0]
    if tag == "const":
        return "Const(value=%d)" % e[1]
    if tag == "symbol":
        return "Symbol(name=%r)" % e[1]
    if tag in ("add", "mul"):
        return "%s(lhs=%s, rhs=%s)" % ("Add" if tag == "add" else "Mul", _repr(e[1]), _repr(e[2]))
    return "%s(lhs=%s, divisor=%d)" % ("FloorDiv" if tag == "floordiv" else "Mod", _repr(e[1]), e[2])


def _commutative(tag, a, b):
    """Flatten nested `tag` nodes, fold their constants, order the remaining
    terms by repr and rebuild left-nested."""
    terms, const = [], 0 if tag == "add" else 1

    def collect(x):
        nonlocal const
        if x[0] == tag:
            collect(x[1])
            collect(x[2])
        elif x[0] == "const":
            const = const + x[1] if tag == "add" else const * x[1]
        else:
            terms.append(x)

    collect(a)
    collect(b)
    if tag == "mul" and const == 0:
        return _c(0)
    if const != (0 if tag == "add" else 1) or not terms:
        terms.append(_c(const))
    terms.sort(key=_repr)
    out = terms[0]
    for t in terms[1:]:
        out = (tag, out, t)
    return out


def cadd(a, b):
    return _commutative("add", a, b)


def cmul(a, b):
    return _commutative("mul", a, b)


_I64 = (-(1 << 63), 1 << 63)


def evaluate(e, bindings, checked=True):
    def ev(x):
        tag = x[0]
        if tag == "const":
            r = x[1]
        elif tag == "symbol":
            r = bindings[x[1]]
        elif tag == "add":
            r = ev(x[1]) + ev(x[2])
        elif tag == "mul":
            r = ev(x[1]) * ev(x[2])
        elif tag == "floordiv":
            r = ev(x[1]) // x[2]
        else:
            r = ev(x[1]) % x[2]
        if checked and not _I64[0] <= r < _I64[1]:
            raise OverflowError("integer_overflow")
        return r
    return ev(e)


def normalize(e):
    """The reference's normal form for comparing expressions
    (artifact.py:364-390): constants folded where they fold without
    overflow, commutative terms ordered."""
    def fold(x):
        try:
            return _c(evaluate(x, {}))
        except (KeyError, OverflowError):
            return x
    tag = e[0]
    if tag in ("add", "mul"):
        a, b = normalize(e[1]), normalize(e[2])
        cand = fold((tag, a, b))
        return cand if cand[0] == "const" else (cadd(a, b) if tag == "add" else cmul(a, b))
    if tag == "floordiv":
        a = normalize(e[1])
        return a if e[2] == 1 else fold(("floordiv", a, e[2]))
    if tag == "mod":
        a = normalize(e[1])
        return _c(0) if e[2] == 1 else fold(("mod", a, e[2]))
    return e


def same_exprs(a, b):
    return len(a) == len(b) and all(normalize(x) == normalize(y) for x, y in zip(a, b))


def dense_strides(shape):
    """Row-major strides in the frontend's normal form (symbolic.py:175-180)."""
    out, running = [], _c(1)
    for d in reversed(shape):
        out.append(running)
        running = cmul(d, running)
    return tuple(reversed(out))


def _manifest_strides(shape):
    """Row-major strides as the exporter writes them into a manifest: the
    innermost is 1, each outer one the product of the next extent and its
    stride, written unfolded (a stride of 1 leaves the extent alone)."""
    out = [_c(1)]
    for d in reversed(shape[1:]):
        inner = out[0]
        out.insert(0, d if inner == _c(1) else ("mul", d, inner))
    return out


def _to_encoder(e):
    tag = e[0]
    if tag == "const":
        return EN.E.c(e[1])
    if tag == "symbol":
        return EN.E.s(e[1])
    a = _to_encoder(e[1])
    b = EN.E.c(e[2]) if tag in ("floordiv", "mod") else _to_encoder(e[2])
    return {"add": EN.add, "mul": EN.mul, "floordiv": EN.floordiv, "mod": EN.mod}[tag](a, b)


def _from_encoder(e, divisor_exprs=False):
    """An encoder expression in the JSON grammar; channel maps keep
    coordinates ("dim", k) and may divide by expressions; a subtraction
    reads as lhs + (-1 * rhs)."""
    k = e.kind
    if k == "const":
        return _c(e.value)
    if k == "sym":
        return ("symbol", e.value)
    if k == "dim":
        return ("dim", e.value)
    a, b = _from_encoder(e.a, divisor_exprs), _from_encoder(e.b, divisor_exprs)
    if k == "sub":
        return ("add", a, ("mul", _c(-1), b))
    if k in ("floordiv", "mod") and not divisor_exprs:
        if b[0] != "const":
            raise ArtifactError("a shape divisor must be a constant")
        return (k, a, b[1])
    return (k, a, b)


# ------------------------------------------------------------ the recipe

def _descriptor(v, where, index=False):
    _keys(v, ("shape", "strides", "offset", "dtype"), where)
    if type(v["shape"]) is not list or type(v["strides"]) is not list:
        raise ArtifactError("compiler manifest %s shape/strides must be arrays" % where)
    if not v["shape"] or len(v["shape"]) != len(v["strides"]):
        raise ArtifactError("compiler manifest %s has invalid rank" % where)
    dtype = _str(v["dtype"], where + ".dtype")
    if dtype not in (("int32", "int64") if index else _TENSOR_DTYPES):
        raise ArtifactError("compiler manifest %s has unsupported dtype" % where)
    return {"shape": tuple(parse_expr(x, where + ".shape") for x in v["shape"]),
            "strides": tuple(parse_expr(x, where + ".strides") for x in v["strides"]),
            "offset": parse_expr(v["offset"], where + ".offset"), "dtype": dtype}


def _same_descriptor(a, b):
    return (a["dtype"] == b["dtype"] and same_exprs(a["shape"], b["shape"])
            and same_exprs(a["strides"], b["strides"])
            and normalize(a["offset"]) == normalize(b["offset"]))


def _param(v, where, manifest):
    """An inline or binding stage parameter; a manifest writes inline bits
    as lowercase hex, a recipe as integers."""
    if v is None:
        return None
    if type(v) is not dict or type(v.get("kind")) is not str:
        raise ArtifactError("compiled recipe has invalid %s" % where)
    if v["kind"] == "inline":
        _keys(v, ("kind", "dtype", "shape", "bits"), where)
        if type(v["shape"]) is not list or type(v["bits"]) is not list:
            raise ArtifactError("compiled recipe %s shape/bits must be arrays" % where)
        bits = tuple(_hex(b, where) if manifest else _int(b, where) for b in v["bits"])
        return {"kind": "inline", "dtype": _str(v["dtype"], where),
                "shape": tuple(_int(s, where) for s in v["shape"]), "bits": bits}
    if v["kind"] == "binding":
        _keys(v, ("kind", "name", "dtype", "extents"), where)
        if type(v["extents"]) is not list:
            raise ArtifactError("compiled recipe %s extents must be an array" % where)
        return {"kind": "binding", "name": _str(v["name"], where), "dtype": _str(v["dtype"], where),
                "extents": tuple(parse_expr(x, where) for x in v["extents"])}
    raise ArtifactError("compiled recipe has unsupported %s kind" % where)


def _hex(v, where):
    if (type(v) is not str or not v or len(v) > 16
            or any(c not in "0123456789abcdef" for c in v)):
        raise ArtifactError("compiler manifest %s bits must be lowercase hex" % where)
    return int(v, 16)


def _same_param(a, b):
    if a is None or b is None:
        return a is None and b is None
    if a["kind"] != b["kind"] or a["dtype"] != b["dtype"]:
        return False
    if a["kind"] == "inline":
        return a["shape"] == b["shape"] and a["bits"] == b["bits"]
    return a["name"] == b["name"] and same_exprs(a["extents"], b["extents"])


class Recipe:
    """A validated recipe in the artifact's JSON form (the reference's
    _decode_recipe, artifact.py:880-961). `json` keeps the object as given,
    so an admitted artifact serializes back to the same bytes."""

    def __init__(self, obj):
        _keys(obj, ("source", "operations", "destination", "direction"), "recipe")
        if type(obj["operations"]) is not list:
            raise ArtifactError("compiled recipe operations must be an array")
        self.direction = _str(obj["direction"], "recipe.direction")
        if self.direction not in ("h2d", "d2h"):
            raise ArtifactError("compiled recipe has unsupported direction")
        self.ops = [self._op(o) for o in obj["operations"]]
        self.source = _descriptor(obj["source"], "recipe.source")
        self.destination = _descriptor(obj["destination"], "recipe.destination")
        self.json = obj

    @staticmethod
    def _op(o):
        if type(o) is not dict or type(o.get("kind")) is not str:
            raise ArtifactError("compiled recipe has invalid operation")
        k = o["kind"]
        if k == "index_select":
            _keys(o, ("kind", "axis", "indices"), "index_select")
            return {"kind": k, "axis": _int(o["axis"], "index_select axis"),
                    "indices": _descriptor(o["indices"], "indices", index=True)}
        if k == "transpose":
            _keys(o, ("kind", "perm"), "transpose")
            if type(o["perm"]) is not list:
                raise ArtifactError("compiled recipe transpose perm must be an array")
            return {"kind": k, "perm": tuple(_int(a, "transpose axis") for a in o["perm"])}
        if k == "reshape":
            _keys(o, ("kind", "shape"), "reshape")
            if type(o["shape"]) is not list:
                raise ArtifactError("compiled recipe reshape shape must be an array")
            return {"kind": k, "shape": tuple(parse_expr(d, "reshape shape") for d in o["shape"])}
        if k == "pad":
            _keys(o, ("kind", "axis", "lo", "hi", "fill"), "pad")
            _keys(o["fill"], ("dtype", "bits"), "fill")
            dtype = _str(o["fill"]["dtype"], "fill dtype")
            bits = _int(o["fill"]["bits"], "fill bits")
            if dtype not in _TENSOR_DTYPES or not 0 <= bits < 1 << _WIDTHS[dtype]:
                raise ArtifactError("compiled recipe has invalid operation")
            return {"kind": k, "axis": _int(o["axis"], "pad axis"), "lo": parse_expr(o["lo"], "pad lo"),
                    "hi": parse_expr(o["hi"], "pad hi"), "fill": (dtype, bits)}
        if k == "cast":
            _keys(o, ("kind", "dtype", "policy"), "cast")
            return {"kind": k, "dtype": _str(o["dtype"], "cast dtype"),
                    "policy": _str(o["policy"], "cast policy")}
        if k in ("quantize", "dequantize"):
            _keys(o, ("kind", "dtype", "policy", "axis", "scale", "zero_point"), k)
            axis = o["axis"]
            if axis is not None:
                axis = _int(axis, k + " axis")
            return {"kind": k, "dtype": _str(o["dtype"], k + " dtype"),
                    "policy": _str(o["policy"], k + " policy"), "axis": axis,
                    "scale": _param(o["scale"], k + " scale", False),
                    "zero_point": _param(o["zero_point"], k + " zero_point", False)}
        raise ArtifactError("compiled recipe has unsupported operation")

    @property
    def typed(self):
        return any(o["kind"] in _TYPED_KINDS for o in self.ops)

    @property
    def indexed(self):
        return any(o["kind"] == "index_select" for o in self.ops)

    @property
    def format_version(self):
        return 3 if self.indexed else 2 if self.typed else 1

    @property
    def parameter_bindings(self):
        """Runtime parameters in first-declaration order, one per name
        (recipe.py:181-188)."""
        seen = []
        for o in self.ops:
            for p in (o.get("scale"), o.get("zero_point")):
                if p and p["kind"] == "binding" and all(q["name"] != p["name"] for q in seen):
                    seen.append(p)
        return seen

    def symbols(self):
        """Every symbol the recipe names (artifact.py:417-442)."""
        names = set()

        def visit(e):
            if e[0] == "symbol":
                names.add(e[1])
            elif e[0] in ("add", "mul"):
                visit(e[1])
                visit(e[2])
            elif e[0] in ("floordiv", "mod"):
                visit(e[1])

        for d in (self.source, self.destination):
            for e in (*d["shape"], *d["strides"], d["offset"]):
                visit(e)
        for o in self.ops:
            if o["kind"] == "reshape":
                for e in o["shape"]:
                    visit(e)
            elif o["kind"] == "pad":
                visit(o["lo"])
                visit(o["hi"])
            elif o["kind"] in _TYPED_KINDS:
                for p in (o.get("scale"), o.get("zero_point")):
                    if p and p["kind"] == "binding":
                        for e in p["extents"]:
                            visit(e)
        return names

    def expected_constraints(self):
        """Divisibility the reshapes' floor divisions need at bind time
        (artifact.py:461-487)."""
        out = []

        def visit(e):
            if e[0] == "floordiv":
                lhs = normalize(e[1])
                if e[2] != 1 and lhs[0] != "const" and (lhs, e[2]) not in out:
                    out.append((lhs, e[2]))
                visit(e[1])
            elif e[0] in ("add", "mul"):
                visit(e[1])
                visit(e[2])
            elif e[0] == "mod":
                visit(e[1])

        for o in self.ops:
            if o["kind"] == "reshape":
                for e in o["shape"]:
                    visit(e)
        return out


def operation_shape(shape, op):
    """The logical shape after one operation (symbolic.py:201-221)."""
    k = op["kind"]
    if k in _TYPED_KINDS:
        return tuple(shape)
    if k == "index_select":
        return (op["indices"]["shape"][0],) + tuple(shape[1:])
    if k == "transpose":
        if sorted(op["perm"]) != list(range(len(shape))):
            raise ArtifactError("unsupported_symbolic_expr: invalid permutation")
        return tuple(shape[i] for i in op["perm"])
    if k == "reshape":
        return tuple(op["shape"])
    if not 0 <= op["axis"] < len(shape):
        raise ArtifactError("unsupported_symbolic_expr: invalid padding axis")
    out = list(shape)
    out[op["axis"]] = cadd(cadd(shape[op["axis"]], op["lo"]), op["hi"])
    return tuple(out)


# ------------------------------------------------------------------- MLIR

def _mexpr(e, quoted=False):
    tag = e[0]
    if tag == "const":
        return str(e[1])
    if tag == "symbol":
        return '"%s"' % e[1] if quoted else e[1]
    if tag in ("add", "mul"):
        return "(%s %s %s)" % (_mexpr(e[1], quoted), "+" if tag == "add" else "*", _mexpr(e[2], quoted))
    return "(%s %s %d)" % (_mexpr(e[1], quoted), tag, e[2])


def _mshape(shape, quoted=False):
    return "[" + ", ".join(_mexpr(d, quoted) for d in shape) + "]"


def _mtype(shape, dtype):
    return "!sym.tensor<%s, %s>" % (_mshape(shape, True), _MLIR[dtype])


def _mliteral(bits, dtype):
    width = _WIDTHS[dtype]
    if dtype.startswith("int"):
        return str(bits if bits < 1 << (width - 1) else bits - (1 << width))
    return "0x%0*X" % (width // 4, bits)


def _mparam(p):
    if p["kind"] == "binding":
        return '#reloc.binding<"%s" : %s, %s>' % (p["name"], _mshape(p["extents"]), _MLIR[p["dtype"]])
    values = [_mliteral(b, p["dtype"]) for b in p["bits"]]
    if p["shape"]:
        return "dense<[%s]> : tensor<%dx%s>" % (", ".join(values), p["shape"][0], _MLIR[p["dtype"]])
    return "dense<%s> : tensor<%s>" % (values[0], _MLIR[p["dtype"]])


def emit_mlir(recipe):
    """The reloc IR text of a recipe: one function from the dense source to
    the destination's logical shape, an op per recipe operation. Its SHA-256
    is the manifest's `input_sha256`."""
    src, dst = recipe.source, recipe.destination
    if src["dtype"] not in _TENSOR_DTYPES or dst["dtype"] not in _TENSOR_DTYPES:
        raise ArtifactError("unsupported_symbolic_expr: unsupported dtype")
    if not recipe.typed and src["dtype"] != dst["dtype"]:
        raise ArtifactError("unsupported_symbolic_expr: unsupported or changed dtype")
    for d, name in ((src, "source"), (dst, "destination")):
        if d["offset"] != _c(0) or tuple(d["strides"]) != dense_strides(d["shape"]):
            raise ArtifactError("unsupported_symbolic_expr: %s_layout: expected dense "
                                "zero-offset tensor" % name)
    current, dtype = src["shape"], src["dtype"]
    index_type = None
    if recipe.indexed:
        ops = recipe.ops
        if (ops[0]["kind"] != "index_select" or len(ops) > 2
                or any(o["kind"] != "cast" for o in ops[1:])):
            raise ArtifactError("unsupported_symbolic_expr: index_select must precede at most "
                                "one cast")
        ix = ops[0]["indices"]
        if tuple(ix["strides"]) != dense_strides(ix["shape"]) or ix["offset"] != _c(0):
            raise ArtifactError("unsupported_symbolic_expr: index operand must describe a dense "
                                "snapshot")
        index_type = _mtype(ix["shape"], ix["dtype"])
    extra = "" if index_type is None else ", %%indices: %s" % index_type
    lines = ["func.func @torch_relocation(%%x: %s%s) -> %s {" % (
        _mtype(current, dtype), extra, _mtype(dst["shape"], dst["dtype"]))]
    value = "%x"
    ops = recipe.ops or [{"kind": "transpose", "perm": tuple(range(len(current)))}]
    for i, op in enumerate(ops):
        target = operation_shape(current, op)
        tdtype = op["dtype"] if op["kind"] in _TYPED_KINDS else dtype
        k = op["kind"]
        if k == "index_select":
            text = "reloc.index_select %s, %%indices axis %d" % (value, op["axis"])
        elif k == "transpose":
            text = "reloc.transpose %s perm [%s]" % (value, ", ".join(map(str, op["perm"])))
        elif k == "reshape":
            text = "reloc.reshape %s to %s" % (value, _mshape(target))
        elif k == "pad":
            fd, fb = op["fill"]
            text = "reloc.pad %s axis %d lo %s hi %s value (%s : %s)" % (
                value, op["axis"], _mexpr(op["lo"]), _mexpr(op["hi"]), _mliteral(fb, fd), _MLIR[fd])
        elif k == "cast":
            text = "reloc.cast %s policy %s" % (value, op["policy"])
        else:
            text = "reloc.%s %s" % (k, value)
            if op["axis"] is not None:
                text += " axis %d" % op["axis"]
            text += " scale(%s)" % _mparam(op["scale"])
            if op["zero_point"] is not None:
                text += " zero_point(%s)" % _mparam(op["zero_point"])
            text += " policy %s" % op["policy"]
        operand = ", " + index_type if k == "index_select" else ""
        lines.append("  %%v%d = %s : %s%s -> %s" % (i, text, _mtype(current, dtype), operand,
                                                     _mtype(target, tdtype)))
        value, current, dtype = "%%v%d" % i, target, tdtype
    if dtype != dst["dtype"]:
        raise ArtifactError("unsupported_symbolic_expr: destination dtype does not match the chain")
    lines.append("  return %s : %s" % (value, _mtype(dst["shape"], dst["dtype"])))
    lines.append("}")
    return "\n".join(lines) + "\n"


# ------------------------------------------------------------- the writer

def _jparam(p):
    if p is None:
        return None
    if p["kind"] == "inline":
        return {"bits": ["%x" % b for b in p["bits"]], "dtype": p["dtype"], "kind": "inline",
                "shape": list(p["shape"])}
    return {"dtype": p["dtype"], "extents": [_list(e) for e in p["extents"]], "kind": "binding",
            "name": p["name"]}


def _jdescriptor(d):
    return {"dtype": d["dtype"], "offset": ["const", 0], "shape": [_list(e) for e in d["shape"]],
            "strides": [_list(e) for e in _manifest_strides(d["shape"])]}


def _encoder_ops(recipe):
    out = []
    for o in recipe.ops:
        k = o["kind"]
        if k == "transpose":
            out.append(EN.Transpose(o["perm"]))
        elif k == "reshape":
            out.append(EN.Reshape(tuple(_to_encoder(e) for e in o["shape"])))
        elif k == "pad":
            out.append(EN.Pad(o["axis"], _to_encoder(o["lo"]), _to_encoder(o["hi"]), bits=o["fill"][1]))
        elif k == "cast":
            out.append(EN.Cast(o["dtype"], o["policy"]))
        elif k in ("quantize", "dequantize"):
            def param(p):
                if p is None:
                    return None
                if p["kind"] == "inline":
                    return EN.InlineParam((), p["dtype"], len(p["shape"]), p["bits"])
                return EN.BindingParam(p["name"], p["dtype"],
                                       tuple(_to_encoder(e) for e in p["extents"]))
            cls = EN.Quantize if k == "quantize" else EN.Dequantize
            out.append(cls(param(o["scale"]), param(o["zero_point"]), o["axis"], o["policy"],
                           o["dtype"]))
        else:
            raise ArtifactError("unsupported recipe operation %r" % k)
    return out


def _plan_for(recipe):
    src = recipe.source
    if recipe.indexed:
        sel = recipe.ops[0]
        if sel["axis"] != 0:
            raise ArtifactError("index_select runs along axis 0")
        ix = sel["indices"]["shape"][0]
        cast = recipe.ops[1]["dtype"] if len(recipe.ops) == 2 else src["dtype"]
        blob = EN.encode_index_select([_to_encoder(e) for e in src["shape"]], src["dtype"],
                                      _to_encoder(ix), sel["indices"]["dtype"], cast)
        return EN.Plan(blob, list(_wire_symbols(blob, 2)), False, [], [], src["dtype"], cast)
    return EN.encode([_to_encoder(e) for e in src["shape"]], src["dtype"], _encoder_ops(recipe))


def compile_recipe(recipe, compiler=None):
    """Fold a recipe (a `Recipe` or its JSON object) into an admitted
    artifact: plan bytes from this package's encoder and the manifest the
    exporter writes for them."""
    if not isinstance(recipe, Recipe):
        recipe = Recipe(recipe)
    try:
        plan = _plan_for(recipe)
    except EN.EncodeError as e:
        raise ArtifactError("unsupported_recipe: %s" % e) from e
    mlir = emit_mlir(recipe).encode("utf-8")
    schema = INDEXED if recipe.indexed else TYPED if recipe.typed else LAYOUT
    m = {"schema_version": schema[0], "wire_version": schema[1], "status": "ok",
         "compiler": dict(compiler or DEFAULT_COMPILER), "plan_count": 1,
         "symbols": list(plan.symbols),
         "logical_source": _jdescriptor(recipe.source),
         "logical_destination": _jdescriptor(recipe.destination),
         "constraints": {"divisibility": [
             {"divisor": d, "expr": _list(_from_encoder(e))} for e, d in plan.divisibility]},
         "plan_sha256": hashlib.sha256(plan.blob).hexdigest(),
         "input_sha256": hashlib.sha256(mlir).hexdigest()}
    if recipe.indexed:
        sel = recipe.ops[0]
        policy = recipe.ops[1]["policy"] if len(recipe.ops) == 2 else "exact"
        ix = sel["indices"]
        m["index_select"] = {"axis": sel["axis"], "policy": policy,
                             "indices": _jdescriptor(ix) | {"dtype": ix["dtype"]}}
    elif recipe.typed:
        stages, rank = [], len(recipe.destination["shape"])
        shape, dtype, si = recipe.source["shape"], recipe.source["dtype"], 0
        for o in recipe.ops:
            if o["kind"] in _TYPED_KINDS:
                st = plan.stages[si]
                axis = -1 if o["kind"] == "cast" or o["axis"] is None else o["axis"]
                stages.append({
                    "axis": axis,
                    "channel": None if st.channel is None else
                    {"dims": rank, "expr": _list(_from_encoder(st.channel, True))},
                    "input_dtype": dtype, "output_dtype": o["dtype"], "policy": o["policy"],
                    "scale": _jparam(o.get("scale")), "shape": [_list(e) for e in shape],
                    "transform": o["kind"], "zero_point": _jparam(o.get("zero_point"))})
                dtype = o["dtype"]
                si += 1
            shape = operation_shape(shape, o)
        m["stages"] = stages
        m["fills"] = [{"bits": "%x" % bits, "dst_axis": axis, "dtype": fdt, "stage": stage}
                      for axis, stage, fdt, bits in plan.fills]
        m["parameters"] = [{"dtype": p["dtype"], "extents": [_list(e) for e in p["extents"]],
                            "name": p["name"]} for p in recipe.parameter_bindings]
    return admit(recipe, plan.blob, json.loads(json.dumps(m)))


# ------------------------------------------------------------- admission

def _decoded(plan, typed, indexed):
    from . import pyreloc as P
    loader = P.load_indexed_plan if indexed else P.load_typed_plan if typed else P.load_plan
    try:
        return loader(plan)
    except P.DecodeError as e:
        raise ArtifactError("compiler published an invalid plan: %s" % e) from e


def _wire_symbols(plan, version):
    if len(plan) < 12 or plan[:4] != b"RPLN":
        raise ArtifactError("compiler plan has invalid wire header")
    if int.from_bytes(plan[4:8], "little") != version:
        raise ArtifactError("compiler plan wire version mismatch")
    count, off, names = int.from_bytes(plan[8:12], "little"), 12, []
    for _ in range(count):
        if off + 4 > len(plan):
            raise ArtifactError("compiler plan has truncated symbol table")
        n = int.from_bytes(plan[off:off + 4], "little")
        off += 4
        if off + n > len(plan):
            raise ArtifactError("compiler plan has truncated symbol name")
        try:
            name = plan[off:off + n].decode("utf-8")
        except UnicodeDecodeError as e:
            raise ArtifactError("compiler plan has invalid symbol name") from e
        if not name.isidentifier() or not name.isascii():
            raise ArtifactError("compiler plan has invalid symbol name")
        names.append(name)
        off += n
    if len(set(names)) != len(names):
        raise ArtifactError("compiler plan has duplicate symbols")
    return tuple(names)


def _compiler(m, schema):
    if _int(m.get("schema_version"), "schema_version") != schema[0]:
        raise ArtifactError("compiler manifest schema version mismatch")
    if _int(m.get("wire_version"), "wire_version") != schema[1]:
        raise ArtifactError("compiler manifest wire version mismatch")
    c = m.get("compiler")
    _keys(c, ("name", "interface_version", "llvm_version", "build_identity"), "compiler")
    ident = (_str(c["name"], "compiler.name"), _int(c["interface_version"], "compiler.interface_version"),
             _str(c["llvm_version"], "compiler.llvm_version"),
             _str(c["build_identity"], "compiler.build_identity"))
    if ident[0] != "sym-reloc-export" or ident[1] != 1:
        raise ArtifactError("compiler manifest identifies an unsupported compiler interface")
    return c


def _constraints(v):
    _keys(v, ("divisibility",), "constraints")
    if type(v["divisibility"]) is not list:
        raise ArtifactError("compiler manifest divisibility constraints must be an array")
    out = []
    for entry in v["divisibility"]:
        _keys(entry, ("expr", "divisor"), "divisibility constraint")
        d = _int(entry["divisor"], "constraint divisor")
        if d <= 0:
            raise ArtifactError("compiler manifest constraint divisor must be positive")
        out.append((normalize(parse_expr(entry["expr"], "constraint")), d))
    return out


def _channel_ok(v, dims, symbols, where):
    if type(v) is not list or not v or type(v[0]) is not str:
        raise ArtifactError("compiler manifest %s has invalid channel expression" % where)
    tag = v[0]
    if tag == "const" and len(v) == 2:
        _int(v[1], where)
    elif tag == "dim" and len(v) == 2:
        if not 0 <= _int(v[1], where) < dims:
            raise ArtifactError("compiler manifest %s channel dimension is out of range" % where)
    elif tag == "symbol" and len(v) == 2:
        if _str(v[1], where) not in symbols:
            raise ArtifactError("compiler manifest %s channel symbol is not a plan symbol" % where)
    elif tag in ("add", "mul", "floordiv", "mod") and len(v) == 3:
        _channel_ok(v[1], dims, symbols, where)
        _channel_ok(v[2], dims, symbols, where)
    else:
        raise ArtifactError("compiler manifest %s has unsupported channel expression" % where)


_STAGE_FIELDS = ("transform", "policy", "input_dtype", "output_dtype", "shape", "scale",
                 "zero_point", "axis", "channel")


def _typed_sections(recipe, m, symbols, decoded):
    """Stages, fills and parameter declarations against the recipe and the
    decoded plan (artifact.py:662-703)."""
    stages, fills, params = m["stages"], m["fills"], m["parameters"]
    if type(stages) is not list or type(fills) is not list or type(params) is not list:
        raise ArtifactError("compiler manifest typed sections must be arrays")
    typed_ops = [o for o in recipe.ops if o["kind"] in _TYPED_KINDS]
    if len(stages) != len(typed_ops) or decoded.num_stages != len(stages):
        raise ArtifactError("compiler manifest stage count does not match the recipe")
    rank = len(recipe.destination["shape"])
    dstages = decoded.stages
    shape, dtype, i = recipe.source["shape"], recipe.source["dtype"], 0
    for o in recipe.ops:
        if o["kind"] in _TYPED_KINDS:
            e, where = stages[i], "stage %d" % i
            _keys(e, _STAGE_FIELDS, where)
            t, pol = _str(e["transform"], where), _str(e["policy"], where)
            ind, outd = _str(e["input_dtype"], where), _str(e["output_dtype"], where)
            if t != o["kind"] or pol != o["policy"] or ind != dtype or outd != o["dtype"]:
                raise ArtifactError("compiler manifest %s does not match the recipe transform" % where)
            if type(e["shape"]) is not list or not same_exprs(
                    tuple(parse_expr(x, where) for x in e["shape"]), shape):
                raise ArtifactError("compiler manifest %s operand shape mismatch" % where)
            axis = _int(e["axis"], where)
            want_axis = -1 if o["kind"] == "cast" or o["axis"] is None else o["axis"]
            if axis != want_axis:
                raise ArtifactError("compiler manifest %s channel axis mismatch" % where)
            if (not _same_param(_param(e["scale"], where, True), o.get("scale"))
                    or not _same_param(_param(e["zero_point"], where, True), o.get("zero_point"))):
                raise ArtifactError("compiler manifest %s parameter mismatch" % where)
            ch = e["channel"]
            if want_axis < 0:
                if ch is not None:
                    raise ArtifactError("compiler manifest %s has a channel map without an axis" % where)
            else:
                _keys(ch, ("dims", "expr"), where + " channel")
                if _int(ch["dims"], where) != rank:
                    raise ArtifactError("compiler manifest %s channel rank is not the result rank"
                                        % where)
                _channel_ok(ch["expr"], rank, symbols, where)
            d = dstages[i]
            if (d["transform"], d["policy"], d["input"], d["output"], d["axis"], d["has_channel"]) != \
                    (t, pol, ind, outd, want_axis, want_axis >= 0):
                raise ArtifactError("compiler plan %s does not match the manifest" % where)
            dtype = o["dtype"]
            i += 1
        shape = operation_shape(shape, o)
    if dtype != recipe.destination["dtype"]:
        raise ArtifactError("compiled recipe chain dtype does not reach the destination dtype")
    pads = [o for o in recipe.ops if o["kind"] == "pad"]
    if len(fills) != len(pads) or decoded.fills != len(fills):
        raise ArtifactError("compiler manifest fill count does not match the recipe")
    got = []
    for f in fills:
        _keys(f, ("dst_axis", "stage", "dtype", "bits"), "fill")
        if not 0 <= _int(f["dst_axis"], "fill dst_axis") < rank:
            raise ArtifactError("compiler manifest fill axis is out of range")
        if not 0 <= _int(f["stage"], "fill stage") <= len(stages):
            raise ArtifactError("compiler manifest fill stage is out of range")
        got.append((_str(f["dtype"], "fill dtype"), _hex(f["bits"], "fill")))
    if sorted(got) != sorted(p["fill"] for p in pads):
        raise ArtifactError("compiler manifest fills do not match the recipe pads")
    declared = []
    for e in params:
        _keys(e, ("name", "dtype", "extents"), "parameter")
        if type(e["extents"]) is not list:
            raise ArtifactError("compiler manifest parameter extents must be an array")
        declared.append((_str(e["name"], "parameter name"), _str(e["dtype"], "parameter dtype"),
                         tuple(parse_expr(x, "parameter extents") for x in e["extents"])))
    want = recipe.parameter_bindings
    if len(declared) != len(want) or any(
            d[0] != w["name"] or d[1] != w["dtype"] or not same_exprs(d[2], w["extents"])
            for d, w in zip(declared, want)):
        raise ArtifactError("compiler manifest parameters do not match the recipe bindings")
    runtime = [(p["name"], p["dtype"], p["rank"]) for p in decoded.parameters]
    if runtime != [(d[0], d[1], len(d[2])) for d in declared]:
        raise ArtifactError("compiler plan parameters do not match the manifest")
    return declared


def _admit_indexed(recipe, mlir, plan, m):
    _keys(m, ("schema_version", "wire_version", "status", "compiler", "plan_count", "symbols",
              "logical_source", "logical_destination", "constraints", "index_select",
              "plan_sha256", "input_sha256"), "indexed manifest")
    compiler = _compiler(m, INDEXED)
    if m["status"] != "ok" or _int(m["plan_count"], "plan_count") != 1:
        raise ArtifactError("indexed manifest must describe exactly one plan")
    ops = recipe.ops
    if ops[0]["kind"] != "index_select" or len(ops) > 2 or any(o["kind"] != "cast" for o in ops[1:]):
        raise ArtifactError("unsupported indexed recipe chain")
    sel, entry = ops[0], m["index_select"]
    _keys(entry, ("axis", "indices", "policy"), "index_select")
    policy = ops[1]["policy"] if len(ops) == 2 else "exact"
    if _int(entry["axis"], "index_select axis") != sel["axis"] or entry["policy"] != policy:
        raise ArtifactError("indexed manifest selection/policy mismatch")
    declared = (_descriptor(m["logical_source"], "logical_source"),
                _descriptor(entry["indices"], "indices", index=True),
                _descriptor(m["logical_destination"], "logical_destination"))
    if any(not _same_descriptor(a, b) for a, b in
           zip(declared, (recipe.source, sel["indices"], recipe.destination))):
        raise ArtifactError("indexed manifest descriptor mismatch")
    if _constraints(m["constraints"]):
        raise ArtifactError("unexpected indexed constraints")
    if (m["plan_sha256"] != hashlib.sha256(plan).hexdigest()
            or m["input_sha256"] != hashlib.sha256(mlir).hexdigest()):
        raise ArtifactError("indexed artifact digest mismatch")
    decoded = _decoded(plan, False, True)
    symbols = m["symbols"]
    if (type(symbols) is not list or any(type(s) is not str for s in symbols)
            or tuple(symbols) != _wire_symbols(plan, 2) or symbols != list(decoded.symbols)):
        raise ArtifactError("indexed manifest symbol table mismatch")
    meta = decoded.metadata
    if meta["axis"] != entry["axis"] or meta["policy"] != entry["policy"]:
        raise ArtifactError("indexed wire selection/policy mismatch")
    for key, want in zip(("source", "indices", "result"), declared):
        shape = tuple(parse_expr(d, key) for d in meta[key]["shape"])
        got = {"shape": shape, "strides": dense_strides(shape), "offset": _c(0),
               "dtype": meta[key]["dtype"]}
        if not _same_descriptor(got, want):
            raise ArtifactError("indexed wire %s descriptor mismatch" % key)
    return compiler, ()


def admit(recipe, plan, manifest):
    """Admit plan bytes and a manifest for a recipe (artifact.py:706-762)."""
    if not isinstance(recipe, Recipe):
        recipe = Recipe(recipe)
    if type(manifest) is not dict:
        raise ArtifactError("compiler manifest must be an object")
    mlir = emit_mlir(recipe).encode("utf-8")
    if recipe.indexed:
        compiler, params = _admit_indexed(recipe, mlir, plan, manifest)
        return CompiledArtifact(recipe, plan, manifest, compiler, params)
    typed = recipe.typed
    schema = TYPED if typed else LAYOUT
    fields = ("schema_version", "wire_version", "status", "compiler", "plan_count", "symbols",
              "logical_source", "logical_destination", "constraints", "plan_sha256",
              "input_sha256") + (("stages", "fills", "parameters") if typed else ())
    _keys(manifest, fields, "success")
    compiler = _compiler(manifest, schema)
    if manifest["status"] != "ok" or _int(manifest["plan_count"], "plan_count") != 1:
        raise ArtifactError("compiler manifest does not describe exactly one successful plan")
    symbols = manifest["symbols"]
    if type(symbols) is not list or any(type(s) is not str for s in symbols):
        raise ArtifactError("compiler manifest symbols must be an array of strings")
    symbols = tuple(symbols)
    decoded = _decoded(plan, typed, False)
    if symbols != _wire_symbols(plan, schema[1]) or symbols != tuple(decoded.symbols):
        raise ArtifactError("compiler manifest symbol order does not match the plan")
    if len(set(symbols)) != len(symbols) or set(symbols) != recipe.symbols():
        raise ArtifactError("compiler manifest symbol set does not match the recipe")
    if not _same_descriptor(_descriptor(manifest["logical_source"], "logical_source"),
                            recipe.source):
        raise ArtifactError("compiler manifest logical source descriptor mismatch")
    if not _same_descriptor(_descriptor(manifest["logical_destination"], "logical_destination"),
                            recipe.destination):
        raise ArtifactError("compiler manifest logical destination descriptor mismatch")
    if sorted(_constraints(manifest["constraints"]), key=repr) != sorted(
            recipe.expected_constraints(), key=repr):
        raise ArtifactError("compiler manifest constraints mismatch")
    params = _typed_sections(recipe, manifest, symbols, decoded) if typed else ()
    if _str(manifest["plan_sha256"], "plan_sha256") != hashlib.sha256(plan).hexdigest():
        raise ArtifactError("compiler manifest plan digest mismatch")
    if _str(manifest["input_sha256"], "input_sha256") != hashlib.sha256(mlir).hexdigest():
        raise ArtifactError("compiler manifest input digest mismatch")
    return CompiledArtifact(recipe, plan, manifest, compiler, params)


class CompiledArtifact:
    """An admitted artifact (the reference's CompiledRecipe): the recipe, the
    plan bytes and the manifest, with the portable serialization."""

    def __init__(self, recipe, plan_bytes, manifest, compiler, parameters):
        self.recipe = recipe
        self.plan_bytes = bytes(plan_bytes)
        self.manifest = manifest
        self.compiler = compiler
        self.parameters = tuple(parameters)

    typed = property(lambda self: self.recipe.typed or self.recipe.indexed and len(self.recipe.ops) > 1)
    indexed = property(lambda self: self.recipe.indexed)
    wire_version = property(lambda self: self.manifest["wire_version"])
    symbols = property(lambda self: tuple(self.manifest["symbols"]))
    format_version = property(lambda self: self.recipe.format_version)

    def load_plan(self):
        """The plan decoded by the native library (pyreloc's loader for its
        wire version)."""
        return _decoded(self.plan_bytes, self.recipe.typed and not self.indexed, self.indexed)

    def bind_symbols(self, source_shape):
        """Wire-symbol values from a concrete source shape: each symbol the
        source descriptor names takes that axis' extent (the same symbol on
        several axes must agree), then the divisibility constraints hold."""
        shape = self.recipe.source["shape"]
        if len(source_shape) != len(shape):
            raise ArtifactError("source_descriptor")
        values = {}
        for e, n in zip(shape, source_shape):
            if e[0] == "const":
                if e[1] != n:
                    raise ArtifactError("source_descriptor")
            elif e[0] == "symbol":
                if values.setdefault(e[1], int(n)) != n:
                    raise ArtifactError("source_descriptor")
        for c in self.manifest.get("constraints", {}).get("divisibility", []):
            if evaluate(parse_expr(c["expr"], "constraint"), values) % c["divisor"]:
                raise ArtifactError("divisibility")
        return {name: values[name] for name in self.symbols}

    def parameter_extents(self, symbols):
        """{name: (dtype, extents)} of each declared runtime parameter under
        bound wire symbols (artifact.py:199-210)."""
        return {name: (dtype, tuple(evaluate(e, symbols) for e in extents))
                for name, dtype, extents in self.parameters}

    def to_bytes(self):
        payload = {"format_version": self.format_version, "manifest": self.manifest,
                   "plan_base64": base64.b64encode(self.plan_bytes).decode("ascii"),
                   "recipe": self.recipe.json}
        return (json.dumps(payload, sort_keys=True, separators=(",", ":")) + "\n").encode("utf-8")

    @classmethod
    def from_bytes(cls, data):
        try:
            payload = json.loads(bytes(data))
        except (TypeError, UnicodeDecodeError, json.JSONDecodeError) as e:
            raise ArtifactError("malformed compiled recipe serialization") from e
        _keys(payload, ("format_version", "manifest", "plan_base64", "recipe"), "artifact")
        version = _int(payload["format_version"], "artifact format_version")
        if version not in (1, 2, 3):
            raise ArtifactError("compiled recipe format version mismatch")
        if type(payload["plan_base64"]) is not str:
            raise ArtifactError("compiled recipe plan_base64 must be a string")
        try:
            plan = base64.b64decode(payload["plan_base64"], validate=True)
        except ValueError as e:
            raise ArtifactError("compiled recipe has invalid plan bytes") from e
        recipe = Recipe(payload["recipe"])
        if version != recipe.format_version:
            raise ArtifactError("compiled recipe format version does not match its recipe")
        return admit(recipe, plan, payload["manifest"])

    def save(self, path):
        Path(path).write_bytes(self.to_bytes())

    @classmethod
    def load(cls, path):
        try:
            data = Path(path).read_bytes()
        except OSError as e:
            raise ArtifactError("unable to read compiled recipe") from e
        return cls.from_bytes(data)
