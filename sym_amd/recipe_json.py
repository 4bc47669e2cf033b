"""Recipes in the reference's JSON form (the `recipe` object of a `.reloc`
artifact, libreloc/python/reloc_torch/artifact.py:816-900) -> encoder ops."""
from . import encoder as EN


def dim(v):
    """["const", n] | ["symbol", name] | nested ["floordiv"/"mul"/"add"...]."""
    if isinstance(v, (int, str)):
        return EN.expr(v)
    tag = v[0]
    if tag == "const":
        return EN.E.c(v[1])
    if tag == "symbol":
        return EN.E.s(v[1])
    a, b = dim(v[1]), dim(v[2])
    return {"floordiv": EN.floordiv, "mul": EN.mul, "add": EN.add, "mod": EN.mod}[tag](a, b)


def _param(p):
    if p is None:
        return None
    if p["kind"] == "inline":
        return EN.InlineParam(values=(), dtype=p["dtype"], rank=len(p.get("shape", [])),
                              bits=tuple(int(b) for b in p["bits"]))
    return EN.BindingParam(p["name"], p["dtype"], tuple(dim(e) for e in p.get("extents", [])))


def ops(recipe):
    out = []
    for o in recipe["operations"]:
        k = o["kind"]
        if k == "transpose":
            out.append(EN.Transpose(tuple(o["perm"])))
        elif k == "reshape":
            out.append(EN.Reshape(tuple(dim(e) for e in o["shape"])))
        elif k == "pad":
            fill = o.get("fill") or {}
            out.append(EN.Pad(o["axis"], dim(o["lo"]), dim(o["hi"]), bits=fill.get("bits", 0)))
        elif k == "cast":
            out.append(EN.Cast(o["dtype"], o.get("policy", "ieee_rne")))
        elif k == "quantize":
            out.append(EN.Quantize(_param(o["scale"]), _param(o.get("zero_point")), o.get("axis"),
                                   o.get("policy", "symmetric_rne"), o.get("dtype", "int8")))
        elif k == "dequantize":
            out.append(EN.Dequantize(_param(o["scale"]), _param(o.get("zero_point")), o.get("axis"),
                                     o.get("policy", "affine"), o.get("dtype", "float32")))
        else:
            raise EN.EncodeError("unsupported recipe operation %r" % k)
    return out


def encode_recipe(recipe):
    src = recipe["source"]
    return EN.encode([dim(e) for e in src["shape"]], src["dtype"], ops(recipe))
