"""Block-permute plans ([B, S, H, D] -> [B, H, S, D] with value stages) that
take the direct permute body or keep the general one.

The direct body (power-of-two H*D, D and store runs; the parameter stage,
if any, per tensor or per channel along H) indexes with shifts and takes a
vector's parameters from its own H coordinate. Every other permute derives
the channel from the dense result offset. Used by the CPU launch checks
(which body each plan gets; every launch verified) and by the GPU parity
test against the oracle.
"""
import numpy as np

from sym_amd import encoder as EN


def _per(n, rng, lo=0.004, hi=0.05):
    return EN.InlineParam(tuple(float(v) for v in rng.uniform(lo, hi, n)), "float32", 1)


def _zp(n, rng):
    return EN.InlineParam(tuple(int(v) for v in rng.integers(-9, 10, n)), "int32", 1)


def cases(B=2, S=64):
    """(name, plan blob, source array, direct expected) per case."""
    rng = np.random.default_rng(20261202)
    perm = EN.Transpose((0, 2, 1, 3))
    out = []

    def add(name, H, D, dtype, ops, direct):
        shape = (B, S, H, D)
        if dtype == "int8":
            x = rng.integers(-128, 128, shape, dtype=np.int8)
        else:
            x = (rng.standard_normal(shape) * 3).astype(dtype)
        out.append((name, EN.encode(list(shape), dtype, [perm] + ops).blob, x, direct))

    # direct: one case per compile-time chain
    add("f16 quant per head", 32, 128, "float16",
        [EN.Cast("float32", "exact"), EN.Quantize(_per(32, rng), axis=1)], True)
    add("f16 quant per tensor", 32, 128, "float16",
        [EN.Cast("float32", "exact"), EN.Quantize(EN.InlineParam((0.03,), "float32", 0))], True)
    add("f16 quant per head, 8 heads of 64", 8, 64, "float16",
        [EN.Cast("float32", "exact"), EN.Quantize(_per(8, rng), axis=1)], True)
    add("f32 quant per head", 16, 128, "float32", [EN.Quantize(_per(16, rng), axis=1)], True)
    add("i8 dequant per head -> f16", 32, 128, "int8",
        [EN.Dequantize(_per(32, rng), zero_point=_zp(32, rng), axis=1), EN.Cast("float16")], True)
    add("i8 dequant per head", 16, 64, "int8",
        [EN.Dequantize(_per(16, rng), zero_point=_zp(16, rng), axis=1)], True)
    add("f32 -> f16", 32, 128, "float32", [EN.Cast("float16")], True)
    add("f16 -> f32", 32, 128, "float16", [EN.Cast("float32", "exact")], True)
    add("f16 layout only", 32, 128, "float16", [], True)
    # general body: the channel is not H, or a division is not a shift
    add("f16 quant per D", 32, 128, "float16",
        [EN.Cast("float32", "exact"), EN.Quantize(_per(128, rng), axis=3)], False)
    add("f16 quant per S", 32, 128, "float16",
        [EN.Cast("float32", "exact"), EN.Quantize(_per(S, rng), axis=2)], False)
    add("f16 quant per batch", 32, 128, "float16",
        [EN.Cast("float32", "exact"), EN.Quantize(_per(B, rng), axis=0)], False)
    add("f16 quant per head, 24 heads", 24, 128, "float16",
        [EN.Cast("float32", "exact"), EN.Quantize(_per(24, rng), axis=1)], False)
    add("f16 quant per head, D = 96", 32, 96, "float16",
        [EN.Cast("float32", "exact"), EN.Quantize(_per(32, rng), axis=1)], False)
    return out


def _chain(rng, dtype, shape):
    """Stages after the [B,S,H,D] -> [B,H,S,D] transpose: one of the chains
    the permute runs, a parameter stage per tensor or along a random axis."""
    axis = [None, 0, 1, 2, 3][int(rng.integers(5))]
    n = 1 if axis is None else shape[(0, 2, 1, 3)[axis]]
    rank = 0 if axis is None else 1
    sc = EN.InlineParam(tuple(float(v) for v in rng.uniform(0.004, 0.05, n)), "float32", rank)
    zp = EN.InlineParam(tuple(int(v) for v in rng.integers(-9, 10, n)), "int32", rank)
    if dtype == "float16":
        return [[], [EN.Cast("float32", "exact")],
                [EN.Cast("float32", "exact"), EN.Quantize(sc, axis=axis)]][int(rng.integers(3))]
    if dtype == "float32":
        return [[EN.Cast("float16")], [EN.Quantize(sc, axis=axis)]][int(rng.integers(2))]
    if dtype == "bfloat16":
        return [EN.Cast("float32", "exact")]
    return [[EN.Dequantize(sc, zero_point=zp, axis=axis)],
            [EN.Dequantize(sc, zero_point=zp, axis=axis), EN.Cast("float16")]][int(rng.integers(2))]


def random_cases(n, seed=7):
    """(name, plan blob, source array) for n random block permutes of
    [B, S, H, D] -> [B, H, S, D] with a random chain; shapes small enough for
    the oracle, H and D powers of two or not."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        dtype = ["float16", "float32", "int8", "bfloat16"][int(rng.integers(4))]
        shape = (int(rng.integers(1, 4)), int(rng.choice([2, 8, 12, 16, 40, 64])),
                 int(rng.choice([2, 3, 4, 6, 8, 16, 24, 32])), int(rng.choice([16, 32, 48, 64, 96, 128])))
        ops = [EN.Transpose((0, 2, 1, 3))] + _chain(rng, dtype, shape)
        try:
            plan = EN.encode(list(shape), dtype, ops)
        except EN.EncodeError:
            continue
        if dtype == "int8":
            x = rng.integers(-128, 128, shape, dtype=np.int8)
        elif dtype == "bfloat16":
            x = (rng.integers(0, 1 << 16, shape, dtype=np.uint32)).astype(np.uint16)
        else:
            x = (rng.standard_normal(shape) * 3).astype(dtype)
        out.append(("%s %s %s" % (dtype, shape, [type(o).__name__ for o in ops[1:]]), plan.blob, x))
    return out
