"""Random relocation recipes for the fuzz tests (tests/test_fuzz.py on the
CPU, tests/test_gpu_fuzz.py on the GPU): chains of transposes, reshapes,
pads and value stages (casts, quantize, dequantize with per-tensor or
per-channel inline parameters) over small random shapes, encoded by
sym_amd.encoder, with random source values that include the special
values of each element type."""
import numpy as np

from sym_amd import encoder as EN

WIDTH = {"float32": 4, "float16": 2, "bfloat16": 2, "int8": 1}
BITS = {1: np.uint8, 2: np.uint16, 4: np.uint32}


def _layout_op(rng, shape, dtype):
    kind = rng.choice(["transpose", "reshape", "pad"])
    if kind == "transpose" and len(shape) >= 2:
        perm = [int(p) for p in rng.permutation(len(shape))]
        return EN.Transpose(tuple(perm)), [shape[p] for p in perm]
    if kind == "reshape":
        if len(shape) >= 2 and rng.random() < 0.5:  # merge two neighbours
            k = int(rng.integers(0, len(shape) - 1))
            new = shape[:k] + [shape[k] * shape[k + 1]] + shape[k + 2:]
            return EN.Reshape(tuple(new)), new
        k = int(rng.integers(0, len(shape)))  # split one axis by a divisor
        divs = [d for d in range(2, shape[k]) if shape[k] % d == 0]
        if divs and len(shape) < 5:
            d = int(rng.choice(divs))
            new = shape[:k] + [shape[k] // d, d] + shape[k + 1:]
            return EN.Reshape(tuple(new)), new
        return None, shape
    axis = int(rng.integers(0, len(shape)))
    lo, hi = int(rng.integers(0, 3)), int(rng.integers(0, 4))
    if lo + hi == 0:
        hi = 1
    if dtype == "int8":
        value = int(rng.integers(-128, 128))
    else:
        value = float(rng.choice([0.0, -0.0, 1.5, -2.25, np.inf]))
    new = list(shape)
    new[axis] += lo + hi
    return EN.Pad(axis, lo, hi, value), new


def _inline(rng, n, per_channel, lo, hi):
    vals = tuple(float(np.float32(v)) for v in rng.uniform(lo, hi, n if per_channel else 1))
    return EN.InlineParam(vals, "float32", 1 if per_channel else 0)


def _stage(rng, shape, dtype):
    axis = int(rng.integers(0, len(shape)))
    per = bool(rng.random() < 0.5)
    if dtype == "float32":
        pick = rng.choice(["f16", "bf16", "quant"])
        if pick == "f16":
            return EN.Cast("float16"), "float16"
        if pick == "bf16":
            return EN.Cast("bfloat16"), "bfloat16"
        return EN.Quantize(_inline(rng, shape[axis], per, 0.005, 0.5),
                           axis=axis if per else None), "int8"
    if dtype in ("float16", "bfloat16"):
        return EN.Cast("float32", "exact"), "float32"
    zp = None
    if rng.random() < 0.3:
        zp = EN.InlineParam(tuple(int(v) for v in rng.integers(-20, 21, shape[axis] if per else 1)),
                            "int32", 1 if per else 0)
    return EN.Dequantize(_inline(rng, shape[axis], per, 0.005, 0.5), zero_point=zp,
                         axis=axis if per else None), "float32"


ALIGNED = [8, 16, 24, 32, 48, 64, 96, 128, 192, 256]


def random_recipe(rng, aligned=False, max_elements=6000):
    """(source shape, source dtype, ops) for one random recipe. `aligned`
    draws extents that are multiples of 8 (up to 256) so that the vector,
    tile and block-permute kernels qualify; otherwise extents are small and
    arbitrary (the element-wise kernel)."""
    rank = int(rng.integers(2 if aligned else 1, 5))
    if aligned:
        max_elements = 1 << 18
    while True:
        if aligned:
            shape = [int(rng.choice(ALIGNED)) if rng.random() < 0.8 else int(rng.integers(1, 6))
                     for _ in range(rank)]
        else:
            shape = [int(rng.integers(1, 48 if rank <= 2 else 12)) for _ in range(rank)]
        if int(np.prod(shape)) <= max_elements:
            break
    dtype = str(rng.choice(["float32", "float16", "int8", "bfloat16"], p=[0.45, 0.25, 0.2, 0.1]))
    ops, cur, cur_t = [], list(shape), dtype
    for _ in range(int(rng.integers(1, 6))):
        if rng.random() < 0.6:
            op, new = _layout_op(rng, cur, cur_t)
            if op is None or int(np.prod(new)) > 4 * max_elements:
                continue
            ops.append(op)
            cur = new
        else:
            op, cur_t = _stage(rng, cur, cur_t)
            ops.append(op)
    return shape, dtype, ops


def transpose_recipe(rng):
    """A tile-transpose shaped recipe: [batch?, A, B] with a swap of the last
    two axes, A and B multiples of 8 (mostly of 64), and value stages before
    or after the swap (the C1/C3 pattern)."""
    dims = [int(rng.choice([64, 128, 192, 256, 320, 96, 40])) for _ in range(2)]
    shape = ([int(rng.integers(1, 4))] if rng.random() < 0.4 else []) + dims
    dtype = str(rng.choice(["float32", "float16", "int8"]))
    r = len(shape)
    perm = tuple(list(range(r - 2)) + [r - 1, r - 2])
    ops, cur, cur_t = [], list(shape), dtype
    if rng.random() < 0.5:
        op, cur_t = _stage(rng, cur, cur_t)
        ops.append(op)
    ops.append(EN.Transpose(perm))
    cur = [cur[p] for p in perm]
    if rng.random() < 0.5:
        op, cur_t = _stage(rng, cur, cur_t)
        ops.append(op)
    return shape, dtype, ops


def random_source(rng, shape, dtype):
    n = int(np.prod(shape))
    if dtype == "int8":
        return rng.integers(-128, 128, n, dtype=np.int8).reshape(shape)
    x = rng.standard_normal(n).astype(np.float32) * np.float32(rng.choice([1.0, 100.0, 1e4]))
    specials = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 65504.0, 65520.0, 2.0 ** -24,
                         2.0 ** -25, 3e38], dtype=np.float32)
    k = min(n, len(specials))
    x[rng.choice(n, k, replace=False)] = specials[:k]
    if dtype == "float32":
        return x.reshape(shape)
    if dtype == "float16":
        with np.errstate(over="ignore"):
            return x.astype(np.float16).reshape(shape)
    return (x.view(np.uint32) >> 16).astype(np.uint16).reshape(shape)  # bfloat16 bits


def make_plan(seed):
    """A random recipe that the encoder accepts: (plan, source array, ops),
    or None when every draw is rejected. Seeds cycle through small arbitrary
    shapes (even), aligned shapes (1 mod 4) and tile transposes (3 mod 4)."""
    rng = np.random.default_rng(seed)
    for _ in range(20):
        if seed % 4 == 3:
            shape, dtype, ops = transpose_recipe(rng)
        else:
            shape, dtype, ops = random_recipe(rng, aligned=bool(seed % 2))
        try:
            plan = EN.encode(shape, dtype, ops)
        except EN.EncodeError:
            continue
        return plan, random_source(rng, shape, dtype), ops
    return None
