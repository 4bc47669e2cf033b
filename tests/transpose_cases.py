"""Random one-byte-source transposes ([R, Q] -> [Q, R], or [B, R, Q] ->
[B, Q, R]) with the value chains the transpose kernel runs: layout only,
dequantize (per tensor or along an axis, with zero points), and
dequantize then cast to f16. Source-contiguous extents Q that are multiples
of 128 take tiles 128 q wide in the rotated order (with f16 or f32
results, 128 c wide byte tiles when R is a multiple of 128 too), others
64-wide tiles; R extents that are
not multiples of the tile leave an edge strip to the element-wise kernel (R = 100 also breaks the 16-byte row alignment of one- and two-byte
results, which then run element-wise throughout). Used by the CPU launch checks (every launch verified, the tile width
asserted) and by the GPU parity test against the oracle.
"""
import numpy as np

from sym_amd import encoder as EN

QS = (64, 128, 192, 256, 384, 1152)
RS = (64, 100, 128, 160, 256, 320)


def _chain(rng, shape):
    """Stages before the transpose: none, a dequantize, or a dequantize and a
    cast to f16; the parameter stage per tensor or along a random axis."""
    kind = int(rng.integers(3))
    if kind == 0:
        return []
    axis = [None] + list(range(len(shape)))
    axis = axis[int(rng.integers(len(axis)))]
    n = 1 if axis is None else shape[axis]
    rank = 0 if axis is None else 1
    sc = EN.InlineParam(tuple(float(v) for v in rng.uniform(0.004, 0.05, n)), "float32", rank)
    zp = EN.InlineParam(tuple(int(v) for v in rng.integers(-9, 10, n)), "int32", rank)
    deq = EN.Dequantize(sc, zero_point=zp if rng.integers(2) else None, axis=axis)
    return [deq] if kind == 1 else [deq, EN.Cast("float16")]


def _fixed(rng):
    """Dequantize -> f16 byte tiles with the scale along the result rows
    (parameters indexed by row: per-channel, all-zero and per-tensor zero
    points, none) and along the result columns (channel from each vector's
    offset)."""
    out = []
    for r, q, axis, zp in ((128, 128, 1, "channel"), (256, 384, 1, "tensor"), (128, 1152, 1, None),
                           (256, 128, 1, "zeros"), (256, 256, 0, "channel"), (384, 128, 0, None)):
        n = (r, q)[axis]
        sc = EN.InlineParam(tuple(float(v) for v in rng.uniform(0.004, 0.05, n)), "float32", 1)
        if zp == "channel":
            z = EN.InlineParam(tuple(int(v) for v in rng.integers(-9, 10, n)), "int32", 1)
        elif zp == "zeros":  # per channel, all 0: the kernel leaves them out
            z = EN.InlineParam((0,) * n, "int32", 1)
        elif zp == "tensor":
            z = EN.InlineParam((int(rng.integers(-9, 10)),), "int32", 0)
        else:
            z = None
        ops = [EN.Dequantize(sc, zero_point=z, axis=axis), EN.Cast("float16")]
        plan = EN.encode([r, q], "int8", ops + [EN.Transpose((1, 0))])
        x = rng.integers(-128, 128, (r, q), dtype=np.int8)
        out.append(("int8 %s dequant axis %d zp %s -> f16" % ((r, q), axis, zp), plan.blob, x, (128, 128)))
    return out


def random_cases(n, seed=11):
    """(name, plan blob, source array, expected (q, c) tile widths): six
    fixed byte-tile cases, then n random one-byte transposes."""
    rng = np.random.default_rng(seed)
    out = _fixed(rng)
    n += len(out)
    while len(out) < n:
        q = int(rng.choice(QS))
        r = int(rng.choice(RS))
        batch = int(rng.integers(0, 3))
        shape = (r, q) if batch == 0 else (batch, r, q)
        perm = (1, 0) if batch == 0 else (0, 2, 1)
        ops = _chain(rng, shape)
        try:
            plan = EN.encode(list(shape), "int8", ops + [EN.Transpose(perm)])
        except EN.EncodeError:
            continue
        x = rng.integers(-128, 128, shape, dtype=np.int8)
        wider = bool(ops)  # f32 or f16 results
        width = (128 if q % 128 == 0 else 64, 128 if q % 128 == 0 and r % 128 == 0 and wider else 64)
        out.append(("int8 %s %s" % (shape, [type(o).__name__ for o in ops]), plan.blob, x, width))
    return out
