"""The five benchmark workloads of this path as recipes + seeded inputs.

Each recipe is folded by sym_amd.encoder into the plan the reference's
exporter would produce (byte-identical on every recipe the reference
recorded; C1 matches its exported `split_transpose` digest). Inputs follow
the configs' distributions with seed 20260710 (the reference suite's
RELOC_SEED, libreloc/python/tests/conftest.py:23).

  C1  README plan: f32[s0] -> reshape [s0//64, 64] -> transpose -> [64, s0//64]
  C2  image batch: f32 NCHW [32,3,224,224] -> pad C 3->4 (0.0) -> NHWC -> f16
  C3  int8 weight [4096,11008] -> dequant(scale[11008], axis 1) -> f16 ->
      transpose -> [11008,4096]   (WeightFetcher's recipe with an f16 result)
  C4  MoE experts: int8 [out,in] -> dequant(scale[out], axis 0) -> f16, row-major
  C5  f16 [B,S,32,128] -> transpose [0,2,1,3] -> f32 -> quantize(scale[32], axis 1)
"""
from dataclasses import dataclass
from typing import Callable, Dict, List, Tuple

import numpy as np

from . import encoder as EN

SEED = 20260710


def c1_plan():
    return EN.encode(["s0"], "float32", [EN.Reshape(("s0 floordiv 64", 64)), EN.Transpose((1, 0))])


def c2_plan(n=32, c=3, h=224, w=224):
    return EN.encode([n, c, h, w], "float32",
                     [EN.Pad(1, 0, 1, 0.0), EN.Transpose((0, 2, 3, 1)), EN.Cast("float16")])


def c3_plan():
    scale = EN.BindingParam("scale", "float32", ("s1",))
    return EN.encode(["s0", "s1"], "int8",
                     [EN.Dequantize(scale, axis=1), EN.Cast("float16"), EN.Transpose((1, 0))])


def c4_plan():
    scale = EN.BindingParam("scale", "float32", ("s0",))
    return EN.encode(["s0", "s1"], "int8", [EN.Dequantize(scale, axis=0), EN.Cast("float16")])


def c5_plan(heads=32, dim=128):
    scale = EN.BindingParam("scale", "float32", (heads,))
    return EN.encode(["B", "S", heads, dim], "float16",
                     [EN.Transpose((0, 2, 1, 3)), EN.Cast("float32"), EN.Quantize(scale, axis=1)])


# ---------------------------------------------------------------- inputs

def c1_input(n, seed=SEED):
    return np.random.default_rng(seed).uniform(-1, 1, n).astype(np.float32)


def c2_input(n=32, c=3, h=224, w=224, seed=SEED):
    return np.random.default_rng(seed).standard_normal((n, c, h, w), dtype=np.float32)


def int8_weight(rows, cols, rng):
    return rng.integers(-127, 128, (rows, cols), dtype=np.int8)


def scales(n, rng, lo=1e-3, hi=2e-2):
    return rng.uniform(lo, hi, n).astype(np.float32)


def c3_input(rows=4096, cols=11008, seed=SEED):
    rng = np.random.default_rng(seed)
    return int8_weight(rows, cols, rng), scales(cols, rng)


def c4_pool(experts=8, hidden=4096, inter=14336, seed=SEED):
    """Per expert: gate/up [inter, hidden], down [hidden, inter] ([out, in])
    int8 with per-output-row f32 scales."""
    rng = np.random.default_rng(seed)
    pool = []
    for _ in range(experts):
        mats = []
        for rows, cols in ((inter, hidden), (inter, hidden), (hidden, inter)):
            mats.append((int8_weight(rows, cols, rng), scales(rows, rng)))
        pool.append(mats)
    return pool


def c4_steps(steps, experts=8, active=2, seed=SEED):
    rng = np.random.default_rng(seed + 1)
    return [tuple(rng.choice(experts, active, replace=False).tolist()) for _ in range(steps)]


def c5_input(b, s, heads=32, dim=128, seed=SEED):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((b, s, heads, dim), dtype=np.float32).astype(np.float16)
    return x, rng.uniform(0.02, 0.05, heads).astype(np.float32)


C5_SHAPES = [(b, s) for b in (1, 8, 64) for s in (128, 1024, 4096)]
C1_SIZES = [128, 192, 256, 16777216]


def param(name, arr):
    """A parameter in pyreloc.bind_typed form."""
    arr = np.ascontiguousarray(arr)
    return {name: (str(arr.dtype), list(arr.shape), arr.tobytes())}
