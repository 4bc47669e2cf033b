"""Helpers that read the committed golden fixtures under tests/golden."""
import glob
import json
import os

import numpy as np

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CORPUS = os.path.join(HERE, "corpus")
NP_BITS = {"float32": np.uint32, "float16": np.uint16, "bfloat16": np.uint16, "uint16": np.uint16,
           "int8": np.uint8, "int32": np.uint32}


def goldens():
    with open(os.path.join(HERE, "goldens.json")) as f:
        return json.load(f)


def path(*parts):
    """A fixture file under tests/golden (e.g. the reference's calibration
    files in tests/golden/calibration)."""
    return os.path.join(HERE, *parts)


def typed_fixtures():
    out = []
    for jf in sorted(glob.glob(os.path.join(CORPUS, "typed", "*.json"))):
        with open(jf) as f:
            meta = json.load(f)
        with open(jf[:-5] + ".bin", "rb") as f:
            blob = f.read()
        out.append((meta, blob))
    return out


def layout_fixtures():
    out = []
    for jf in sorted(glob.glob(os.path.join(CORPUS, "*.json"))):
        with open(jf) as f:
            meta = json.load(f)
        with open(jf[:-5] + ".bin", "rb") as f:
            blob = f.read()
        out.append((meta, blob))
    return out


def fixture_params(meta):
    """{name: (dtype name, shape, little-endian bytes)} of a typed fixture."""
    out = {}
    for name, pv in meta.get("parameters", {}).items():
        arr = np.array([int(x, 16) for x in pv["bits"]], dtype=NP_BITS[pv["dtype"]])
        out[name] = (pv["dtype"], list(pv["shape"]), arr.tobytes())
    return out


def bits_array(entry):
    return np.array([int(x, 16) for x in entry["bits"]], dtype=NP_BITS[entry["dtype"]])
