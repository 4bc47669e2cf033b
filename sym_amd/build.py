"""Build librelx.so in-tree with hipcc for gfx950.

    python -m sym_amd.build        # or: from sym_amd.build import build; build()

Objects go to sym_amd/_build/, the library to sym_amd/librelx.so (both
git-ignored; the .so travels to the GPU box with the tree).
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "librelx.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("RELX_OFFLOAD_ARCH", "gfx950")

# Value stages must keep every rounding: no contraction, no fast math, keep
# denormals. Packed-FP32 instructions are disabled for all HIP code.
COMMON = ["-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-fno-fast-math", "-Wall",
          "-Wno-unused-command-line-argument"]
DEVICE = ["--offload-arch=" + ARCH, "-mcode-object-version=5", "-fno-gpu-flush-denormals-to-zero",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
SOURCES = ["plan.cpp", "program.cpp", "runtime.cpp", "workers.cpp", "indexed.cpp", "transfer.cpp",
           "capi.cpp",
           "kernels.hip",
           "k_stream_fast.hip", "k_stream_generic.hip", "k_transpose.hip", "k_interleave.hip",
           "k_interleave_generic.hip", "k_permute.hip", "k_gather.hip", "k_copy.hip", "noalloc.hip"]


# The one-level interleave takes its hot arguments as leading scalars that
# the dispatch preloads into scalar registers.
EXTRA = {"k_interleave.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"]}


def _compile(src):
    obj = os.path.join(OUT_DIR, os.path.basename(src) + ".o")
    cmd = [HIPCC] + COMMON + DEVICE + EXTRA.get(src, []) + ["-I" + CSRC, "-c",
                                                            os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".hip"):
        cmd[1:1] = ["-x", "hip"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "packed-fp32-ops"
    err = "\n".join(l for l in (r.stderr or "").splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError("compile failed: %s\n%s" % (" ".join(cmd), err))
    return obj, err


def build(verbose=False):
    os.makedirs(OUT_DIR, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(os.cpu_count() or 8, len(SOURCES), 16)) as ex:
        results = list(ex.map(_compile, SOURCES))
    for obj, err in results:
        if verbose and err.strip():
            print(err, file=sys.stderr)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", tmp] + \
        [o for o, _ in results] + ["-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed: %s\n%s" % (" ".join(cmd), r.stderr))
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
