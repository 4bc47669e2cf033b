"""Every module of the package imports as the first import of a fresh
interpreter (transfer and dispatch import pyreloc, whose pyreloc-named
re-exports of them resolve on first use), and the re-exported names are
the defining modules' objects. No device is touched."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
MODULES = ["pyreloc", "transfer", "dispatch", "artifact", "encoder", "recipe_json", "workloads",
           "build", "_native", "_hostmath"]


@pytest.mark.parametrize("mod", MODULES)
def test_module_imports_first(mod):
    r = subprocess.run([sys.executable, "-c", "import sym_amd.%s" % mod], cwd=ROOT,
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]


def test_reexports_are_the_defining_objects():
    from sym_amd import dispatch as D
    from sym_amd import pyreloc as P
    from sym_amd import transfer as T
    for mod, names in P._REEXPORTS.items():
        src = T if mod == "transfer" else D
        for name in names:
            assert getattr(P, name) is getattr(src, name), name
            assert name in dir(P)
    with pytest.raises(AttributeError):
        P.no_such_name  # noqa: B018
