"""Extract golden DATA (hex wire blobs, witness vectors, recorded digests) from
the reference's own test fixtures into tests/golden/goldens.json.

Runs only where /root/reference is mounted (the build container); the JSON it
writes is committed, so nothing reads the reference at test time. The copied
items are data: hex byte strings the reference's tests decode, the numeric
witness tables of docs/reloc-typed-semantics.md section 6, and plan digests.

Sources:
  libreloc/test/TypedGoldens.h:30-164      typed wire v1 hex blobs
  libreloc/test/TypedDecodeTest.cpp:43-49  v0 identity golden (181 bytes)
  libreloc/test/DecodeTest.cpp:41-120      v0 identity/reference/pad/degraded
  docs/runtime-evidence/cuda.json:40-60    exported example plan digests
  test/dialect/reloc/indexed_export_check.py:50-57  frozen wire v2 bytes
                                           (static f32[8,5], i64[3] -> f32[3,5])
"""
import json
import pathlib
import re

REF = pathlib.Path("/root/reference")
OUT = pathlib.Path(__file__).resolve().parent / "goldens.json"


def hex_constants(path):
    text = path.read_text()
    out = {}
    for m in re.finditer(r"(k\w+Hex)\s*=\s*((?:\s*\"[0-9a-f]*\")+)\s*;", text):
        out[m.group(1)] = "".join(re.findall(r"\"([0-9a-f]*)\"", m.group(2)))
    return out


def main():
    typed = hex_constants(REF / "libreloc/test/TypedGoldens.h")
    v0 = hex_constants(REF / "libreloc/test/DecodeTest.cpp")
    v0.update({"kIdentityV0Hex": hex_constants(REF / "libreloc/test/TypedDecodeTest.cpp")["kIdentityV0Hex"]})
    evidence = json.loads((REF / "docs/runtime-evidence/cuda.json").read_text())
    digests = []

    def walk(node, key=None):
        if isinstance(node, dict):
            if "plan_sha256" in node and "plan_bytes" in node:
                digests.append({"recipe": key, "plan_bytes": node["plan_bytes"],
                                "plan_sha256": node["plan_sha256"],
                                "symbols": node.get("symbols", []),
                                "constraints": node.get("constraints", {})})
            for k, v in node.items():
                walk(v, k)
        elif isinstance(node, list):
            for v in node:
                walk(v, key)

    walk(evidence)
    check = (REF / "test/dialect/reloc/indexed_export_check.py").read_text()
    m = re.search(r"identity\.hex\(\) == \(((?:\s*'[0-9a-f]*')+)\s*\)", check)
    indexed = {"static_f32_8x5_i64_3_exact": "".join(re.findall(r"'([0-9a-f]*)'", m.group(1)))}
    OUT.write_text(json.dumps({"typed_v1": typed, "layout_v0": v0, "exported_plan_digests": digests,
                               "indexed_v2": indexed},
                              indent=1, sort_keys=True) + "\n")
    print("wrote", OUT, len(typed), "typed,", len(v0), "v0,", len(digests), "digests")


if __name__ == "__main__":
    main()
