"""Convert the reference's golden-vector DATA file into a JSON fixture.

Source: tests/data/reference_vectors.txt in the reference tree (19 cases: 11
GEMM, 4 bias_act, 3 row_reduce, 1 row_softmax).  The file is data -- inputs and
expected outputs as 8-hex-digit IEEE-754 f32 bit patterns -- so the fixture keeps
the bit patterns unchanged and only re-encodes the container as JSON, because the
reference tree is not available on the GPU box.

Usage:  python tests/golden/import_reference_vectors.py [path/to/reference_vectors.txt]
Writes: tests/golden/reference_vectors.json
"""
from __future__ import annotations

import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
DEFAULT_SRC = "/root/reference/tests/data/reference_vectors.txt"
OUT = os.path.join(HERE, "reference_vectors.json")


def parse(text: str) -> list[dict]:
    """Parse the case/end block format: `case NAME`, `kind K`, `mode M`,
    `int NAME V`, `float NAME HEX`, `array NAME COUNT` followed by COUNT hex
    tokens over the next lines, and `end`."""
    cases: list[dict] = []
    cur: dict | None = None
    toks: list[str] = []
    want = 0
    arr_name = ""
    for raw in text.splitlines():
        line = raw.strip()
        if not line or line.startswith("#"):
            continue
        if want:
            toks.extend(line.split())
            if len(toks) >= want:
                if len(toks) != want:
                    raise ValueError(f"array {arr_name}: expected {want} tokens, got {len(toks)}")
                cur["arrays"][arr_name] = toks
                toks, want = [], 0
            continue
        parts = line.split()
        head = parts[0]
        if head == "case":
            cur = {"name": parts[1], "ints": {}, "floats": {}, "arrays": {}}
        elif head == "end":
            cases.append(cur)
            cur = None
        elif head in ("kind", "mode"):
            cur[head] = parts[1]
        elif head == "int":
            cur["ints"][parts[1]] = int(parts[2])
        elif head == "float":
            cur["floats"][parts[1]] = parts[2]
        elif head == "array":
            arr_name, want = parts[1], int(parts[2])
            toks = []
            if want == 0:
                cur["arrays"][arr_name] = []
        else:
            raise ValueError(f"unknown directive {head!r}")
    return cases


def main(argv: list[str]) -> int:
    src = argv[1] if len(argv) > 1 else DEFAULT_SRC
    with open(src) as f:
        cases = parse(f.read())
    doc = {
        "source": "reference tests/data/reference_vectors.txt (data, hex f32 bit patterns)",
        "encoding": "every float is an 8-hex-digit IEEE-754 binary32 bit pattern",
        "cases": cases,
    }
    with open(OUT, "w") as f:
        json.dump(doc, f, indent=1)
        f.write("\n")
    print(f"wrote {len(cases)} cases to {OUT}")
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
