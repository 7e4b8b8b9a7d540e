"""Writes tests/golden/alloc_fragmentation.json: the reference's published
fragmentation tables for its allocator benchmark's three traces (RESULTS.md
section 2b, the generated blocks s2b-frag-uniform, s2b-frag-dl and
s2b-frag-bypass).  The traces come from a fixed seed, so the figures are
deterministic on any machine (the reference says so in each block's header).

Read as text from the reference tree; run where it is present:

    python tests/golden/make_alloc_fragmentation.py [/root/reference/RESULTS.md]
"""
from __future__ import annotations

import json
import os
import re
import sys

BLOCKS = {"s2b-frag-uniform": "uniform_pow2", "s2b-frag-dl": "dl_transformer",
          "s2b-frag-bypass": "dl_transformer_bypass"}
COLS = ["peak_reserved", "peak_blocks", "peak_requested", "block_eff", "reserv_eff",
        "utilisation", "internal_waste", "largest_free_at_end", "oom"]


def main(path: str = "/root/reference/RESULTS.md") -> None:
    text = open(path).read()
    out = {"source": "reference RESULTS.md section 2b (generated blocks "
                     + ", ".join(BLOCKS) + ")", "traces": {}}
    for block, trace in BLOCKS.items():
        m = re.search(r"<!-- BEGIN GENERATED id=" + re.escape(block) + r" .*?-->(.*?)"
                      r"<!-- END GENERATED id=" + re.escape(block), text, re.S)
        assert m, block
        rows = {}
        for line in m.group(1).splitlines():
            cells = [c.strip() for c in line.strip().strip("|").split("|")]
            if len(cells) == 10 and cells[0] in ("raw", "buddy", "freelist"):
                rows[cells[0]] = dict(zip(COLS, cells[1:]))
        assert set(rows) == {"raw", "buddy", "freelist"}, (block, rows)
        out["traces"][trace] = rows
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "alloc_fragmentation.json")
    with open(dst, "w") as f:
        json.dump(out, f, indent=1)
    print(f"wrote {dst}")


if __name__ == "__main__":
    main(*sys.argv[1:])
