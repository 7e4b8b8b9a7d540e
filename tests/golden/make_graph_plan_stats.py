"""Writes tests/golden/graph_plan_stats.json: the plan statistics of the
reference graph bench's five graphs as the reference published them (RESULTS.md
section 4, generated block s4-graph): for each graph and schedule policy, the
streams used out of those requested, the peak arena bytes and the naive (one
buffer per tensor) bytes.  They are functions of the graph, the schedule policy,
the memory policy (happens-before reuse, bench/graph_bench.cpp:333) and the
stream count only, so they hold on any machine; the timing columns are left out.

Read as text from the reference tree; run where it is present:

    python tests/golden/make_graph_plan_stats.py [/root/reference/RESULTS.md]
"""
from __future__ import annotations

import json
import os
import re
import sys


def main(path: str = "/root/reference/RESULTS.md") -> None:
    text = open(path).read()
    m = re.search(r"<!-- BEGIN GENERATED id=s4-graph .*?-->(.*?)<!-- END GENERATED id=s4-graph",
                  text, re.S)
    assert m
    graphs = {}
    for line in m.group(1).splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) != 9 or cells[0] in ("Graph", "---") or cells[0].startswith("-"):
            continue
        used, requested = (int(x) for x in cells[2].split("/"))
        peak = int(cells[6].split()[0].replace(",", ""))
        naive = int(cells[7].split()[0].replace(",", ""))
        graphs.setdefault(cells[0], {})[cells[1]] = {
            "streams_used": used, "streams_requested": requested,
            "arena_bytes": peak, "naive_bytes": naive}
    assert len(graphs) == 5 and all(len(v) == 3 for v in graphs.values()), graphs
    out = {"source": "reference RESULTS.md section 4, generated block s4-graph",
           "memory_policy": "reuse_happens_before", "graphs": graphs}
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "graph_plan_stats.json")
    with open(dst, "w") as f:
        json.dump(out, f, indent=1)
    print(f"wrote {dst}")


if __name__ == "__main__":
    main(*sys.argv[1:])
