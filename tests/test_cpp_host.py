"""Runs the C++ host-layer test binary (tests/cpp/test_host.cpp) on the CPU:
graph, scheduler, happens-before, memory planner, buddy allocator, tile and
occupancy arithmetic, online-softmax algebra and launcher argument checks."""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CPP = os.path.join(HERE, "cpp")


def _binary(name: str) -> str:
    subprocess.run(["make", "-s", "-C", CPP], check=True)
    path = os.path.join(CPP, "bin", name)
    assert os.path.exists(path), f"{path} was not built"
    return path


def test_host_layers():
    r = subprocess.run([_binary("test_host")], capture_output=True, text=True, timeout=300)
    print(r.stdout[-4000:])
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-2000:]
    assert "0 failures" in r.stdout
