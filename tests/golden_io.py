"""Loading of the committed golden fixtures (hex-encoded f32 bit patterns)."""
from __future__ import annotations

import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")


def _arr(tokens) -> np.ndarray:
    return np.array([int(t, 16) for t in tokens], dtype=np.uint32).view(np.float32)


def _flt(token: str) -> float:
    return float(np.array([int(token, 16)], dtype=np.uint32).view(np.float32)[0])


def load(name: str) -> list[dict]:
    """Returns cases with arrays decoded to float32 numpy arrays."""
    with open(os.path.join(GOLDEN, name)) as f:
        doc = json.load(f)
    out = []
    for c in doc["cases"]:
        out.append({
            "name": c["name"],
            "kind": c["kind"],
            "mode": c["mode"],
            "ints": dict(c["ints"]),
            "floats": {k: _flt(v) for k, v in c["floats"].items()},
            "arrays": {k: _arr(v) for k, v in c["arrays"].items()},
        })
    return out


def all_cases() -> list[dict]:
    return load("reference_vectors.json") + load("mcke_golden.json")


def bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
