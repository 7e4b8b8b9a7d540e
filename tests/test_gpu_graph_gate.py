"""The numerics gate can fail: GraphExecutor::validate_numerics() on a graph whose
first node returns a different answer on every launch (tests/cpp/gate_probe.cpp,
run in-process through tests/cpp/bin/libgate_probe.so).

Counterpart of the reference's test_numerics_gate_catches_nondeterminism
(tests/test_graph_host.cpp:1558-1597): a gate that never fires is not a gate.  The
flaky op must be caught as run-to-run variance within the first plan (the way a
real race shows), and the same graph with the op made deterministic must pass --
so the failure comes from the op's answers, not from the harness."""
from __future__ import annotations

import ctypes as C
import os

import pytest

pytestmark = pytest.mark.gpu

LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "bin", "libgate_probe.so")


def _probe(nondeterministic: int, repeats: int):
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is missing: build with `make -C tests/cpp`")
    lib = C.CDLL(LIB)
    lib.mcke_test_gate_probe.restype = C.c_int
    lib.mcke_test_gate_probe.argtypes = [C.c_int, C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int),
                                         C.c_char_p, C.c_size_t]
    passed, configs = C.c_int(-1), C.c_int(-1)
    buf = C.create_string_buffer(4096)
    rc = lib.mcke_test_gate_probe(nondeterministic, repeats, C.byref(passed), C.byref(configs),
                                  buf, len(buf))
    detail = buf.value.decode()
    print(f"nondeterministic={nondeterministic}: passed={passed.value} configs={configs.value}: {detail}")
    assert rc == 0, detail
    return passed.value, configs.value, detail


def test_gate_fires_on_run_to_run_variance(gpu):
    passed, configs, detail = _probe(1, 3)
    assert passed == 0, detail
    # Caught inside the first configuration, as run-to-run variance of the flaky
    # node's output, naming the run, the tensor and the two bit patterns.
    assert configs == 1, detail
    assert detail.startswith("sequential / per-tensor: "), detail
    assert "run 1 differs from run 0 in 'flaky' at element 0" in detail, detail
    # Launches 1 and 2 wrote 1.5 (0x3fc00000) and 2.0 (0x40000000).
    assert "0x3fc00000 then 0x40000000" in detail, detail


def test_gate_passes_the_same_graph_when_deterministic(gpu):
    passed, configs, detail = _probe(0, 3)
    assert passed == 1, detail
    assert configs == 9, detail
    assert detail.startswith("bitwise identical: 9 plans x 3 runs each"), detail
