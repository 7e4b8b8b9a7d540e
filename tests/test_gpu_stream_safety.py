"""GPU race test of the allocators' stream-ordered reuse (tests/cpp/stream_safety.cpp,
the counterpart of the reference's tests/test_stream_safety.cu), run in-process
through tests/cpp/bin/libstream_safety.so: a reader on one stream is held by a
host-released flag (a bounded poll) while the freed block is requested from
another stream.  The naive pool must be caught corrupting; the buddy and FreeList
allocators, under every reuse policy, must stay clean."""
from __future__ import annotations

import ctypes as C
import os

import pytest

pytestmark = pytest.mark.gpu

LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "bin", "libstream_safety.so")


def test_stream_safety_arms(gpu):
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is missing: build with `make -C tests/cpp`")
    lib = C.CDLL(LIB)
    lib.mcke_test_stream_safety.restype = C.c_int
    lib.mcke_test_stream_safety.argtypes = [C.c_char_p, C.c_size_t]
    buf = C.create_string_buffer(1 << 16)
    rc = lib.mcke_test_stream_safety(buf, len(buf))
    report = buf.value.decode()
    print(report)
    assert rc == 0, report
    assert "naive_pool" in report and "all arms PASS" in report
