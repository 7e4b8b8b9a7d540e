"""The C-ABI library, without a GPU: it loads, exports every symbol the header
declares, and rejects bad arguments before any device work (reference error
conventions: kernels.hpp:78-86, bias_act.cu:208-229, reduce.cu:224-295,
softmax.cu:177-199, gemm.cu:829-882).

The argument-validation tests pass fake device pointers, which is only safe
because every call here is rejected before a launch; they are skipped when a GPU
is visible (the GPU suite repeats them with real buffers).
"""
from __future__ import annotations

import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mcke_amd.h")
GRAPH_HEADER = os.path.join(ROOT, "include", "mcke_graph.h")


def _declared_functions(header: str = HEADER) -> list[str]:
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mcke_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = _declared_functions()
    for must in ("mcke_launch_gemm_f32", "mcke_launch_bias_act_f32", "mcke_launch_row_reduce_f32",
                 "mcke_launch_row_reduce_ws_f32", "mcke_launch_row_softmax_f32",
                 "mcke_row_reduce_workspace_bytes", "mcke_gemm_kernel_attrs", "mcke_last_error",
                 "mcke_rt_stream_create", "mcke_rt_event_elapsed_ms", "mcke_rt_malloc"):
        assert must in names


def test_library_exports_every_declared_symbol(mcke):
    L = mcke.lib()
    for name in _declared_functions():
        assert hasattr(L, name), f"{name} declared in mcke_amd.h but not exported"
    out = subprocess.run(["nm", "-D", "--defined-only", mcke.library_path()],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\sT\s(mcke_\w+)", out))
    assert set(_declared_functions()) <= exported
    assert mcke.lib().mcke_abi_version() == 1


def test_host_library_exports_every_graph_symbol(mcke):
    from mcke_amd import graph
    L = graph.host_lib()
    names = _declared_functions(GRAPH_HEADER)
    assert "mcke_executor_validate_numerics" in names and "mcke_graph_add_gemm" in names
    for name in names:
        assert hasattr(L, name), f"{name} declared in mcke_graph.h but not exported"
    out = subprocess.run(["nm", "-D", "--defined-only", graph.host_library_path()],
                         capture_output=True, text=True, check=True).stdout
    assert set(names) <= set(re.findall(r"\sT\s(mcke_\w+)", out))


def test_graph_builder_without_gpu(mcke):
    """Graph construction and shape inference are host-only."""
    from mcke_amd import graph
    g, t = graph.mlp_block(64, 32, 128)
    assert g.shape(t["gemm1"]) == (64, 128) and g.shape(t["y"]) == (64, 32)
    g2 = graph.Graph()
    x = g2.add_input((4, 4), "x")
    b = g2.add_input((5,), "b")
    import pytest as _pt
    with _pt.raises(mcke.MckeError) as ei:
        g2.add_bias_act(x, b, "bad")
    assert ei.value.status.code == mcke.StatusCode.kInvalidArgument
    with _pt.raises(mcke.MckeError):
        g2.add_gemm(x, x, "tiled_no_tile", variant=mcke.GemmVariant.kTiledSmem)


def test_fused_gemm_node_without_gpu(mcke):
    """GemmBiasAct nodes: shapes, the checks at build time, and the fused MLP's
    tensors matching the unfused one's."""
    from mcke_amd import graph
    g, t = graph.mlp_block_fused(64, 32, 128)
    assert g.shape(t["h"]) == (64, 128) and g.shape(t["z"]) == (64, 32)
    assert g.shape(t["y"]) == (64, 32)
    g2 = graph.Graph()
    a = g2.add_input((8, 16), "a")
    b = g2.add_input((16, 12), "b")
    ok_bias, bad_bias = g2.add_input((12,), "bias"), g2.add_input((16,), "bias16")
    assert g2.shape(g2.add_gemm_bias_act(a, b, ok_bias, "y")) == (8, 12)
    IA = mcke.StatusCode.kInvalidArgument
    for args in ((a, b, bad_bias), (a, a, ok_bias), (b, b, ok_bias)):
        with pytest.raises(mcke.MckeError) as ei:
            g2.add_gemm_bias_act(*args, "bad")
        assert ei.value.status.code == IA
    with pytest.raises(mcke.MckeError):                       # not a kMfmaF32 tile
        g2.add_gemm_bias_act(a, b, ok_bias, "bad_tile", tile=mcke.GemmTile(128, 128, 8, 8, 8))
    with pytest.raises(mcke.MckeError):                       # unknown activation
        g2.add_gemm_bias_act(a, b, ok_bias, "bad_act", act=7)


def test_graph_dtypes_without_gpu(mcke):
    """16-bit inputs: only GEMM nodes take them; the output dtype follows the op."""
    from mcke_amd import graph
    import pytest as _pt
    IA = mcke.StatusCode.kInvalidArgument
    g = graph.Graph()
    x = g.add_input((64, 32), "x", dtype=2)          # bf16
    w = g.add_input((32, 48), "w", dtype=2)
    wh = g.add_input((32, 48), "wh", dtype=1)        # f16
    b = g.add_input((48,), "b")                      # f32
    h = g.add_gemm_lp(x, w, "g")                     # f32 C
    assert g.shape(h) == (64, 48)
    g.add_bias_act(h, b, "act")                      # f32 from here on
    h16 = g.add_gemm_lp(x, w, "g16", out_dtype=2)    # bf16 C
    for bad in (lambda: g.add_bias_act(h16, b, "act16"),          # f32-only op on bf16
                lambda: g.add_softmax(x, "sm"),
                lambda: g.add_gemm_lp(x, wh, "mixed"),             # bf16 x f16
                lambda: g.add_gemm_lp(x, w, "odd_out", out_dtype=1),
                lambda: g.add_gemm(x, w, "f32_variant_on_bf16"),
                lambda: g.add_gemm_lp(b, b, "f32_inputs"),
                lambda: g.add_gemm_lp(x, w, "tile", tile=mcke.GemmTile(256, 256, 32, 16, 16))):
        with _pt.raises(mcke.MckeError) as ei:
            bad()
        assert ei.value.status.code == IA, ei.value


def test_enum_values_match_reference(mcke):
    assert [int(v) for v in mcke.Activation] == [0, 1, 2, 3]
    assert [int(v) for v in mcke.ReduceKind] == [0, 1, 2]
    assert [int(v) for v in mcke.ReduceVariant] == [0, 1, 2]
    assert [int(v) for v in mcke.SoftmaxVariant] == [0, 1]
    V = mcke.GemmVariant
    assert (V.kNaive, V.kTiledSmem, V.kTiledRegBlock, V.kWarpTile, V.kCublasRef,
            V.kWarpTileNoDbuf, V.kWarpTileVec4, V.kNaiveUncoalesced, V.kMfmaF32) == tuple(range(9))
    assert [int(c) for c in mcke.StatusCode] == list(range(7))
    # DType, include/mcke/core/dtype.hpp:33-41: kF32, kF16, kBF16 first.
    assert (int(mcke.DType.kF32), int(mcke.DType.kF16), int(mcke.DType.kBF16)) == (0, 1, 2)


def test_host_generators_match_oracle(mcke, orc):
    import numpy as np
    for seed, lo, hi in ((0x6E33A, -1.0, 1.0), (3, 0.0, 1.0), (0xB1A5B1A5, -0.5, 0.5)):
        assert np.array_equal(mcke.fill_random(10001, seed, lo, hi).view(np.uint32),
                              orc.fill_random(10001, seed, lo, hi).view(np.uint32))
    for seed, mu, sigma in ((1, 0.0, 1.0), (2, 0.0, 2.0), (3, 0.0, 0.02)):
        assert np.array_equal(mcke.fill_normal(10001, seed, mu, sigma).view(np.uint32),
                              orc.fill_normal(10001, seed, mu, sigma).view(np.uint32))


def test_max_vector_width(mcke):
    assert mcke.max_vector_width_f32(0x1000, 4096) == 4
    assert mcke.max_vector_width_f32(0x1000, 4098) == 2
    assert mcke.max_vector_width_f32(0x1008, 4096) == 2
    assert mcke.max_vector_width_f32(0x1004, 4096) == 1
    assert mcke.max_vector_width_f32(0x1000, 7) == 1


def test_workspace_query(mcke):
    TP = mcke.ReduceVariant.kTwoPass
    assert mcke.row_reduce_workspace_bytes(8192, 8192, mcke.ReduceVariant.kWarpShuffle) == 0
    assert mcke.row_reduce_workspace_bytes(0, 100, TP) == 0
    assert mcke.row_reduce_workspace_bytes(8192, 8192, TP) == 8192 * 4          # split 1
    assert mcke.row_reduce_workspace_bytes(1, 1 << 26, TP) == 256 * 4           # full sum
    assert mcke.row_reduce_workspace_bytes(64, 524288, TP) == 64 * 4 * 4
    assert mcke.row_reduce_workspace_bytes(1, 1000, TP) == 4                    # short row


def test_default_mfma_tile(mcke):
    """The rule weighs each tile's sustained rate by how evenly its tile count fills
    whole rounds of CUs (256 on a CPU-only host, gfx950's count)."""
    t = mcke.gemm_mfma_default_tile(8192, 8192, 8192)
    assert t.astuple() == (256, 256, 32, 16, 16)
    assert mcke.gemm_mfma_default_tile(4096, 4096, 4096).astuple() == (256, 256, 32, 16, 16)
    assert mcke.gemm_mfma_default_tile(4096, 4096, 16384).astuple() == (256, 256, 32, 16, 16)
    assert mcke.gemm_mfma_default_tile(8192, 8192, 512).astuple() == (256, 256, 32, 16, 16)
    # 6144^3: 576 tiles of 256 fill 2.25 rounds; 2304 tiles of 128 fill 9.
    assert mcke.gemm_mfma_default_tile(6144, 6144, 6144).astuple() == (128, 128, 32, 8, 8)
    assert mcke.gemm_mfma_default_tile(2048, 2048, 2048).astuple() == (128, 128, 32, 8, 8)
    assert mcke.gemm_mfma_default_tile(2048, 2048, 8192).astuple() == (128, 128, 32, 8, 8)
    # 3072^3: 576 tiles of 128 fill 2.25 rounds; 2304 tiles of 64 fill 9.
    assert mcke.gemm_mfma_default_tile(3072, 3072, 3072).astuple() == (64, 64, 32, 4, 4)
    assert mcke.gemm_mfma_default_tile(1024, 1024, 1024).astuple() == (64, 64, 32, 4, 4)
    # 512^3: 64 tiles of 64 fill a quarter round; 256 tiles of 32 fill one.
    assert mcke.gemm_mfma_default_tile(512, 512, 512).astuple() == (32, 32, 32, 2, 2)
    assert mcke.gemm_mfma_default_tile(256, 256, 256).astuple() == (32, 32, 32, 2, 2)
    assert mcke.gemm_mfma_default_tile(1, 1, 1).astuple() == (32, 32, 32, 2, 2)


# ---------------------------------------------------------------------------
# Argument validation with fake pointers (rejected before any launch)
# ---------------------------------------------------------------------------
def _no_gpu(mcke) -> bool:
    try:
        return mcke.device_count() == 0
    except Exception:
        return True


@pytest.fixture()
def cpu_only(mcke):
    if not _no_gpu(mcke):
        pytest.skip("a GPU is visible: these calls pass fake device addresses, so they run only "
                    "where a missed rejection cannot launch a kernel on them")
    return mcke


X, Y, B, W = 0x10000, 0x20000, 0x30000, 0x40000   # fake, 256-byte aligned


def test_empty_extents_are_ok_without_launch(cpu_only):
    m = cpu_only
    assert m.launch_bias_act_f32(X, B, Y, 0, 10, 3, 4).ok()
    assert m.launch_bias_act_f32(None, None, None, 5, 0, 3, 4).ok()
    assert m.launch_row_reduce_f32(X, Y, 0, 5, 0, 1).ok()
    assert m.launch_row_softmax_f32(X, Y, 7, 0, 1).ok()
    assert m.launch_gemm_f32(X, B, Y, 0, 5, 5, 1.0, 0.0, m.GemmVariant.kMfmaF32,
                             m.MFMA_TILES[0]).ok()
    assert m.launch_activation_f32(X, Y, 0, 3, 4).ok()
    assert m.launch_vector_add_f32(X, B, Y, 0).ok()


def test_bias_act_rejections(cpu_only):
    m = cpu_only
    IA = m.StatusCode.kInvalidArgument
    assert m.launch_bias_act_f32(X, None, Y, 4, 8, 3, 4).code == IA           # null bias
    assert m.launch_bias_act_f32(None, B, Y, 4, 8, 3, 4).code == IA           # null x
    assert m.launch_bias_act_f32(X, B, Y, -1, 8, 3, 4).code == IA             # negative
    assert m.launch_bias_act_f32(X, B, Y, 4, 8, 3, 3).code == IA              # vw 3
    st = m.launch_bias_act_f32(X, B, Y, 4, 6, 3, 4)                           # cols % vw
    assert st.code == IA and "multiple of vector_width" in st.message
    assert m.launch_bias_act_f32(X + 4, B, Y, 4, 8, 3, 4).code == IA          # misaligned x
    assert m.launch_bias_act_f32(X, B + 8, Y, 4, 8, 3, 4).code == IA          # misaligned bias
    assert m.launch_bias_act_f32(X, B, X, 4, 8, 3, 4).code == IA              # in place
    assert m.launch_bias_act_f32(X, B, Y, 4, 8, 9, 4).code == IA              # bad act
    assert m.launch_activation_f32(X, Y, 6, 3, 4).code == IA                  # n % vw
    st = m.launch_bias_act_f32(X, B, Y, 1, 1 << 33, 3, 1)                    # grid x > 2^32 lanes
    assert st.code == IA and "32-bit work size" in st.message


def test_reduce_rejections(cpu_only):
    m = cpu_only
    IA = m.StatusCode.kInvalidArgument
    TP = m.ReduceVariant.kTwoPass
    st = m.launch_row_reduce_f32(X, Y, 4, 8, 0, TP)                           # 7-arg kTwoPass
    assert st.code == m.StatusCode.kUnimplemented
    assert m.launch_row_reduce_f32(X, Y, 4, 8, 0, TP, None, 0, None).code == IA
    need = m.row_reduce_workspace_bytes(1, 1 << 20, TP)
    assert m.launch_row_reduce_f32(X, Y, 1, 1 << 20, 0, TP, W, need - 4, None).code == IA
    assert m.launch_row_reduce_f32(X, Y, -2, 8, 0, 1).code == IA
    assert m.launch_row_reduce_f32(None, Y, 2, 8, 0, 1).code == IA
    assert m.launch_row_reduce_f32(X, Y, 2, 8, 7, 1).code == IA               # bad kind
    assert m.launch_row_reduce_f32(X, Y, 1 << 31, 8, 0, 1).code == IA         # rows > 2^31-1


def test_softmax_rejections(cpu_only):
    m = cpu_only
    IA = m.StatusCode.kInvalidArgument
    assert m.launch_row_softmax_f32(X, X, 4, 8, 1).code == IA
    assert m.launch_row_softmax_f32(X, None, 4, 8, 1).code == IA
    assert m.launch_row_softmax_f32(X, Y, -4, 8, 1).code == IA
    assert m.launch_row_softmax_f32(X, Y, 1 << 31, 8, 1).code == IA
    assert m.launch_row_softmax_f32(X, Y, 4, 8, 5).code == IA


def test_gemm_rejections(cpu_only):
    m = cpu_only
    IA = m.StatusCode.kInvalidArgument
    V, T = m.GemmVariant, m.GemmTile
    good = m.MFMA_TILES[0]
    assert m.launch_gemm_f32(X, B, X, 8, 8, 8, 1, 0, V.kMfmaF32, good).code == IA   # a == c
    assert m.launch_gemm_f32(X, B, B, 8, 8, 8, 1, 0, V.kMfmaF32, good).code == IA   # b == c
    assert m.launch_gemm_f32(X, B, Y, -8, 8, 8, 1, 0, V.kMfmaF32, good).code == IA
    assert m.launch_gemm_f32(X, None, Y, 8, 8, 8, 1, 0, V.kMfmaF32, good).code == IA
    assert m.launch_gemm_f32(X, B, Y, 1 << 31, 8, 8, 1, 0, V.kMfmaF32, good).code == IA
    # unsupported (variant, tile) pairs: no fallback
    assert m.launch_gemm_f32(X, B, Y, 8, 8, 8, 1, 0, V.kTiledSmem, T()).code == IA
    assert m.launch_gemm_f32(X, B, Y, 8, 8, 8, 1, 0, V.kWarpTile, T(32, 32, 32, 1, 1)).code == IA
    st = m.launch_gemm_f32(X, B, Y, 8, 8, 8, 1, 0, V.kMfmaF32, T(128, 128, 8, 8, 8))
    assert st.code == IA and "no fallback" in st.message
    assert m.launch_gemm_f32(X, B, Y, 8, 8, 8, 1, 0, V.kMfmaF32, T(100, 128, 8, 8, 8)).code == IA
    assert m.launch_gemm_f32(X, B, Y, 8, 8, 8, 1, 0, 42, good).code == IA
    # the ladder's 2-D grid caps the row tiles at 65535
    assert m.launch_gemm_f32(X, B, Y, 65536 * 4 + 1, 8, 8, 1, 0, V.kNaive, T()).code == IA
    # tiles x lanes beyond the grid's 32-bit work size: 4096^2 32 x 32 tiles of 256 lanes,
    # and 2^26 column tiles of 64 lanes for the uncoalesced ladder kernel
    st = m.launch_gemm_f32(X, B, Y, 1 << 17, 1 << 17, 8, 1, 0, V.kMfmaF32, T(32, 32, 32, 2, 2))
    assert st.code == IA and "32-bit work size" in st.message
    st = m.launch_gemm_f32(X, B, Y, 8, 1 << 28, 8, 1, 0, V.kNaiveUncoalesced, T())
    assert st.code == IA and "32-bit work size" in st.message


def test_gemm_bias_act_rejections(cpu_only):
    """The fused GEMM + bias + activation entry point: launch_gemm_f32's kMfmaF32
    validation plus the bias, the activation and the output's aliasing."""
    m = cpu_only
    IA = m.StatusCode.kInvalidArgument
    T = m.GemmTile
    good = m.MFMA_TILES[0]
    f = m.launch_gemm_bias_act_f32
    assert f(X, B, W, Y, 0, 8, 8, 1, 3, good).ok()                  # empty: no launch
    assert f(None, None, None, None, 8, 0, 8, 1, 3, good).ok()
    assert f(X, B, None, Y, 8, 8, 8, 1, 3, good).code == IA         # null bias
    assert f(X, None, W, Y, 8, 8, 8, 1, 3, good).code == IA         # null b
    assert f(X, B, W, None, 8, 8, 8, 1, 3, good).code == IA         # null y
    for out in (X, B, W):                                           # y aliases an input
        assert f(X, B, W, out, 8, 8, 8, 1, 3, good).code == IA
    assert f(X, B, W, Y, -8, 8, 8, 1, 3, good).code == IA
    assert f(X, B, W, Y, 8, 8, -1, 1, 3, good).code == IA
    assert f(X, B, W, Y, 8, 8, 1 << 31, 1, 3, good).code == IA
    st = f(X, B, W, Y, 8, 8, 8, 1, 4, good)                         # bad activation
    assert st.code == IA and "Activation" in st.message
    assert f(X, B, W, Y, 8, 8, 8, 1, -1, good).code == IA
    st = f(X, B, W, Y, 8, 8, 8, 1, 3, T(128, 128, 8, 8, 8))         # not a kMfmaF32 tile
    assert st.code == IA and "no fallback" in st.message
    st = f(X, B, W, Y, 1 << 17, 1 << 17, 8, 1, 3, T(32, 32, 32, 2, 2))
    assert st.code == IA and "32-bit work size" in st.message


def test_default_lp_tile(mcke):
    assert mcke.gemm_lp_default_tile(8192, 8192, 8192).astuple() == (256, 256, 64, 16, 16)
    assert mcke.gemm_lp_default_tile(4096, 4096, 4096).astuple() == (256, 256, 64, 16, 16)
    assert mcke.gemm_lp_default_tile(2048, 2048, 2048).astuple() == (128, 128, 64, 8, 8)
    assert mcke.gemm_lp_default_tile(1024, 1024, 1024).astuple() == (64, 64, 64, 4, 4)


def test_gemm_lp_rejections(cpu_only):
    m = cpu_only
    IA = m.StatusCode.kInvalidArgument
    D, T = m.DType, m.GemmTile
    good = m.LP_TILES[0]
    bf, f16, f32 = D.kBF16, D.kF16, D.kF32
    assert m.launch_gemm_lp(X, B, Y, bf, f32, 0, 8, 8, 1, 0, good).ok()              # m == 0
    assert m.launch_gemm_lp(None, None, None, bf, bf, 8, 0, 8, 1, 0, good).ok()      # n == 0
    assert m.launch_gemm_lp(X, B, X, bf, f32, 8, 8, 8, 1, 0, good).code == IA        # a == c
    assert m.launch_gemm_lp(X, B, B, f16, f16, 8, 8, 8, 1, 0, good).code == IA       # b == c
    assert m.launch_gemm_lp(X, B, Y, bf, f32, -8, 8, 8, 1, 0, good).code == IA
    assert m.launch_gemm_lp(X, None, Y, bf, f32, 8, 8, 8, 1, 0, good).code == IA
    assert m.launch_gemm_lp(X, B, Y, bf, f32, 8, 8, 1 << 31, 1, 0, good).code == IA
    st = m.launch_gemm_lp(X, B, Y, f32, f32, 8, 8, 8, 1, 0, good)                    # fp32 in
    assert st.code == IA and "ab_dtype" in st.message
    st = m.launch_gemm_lp(X, B, Y, bf, f16, 8, 8, 8, 1, 0, good)                     # mixed out
    assert st.code == IA and "c_dtype" in st.message
    st = m.launch_gemm_lp(X, B, Y, bf, f32, 8, 8, 8, 1, 0, T(256, 256, 32, 16, 16))  # fp32 tile
    assert st.code == IA and "no fallback" in st.message
    st, _ = m.gemm_lp_kernel_attrs(f16, f32, T(128, 128, 8, 8, 8))
    assert st.code == IA
    st = m.launch_gemm_lp(X, B, Y, bf, f32, 1 << 18, 1 << 18, 64, 1, 0, T(64, 64, 64, 4, 4))
    assert st.code == IA and "32-bit work size" in st.message                       # 2^24 tiles
