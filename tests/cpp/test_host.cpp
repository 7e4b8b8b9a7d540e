// test_host.cpp -- CPU tests of the C++ host layers (no GPU needed).
//
// Covers: Status/StatusOr, GemmTile validity and the CDNA occupancy model, the
// double-buffer schedule, the online-softmax algebra, the kernels.hpp launchers'
// argument rejection (fake pointers, only when no GPU is visible), Shape, the
// graph (finalize, depth/ALAP/slack, dead nodes, live ranges), the three stream
// policies with their event and wait counts, happens-before, the memory planner
// (exact bytes, unsafe arm flagged by the race verifier, random-DAG fuzz) and the
// buddy allocator on host memory with fake streams.  Expected values are derived
// in the comments next to each check.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <random>
#include <set>
#include <string>

#include <unistd.h>

#include "check.hpp"
#include "../../mini-cuda-kernel-engine_amd/csrc/fast_div.hpp"
#include "mcke/graph/cost_model.hpp"
#include "mcke/graph/executor.hpp"
#include "mcke/graph/graph.hpp"
#include "mcke/graph/memory_plan.hpp"
#include "mcke/graph/schedule.hpp"
#include "mcke/kernels/kernels.hpp"
#include "mcke/kernels/softmax_online.hpp"
#include "mcke/memory/buddy_allocator.hpp"
#include "mcke/memory/buddy_math.hpp"
#include "mcke/memory/freelist_allocator.hpp"
#include "mcke/profiling/host_timer.hpp"
#include "mcke/profiling/profiler.hpp"

using namespace mcke;
namespace K = mcke::kernels;

// ---------------------------------------------------------------------------
TEST(status_and_statusor) {
  CHECK(OkStatus().ok());
  const Status s = InvalidArgumentError("bad");
  CHECK(!s.ok() && s.code() == StatusCode::kInvalidArgument && s.to_string() == "InvalidArgument: bad");
  StatusOr<int> v = 7;
  CHECK(v.ok() && *v == 7);
  StatusOr<int> e = UnimplementedError("x");
  CHECK(!e.ok() && e.status().code() == StatusCode::kUnimplemented);
  CHECK(static_cast<int>(StatusCode::kDeviceError) == MCKE_STATUS_DEVICE_ERROR);
  auto f = []() -> Status {
    MCKE_ASSIGN_OR_RETURN(int a, StatusOr<int>(3));
    MCKE_ASSIGN_OR_RETURN(int b, StatusOr<int>(InternalError("stop")));
    return a + b > 0 ? OkStatus() : InternalError("unreachable");
  };
  CHECK(f().code() == StatusCode::kInternal);
}

// ---------------------------------------------------------------------------
TEST(gemm_tile_validity_wave64) {
  CHECK_EQ(K::threads_per_block(K::GemmTile{}), 256);
  CHECK(K::tile_is_self_consistent(K::GemmTile{}));
  CHECK(K::tile_is_self_consistent(K::GemmTile{32, 32, 32, 1, 1}));        // 1024 lanes
  CHECK(!K::tile_is_self_consistent(K::GemmTile{16, 16, 8, 4, 4}));        // 16 lanes: not a wave
  // 64x32 with 4x4: (16 x 8) = 128 lanes (2 waves); bm*bk = 512 and bk*bn = 256 both divide by 128.
  CHECK(K::tile_is_self_consistent(K::GemmTile{64, 32, 8, 4, 4}));
  CHECK(K::threads_per_block(K::GemmTile{64, 32, 8, 4, 4}) == 128);
  // 32x32 with 4x4: 64 lanes, but bk*bn = 8*32 = 256 and bm*bk = 256 divide: valid;
  // 32x16 with 4x4: 32 lanes, half a wave: invalid.
  CHECK(K::tile_is_self_consistent(K::GemmTile{32, 32, 8, 4, 4}));
  CHECK(!K::tile_is_self_consistent(K::GemmTile{32, 16, 8, 4, 4}));
  CHECK(!K::tile_is_self_consistent(K::GemmTile{128, 128, 8, 0, 8}));
  CHECK(!K::tile_is_self_consistent(K::GemmTile{100, 128, 8, 8, 8}));      // 100 % 8 != 0
  for (const auto& t : {K::GemmTile{256, 256, 32, 16, 16}, K::GemmTile{256, 256, 16, 16, 16},
                        K::GemmTile{128, 128, 32, 8, 8}, K::GemmTile{128, 128, 16, 8, 8},
                        K::GemmTile{64, 64, 32, 4, 4}, K::GemmTile{32, 32, 32, 2, 2}}) {
    CHECK(K::tile_is_self_consistent(t));
    CHECK_EQ(K::threads_per_block(t), 256);
    CHECK(K::gemm_tile_is_supported(K::GemmVariant::kMfmaF32, t));
    CHECK(!K::gemm_tile_is_supported(K::GemmVariant::kWarpTile, t));
  }
  CHECK(!K::gemm_tile_is_supported(K::GemmVariant::kMfmaF32, K::GemmTile{}));
  CHECK(!K::gemm_tile_is_supported(K::GemmVariant::kMfmaF32, K::GemmTile{32, 32, 16, 2, 2}));
  // The launcher's default tile is always one the host model accepts.
  for (std::int64_t n : {1, 100, 256, 512, 1024, 3072, 4096, 6144, 8192})
    CHECK(K::gemm_tile_is_supported(K::GemmVariant::kMfmaF32, K::mfma_default_tile(n, n, n)));
  CHECK(K::gemm_tile_is_supported(K::GemmVariant::kWarpTile, K::GemmTile{}));
  CHECK(!K::gemm_tile_is_supported(K::GemmVariant::kTiledSmem, K::GemmTile{}));
  CHECK(K::gemm_tile_is_supported(K::GemmVariant::kTiledSmem, K::GemmTile{32, 32, 32, 1, 1}));
  CHECK(K::gemm_tile_is_supported(K::GemmVariant::kNaive, K::GemmTile{1, 2, 3, 4, 5}));   // ignores the tile
  CHECK(K::gemm_tile_is_supported(K::GemmVariant::kCublasRef, K::GemmTile{1, 2, 3, 4, 5}));
  // smem: (bk*(bm+pad) + bk*bn) floats, doubled when double-buffered.
  CHECK_EQ(K::smem_bytes(K::GemmTile{}, false), std::size_t{8192});
  CHECK_EQ(K::smem_bytes(K::GemmTile{}, true, 4), std::size_t{(8 * 132 + 8 * 128) * 4 * 2});
  CHECK_EQ(static_cast<int>(K::GemmVariant::kMfmaF32), 8);
}

TEST(dbuf_schedule_exhaustive) {
  for (std::int64_t n = 0; n <= 200; ++n) {
    const auto s = K::dbuf_schedule(n);
    CHECK_EQ(s.pair_iters * 2 + (s.has_tail ? 1 : 0), n);
    CHECK(s.has_tail == (n % 2 == 1));
  }
  CHECK_EQ(K::dbuf_schedule(-3).pair_iters, 0);
}

TEST(occupancy_model_cdna) {
  const DeviceInfo d = mi355x_device_info();
  // 256 lanes = 4 waves = 1 wave per SIMD per workgroup.
  // 512 VGPRs (the 256x256 MFMA tile): 512/512 = 1 wave per SIMD -> 1 workgroup;
  // LDS 139264 B rounds to 139264 (512-multiple) -> 160K/139264 = 1.
  auto e = K::occupancy_blocks_per_sm(d, 256, 512, 139264);
  CHECK_EQ(e.blocks_per_sm, 1);
  CHECK(e.tied);   // registers and LDS both allow exactly 1
  // 168 VGPRs -> round to 168 -> 512/168 = 3 waves per SIMD; LDS 69632 -> 2 per CU.
  e = K::occupancy_blocks_per_sm(d, 256, 168, 69632);
  CHECK_EQ(e.by_registers, 3);
  CHECK_EQ(e.by_smem, 2);
  CHECK_EQ(e.blocks_per_sm, 2);
  CHECK(e.limiter == K::OccupancyLimiter::kSharedMemory);
  CHECK(std::fabs(e.occupancy - 512.0 / 2048.0) < 1e-12);
  // No LDS, 32 VGPRs: registers allow 512/32 = 16 -> capped at 8 waves per SIMD;
  // lanes cap 2048/256 = 8 blocks; 8 ties with registers -> the lanes cap is reported.
  e = K::occupancy_blocks_per_sm(d, 256, 32, 0);
  CHECK_EQ(e.by_registers, 8);
  CHECK_EQ(e.by_threads, 8);
  CHECK_EQ(e.blocks_per_sm, 8);
  CHECK(e.limiter == K::OccupancyLimiter::kThreadsPerSm && e.tied);
  // 1024-lane workgroup = 16 waves = 4 per SIMD: 100 VGPRs -> round 104 -> 4 waves/SIMD -> 1 block.
  e = K::occupancy_blocks_per_sm(d, 1024, 100, 0);
  CHECK_EQ(e.by_registers, 1);
  CHECK_EQ(e.blocks_per_sm, 1);
  // Will not launch: LDS beyond the CU, or more lanes than a workgroup may have.
  CHECK(K::occupancy_blocks_per_sm(d, 256, 64, 200 * 1024).limiter == K::OccupancyLimiter::kInvalid);
  CHECK(K::occupancy_blocks_per_sm(d, 2048, 64, 0).blocks_per_sm == 0);
  CHECK(K::occupancy_blocks_per_sm(DeviceInfo{}, 256, 64, 0).blocks_per_sm == 0);
}

// ---------------------------------------------------------------------------
TEST(online_softmax_algebra) {
  const K::OnlineState id = K::online_identity();
  const K::OnlineState e = K::online_combine(id, id);
  CHECK(!std::isnan(e.m) && !std::isnan(e.d) && e.d == 0.0f);
  std::mt19937 rng(3);
  std::normal_distribution<float> nd(0.f, 5.f);
  for (int n : {1, 2, 17, 64, 1000}) {
    std::vector<float> x(n);
    for (auto& v : x) v = nd(rng);
    K::OnlineState s = id;
    for (float v : x) s = K::online_update(s, v);
    double m = -INFINITY;
    for (float v : x) m = std::max(m, static_cast<double>(v));
    double d = 0;
    for (float v : x) d += std::exp(static_cast<double>(v) - m);
    CHECK(s.m == static_cast<float>(m));
    CHECK(std::fabs(s.d - d) <= 1e-5 * d);
    // split into two halves and combine (both orders)
    K::OnlineState a = id, b = id;
    for (int i = 0; i < n; ++i) (i < n / 2 ? a : b) = K::online_update(i < n / 2 ? a : b, x[i]);
    const K::OnlineState ab = K::online_combine(a, b), ba = K::online_combine(b, a);
    CHECK(ab.m == ba.m && std::fabs(ab.d - ba.d) <= 1e-6f * ab.d);
    CHECK(std::fabs(ab.d - d) <= 1e-5 * d);
  }
}

// ---------------------------------------------------------------------------
static bool no_gpu() { return device_count() == 0; }

TEST(launchers_reject_bad_arguments_without_launching) {
  if (!no_gpu()) {
    std::printf("  (skipped: a GPU is visible)\n");
    return;
  }
  auto* X = reinterpret_cast<float*>(0x10000);
  auto* Y = reinterpret_cast<float*>(0x20000);
  auto* B = reinterpret_cast<float*>(0x30000);
  rt::StreamHandle s{};
  CHECK(K::launch_bias_act_f32(X, B, Y, 0, 8, K::Activation::kGeluTanh, 4, s).ok());
  CHECK(K::launch_bias_act_f32(X, B, X, 4, 8, K::Activation::kGeluTanh, 4, s).code() == StatusCode::kInvalidArgument);
  CHECK(K::launch_bias_act_f32(X, B, Y, 4, 6, K::Activation::kGeluTanh, 4, s).code() == StatusCode::kInvalidArgument);
  CHECK(K::launch_row_reduce_f32(X, Y, 4, 8, K::ReduceKind::kSum, K::ReduceVariant::kTwoPass, s).code() ==
        StatusCode::kUnimplemented);
  CHECK(K::launch_row_softmax_f32(X, X, 4, 8, K::SoftmaxVariant::kOnlineOnePass, s).code() ==
        StatusCode::kInvalidArgument);
  CHECK(K::launch_gemm_f32(X, B, X, 8, 8, 8, 1.f, 0.f, K::GemmVariant::kMfmaF32, K::GemmTile{256, 256, 32, 16, 16}, s)
            .code() == StatusCode::kInvalidArgument);
  const Status st = K::launch_gemm_f32(X, B, Y, 8, 8, 8, 1.f, 0.f, K::GemmVariant::kTiledSmem, K::GemmTile{}, s);
  CHECK(st.code() == StatusCode::kInvalidArgument && st.message().find("no fallback") != std::string::npos);
  CHECK(K::max_vector_width_f32(X, 4096) == 4 && K::max_vector_width_f32(X, 4094) == 2);
  CHECK(K::row_reduce_workspace_bytes(1, 1 << 26, K::ReduceVariant::kTwoPass) == 256 * 4);
  CHECK(K::mfma_default_tile(8192, 8192, 8192).bm == 256);
}

// ---------------------------------------------------------------------------
TEST(shape_basics) {
  const Shape s{2, 3, 4};
  CHECK(s.rank() == 3 && s.numel() == 24 && s.rows() == 6 && s.cols() == 4);
  CHECK(s.stride(0) == 12 && s.stride(1) == 4 && s.stride(2) == 1 && s.is_contiguous());
  CHECK(s.bytes(DType::kF32) == 96 && s.to_string() == "[2,3,4]");
  const dim_t idx[3] = {1, 2, 3};
  CHECK(s.offset_of(idx) == 23);
  CHECK(Shape{5}.rows() == 1 && Shape{5}.cols() == 5);
}

// ---------------------------------------------------------------------------
// Graph builders (the reference's bench topologies, graph_bench.cpp:120-215).
static OpPtr bias_act(BiasActParams::Act a = BiasActParams::Act::kGeluTanh) {
  BiasActParams p;
  p.act = a;
  return std::make_unique<BiasActOp>(p);
}

struct Built {
  Graph g;
  std::vector<TensorId> inputs, outputs;
};

static Built chain(int n, dim_t rows, dim_t cols) {
  Built b;
  const TensorId x = *b.g.add_input(Shape{rows, cols}, DType::kF32, "x");
  const TensorId bi = *b.g.add_input(Shape{cols}, DType::kF32, "bias");
  b.inputs = {x, bi};
  TensorId cur = x;
  for (int i = 0; i < n; ++i) cur = (*b.g.add_node(bias_act(), {cur, bi}, "n" + std::to_string(i)))[0];
  (void)b.g.mark_output(cur);
  b.outputs = {cur};
  (void)b.g.finalize();
  return b;
}

static Built fanout(int branches, int depth, dim_t rows, dim_t cols) {
  Built b;
  const TensorId x = *b.g.add_input(Shape{rows, cols}, DType::kF32, "x");
  const TensorId bi = *b.g.add_input(Shape{cols}, DType::kF32, "bias");
  b.inputs = {x, bi};
  for (int k = 0; k < branches; ++k) {
    TensorId cur = x;
    for (int d = 0; d < depth; ++d)
      cur = (*b.g.add_node(bias_act(), {cur, bi}, "b" + std::to_string(k) + "n" + std::to_string(d)))[0];
    (void)b.g.mark_output(cur);
    b.outputs.push_back(cur);
  }
  (void)b.g.finalize();
  return b;
}

// a -> {b, c} -> d (diamond)
static Built diamond(dim_t rows, dim_t cols) {
  Built b;
  const TensorId x = *b.g.add_input(Shape{rows, cols}, DType::kF32, "x");
  const TensorId bi = *b.g.add_input(Shape{cols}, DType::kF32, "bias");
  const TensorId a = (*b.g.add_node(bias_act(), {x, bi}, "a"))[0];
  const TensorId l = (*b.g.add_node(bias_act(), {a, bi}, "l"))[0];
  const TensorId r = (*b.g.add_node(std::make_unique<ReduceOp>(ReduceParams{}), {a}, "r"))[0];
  GemmParams gp;
  gp.variant = K::GemmVariant::kMfmaF32;
  gp.auto_tile = true;
  // d = l (rows x cols) times a [cols x cols] weight: use a second input.
  const TensorId w = *b.g.add_input(Shape{cols, cols}, DType::kF32, "w");
  const TensorId d = (*b.g.add_node(std::make_unique<GemmOp>(gp), {l, w}, "d"))[0];
  (void)b.g.mark_output(d);
  (void)b.g.mark_output(r);
  b.outputs = {d, r};
  (void)b.g.finalize();
  return b;
}

TEST(graph_finalize_depths_and_dead_nodes) {
  Built b = diamond(64, 64);
  CHECK(b.g.finalized());
  // nodes: 0 a (depth 0), 1 l (1), 2 r (1), 3 d (2)
  CHECK(b.g.node(0).depth == 0 && b.g.node(1).depth == 1 && b.g.node(2).depth == 1 && b.g.node(3).depth == 2);
  // r's only successor... r has none; its ALAP depth is the critical depth (2), slack 1.
  CHECK(b.g.node(2).alap_depth == 2 && b.g.node(2).slack == 1);
  CHECK(b.g.node(1).slack == 0 && b.g.node(0).slack == 0);
  CHECK(b.g.dead_nodes().empty());
  CHECK(*b.g.max_level_width() == 2);
  CHECK(b.g.node(3).preds == std::vector<NodeId>{1});
  CHECK((b.g.node(0).succs == std::vector<NodeId>{1, 2}));

  // A node that reaches no output is dead.
  Graph g;
  const TensorId x = *g.add_input(Shape{4, 4}, DType::kF32, "x");
  const TensorId bi = *g.add_input(Shape{4}, DType::kF32, "b");
  const TensorId y = (*g.add_node(bias_act(), {x, bi}, "live"))[0];
  (void)(*g.add_node(bias_act(), {x, bi}, "dead"));
  CHECK_OK(g.mark_output(y));
  CHECK_OK(g.finalize());
  CHECK(g.dead_nodes() == std::vector<NodeId>{1});
}

TEST(graph_errors) {
  Graph g;
  CHECK(g.finalize().code() == StatusCode::kFailedPrecondition);   // no nodes
  CHECK(g.add_input(Shape{0, 4}, DType::kF32, "bad").status().code() == StatusCode::kInvalidArgument);
  const TensorId x = *g.add_input(Shape{4, 4}, DType::kF32, "x");
  const TensorId bi = *g.add_input(Shape{5}, DType::kF32, "b");
  CHECK(g.add_node(bias_act(), {x, bi}, "mismatch").status().code() == StatusCode::kInvalidArgument);
  CHECK(g.add_node(bias_act(), {x, 99}, "oob").status().code() == StatusCode::kInvalidArgument);
  CHECK(g.add_node(nullptr, {x}, "null").status().code() == StatusCode::kInvalidArgument);
  const TensorId b4 = *g.add_input(Shape{4}, DType::kF32, "b4");
  (void)(*g.add_node(bias_act(), {x, b4}, "ok"));
  CHECK(g.finalize().code() == StatusCode::kInvalidArgument);      // no outputs
  GemmParams gp;
  gp.beta = 1.0f;
  CHECK(g.add_node(std::make_unique<GemmOp>(gp), {x, x}, "beta").status().code() == StatusCode::kUnimplemented);
  GemmParams bad_tile;
  bad_tile.variant = K::GemmVariant::kTiledSmem;   // default tile is not (32,32,32,1,1)
  CHECK(g.add_node(std::make_unique<GemmOp>(bad_tile), {x, x}, "tile").status().code() ==
        StatusCode::kInvalidArgument);
  SoftmaxParams unstable;
  unstable.numerically_stable = false;
  CHECK(g.add_node(std::make_unique<SoftmaxOp>(unstable), {x}, "u").status().code() == StatusCode::kUnimplemented);
  ReduceParams axis0;
  axis0.axis = 0;
  CHECK(g.add_node(std::make_unique<ReduceOp>(axis0), {x}, "ax").status().code() == StatusCode::kInvalidArgument);
}

TEST(op_costs_are_the_ideal_formulas) {
  GemmParams gp;
  const GemmOp gemm(gp);
  const OpCost g = gemm.cost({Shape{8192, 8192}, Shape{8192, 8192}});
  CHECK(g.flops == 2ull * 8192 * 8192 * 8192);
  CHECK(g.bytes == 3ull * 8192 * 8192 * 4);
  const OpCost ba = BiasActOp(BiasActParams{BiasActParams::Act::kGeluTanh}).cost({Shape{16384, 4096}, Shape{4096}});
  CHECK(ba.bytes == 536887296ull && ba.flops == 10ull * 16384 * 4096);
  CHECK(BiasActOp(BiasActParams{BiasActParams::Act::kGeluErf}).cost({Shape{2, 2}, Shape{2}}).flops == 4 * 22);
  CHECK(BiasActOp(BiasActParams{BiasActParams::Act::kNone}).cost({Shape{2, 2}, Shape{2}}).flops == 4);
  const OpCost rs = ReduceOp(ReduceParams{}).cost({Shape{8192, 8192}});
  CHECK(rs.bytes == 268468224ull && rs.flops == 8192ull * 8191);
  ReduceParams mx;
  mx.kind = ReduceParams::Kind::kMax;
  CHECK(ReduceOp(mx).cost({Shape{8192, 8192}}).flops == 0);
  const OpCost sm = SoftmaxOp(SoftmaxParams{}).cost({Shape{32768, 4096}});
  CHECK(sm.bytes == 1073741824ull && sm.flops == 5ull * 32768 * 4096);
  // shapes
  CHECK((*ReduceOp(ReduceParams{}).infer_shapes({Shape{3, 5, 7}}))[0] == (Shape{3, 5}));
  CHECK((*ReduceOp(ReduceParams{}).infer_shapes({Shape{7}}))[0] == (Shape{1}));
  // roofline time: a 8192^3 GEMM at 157.3 TFLOP/s vs its bytes at 8 TB/s: compute-bound.
  const Roofline rl = mi355x_roofline();
  CHECK(!rl.memory_bound(g.arithmetic_intensity()) && rl.memory_bound(ba.arithmetic_intensity()));
  CHECK(std::fabs(rl.ridge_point_ai() - 157.3e12 / 8e12) < 1e-9);
}

// The roofline cost model that balances streams (the reference's
// test_cost_model_roofline, tests/test_graph_host.cpp:816-858), on MI355X's
// published figures: a 4096^3 GEMM is 1.374e11 flops / 157.3e12 = 0.874 ms of
// arithmetic against 201 MB / 8e12 = 0.025 ms of traffic (compute-bound); softmax
// 8192 x 4096 is 2.68e8 B / 8e12 = 0.0336 ms of traffic against 1.68e8 flops /
// 157.3e12 = 0.0011 ms (memory-bound).  A zero roofline costs 0, not infinity.
TEST(cost_model_roofline) {
  const Roofline rl = mi355x_roofline();
  const OpCost gc = GemmOp(GemmParams{}).cost({Shape{4096, 4096}, Shape{4096, 4096}});
  const double g_ms = plan_cost_ms(gc, rl);
  CHECK(std::fabs(g_ms - 2.0 * 4096.0 * 4096.0 * 4096.0 / 157.3e12 * 1e3) < 1e-9);
  CHECK(!op_is_memory_bound(gc, rl));
  const OpCost sc = SoftmaxOp(SoftmaxParams{}).cost({Shape{8192, 4096}});
  const double s_ms = plan_cost_ms(sc, rl);
  CHECK(std::fabs(s_ms - 2.0 * 8192.0 * 4096.0 * 4.0 / 8e12 * 1e3) < 1e-12);
  CHECK(op_is_memory_bound(sc, rl));
  CHECK(g_ms / s_ms > 20.0);
  const Roofline zero{};
  CHECK(plan_cost_ms(gc, zero) == 0.0);
  CHECK(zero.attainable_tflops(1.0) == 0.0 && zero.ridge_point_ai() == 0.0);
}

// Profiler::summary_table keeps three decimals on every row, not only the first
// (the reference's test_summary_table_precision, tests/test_host_core.cpp:2448-2483:
// a sticky setprecision(1) from the %peak column once cut rows 2.. to one
// decimal), with its frozen column widths; write_csv writes the reference's
// 13 columns (src/core/profiler.cpp:95-113) with each derived column computed
// from the record.
TEST(profiler_summary_table_and_csv) {
  Profiler prof;
  KernelRecord a;
  a.name = "k";
  a.variant = "first";
  a.median_ms = 1.23456;
  a.min_ms = 1.11111;
  a.flops = 100;
  a.bytes = 400;
  a.iterations = 20;
  KernelRecord b = a;
  b.variant = "second";
  b.median_ms = 0.52349;
  b.min_ms = 0.51237;
  prof.add(a);
  prof.add(b);
  Roofline rl;
  rl.peak_gb_s = 235.4;
  rl.peak_tflops = 8.130;
  const std::string t = prof.summary_table(rl);
  for (const char* s : {"1.235", "1.111", "0.523", "0.512"}) CHECK(t.find(s) != std::string::npos);
  CHECK(t.find(std::string(117, '-')) != std::string::npos);
  // A data row: 22 + 30 + 10 + 10 + 10 + 10 + 8 + 10 characters, then "  memory".
  const std::size_t row2 = t.find("k     ", t.find("first"));
  CHECK(row2 != std::string::npos);
  const std::string line = t.substr(row2, t.find('\n', row2) - row2);
  CHECK(line.size() == 110 + 8 && line.substr(110) == "  memory");
  CHECK(line.substr(22, 6) == "second");

  const std::string path = "/tmp/mcke_test_profiler_" + std::to_string(::getpid()) + ".csv";
  CHECK_OK(prof.write_csv(path, rl));
  std::FILE* f = std::fopen(path.c_str(), "r");
  CHECK(f != nullptr);
  std::string text;
  char chunk[512];
  while (std::size_t got = std::fread(chunk, 1, sizeof chunk, f)) text.append(chunk, got);
  std::fclose(f);
  std::remove(path.c_str());
  // Default stream precision (6 significant digits): 400 B / 1.23456 ms = 0.000324002 GB/s,
  // 100 flops -> 8.1e-08 TFLOP/s; AI 0.25 < ridge 34.5 -> memory; attainable
  // 0.25 x 235.4 GB/s = 0.05885 TFLOP/s; efficiency 8.10005e-08 / 0.05885 = 1.37639e-04 %.
  CHECK(text ==
        "kernel,variant,median_ms,min_ms,iterations,ideal_flops,ideal_bytes,achieved_gb_s,"
        "achieved_tflops,arithmetic_intensity,attainable_tflops,efficiency_pct,bound\n"
        "k,first,1.23456,1.11111,20,100,400,0.000324002,8.10005e-08,0.25,0.05885,0.000137639,memory\n"
        "k,second,0.52349,0.51237,20,100,400,0.000764102,1.91026e-07,0.25,0.05885,0.000324597,memory\n");
  CHECK(!prof.write_csv("/nonexistent-dir/x.csv", rl).ok());
}

// ---------------------------------------------------------------------------
TEST(schedule_fanout_policies) {
  Built b = fanout(4, 4, 64, 64);
  const Roofline rl{1.0, 8000.0};
  // chain-greedy: every branch continues its own stream -> no events, no waits.
  auto cg = plan_streams(b.g, SchedulePolicy::kChainGreedy, 4, rl);
  CHECK(cg.ok());
  CHECK_EQ(cg->num_streams_used, std::size_t{4});
  CHECK_EQ(cg->num_events, std::size_t{0});
  CHECK_EQ(cg->waits_dedup, std::size_t{0});
  CHECK_OK(verify_plan_ordering(b.g, *cg));
  // level-parallel: 3 level boundaries x 4 streams x 3 other streams = 36 waits;
  // every node of levels 0..2 is waited on -> 12 records.
  auto lp = plan_streams(b.g, SchedulePolicy::kLevelParallel, 4, rl);
  CHECK(lp.ok());
  CHECK_EQ(lp->num_events, std::size_t{12});
  CHECK_EQ(lp->waits_raw, std::size_t{36});
  CHECK_EQ(lp->waits_dedup, std::size_t{36});
  CHECK_OK(verify_plan_ordering(b.g, *lp));
  // sequential: one stream, nothing to record.
  auto sq = plan_streams(b.g, SchedulePolicy::kSequential, 4, rl);
  CHECK(sq.ok() && sq->num_streams_used == 1 && sq->num_events == 0);
  // more streams than nodes in a level: only 4 used.
  auto cg8 = plan_streams(b.g, SchedulePolicy::kChainGreedy, 8, rl);
  CHECK(cg8.ok() && cg8->num_streams_used == 4 && cg8->num_streams_requested == 8);
  CHECK(plan_streams(b.g, SchedulePolicy::kChainGreedy, 0, rl).status().code() == StatusCode::kInvalidArgument);
}

TEST(schedule_chain_has_no_events) {
  Built b = chain(16, 32, 32);
  const Roofline rl{1.0, 8000.0};
  for (auto p : {SchedulePolicy::kSequential, SchedulePolicy::kLevelParallel, SchedulePolicy::kChainGreedy}) {
    auto sa = plan_streams(b.g, p, 4, rl);
    CHECK(sa.ok());
    // width 1: one stream is enough for every policy, so no cross-stream events.
    CHECK_EQ(sa->num_streams_used, std::size_t{1});
    CHECK_EQ(sa->num_events, std::size_t{0});
  }
}

TEST(schedule_diamond_and_happens_before) {
  Built b = diamond(64, 64);
  auto sa = plan_streams(b.g, SchedulePolicy::kChainGreedy, 2, Roofline{1.0, 8000.0});
  CHECK(sa.ok());
  // topo: a(0), l(1), r(2), d(3).  a -> s0; l: one pred (a) not continued -> s0;
  // r: one pred (a) already continued -> least loaded stream = s1; d: pred l -> s0.
  CHECK(sa->stream_of[0] == 0 && sa->stream_of[1] == 0 && sa->stream_of[2] == 1 && sa->stream_of[3] == 0);
  // r waits on a's event: one record, one wait.
  CHECK_EQ(sa->num_events, std::size_t{1});
  CHECK_EQ(sa->waits_dedup, std::size_t{1});
  auto hb = sa->happens_before();
  CHECK(hb.ok());
  CHECK(hb->precedes(0, 1) && hb->precedes(0, 2) && hb->precedes(0, 3) && hb->precedes(1, 3));
  CHECK(hb->concurrent(2, 3) && hb->concurrent(1, 2));
  CHECK(!hb->precedes(3, 0));
}

TEST(schedule_prunes_waits_implied_by_clocks) {
  // P, X from x; Q = P.X; R = ba(P); Z = P.Q.  Chain-greedy on 3 streams at
  // 1 TFLOP/s: P -> s0, X -> s1, Q (two preds) -> s2 waiting on P and X, R (P's
  // heir) -> s0, Z (two preds) -> the least-loaded s1.  Z needs P and Q; Q has
  // already waited on P, so one wait (on Q) orders both: 4 cross-stream needs,
  // 3 waits, 3 events (P, X, Q).
  Graph g;
  const TensorId x = *g.add_input(Shape{64, 64}, DType::kF32, "x");
  const TensorId bi = *g.add_input(Shape{64}, DType::kF32, "b");
  GemmParams gp;
  gp.variant = K::GemmVariant::kMfmaF32;
  gp.auto_tile = true;
  const TensorId p = (*g.add_node(bias_act(), {x, bi}, "P"))[0];
  const TensorId xx = (*g.add_node(bias_act(), {x, bi}, "X"))[0];
  const TensorId q = (*g.add_node(std::make_unique<GemmOp>(gp), {p, xx}, "Q"))[0];
  const TensorId r = (*g.add_node(bias_act(), {p, bi}, "R"))[0];
  const TensorId z = (*g.add_node(std::make_unique<GemmOp>(gp), {p, q}, "Z"))[0];
  CHECK_OK(g.mark_output(r));
  CHECK_OK(g.mark_output(z));
  CHECK_OK(g.finalize());
  auto sa = plan_streams(g, SchedulePolicy::kChainGreedy, 3, Roofline{1.0, 8000.0});
  CHECK(sa.ok());
  // scheduled order P(0) X(1) Q(2) R(3) Z(4)
  CHECK((sa->stream_of == std::vector<std::uint16_t>{0, 1, 2, 0, 1}));
  CHECK_EQ(sa->waits_raw, std::size_t{4});
  CHECK_EQ(sa->waits_dedup, std::size_t{3});
  CHECK_EQ(sa->num_events, std::size_t{3});
  CHECK_EQ(sa->waits_of[4].size(), std::size_t{1});
  CHECK_EQ(sa->waits_of[4][0], sa->record_of[2]);
  CHECK_OK(verify_plan_ordering(g, *sa));
  auto hb = sa->happens_before();
  CHECK(hb.ok() && hb->precedes(0, 4) && hb->precedes(2, 4) && hb->concurrent(3, 4));
}

TEST(happens_before_rejects_malformed) {
  // two nodes sharing an issue index on one stream
  CHECK(!HappensBefore::build(1, {0, 0}, {0, 0}, {kNoEventId, kNoEventId}, {{}, {}}, {0, 1}).ok());
  // waiting on an event nobody records
  CHECK(!HappensBefore::build(2, {0, 1}, {0, 0}, {kNoEventId, kNoEventId}, {{}, {7}}, {0, 1}).ok());
  // gap in the issue indices
  CHECK(!HappensBefore::build(1, {0, 0}, {0, 2}, {kNoEventId, kNoEventId}, {{}, {}}, {0, 1}).ok());
  // stream out of range
  CHECK(!HappensBefore::build(1, {0, 1}, {0, 0}, {kNoEventId, kNoEventId}, {{}, {}}, {0, 1}).ok());
  // a well-formed cross-stream edge
  auto hb = HappensBefore::build(2, {0, 1}, {0, 0}, {0, kNoEventId}, {{}, {0}}, {0, 1});
  CHECK(hb.ok() && hb->precedes(0, 1) && !hb->precedes(1, 0));
}

// ---------------------------------------------------------------------------
TEST(memory_chain16_exact_bytes) {
  Built b = chain(16, 64, 64);   // every tensor 16 KiB, bias 256 B
  auto sa = plan_streams(b.g, SchedulePolicy::kSequential, 1, Roofline{1.0, 8000.0});
  auto hb = sa->happens_before();
  auto mp = plan_memory(b.g, *sa, *hb, MemoryPolicy::kReuseHappensBefore);
  CHECK(mp.ok());
  // x, 16 node outputs (last is the graph output), bias: 17 x 16 KiB + 256 naive.
  CHECK_EQ(mp->naive_bytes, std::size_t{17 * 16384 + 256});
  // x + two ping-pong intermediates + the output + the bias.
  CHECK_EQ(mp->arena_bytes, std::size_t{4 * 16384 + 256});
  CHECK_EQ(mp->buffers_used, std::size_t{5});
  CHECK_OK(verify_no_buffer_races(b.g, *sa, *hb, *mp));
  auto per = plan_memory(b.g, *sa, *hb, MemoryPolicy::kAllocPerTensor);
  CHECK(per.ok() && per->arena_bytes == per->naive_bytes);
  for (std::size_t t = 0; t < b.g.num_tensors(); ++t) CHECK(mp->offset_of[t] % kDeviceAlignment == 0);
}

TEST(memory_unsafe_arm_is_flagged) {
  // Fan-out on 4 streams: branches run concurrently.  Topological-position reuse
  // lets a later branch's tensor take an earlier branch's bytes with no ordering
  // between them: the race verifier must reject that plan, and the
  // happens-before plan must pass.
  Built b = fanout(4, 4, 64, 64);
  auto sa = plan_streams(b.g, SchedulePolicy::kChainGreedy, 4, Roofline{1.0, 8000.0});
  auto hb = sa->happens_before();
  auto naive = plan_memory(b.g, *sa, *hb, MemoryPolicy::kReuseTopoNaive);
  CHECK(naive.ok());
  CHECK(verify_no_buffer_races(b.g, *sa, *hb, *naive).code() == StatusCode::kInternal);
  auto safe = plan_memory(b.g, *sa, *hb, MemoryPolicy::kReuseHappensBefore);
  CHECK(safe.ok());
  CHECK_OK(verify_no_buffer_races(b.g, *sa, *hb, *safe));
  auto same = plan_memory(b.g, *sa, *hb, MemoryPolicy::kReuseSameStream);
  CHECK_OK(verify_no_buffer_races(b.g, *sa, *hb, *same));
  // Concurrency costs memory: 4 streams need more arena than 1.
  auto sa1 = plan_streams(b.g, SchedulePolicy::kSequential, 1, Roofline{1.0, 8000.0});
  auto hb1 = sa1->happens_before();
  auto one = plan_memory(b.g, *sa1, *hb1, MemoryPolicy::kReuseHappensBefore);
  CHECK(one->arena_bytes < safe->arena_bytes);
}

TEST(memory_and_schedule_fuzz_random_dags) {
  std::mt19937 rng(1234);
  for (int trial = 0; trial < 60; ++trial) {
    Graph g;
    const dim_t n = 32;
    std::vector<TensorId> pool{*g.add_input(Shape{n, n}, DType::kF32, "x")};
    const TensorId bi = *g.add_input(Shape{n}, DType::kF32, "b");
    const int nodes = 4 + static_cast<int>(rng() % 20);
    for (int i = 0; i < nodes; ++i) {
      const TensorId src = pool[rng() % pool.size()];
      const int kind = static_cast<int>(rng() % 3);
      TensorId out;
      if (kind == 0) {
        out = (*g.add_node(bias_act(), {src, bi}, "ba" + std::to_string(i)))[0];
      } else if (kind == 1) {
        out = (*g.add_node(std::make_unique<SoftmaxOp>(SoftmaxParams{}), {src}, "sm" + std::to_string(i)))[0];
      } else {
        const TensorId other = pool[rng() % pool.size()];
        GemmParams gp;
        gp.variant = K::GemmVariant::kMfmaF32;
        gp.auto_tile = true;
        out = (*g.add_node(std::make_unique<GemmOp>(gp), {src, other}, "mm" + std::to_string(i)))[0];
      }
      pool.push_back(out);
    }
    (void)g.mark_output(pool.back());
    if (rng() % 2) (void)g.mark_output(pool[pool.size() / 2]);
    CHECK_OK(g.finalize());
    for (auto sp : {SchedulePolicy::kSequential, SchedulePolicy::kLevelParallel, SchedulePolicy::kChainGreedy}) {
      for (int streams : {1, 2, 3, 4}) {
        auto sa = plan_streams(g, sp, streams, Roofline{1.0, 8000.0});
        if (!sa.ok()) {
          CHECK(false);
          continue;
        }
        CHECK_OK(verify_plan_ordering(g, *sa));
        auto hb = sa->happens_before();
        CHECK(hb.ok());
        for (auto mpol : {MemoryPolicy::kAllocPerTensor, MemoryPolicy::kReuseSameStream,
                          MemoryPolicy::kReuseHappensBefore}) {
          auto mp = plan_memory(g, *sa, *hb, mpol);
          CHECK(mp.ok());
          CHECK_OK(verify_no_buffer_races(g, *sa, *hb, *mp));
          CHECK(mp->arena_bytes <= mp->naive_bytes);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Buddy allocator on host memory with fake streams.
class HostBuddy : public BuddyAllocator {
 public:
  using BuddyAllocator::BuddyAllocator;
  // The base destructor would reach the base seams (hipFree on host memory).
  ~HostBuddy() override { release_all(); }
  mutable std::set<rt::StreamHandle> busy;
  int raw_allocs = 0, raw_frees = 0;

 protected:
  bool stream_completed(rt::StreamHandle s) const override { return busy.count(s) == 0; }
  void wait_stream(rt::StreamHandle s) const override { busy.erase(s); }
  StatusOr<void*> raw_alloc(std::size_t bytes) override {
    ++raw_allocs;
    void* p = std::aligned_alloc(256, bytes);
    if (!p) return OutOfMemoryError("host aligned_alloc failed");
    return p;
  }
  void raw_free(void* p) override {
    ++raw_frees;
    std::free(p);
  }
};

static rt::StreamHandle fake_stream(std::uintptr_t id) { return reinterpret_cast<rt::StreamHandle>(id * 0x100); }

static BuddyConfig small_cfg(ReusePolicy p) {
  BuddyConfig c;
  c.initial_slab_bytes = 1 << 20;
  c.large_alloc_threshold = 4 << 20;
  c.reuse_policy = p;
  return c;
}

// Destruction returns every slab and bypass allocation through the subclass's
// own memory seam, and waits for parked blocks' streams through its own
// completion seam (release_all() from the subclass destructor).
struct SeamLedger {
  int allocs = 0, frees = 0, waits = 0;
};
class LedgerBuddy : public BuddyAllocator {
 public:
  LedgerBuddy(BuddyConfig c, SeamLedger* l) : BuddyAllocator(c), l_(l) {}
  ~LedgerBuddy() override { release_all(); }

 protected:
  bool stream_completed(rt::StreamHandle) const override { return false; }
  void wait_stream(rt::StreamHandle) const override { ++l_->waits; }
  StatusOr<void*> raw_alloc(std::size_t bytes) override {
    ++l_->allocs;
    return std::aligned_alloc(256, bytes);
  }
  void raw_free(void* p) override {
    ++l_->frees;
    std::free(p);
  }

 private:
  SeamLedger* l_;
};
class LedgerFreeList : public FreeListAllocator {
 public:
  LedgerFreeList(FreeListConfig c, SeamLedger* l) : FreeListAllocator(c), l_(l) {}
  ~LedgerFreeList() override { release_all(); }

 protected:
  bool stream_completed(rt::StreamHandle) const override { return false; }
  void wait_stream(rt::StreamHandle) const override { ++l_->waits; }
  StatusOr<void*> raw_alloc(std::size_t bytes) override {
    ++l_->allocs;
    return std::aligned_alloc(256, bytes);
  }
  void raw_free(void* p) override {
    ++l_->frees;
    std::free(p);
  }

 private:
  SeamLedger* l_;
};

TEST(allocators_release_through_subclass_seams) {
  SeamLedger lb;
  {
    LedgerBuddy b(small_cfg(ReusePolicy::kCoarseStreamPoll), &lb);
    auto a = b.allocate(1000, fake_stream(1));
    auto big = b.allocate(8 << 20, fake_stream(1));     // above the threshold: bypass
    CHECK(a.ok() && big.ok());
    CHECK_OK(b.deallocate(*a, fake_stream(1)));          // parked: its stream never completes
  }
  CHECK_EQ(lb.allocs, 2);
  CHECK_EQ(lb.frees, 2);
  CHECK(lb.waits >= 1);
  SeamLedger lf;
  {
    FreeListConfig c;
    c.slab_bytes = 1 << 20;
    LedgerFreeList f(c, &lf);
    CHECK_OK(f.config_status());
    auto a = f.allocate(1000, fake_stream(2));
    CHECK(a.ok());
    CHECK_OK(f.deallocate(*a, fake_stream(2)));
  }
  CHECK(lf.allocs >= 1);
  CHECK_EQ(lf.frees, lf.allocs);
  CHECK(lf.waits >= 1);
}

TEST(buddy_sizes_split_merge_validate) {
  HostBuddy b(small_cfg(ReusePolicy::kCoarseStreamPoll));
  const auto s1 = fake_stream(1);
  auto a = b.allocate(1000, s1);
  CHECK(a.ok() && a->bytes == 1024 && a->requested_bytes == 1000);
  CHECK(reinterpret_cast<std::uintptr_t>(a->ptr) % 256 == 0);
  auto c = b.allocate(100, s1);   // rounds up to the 256-byte minimum block
  CHECK(c.ok() && c->bytes == 256);
  CHECK_OK(b.validate());
  CHECK_EQ(b.stats().bytes_in_use, std::size_t{1280});
  CHECK_EQ(b.raw_allocs, 1);
  CHECK_OK(b.deallocate(*a, s1));
  CHECK_OK(b.deallocate(*c, s1));
  CHECK_OK(b.validate());
  // After the parked blocks are reclaimed (same stream), the slab merges back to
  // one 1 MiB block: a 1 MiB request fits without a new slab.
  auto whole = b.allocate(1 << 20, s1);
  CHECK(whole.ok() && whole->bytes == (1u << 20));
  CHECK_EQ(b.raw_allocs, 1);
  CHECK_OK(b.validate());
  CHECK(b.stats().largest_free_block == 0);
}

TEST(buddy_stream_ordered_reuse) {
  for (ReusePolicy pol : {ReusePolicy::kSameStreamOnly, ReusePolicy::kCoarseStreamPoll}) {
    HostBuddy b(small_cfg(pol));
    const auto s1 = fake_stream(1), s2 = fake_stream(2);
    auto a = b.allocate(64 << 10, s1);
    void* first = a->ptr;
    b.busy.insert(s1);                      // s1 still has queued work using the block
    CHECK_OK(b.deallocate(*a, s1));
    CHECK_EQ(b.stats().deferred_reuses, std::uint64_t{1});
    auto on_s1 = b.allocate(64 << 10, s1);  // same stream: safe immediately
    CHECK(on_s1->ptr == first);
    CHECK_OK(b.deallocate(*on_s1, s1));
    auto on_s2 = b.allocate(64 << 10, s2);  // other stream, s1 busy: never the same bytes
    CHECK(on_s2->ptr != first);
    CHECK_OK(b.deallocate(*on_s2, s2));
    b.busy.erase(s1);                       // s1 drains
    auto later = b.allocate(64 << 10, s2);
    if (pol == ReusePolicy::kCoarseStreamPoll)
      CHECK(later->ptr == first);           // the poll sees s1 idle and releases the block
    else
      CHECK(later->ptr != first || b.stats().blocking_drains > 0);
    CHECK_OK(b.validate());
  }
}

TEST(buddy_blocking_drain_and_oom) {
  BuddyConfig cfg = small_cfg(ReusePolicy::kCoarseStreamPoll);
  cfg.max_total_bytes = 1 << 20;
  HostBuddy b(cfg);
  const auto s1 = fake_stream(1), s2 = fake_stream(2);
  auto a = b.allocate(1 << 20, s1);
  CHECK(a.ok());
  b.busy.insert(s1);
  CHECK_OK(b.deallocate(*a, s1));
  // s2 needs the whole slab; the only copy is parked behind busy s1, and the cap
  // forbids a new slab: the allocator must wait for s1 (a counted blocking drain).
  auto c = b.allocate(1 << 20, s2);
  CHECK(c.ok() && c->ptr == a->ptr);
  CHECK_EQ(b.stats().blocking_drains, std::uint64_t{1});
  // Nothing left and the cap reached: out of memory, counted.
  auto d = b.allocate(256, s2);
  CHECK(!d.ok() && d.status().code() == StatusCode::kOutOfMemory);
  CHECK_EQ(b.stats().oom_events, std::uint64_t{1});
  CHECK_OK(b.deallocate(*c, s2));
  CHECK_OK(b.validate());
}

TEST(buddy_growth_bypass_and_trim) {
  HostBuddy b(small_cfg(ReusePolicy::kCoarseStreamPoll));
  const auto s1 = fake_stream(1);
  auto a = b.allocate(768 << 10, s1);      // 1 MiB block: the whole first slab
  auto c = b.allocate(512 << 10, s1);      // needs a second slab (growth x2 -> 2 MiB)
  CHECK(a.ok() && c.ok());
  CHECK_EQ(b.raw_allocs, 2);
  CHECK_EQ(b.stats().bytes_reserved, std::size_t{3 << 20});
  auto big = b.allocate(8 << 20, s1);      // above the 4 MiB threshold: its own hipMalloc
  CHECK(big.ok() && big->slab_id == kBypassSlabId && big->bytes == std::size_t{8 << 20});
  CHECK_EQ(b.raw_allocs, 3);
  CHECK_OK(b.deallocate(*big, s1));
  CHECK_EQ(b.raw_frees, 1);
  CHECK_OK(b.deallocate(*c, s1));
  CHECK_OK(b.trim());                      // the second slab is empty again: released
  CHECK_EQ(b.raw_frees, 2);
  CHECK_EQ(b.stats().bytes_reserved, std::size_t{1 << 20});
  CHECK_OK(b.validate());
  CHECK_OK(b.deallocate(*a, s1));
  CHECK(b.deallocate(*a, s1).code() == StatusCode::kFailedPrecondition);   // double free
}

// Handles that name no live block (the reference's test_buddy_bad_handles,
// tests/test_host_core.cpp:717-748): a double free is a failed precondition; a
// live pointer with the wrong slab or block id, or a pointer from elsewhere, an
// invalid argument (and the block stays live); a null pointer is a no-op.
TEST(buddy_bad_handles) {
  HostBuddy b(small_cfg(ReusePolicy::kCoarseStreamPoll));
  const auto s1 = fake_stream(1);
  auto keep = b.allocate(4096, s1);
  auto r = b.allocate(1024, s1);
  CHECK(keep.ok() && r.ok());
  Allocation bad = *keep;
  bad.slab_id = 99;
  CHECK(b.deallocate(bad, s1).code() == StatusCode::kInvalidArgument);
  bad = *keep;
  bad.block_id = 100000;
  CHECK(b.deallocate(bad, s1).code() == StatusCode::kInvalidArgument);
  CHECK_EQ(b.stats().bytes_in_use, std::size_t{4096 + 1024});   // both still live
  CHECK_OK(b.deallocate(*r, s1));
  CHECK(b.deallocate(*r, s1).code() == StatusCode::kFailedPrecondition);
  std::vector<char> elsewhere(4096);
  bad = *keep;
  bad.ptr = elsewhere.data();
  CHECK(b.deallocate(bad, s1).code() == StatusCode::kInvalidArgument);
  bad.ptr = nullptr;
  CHECK_OK(b.deallocate(bad, s1));                             // free(nullptr) convention
  CHECK_OK(b.validate());
  CHECK_OK(b.deallocate(*keep, s1));
  CHECK_OK(b.validate());
}

// The rounding a block costs, pinned (the reference's test_buddy_internal_waste,
// tests/test_host_core.cpp:537-565): each block is the next power of two, and the
// stats add up the requests and the blocks.
TEST(buddy_internal_waste) {
  HostBuddy b(small_cfg(ReusePolicy::kCoarseStreamPoll));
  const std::pair<std::size_t, std::size_t> cases[] = {{257, 512}, {768, 1024}, {3072, 4096},
                                                       {4097, 8192}};
  std::size_t ask = 0, blocks = 0;
  std::vector<Allocation> live;
  for (const auto& [want, block] : cases) {
    auto r = b.allocate(want, fake_stream(1));
    CHECK(r.ok());
    CHECK_EQ(r->bytes, block);
    CHECK_EQ(r->internal_waste(), block - want);
    ask += want;
    blocks += block;
    live.push_back(*r);
  }
  const AllocatorStats st = b.stats();
  CHECK_EQ(st.bytes_requested, ask);
  CHECK_EQ(st.bytes_in_use, blocks);
  CHECK_EQ(st.internal_waste(), blocks - ask);
  for (const Allocation& a : live) CHECK_OK(b.deallocate(a, fake_stream(1)));
  CHECK_EQ(b.stats().internal_waste(), std::size_t{0});
}

// Random churn with ground truth the test keeps itself (the reference's
// test_buddy_property_no_overlap, tests/test_host_core.cpp:436-535): every block is
// aligned and large enough, no two live blocks overlap, and a byte pattern written
// over each block's whole usable size is intact when it is freed (which bookkeeping
// that only agrees with itself would not show).  The slabs are host memory here;
// where a block lives is the allocator's integer arithmetic either way.
template <class A, class SizeFn>
static void churn_no_overlap(A& alloc, SizeFn size_of, std::size_t block_floor, int iters,
                             std::uint64_t seed) {
  struct LiveBlock {
    Allocation a;
    rt::StreamHandle s;
    unsigned char magic;
  };
  std::vector<LiveBlock> live;
  std::uint64_t rng = seed;
  auto next = [&] { rng = rng * 6364136223846793005ULL + 1442695040888963407ULL; return rng >> 33; };
  std::size_t in_use = 0, requested = 0;
  int overlap = 0, magic = 0, shape = 0;
  for (int it = 0; it < iters; ++it) {
    if (live.empty() || next() % 100 < 60) {
      const std::size_t want = size_of(next());
      const auto s = fake_stream(1 + next() % 2);
      auto r = alloc.allocate(want, s);
      CHECK(r.ok());
      if (!r.ok()) continue;
      if (r->bytes < want || r->bytes < block_floor || r->requested_bytes != want ||
          reinterpret_cast<std::uintptr_t>(r->ptr) % 256 != 0)
        ++shape;
      const auto m = static_cast<unsigned char>(1 + it % 251);
      std::memset(r->ptr, m, r->bytes);
      live.push_back({*r, s, m});
      in_use += r->bytes;
      requested += want;
    } else {
      const std::size_t i = next() % live.size();
      const LiveBlock l = live[i];
      const auto* p = static_cast<const unsigned char*>(l.a.ptr);
      for (std::size_t k = 0; k < l.a.bytes; ++k)
        if (p[k] != l.magic) {
          ++magic;
          break;
        }
      CHECK_OK(alloc.deallocate(l.a, l.s));
      live.erase(live.begin() + static_cast<std::ptrdiff_t>(i));
      in_use -= l.a.bytes;
      requested -= l.a.requested_bytes;
    }
    if (it % 97 == 0) {
      std::vector<std::pair<std::uintptr_t, std::uintptr_t>> iv;
      for (const LiveBlock& l : live)
        iv.emplace_back(reinterpret_cast<std::uintptr_t>(l.a.ptr),
                        reinterpret_cast<std::uintptr_t>(l.a.ptr) + l.a.bytes);
      std::sort(iv.begin(), iv.end());
      for (std::size_t k = 1; k < iv.size(); ++k)
        if (iv[k].first < iv[k - 1].second) ++overlap;
      CHECK_OK(alloc.validate());
    }
    CHECK_EQ(alloc.stats().bytes_in_use, in_use);
    CHECK_EQ(alloc.stats().bytes_requested, requested);
  }
  CHECK_EQ(overlap, 0);
  CHECK_EQ(magic, 0);
  CHECK_EQ(shape, 0);
  for (const LiveBlock& l : live) CHECK_OK(alloc.deallocate(l.a, l.s));
  CHECK_EQ(alloc.stats().bytes_in_use, std::size_t{0});
  CHECK_OK(alloc.validate());
}

TEST(buddy_property_no_overlap) {
  for (ReusePolicy pol : {ReusePolicy::kSameStreamOnly, ReusePolicy::kCoarseStreamPoll}) {
    HostBuddy b(small_cfg(pol));
    const std::size_t sizes[] = {1, 255, 256, 257, 768, 3072, 4097, 8192, 100000};
    churn_no_overlap(b, [&](std::uint64_t r) { return sizes[r % 9]; }, 256, 20000, 0x1234567);
  }
}

// ---------------------------------------------------------------------------
// FreeList allocator on host memory with fake streams.
class HostFreeList : public FreeListAllocator {
 public:
  using FreeListAllocator::FreeListAllocator;
  // The base destructor would reach the base seams (hipFree on host memory).
  ~HostFreeList() override { release_all(); }
  mutable std::set<rt::StreamHandle> busy;
  int raw_allocs = 0, raw_frees = 0;

 protected:
  bool stream_completed(rt::StreamHandle s) const override { return busy.count(s) == 0; }
  void wait_stream(rt::StreamHandle s) const override { busy.erase(s); }
  StatusOr<void*> raw_alloc(std::size_t bytes) override {
    ++raw_allocs;
    void* p = std::aligned_alloc(256, bytes);
    if (!p) return OutOfMemoryError("host aligned_alloc failed");
    return p;
  }
  void raw_free(void* p) override {
    ++raw_frees;
    std::free(p);
  }
};

static FreeListConfig fl_cfg(ReusePolicy p) {
  FreeListConfig c;
  c.slab_bytes = 4 << 20;
  c.small_class_granularity = 512;
  c.small_large_split = 64 << 10;
  c.large_alloc_threshold = 2 << 20;
  c.reuse_policy = p;
  return c;
}

TEST(freelist_size_classes) {
  HostFreeList f(fl_cfg(ReusePolicy::kCoarseStreamPoll));
  CHECK_OK(f.config_status());
  // 128 linear classes of 512 B up to 64 KiB, then 128, 256, ..., 2048 KiB.
  CHECK_EQ(f.size_class_of(1), std::size_t{0});
  CHECK_EQ(f.size_class_of(512), std::size_t{0});
  CHECK_EQ(f.size_class_of(513), std::size_t{1});
  CHECK_EQ(f.size_class_of(64 << 10), std::size_t{127});
  CHECK_EQ(f.size_class_of((64 << 10) + 1), std::size_t{128});
  CHECK_EQ(f.size_class_of(128 << 10), std::size_t{128});
  CHECK_EQ(f.size_class_of((128 << 10) + 1), std::size_t{129});
  CHECK_EQ(f.size_class_of(2 << 20), std::size_t{132});
  CHECK_EQ(f.num_classes(), std::size_t{133});
  for (std::size_t c = 0; c < f.num_classes(); ++c) {
    const std::size_t b = f.class_block_bytes(c);
    CHECK_EQ(f.size_class_of(b), c);                          // a block is the top of its class
    if (c > 0) CHECK(f.size_class_of(f.class_block_bytes(c - 1) + 1) == c);
  }
  FreeListConfig bad = fl_cfg(ReusePolicy::kCoarseStreamPoll);
  bad.small_class_granularity = 384;
  HostFreeList g(bad);
  CHECK(g.config_status().code() == StatusCode::kInvalidArgument);
  CHECK(g.allocate(100, fake_stream(1)).status().code() == StatusCode::kInvalidArgument);
}

TEST(freelist_carve_cache_reuse) {
  HostFreeList f(fl_cfg(ReusePolicy::kCoarseStreamPoll));
  const auto s1 = fake_stream(1);
  auto a = f.allocate(1000, s1);
  CHECK(a.ok() && a->bytes == 1024 && a->requested_bytes == 1000);
  CHECK(reinterpret_cast<std::uintptr_t>(a->ptr) % 256 == 0);
  auto b = f.allocate(100 << 10, s1);                         // class 128 KiB
  CHECK(b.ok() && b->bytes == std::size_t{128 << 10});
  CHECK_EQ(f.raw_allocs, 1);
  CHECK_EQ(f.stats().bytes_in_use, std::size_t{1024 + (128 << 10)});
  CHECK_OK(f.validate());
  CHECK_OK(f.deallocate(*a, s1));
  auto c = f.allocate(600, s1);                               // same class, same stream
  CHECK(c.ok() && c->ptr == a->ptr);
  CHECK_EQ(f.stats().reuse_hits, std::uint64_t{1});
  auto d = f.allocate(1000, s1);                              // cache empty: carved anew
  CHECK(d.ok() && d->ptr != a->ptr);
  CHECK_OK(f.validate());
  CHECK_OK(f.deallocate(*b, s1));
  CHECK_OK(f.deallocate(*c, s1));
  CHECK_OK(f.deallocate(*d, s1));
  CHECK(f.deallocate(*d, s1).code() == StatusCode::kFailedPrecondition);   // double free
  CHECK_OK(f.validate());
  CHECK_EQ(f.stats().bytes_in_use, std::size_t{0});
}

TEST(freelist_stream_ordered_reuse) {
  for (ReusePolicy pol : {ReusePolicy::kSameStreamOnly, ReusePolicy::kCoarseStreamPoll}) {
    HostFreeList f(fl_cfg(pol));
    const auto s1 = fake_stream(1), s2 = fake_stream(2);
    auto a = f.allocate(64 << 10, s1);
    void* first = a->ptr;
    f.busy.insert(s1);
    CHECK_OK(f.deallocate(*a, s1));
    CHECK_EQ(f.stats().deferred_reuses, std::uint64_t{1});
    auto on_s1 = f.allocate(64 << 10, s1);                    // same stream: safe at once
    CHECK(on_s1->ptr == first);
    CHECK_OK(f.deallocate(*on_s1, s1));
    auto on_s2 = f.allocate(64 << 10, s2);                    // s1 busy: never the same bytes
    CHECK(on_s2->ptr != first);
    CHECK_OK(f.deallocate(*on_s2, s2));
    f.busy.erase(s1);
    auto later = f.allocate(64 << 10, s2);
    if (pol == ReusePolicy::kCoarseStreamPoll)
      CHECK(later->ptr == first || later->ptr == on_s2->ptr);   // both blocks are reusable now
    else
      CHECK(later->ptr == on_s2->ptr);                         // only s2's own block
    CHECK_OK(f.validate());
  }
}

TEST(freelist_split_blocking_drain_and_oom) {
  FreeListConfig cfg = fl_cfg(ReusePolicy::kCoarseStreamPoll);
  cfg.split_large_blocks = true;
  cfg.max_total_bytes = 4 << 20;
  HostFreeList f(cfg);
  const auto s1 = fake_stream(1), s2 = fake_stream(2);
  auto big = f.allocate(2 << 20, s1);                         // 2 MiB class
  CHECK(big.ok());
  CHECK_OK(f.deallocate(*big, s1));
  // A 1 MiB request on the same stream cuts its block from the cached 2 MiB one;
  // the 1 MiB tail is cached in its own class.
  auto half = f.allocate(1 << 20, s1);
  CHECK(half.ok() && half->ptr == big->ptr && half->bytes == std::size_t{1 << 20});
  auto tail = f.allocate(1 << 20, s1);
  CHECK(tail.ok() && static_cast<char*>(tail->ptr) == static_cast<char*>(big->ptr) + (1 << 20));
  CHECK_EQ(f.raw_allocs, 1);
  CHECK_OK(f.validate());
  // Fill the rest of the only slab the cap allows, park a block behind busy s1,
  // and ask on s2: the allocator waits for s1 (a counted blocking drain).
  auto rest = f.allocate(2 << 20, s1);
  CHECK(rest.ok());
  f.busy.insert(s1);
  CHECK_OK(f.deallocate(*rest, s1));
  auto again = f.allocate(2 << 20, s2);
  CHECK(again.ok() && again->ptr == rest->ptr);
  CHECK_EQ(f.stats().blocking_drains, std::uint64_t{1});
  auto none = f.allocate(512, s2);                            // slab full, cap reached
  CHECK(!none.ok() && none.status().code() == StatusCode::kOutOfMemory);
  CHECK_EQ(f.stats().oom_events, std::uint64_t{1});
  CHECK_OK(f.deallocate(*half, s1));
  CHECK_OK(f.deallocate(*tail, s1));
  CHECK_OK(f.deallocate(*again, s2));
  CHECK_OK(f.validate());
}

// max_total_bytes caps the pools' slabs only: a bypass allocation larger than the
// cap is the caller's own and does not stop the pool growing (the reference's
// checks, buddy_allocator.cpp:185-195 and freelist_allocator.cpp:134-143; its
// allocator bench's dl_transformer_bypass trace needs exactly this).
TEST(max_total_bytes_caps_slabs_not_bypass) {
  {
    BuddyConfig cfg = small_cfg(ReusePolicy::kCoarseStreamPoll);
    cfg.max_total_bytes = 3 << 20;                       // room for 1 MiB + 2 MiB of slabs
    HostBuddy b(cfg);
    const auto s1 = fake_stream(1);
    auto big = b.allocate(16 << 20, s1);                 // bypass, 16 MiB > the cap
    CHECK(big.ok() && big->slab_id == kBypassSlabId);
    auto a = b.allocate(1 << 20, s1);                    // first slab (1 MiB)
    auto c = b.allocate(1 << 20, s1);                    // second slab (2 MiB): 3 MiB in slabs
    CHECK(a.ok() && c.ok());
    CHECK_EQ(b.stats().bytes_reserved, std::size_t{(16 + 3) << 20});
    auto d = b.allocate(1 << 20, s1);                    // fits the second slab
    CHECK(d.ok());
    auto e = b.allocate(1 << 20, s1);                    // a third slab would pass the cap
    CHECK(!e.ok() && e.status().code() == StatusCode::kOutOfMemory);
    for (auto* x : {&*big, &*a, &*c, &*d}) CHECK_OK(b.deallocate(*x, s1));
    CHECK_OK(b.validate());
  }
  {
    FreeListConfig cfg = fl_cfg(ReusePolicy::kCoarseStreamPoll);
    cfg.max_total_bytes = 8 << 20;                       // two 4 MiB slabs
    HostFreeList f(cfg);
    const auto s1 = fake_stream(1);
    auto big = f.allocate(32 << 20, s1);                 // bypass, 32 MiB > the cap
    CHECK(big.ok() && big->slab_id == kBypassSlabId);
    std::vector<Allocation> held;
    for (int i = 0; i < 4; ++i) {                        // 4 x 2 MiB blocks: both slabs
      auto x = f.allocate(2 << 20, s1);
      CHECK(x.ok());
      if (x.ok()) held.push_back(*x);
    }
    auto over = f.allocate(2 << 20, s1);                 // a third slab would pass the cap
    CHECK(!over.ok() && over.status().code() == StatusCode::kOutOfMemory);
    CHECK_OK(f.deallocate(*big, s1));
    for (const Allocation& x : held) CHECK_OK(f.deallocate(x, s1));
  }
}

TEST(freelist_bypass_trim_and_random_walk) {
  HostFreeList f(fl_cfg(ReusePolicy::kCoarseStreamPoll));
  const auto s1 = fake_stream(1), s2 = fake_stream(2);
  auto big = f.allocate(8 << 20, s1);                         // above the 2 MiB threshold
  CHECK(big.ok() && big->slab_id == kBypassSlabId && big->bytes == std::size_t{8 << 20});
  CHECK_OK(f.deallocate(*big, s1));
  CHECK_EQ(f.raw_frees, 1);
  // Random walk over sizes and streams; validate() after every step.
  std::uint64_t rng = 0x1234567;
  auto next = [&] { rng = rng * 6364136223846793005ULL + 1442695040888963407ULL; return rng >> 33; };
  std::vector<std::pair<Allocation, rt::StreamHandle>> held;
  for (int step = 0; step < 400; ++step) {
    if (held.size() < 24 && (next() % 3 != 0 || held.empty())) {
      const std::size_t sz = 1 + next() % (next() % 4 == 0 ? (2 << 20) : (48 << 10));
      const auto st = (next() & 1) ? s1 : s2;
      auto a = f.allocate(sz, st);
      CHECK(a.ok());
      if (a.ok()) {
        CHECK(a->bytes >= sz && a->bytes == f.class_block_bytes(f.size_class_of(sz)));
        held.emplace_back(*a, st);
      }
    } else {
      const std::size_t i = next() % held.size();
      CHECK_OK(f.deallocate(held[i].first, held[i].second));
      held.erase(held.begin() + static_cast<std::ptrdiff_t>(i));
    }
    CHECK_OK(f.validate());
  }
  for (auto& [a, st] : held) CHECK_OK(f.deallocate(a, st));
  CHECK_EQ(f.stats().bytes_in_use, std::size_t{0});
  const int frees_before = f.raw_frees;
  CHECK_OK(f.trim());                                         // every slab is empty: all released
  CHECK(f.raw_frees > frees_before);
  CHECK_EQ(f.stats().bytes_reserved, std::size_t{0});
  CHECK_OK(f.validate());
  auto fresh = f.allocate(4096, s1);                          // a new slab after the trim
  CHECK(fresh.ok());
  CHECK_OK(f.deallocate(*fresh, s1));
}

TEST(freelist_property_no_overlap) {
  for (ReusePolicy pol : {ReusePolicy::kSameStreamOnly, ReusePolicy::kCoarseStreamPoll}) {
    HostFreeList f(fl_cfg(pol));
    const std::size_t sizes[] = {1, 100, 512, 513, 4096, 65536, 65537, 300000, 1 << 20};
    churn_no_overlap(f, [&](std::uint64_t r) { return sizes[r % 9]; }, 512, 20000, 0x7654321);
  }
}

// The defining difference, head to head (the reference's test_freelist_no_coalescing,
// tests/test_host_core.cpp:962-1010): carve a whole slab into 512 B blocks and free
// two adjacent ones.  Buddy merges them into a 1 KiB block that a 1 KiB request
// reuses in place; FreeList keeps two 512 B blocks, so a 1 KiB request needs a new
// slab.
TEST(freelist_no_coalescing_vs_buddy) {
  {
    FreeListConfig c = fl_cfg(ReusePolicy::kCoarseStreamPoll);
    c.slab_bytes = 64 << 10;
    HostFreeList f(c);
    std::vector<Allocation> live;
    for (int i = 0; i < 128; ++i) {
      auto x = f.allocate(512, fake_stream(1));
      CHECK(x.ok());
      live.push_back(*x);
    }
    CHECK_EQ(f.raw_allocs, 1);
    CHECK_EQ(f.stats().largest_free_block, std::size_t{0});     // the slab is fully carved
    CHECK(static_cast<char*>(live[1].ptr) == static_cast<char*>(live[0].ptr) + 512);
    CHECK_OK(f.deallocate(live[0], fake_stream(1)));
    CHECK_OK(f.deallocate(live[1], fake_stream(1)));
    CHECK_OK(f.settle_pending());
    CHECK_EQ(f.stats().largest_free_block, std::size_t{512});   // not merged
    auto k = f.allocate(1024, fake_stream(1));
    CHECK(k.ok() && k->ptr != live[0].ptr);
    CHECK_EQ(f.raw_allocs, 2);
    CHECK_OK(f.validate());
    CHECK_OK(f.deallocate(*k, fake_stream(1)));
    for (std::size_t i = 2; i < live.size(); ++i) CHECK_OK(f.deallocate(live[i], fake_stream(1)));
  }
  {
    BuddyConfig c = small_cfg(ReusePolicy::kCoarseStreamPoll);
    c.initial_slab_bytes = 64 << 10;
    HostBuddy b(c);
    std::vector<Allocation> live;
    for (int i = 0; i < 128; ++i) {
      auto x = b.allocate(512, fake_stream(1));
      CHECK(x.ok());
      live.push_back(*x);
    }
    CHECK_EQ(b.raw_allocs, 1);
    CHECK_EQ(b.stats().largest_free_block, std::size_t{0});
    CHECK(static_cast<char*>(live[1].ptr) == static_cast<char*>(live[0].ptr) + 512);
    // block_id is the node in heap order over the 64 KiB slab's tree: the first two
    // 512 B blocks are the leftmost leaves of level 7, siblings.
    CHECK_EQ(live[0].block_id, static_cast<std::uint32_t>(buddy::heap_index(7, 0)));
    CHECK_EQ(static_cast<std::size_t>(live[1].block_id), buddy::buddy_of(live[0].block_id));
    CHECK_EQ(buddy::offset_of(live[127].block_id, 16), std::size_t{127 * 512});
    CHECK_OK(b.deallocate(live[0], fake_stream(1)));
    CHECK_OK(b.deallocate(live[1], fake_stream(1)));
    CHECK_OK(b.settle_pending());
    CHECK_EQ(b.stats().largest_free_block, std::size_t{1024});  // the two buddies merged
    auto k = b.allocate(1024, fake_stream(1));
    CHECK(k.ok() && k->ptr == live[0].ptr);
    CHECK_EQ(b.raw_allocs, 1);
    CHECK_OK(b.validate());
    CHECK_OK(b.deallocate(*k, fake_stream(1)));
    for (std::size_t i = 2; i < live.size(); ++i) CHECK_OK(b.deallocate(live[i], fake_stream(1)));
  }
}

// Nearest-rank percentiles at the sizes where an off-by-one hides (the reference's
// test_latency_stats_edge_cases, tests/test_host_core.cpp:1194-1256), the histogram's
// buckets, and a self-consistent clock calibration.
TEST(latency_stats_nearest_rank_and_calibration) {
  {
    LatencyStats s(1);
    s.add(777);
    s.finalize();
    for (double p : {0.0, 50.0, 99.9, 100.0}) CHECK_EQ(s.percentile(p), std::uint64_t{777});
    CHECK_EQ(s.min(), std::uint64_t{777});
    CHECK_EQ(s.max(), std::uint64_t{777});
  }
  {
    LatencyStats s(2);
    s.add(20);
    s.add(10);
    s.finalize();
    CHECK_EQ(s.percentile(0.0), std::uint64_t{10});
    CHECK_EQ(s.percentile(100.0), std::uint64_t{20});
    CHECK_EQ(s.median(), std::uint64_t{10});                 // rank ceil(0.5 * 2) = 1: the lower
  }
  {
    LatencyStats s(5);
    for (int i = 0; i < 5; ++i) s.add(42);
    s.finalize();
    CHECK_EQ(s.median(), std::uint64_t{42});
    CHECK_EQ(s.p99(), std::uint64_t{42});
    CHECK(std::fabs(s.mean_ns() - 42.0) < 1e-9);
  }
  {
    LatencyStats s(100);
    for (int i = 100; i >= 1; --i) s.add(static_cast<std::uint64_t>(i));
    CHECK(!s.is_finalized());
    s.finalize();
    CHECK(s.is_finalized());
    CHECK_EQ(s.percentile(1.0), std::uint64_t{1});
    CHECK_EQ(s.median(), std::uint64_t{50});
    CHECK_EQ(s.p90(), std::uint64_t{90});
    CHECK_EQ(s.p99(), std::uint64_t{99});
    CHECK_EQ(s.p999(), std::uint64_t{100});                  // rank ceil(99.9) = 100
    CHECK_EQ(s.percentile(100.0), std::uint64_t{100});
    CHECK(std::fabs(s.mean_ns() - 50.5) < 1e-9);
    // Buckets of a 10 ns floor: [0,10] holds 1..10, (10,20] 11..20, (20,40],
    // (40,80], (80,160] the rest.
    CHECK(s.log2_histogram(10) == "    <= 10 ns: 10\n    <= 20 ns: 10\n    <= 40 ns: 20\n"
                                  "    <= 80 ns: 40\n    <= 160 ns: 20\n");
  }
  {
    LatencyStats s(0);
    s.finalize();
    CHECK(s.empty());
    CHECK_EQ(s.count(), std::size_t{0});
    CHECK_EQ(s.median(), std::uint64_t{0});
    CHECK_EQ(s.max(), std::uint64_t{0});
    CHECK(s.mean_ns() == 0.0);
    CHECK(s.log2_histogram(10) == "  (no samples)\n");
  }
  const ClockCalibration cal = ClockCalibration::measure(20000);
  CHECK(cal.floor_ns > 0);
  CHECK(cal.floor_ns >= cal.tick_ns && cal.floor_ns >= cal.paired_median_ns);
  CHECK(cal.is_below_floor(cal.floor_ns));
  CHECK(!cal.is_below_floor(cal.floor_ns * 1000));
  CHECK(!cal.describe().empty());
  HostTimer t;
  t.start();
  volatile double sink = 0;
  for (int i = 0; i < 100000; ++i) sink = sink + std::sqrt(static_cast<double>(i));
  CHECK(t.stop_ns() > 0);
}

// The tree arithmetic at run time as well as at compile time: every node of a
// 12-level tree round-trips through (level, index) and offset, children and
// buddies are consistent, and level_for_size picks the smallest block that holds a
// request (the reference's test_buddy_math / test_buddy_geometry).
TEST(buddy_math_tree_arithmetic) {
  using namespace buddy;
  CHECK(is_power_of_two(1) && is_power_of_two(4096) && !is_power_of_two(0) && !is_power_of_two(768));
  CHECK_EQ(align_up(257, 256), std::size_t{512});
  CHECK_EQ(align_up(512, 256), std::size_t{512});
  const unsigned arena = 20, minb = 8, L = max_level(arena, minb);
  CHECK_EQ(L, 12u);
  CHECK_EQ(node_count(L), (std::size_t{1} << 13) - 1);
  for (std::size_t n = 0; n < node_count(L); ++n) {
    const unsigned lv = level_of(n);
    CHECK(heap_index(lv, index_in_level(n)) == n);
    CHECK(index_in_level(n) < nodes_at_level(lv));
    CHECK(node_at(offset_of(n, arena), lv, arena) == n);
    CHECK(offset_of(n, arena) % block_bytes_at_level(arena, lv) == 0);
    if (!is_root(n)) {
      CHECK(buddy_of(buddy_of(n)) == n && parent_of(buddy_of(n)) == parent_of(n));
      CHECK((offset_of(n, arena) ^ block_bytes_at_level(arena, lv)) == offset_of(buddy_of(n), arena));
    }
    if (lv < L) {
      CHECK(parent_of(left_child_of(n)) == n && parent_of(right_child_of(n)) == n);
      CHECK(offset_of(left_child_of(n), arena) == offset_of(n, arena));
    }
  }
  for (std::size_t bytes : {std::size_t{1}, std::size_t{255}, std::size_t{256}, std::size_t{257},
                            std::size_t{4097}, std::size_t{1} << 19, (std::size_t{1} << 19) + 1,
                            std::size_t{1} << 20}) {
    const unsigned lv = level_for_size(bytes, arena, minb);
    CHECK(block_bytes_at_level(arena, lv) >= bytes);
    CHECK(lv == L || block_bytes_at_level(arena, lv + 1) < std::max(bytes, std::size_t{256}));
  }
  CHECK_EQ(level_for_size((std::size_t{1} << 20) + 1, arena, minb), L + 1);
}

TEST(first_bit_mismatch_helper) {
  const std::uint32_t x[4] = {1, 2, 3, 4};
  std::uint32_t y[4] = {1, 2, 3, 4};
  CHECK_EQ(first_bit_mismatch(x, y, 16), std::size_t{16});
  y[2] = 7;
  CHECK_EQ(first_bit_mismatch(x, y, 16), std::size_t{8});
}

// The multiply-shift division the flat-grid bias+act kernel uses to split a
// workgroup index into row and strip: equal to n / d for every divisor 1..4096
// and the extreme divisors, at dividends around every multiple of d in range
// and at the ends of [0, 2^31).
TEST(fast_div_matches_division) {
  std::vector<std::uint32_t> divisors;
  for (std::uint32_t d = 1; d <= 4096; ++d) divisors.push_back(d);
  for (std::uint32_t d : {6553u, 65535u, 65536u, 65537u, 1000003u, 16777215u, 16777216u,
                          0x7FFFFFFEu, 0x7FFFFFFFu, 0x80000000u})
    divisors.push_back(d);
  std::mt19937 rng(12345);
  int bad = 0;
  for (std::uint32_t d : divisors) {
    const mcke_amd::FastDivU32 f = mcke_amd::FastDivU32::make(d);
    auto one = [&](std::uint64_t n) {
      if (n >= 0x80000000ull) return;
      const auto n32 = static_cast<std::uint32_t>(n);
      if (f.div(n32) != n32 / d) ++bad;
    };
    for (std::uint64_t n = 0; n < 3000; ++n) one(n);
    for (std::uint64_t n = 0x7FFFFFFFull; n > 0x7FFFFFFFull - 3000; --n) one(n);
    // Around multiples of d spread over the range.
    const std::uint64_t step = std::max<std::uint64_t>(d, (0x80000000ull / 2000) / d * d);
    for (std::uint64_t q = step; q < 0x80000000ull; q += step) {
      one(q - 1);
      one(q);
      one(q + 1);
    }
    for (int i = 0; i < 2000; ++i) one(rng() & 0x7FFFFFFFu);
  }
  CHECK(bad == 0);
}

int main(int argc, char** argv) { return check::run_all(argc, argv); }
