// profiler_probe.cpp -- Profiler::time_op on the GPU, the way the reference's
// benches use it (bench/bias_act_bench.cpp:182-184, bench/gemm_bench.cpp:312-316):
// an rt::Stream, launches through the C++ launcher API (mcke::kernels), one
// KernelRecord per op with the ideal flops/bytes of its Op::cost(), then
// Profiler::write_csv and summary_table against the MI355X roofline.
//
// Built into tests/cpp/bin/libprofiler_probe.so and run in-process by
// tests/test_gpu_profiler.py through mcke_test_profiler_probe(): the caller owns
// every device buffer; the probe times
//   record 0: bias + GELU(tanh), y = act(x + bias), x [rows x cols], vw = 4;
//   record 1: C = A B, n x n x n, kMfmaF32 with the default tile;
// `warmup` untimed launches then `iters` timed ones each, so the outputs hold
// the result of the last launch.  Returns 0 with med_ms[2], min_ms[2] filled and
// the summary table in `detail`; 2 on an error (message in `detail`).
#include <cstdint>
#include <cstdio>
#include <string>

#include "mcke/graph/op.hpp"
#include "mcke/kernels/kernels.hpp"
#include "mcke/profiling/profiler.hpp"
#include "mcke/runtime/stream.hpp"

using namespace mcke;
namespace K = mcke::kernels;

namespace {

int fail(char* detail, std::size_t n, const std::string& what) {
  if (detail && n) std::snprintf(detail, n, "%s", what.c_str());
  return 2;
}

}  // namespace

extern "C" int mcke_test_profiler_probe(const float* x, const float* bias, float* y,
                                        std::int64_t rows, std::int64_t cols, const float* a,
                                        const float* b, float* c, std::int64_t n, int warmup,
                                        int iters, const char* csv_path, double* med_ms,
                                        double* min_ms, char* detail, std::size_t detail_len) {
  StatusOr<rt::Stream> st = rt::Stream::create();
  if (!st.ok()) return fail(detail, detail_len, st.status().to_string());
  const rt::Stream& stream = *st;

  Profiler prof;
  const OpCost ba_cost = BiasActOp(BiasActParams{BiasActParams::Act::kGeluTanh})
                             .cost({Shape{rows, cols}, Shape{cols}});
  StatusOr<KernelRecord> r0 = prof.time_op(
      "bias_act", "gelu_tanh_vw4", stream, ba_cost.flops, ba_cost.bytes, warmup, iters,
      [&](const rt::Stream& s) {
        return K::launch_bias_act_f32(x, bias, y, rows, cols, K::Activation::kGeluTanh, 4,
                                      s.native());
      });
  if (!r0.ok()) return fail(detail, detail_len, "bias_act: " + r0.status().to_string());

  const OpCost g_cost = GemmOp(GemmParams{}).cost({Shape{n, n}, Shape{n, n}});
  const K::GemmTile tile = K::mfma_default_tile(n, n, n);
  StatusOr<KernelRecord> r1 = prof.time_op(
      "gemm", "mfma_f32", stream, g_cost.flops, g_cost.bytes, warmup, iters,
      [&](const rt::Stream& s) {
        return K::launch_gemm_f32(a, b, c, n, n, n, 1.0f, 0.0f, K::GemmVariant::kMfmaF32, tile,
                                  s.native());
      });
  if (!r1.ok()) return fail(detail, detail_len, "gemm: " + r1.status().to_string());

  const Roofline rl = mi355x_roofline();
  if (Status w = prof.write_csv(csv_path, rl); !w.ok()) return fail(detail, detail_len, w.to_string());
  for (int i = 0; i < 2; ++i) {
    med_ms[i] = prof.records()[static_cast<std::size_t>(i)].median_ms;
    min_ms[i] = prof.records()[static_cast<std::size_t>(i)].min_ms;
  }
  if (detail && detail_len) std::snprintf(detail, detail_len, "%s", prof.summary_table(rl).c_str());
  return 0;
}
