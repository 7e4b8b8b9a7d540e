// gate_probe.cpp -- shows on the GPU that GraphExecutor::validate_numerics() can
// fail: the counterpart of the reference's test_numerics_gate_catches_nondeterminism
// (tests/test_graph_host.cpp:1558-1597, with its nondeterministic FakeOp at
// :311-389), which runs on the reference's host backend; this executor runs on HIP,
// so the stand-in op here launches a device fill.
//
// FlakyOp writes every output element with the bits of (1 + 0.5 * calls) where
// `calls` counts its launches -- a different answer on every run, the simplest
// stand-in for a race.  Its deterministic control writes 1.5 on every run.
//
// Built into tests/cpp/bin/libgate_probe.so and run in-process by
// tests/test_gpu_graph_gate.py through mcke_test_gate_probe(): 0 on success with
// *passed and the gate's detail filled in, 2 on a harness error (message in
// `detail`).
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "mcke/core/device.hpp"
#include "mcke/graph/executor.hpp"
#include "mcke/graph/graph.hpp"
#include "mcke/memory/buddy_allocator.hpp"
#include "mcke_amd.h"

using namespace mcke;

namespace {

class FlakyOp final : public Op {
 public:
  explicit FlakyOp(bool nondet) : nondet_(nondet) {}
  [[nodiscard]] std::string_view type_name() const override { return "Flaky"; }
  [[nodiscard]] Status launch(const OpContext& ctx, const std::vector<Tensor>& inputs,
                              const std::vector<Tensor>& outputs) override {
    if (inputs.size() != 1 || outputs.size() != 1) return InternalError("FlakyOp: one input, one output");
    ++calls_;
    const float v = 1.0f + 0.5f * static_cast<float>(nondet_ ? calls_ : 1);
    std::uint32_t bits;
    std::memcpy(&bits, &v, sizeof bits);
    const Tensor& o = outputs[0];
    if (int rc = mcke_fill_u32_async(o.data_ptr(), bits, static_cast<std::size_t>(o.numel()),
                                     static_cast<void*>(ctx.stream)))
      return InternalError(std::string("FlakyOp: mcke_fill_u32_async: ") + mcke_last_error() +
                           " (status " + std::to_string(rc) + ")");
    return OkStatus();
  }
  [[nodiscard]] StatusOr<std::vector<Shape>> infer_shapes(const std::vector<Shape>& in) const override {
    if (in.size() != 1) return InvalidArgumentError("FlakyOp: one input");
    return std::vector<Shape>{in[0]};
  }
  [[nodiscard]] OpCost cost(const std::vector<Shape>& in) const override {
    OpCost c;
    c.bytes = static_cast<std::uint64_t>(in[0].numel()) * 2u * sizeof(float);
    return c;
  }

 private:
  bool nondet_;
  int calls_ = 0;
};

void put(char* dst, std::size_t cap, const std::string& s) {
  if (!dst || cap == 0) return;
  const std::size_t n = s.size() < cap - 1 ? s.size() : cap - 1;
  std::memcpy(dst, s.data(), n);
  dst[n] = '\0';
}

}  // namespace

extern "C" int mcke_test_gate_probe(int nondeterministic, int repeats, int* passed, int* configs_compared,
                                    char* detail, std::size_t detail_cap) {
  auto fail = [&](const Status& s) {
    put(detail, detail_cap, "harness: " + s.message());
    return 2;
  };
  if (!passed || !configs_compared) {
    put(detail, detail_cap, "harness: null output argument");
    return 2;
  }
  Graph g;
  auto x = g.add_input(Shape{64, 64}, DType::kF32, "x");
  if (!x.ok()) return fail(x.status());
  auto n = g.add_node(std::make_unique<FlakyOp>(nondeterministic != 0), {*x}, "flaky");
  if (!n.ok()) return fail(n.status());
  // A second node downstream, so the level-parallel and chain-greedy plans have
  // an edge to order.
  auto n2 = g.add_node(std::make_unique<FlakyOp>(false), {(*n)[0]}, "after");
  if (!n2.ok()) return fail(n2.status());
  if (Status s = g.mark_output((*n)[0]); !s.ok()) return fail(s);
  if (Status s = g.mark_output((*n2)[0]); !s.ok()) return fail(s);
  if (Status s = g.finalize(); !s.ok()) return fail(s);

  auto dev = query_device(0);
  if (!dev.ok()) return fail(dev.status());
  BuddyAllocator alloc;
  ExecutorOptions opts;
  opts.validate_numerics = true;
  opts.num_streams = 2;
  GraphExecutor ex(std::move(g), alloc, *dev, opts);
  if (Status s = ex.plan(); !s.ok()) return fail(s);
  std::vector<float> host(64 * 64, 2.0f);
  if (Status s = ex.set_input(*x, host.data(), host.size() * sizeof(float)); !s.ok()) return fail(s);
  auto res = ex.validate_numerics(repeats);
  if (!res.ok()) return fail(res.status());
  *passed = res->passed ? 1 : 0;
  *configs_compared = res->configs_compared;
  put(detail, detail_cap, res->detail);
  return 0;
}
