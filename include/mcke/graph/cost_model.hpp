// mcke/graph/cost_model.hpp -- roofline time of an op from its ideal cost
// (reference include/mcke/graph/cost_model.hpp:62-78): max(flops / peak,
// bytes / bandwidth).  Used to balance streams, never reported as a measurement.
#pragma once

#include <algorithm>

#include "mcke/graph/op.hpp"
#include "mcke/profiling/profiler.hpp"

namespace mcke {

[[nodiscard]] inline double plan_cost_ms(const OpCost& c, const Roofline& rl) {
  const double t_compute = rl.peak_tflops > 0.0 ? static_cast<double>(c.flops) / (rl.peak_tflops * 1e12) : 0.0;
  const double t_memory = rl.peak_gb_s > 0.0 ? static_cast<double>(c.bytes) / (rl.peak_gb_s * 1e9) : 0.0;
  return std::max(t_compute, t_memory) * 1e3;
}

[[nodiscard]] inline bool op_is_memory_bound(const OpCost& c, const Roofline& rl) {
  return rl.memory_bound(c.arithmetic_intensity());
}

}  // namespace mcke
