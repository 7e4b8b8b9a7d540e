// mcke/graph/memory_plan.hpp -- placement of every tensor in one arena.
//
// Same API as the reference's include/mcke/graph/memory_plan.hpp and
// memory_plan.cpp:40-267.  Tensors are placed largest first (ties by id), each
// in the smallest 256-byte aligned gap between the already placed tensors it may
// not share with (or past them).  Two tensors may share bytes when both are
// intermediates and, under the policy, every access of one is ordered before the
// other's producer:
//   kAllocPerTensor      never (the baseline);
//   kReuseTopoNaive      by position in the topological order only -- UNSAFE
//                        across streams, kept to show what the race check finds;
//   kReuseSameStream     all accesses on the producer's stream and ordered;
//   kReuseHappensBefore  all accesses happen-before the producer (any stream).
// verify_no_buffer_races re-checks every overlapping pair against happens-before.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "mcke/core/status.hpp"
#include "mcke/graph/graph.hpp"
#include "mcke/graph/happens_before.hpp"
#include "mcke/graph/schedule.hpp"

namespace mcke {

enum class MemoryPolicy : std::uint8_t {
  kAllocPerTensor,
  kReuseTopoNaive,
  kReuseSameStream,
  kReuseHappensBefore,
};

inline constexpr std::size_t kNoOffset = static_cast<std::size_t>(-1);

struct MemoryPlan {
  MemoryPolicy policy = MemoryPolicy::kReuseHappensBefore;
  std::vector<std::size_t> offset_of;
  std::vector<std::size_t> bytes_of;   // padded to kDeviceAlignment
  std::size_t arena_bytes = 0;
  std::size_t naive_bytes = 0;
  std::size_t input_bytes = 0, intermediate_bytes = 0, output_bytes = 0;
  std::vector<std::size_t> workspace_bytes;   // per stream
  std::size_t buffers_used = 0;
  [[nodiscard]] std::string describe() const;
};

[[nodiscard]] StatusOr<MemoryPlan> plan_memory(const Graph& g, const StreamAssignment& sa,
                                               const HappensBefore& hb, MemoryPolicy policy);

[[nodiscard]] Status verify_no_buffer_races(const Graph& g, const StreamAssignment& sa,
                                            const HappensBefore& hb, const MemoryPlan& mp);

}  // namespace mcke
