// mcke/graph/schedule.hpp -- assignment of graph nodes to streams, with the
// events that order cross-stream dependencies.
//
// Same API as the reference's include/mcke/graph/schedule.hpp:49-108:
//   kSequential     every node on stream 0 in topological order;
//   kLevelParallel  nodes of one ASAP level spread round-robin over the streams,
//                   with a barrier between consecutive levels (the first node of
//                   level d+1 on each stream waits for the last node of level d
//                   on every other stream);
//   kChainGreedy    a node whose only live predecessor has not passed its stream
//                   on to another node yet inherits that stream; every other node
//                   goes to the least-loaded stream (load = roofline time of its
//                   ideal cost); every cross-stream predecessor must be ordered.
// Cross-stream orderings become event waits, except where the waiting node's
// vector clock already covers the producer (through its stream's earlier nodes
// or an earlier wait); only producers left with a waiter record an event.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "mcke/core/status.hpp"
#include "mcke/graph/graph.hpp"
#include "mcke/graph/happens_before.hpp"
#include "mcke/profiling/profiler.hpp"

namespace mcke {

enum class SchedulePolicy : std::uint8_t { kSequential, kLevelParallel, kChainGreedy };

struct StreamAssignment {
  std::vector<NodeId> nodes;                      // scheduled index -> NodeId
  std::vector<std::uint16_t> stream_of;
  std::vector<std::uint32_t> issue_of;
  std::vector<std::uint32_t> record_of;           // event id or kNoEventId
  std::vector<std::vector<std::uint32_t>> waits_of;
  std::vector<std::uint32_t> order;               // issue order (scheduled indices)
  std::size_t num_streams_used = 0;
  std::size_t num_streams_requested = 0;
  std::size_t num_events = 0;
  std::size_t waits_raw = 0;
  std::size_t waits_dedup = 0;
  std::vector<double> stream_load_ms;
  [[nodiscard]] std::string describe() const;
  [[nodiscard]] StatusOr<HappensBefore> happens_before() const;
};

[[nodiscard]] StatusOr<StreamAssignment> plan_streams(const Graph& g, SchedulePolicy policy,
                                                      int num_streams, const Roofline& rl);

// Every graph dependency must be ordered by the schedule's happens-before.
[[nodiscard]] Status verify_plan_ordering(const Graph& g, const StreamAssignment& sa);

}  // namespace mcke
