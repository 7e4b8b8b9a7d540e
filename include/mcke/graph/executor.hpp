// mcke/graph/executor.hpp -- plans a graph onto streams and an arena, then
// replays it.
//
// Same API as the reference's include/mcke/graph/executor.hpp and
// executor.cpp:39-619:
//   plan()       finalize, schedule (plan_streams + verify_plan_ordering),
//                happens-before, memory plan (+ verify_no_buffer_races), create
//                streams / events / arena / per-stream workspaces, bind tensors;
//   run_async()  fork (stream 0 records, the others wait), per node: its waits,
//                optional timing probes, Op::launch, its record; join back onto
//                stream 0.  Never synchronises the host.  With poison_buffers the
//                arena (outside the input ranges) is refilled each run with a
//                pattern that changes per iteration;
//   validate_numerics()  runs {sequential, level-parallel, chain-greedy} x
//                {per-tensor, same-stream, happens-before} plans `repeats` times
//                each with poisoning on and requires every output to be bitwise
//                identical to the sequential/per-tensor golden run.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "mcke/core/device.hpp"
#include "mcke/core/status.hpp"
#include "mcke/graph/graph.hpp"
#include "mcke/graph/happens_before.hpp"
#include "mcke/graph/memory_plan.hpp"
#include "mcke/graph/schedule.hpp"
#include "mcke/memory/allocator.hpp"
#include "mcke/profiling/profiler.hpp"
#include "mcke/runtime/stream.hpp"
#include "mcke/tensor/tensor.hpp"

namespace mcke {

struct ExecutorOptions {
  SchedulePolicy schedule = SchedulePolicy::kChainGreedy;
  MemoryPolicy memory = MemoryPolicy::kReuseHappensBefore;
  int num_streams = 4;
  bool profile = false;        // per-node timing events (probe ring)
  int profile_slots = 32;      // probe ring depth
  bool validate_numerics = false;
  bool poison_buffers = false;
  std::uint32_t poison_pattern = 0x7F7F7F7Fu;
};

[[nodiscard]] std::size_t first_bit_mismatch(const void* a, const void* b, std::size_t bytes);

struct NumericsResult {
  bool passed = false;
  int configs_compared = 0;
  int repeats = 0;
  std::size_t elements_compared = 0;
  std::string detail;
};

struct NodeTiming {
  NodeId node = kInvalidNode;
  std::string name;
  int stream_idx = 0;
  double median_ms = 0.0;
  double min_ms = 0.0;
  std::uint64_t flops = 0, bytes = 0;
  int samples = 0;
};

inline constexpr std::uint32_t kNoEvent = 0xFFFFFFFFu;

struct ScheduledNode {
  NodeId node = kInvalidNode;
  std::uint16_t stream_idx = 0;
  std::uint16_t issue_index = 0;
  std::uint32_t wait_offset = 0;
  std::uint32_t wait_count = 0;
  std::uint32_t record_event = kNoEvent;
};

class ExecutionPlan {
 public:
  [[nodiscard]] const std::vector<ScheduledNode>& nodes() const noexcept { return sched_; }
  [[nodiscard]] std::size_t num_streams() const noexcept { return streams_.size(); }
  [[nodiscard]] std::size_t peak_memory_bytes() const noexcept { return peak_bytes_; }
  [[nodiscard]] std::size_t naive_memory_bytes() const noexcept { return naive_bytes_; }
  [[nodiscard]] const std::vector<std::uint32_t>& wait_pool() const noexcept { return wait_pool_; }
  [[nodiscard]] std::string describe() const;
  [[nodiscard]] const StreamAssignment& stream_plan() const noexcept { return streams_plan_; }
  [[nodiscard]] const MemoryPlan& memory_plan() const noexcept { return memory_plan_; }
  [[nodiscard]] std::size_t intra_events() const noexcept { return streams_plan_.num_events; }
  [[nodiscard]] std::size_t intra_waits() const noexcept { return streams_plan_.waits_dedup; }
  [[nodiscard]] std::size_t forkjoin_events() const noexcept {
    const std::size_t k = streams_plan_.num_streams_used;
    return k <= 1 ? 0 : k + 2 * (k - 1);
  }
  [[nodiscard]] rt::StreamHandle stream(std::size_t i) const { return streams_[i].native(); }

 private:
  friend class GraphExecutor;
  std::vector<ScheduledNode> sched_;
  std::vector<std::uint32_t> wait_pool_;
  std::vector<rt::Stream> streams_;
  std::vector<rt::Event> events_;
  std::vector<rt::Event> fork_event_;
  std::vector<rt::Event> join_events_;
  std::vector<rt::Event> probes_;
  int probe_slots_ = 0;
  int iteration_ = 0;
  StreamAssignment streams_plan_;
  MemoryPlan memory_plan_;
  std::shared_ptr<Storage> arena_;
  std::vector<std::shared_ptr<Storage>> workspaces_;
  std::vector<std::pair<std::size_t, std::size_t>> input_byte_ranges_;
  std::vector<std::vector<Tensor>> node_inputs_;
  std::vector<std::vector<Tensor>> node_outputs_;
  std::vector<Tensor> bound_;
  std::shared_ptr<Storage> poison_src_;   // device-side pattern for poisoning
  std::size_t peak_bytes_ = 0;
  std::size_t naive_bytes_ = 0;
};

class GraphExecutor {
 public:
  GraphExecutor(Graph graph, DeviceAllocator& alloc, DeviceInfo device, ExecutorOptions opts = {});
  ~GraphExecutor();

  [[nodiscard]] Status plan();
  [[nodiscard]] Status set_input(TensorId t, const void* host_data, std::size_t bytes);
  [[nodiscard]] Status run_async();
  // Captures one iteration of run_async() into a HIP graph and instantiates it;
  // every later run_async() replays that graph with one launch on stream 0
  // instead of re-issuing the plan's launches and events.  A single-stream plan
  // is stream-captured whole.  A plan on several streams is assembled node by
  // node: each node's launches are captured on its own stream into a child
  // graph, and the child joins the parent graph after the previous node of its
  // stream and after the nodes that record the events it waits on, so the
  // graph's edges are exactly the plan's stream order and cross-stream events;
  // no capture spans two streams.  The reference plans this step as
  // capture_cuda_graph (include/mcke/graph/executor.hpp:23-27).  Refused with
  // per-node timing probes (their events would be frozen into the graph) and
  // with the vendor-library GEMM (its internals are not ours to vet for memset
  // nodes).  With poison_buffers the pattern captured is the capture
  // iteration's.  plan() drops the captured graph, since it binds the old plan's
  // buffers.
  [[nodiscard]] Status capture_graph();
  [[nodiscard]] bool captured() const noexcept { return graph_exec_ != nullptr; }
  [[nodiscard]] Status synchronize();
  [[nodiscard]] Status run_sync() {
    MCKE_RETURN_IF_ERROR(run_async());
    return synchronize();
  }
  [[nodiscard]] StatusOr<Tensor> output(TensorId t) const;
  [[nodiscard]] StatusOr<Tensor> any_bound_tensor(TensorId t) const;
  [[nodiscard]] Status collect_timings();
  [[nodiscard]] StatusOr<NumericsResult> validate_numerics(int repeats = 20);
  [[nodiscard]] const std::vector<NodeTiming>& node_timings() const noexcept { return node_timings_; }
  [[nodiscard]] const ExecutionPlan& plan_ref() const { return plan_; }
  [[nodiscard]] const Profiler& profiler() const { return profiler_; }
  [[nodiscard]] const Graph& graph() const { return graph_; }
  [[nodiscard]] ExecutorOptions& options() { return opts_; }

 private:
  // Drains the plan's streams, returns its storages to the allocator while the
  // streams they were last used on still exist, then drops the plan.
  void release_plan();
  [[nodiscard]] Status issue_plan();   // one iteration's launches, events and fills
  [[nodiscard]] Status issue_poison(rt::Stream& s0);   // the poison fills of one iteration
  [[nodiscard]] Status launch_node(std::size_t i, rt::Stream& st);   // scheduled node i's op
  [[nodiscard]] Status assemble_across_streams(void** out_exec);
  void release_capture();

  Graph graph_;
  DeviceAllocator& alloc_;
  DeviceInfo device_;
  ExecutorOptions opts_;
  ExecutionPlan plan_;
  Profiler profiler_;
  std::vector<NodeTiming> node_timings_;
  std::vector<std::pair<TensorId, std::vector<char>>> input_cache_;
  bool planned_ = false;
  void* graph_exec_ = nullptr;   // hipGraphExec_t of the captured iteration
  // hipGraph_t of each node's capture (multi-stream plans), kept until the
  // executable graph assembled from them is released.
  std::vector<void*> capture_parts_;
};

}  // namespace mcke
