// mcke/graph/executor.hpp -- plans a graph onto streams and an arena, then
// replays it.
//
// Same API as the reference's include/mcke/graph/executor.hpp and
// executor.cpp:39-619:
//   plan()       finalize, schedule (plan_streams + verify_plan_ordering),
//                happens-before, memory plan (+ verify_no_buffer_races), create
//                streams / events / arena / per-stream workspaces, bind tensors,
//                and compile one iteration into a list of host steps;
//   run_async()  issues that list: fork (stream 0 records, the others wait), per
//                node its waits, optional timing stamps, Op::launch and its
//                record, then the join back onto stream 0.  Never synchronises
//                the host.  With poison_buffers the arena (outside the graph
//                inputs) is refilled first with a pattern that changes per run;
//   validate_numerics()  runs {sequential, level-parallel, chain-greedy} x
//                {per-tensor, same-stream, happens-before} plans `repeats` times
//                each with poisoning on and requires every output to be bitwise
//                identical to the sequential/per-tensor run.
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

// What capture_if_faster() measured and kept (no reference counterpart).
struct CaptureDecision {
  bool captured = false;          // the graph was kept: run_async() replays it
  double eager_us_per_run = 0.0;  // best block, host wall time per run issued eagerly
  double replay_us_per_run = 0.0; // best block, host wall time per replayed run
  int trials = 0;                 // runs per block (two blocks each way, alternating)
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
  [[nodiscard]] std::size_t num_streams() const noexcept { return lanes_.size(); }
  [[nodiscard]] std::size_t peak_memory_bytes() const noexcept { return arena_bytes_; }
  [[nodiscard]] std::size_t naive_memory_bytes() const noexcept { return unshared_bytes_; }
  [[nodiscard]] const std::vector<std::uint32_t>& wait_pool() const noexcept { return wait_pool_; }
  [[nodiscard]] std::string describe() const;
  [[nodiscard]] const StreamAssignment& stream_plan() const noexcept { return schedule_; }
  [[nodiscard]] const MemoryPlan& memory_plan() const noexcept { return memory_; }
  [[nodiscard]] std::size_t intra_events() const noexcept { return schedule_.num_events; }
  [[nodiscard]] std::size_t intra_waits() const noexcept { return schedule_.waits_dedup; }
  [[nodiscard]] std::size_t forkjoin_events() const noexcept {
    const std::size_t k = schedule_.num_streams_used;
    return k <= 1 ? 0 : k + 2 * (k - 1);
  }
  [[nodiscard]] rt::StreamHandle stream(std::size_t i) const { return lanes_[i].native(); }

 private:
  friend class GraphExecutor;
  // One step of an iteration as the host issues it.  plan() compiles the whole
  // iteration (fork, every node's waits / timing stamps / launch / record, join)
  // into this list once; run_async() walks it.
  struct Step {
    enum class Kind : std::uint8_t { kWait, kRecord, kStampStart, kStampStop, kLaunch };
    Kind kind = Kind::kLaunch;
    std::uint16_t lane = 0;    // index into lanes_
    std::uint32_t arg = 0;     // signal index (kWait, kRecord), scheduled node (the rest)
  };
  std::vector<ScheduledNode> sched_;
  std::vector<std::uint32_t> wait_pool_;
  std::vector<rt::Stream> lanes_;
  // Cross-stream events [0, E), then the fork event (E), then one join event per
  // lane after the first (E + 1 ...).
  std::vector<rt::Event> signals_;
  std::vector<rt::Event> stamps_;   // timing stamps: (node * stamp_slots_ + slot) * 2 + {0 start, 1 stop}
  std::vector<Step> program_;
  int stamp_slots_ = 0;
  int runs_ = 0;                     // iterations issued (selects the stamp slot and the poison pattern)
  StreamAssignment schedule_;
  MemoryPlan memory_;
  std::shared_ptr<Storage> arena_;
  std::vector<std::shared_ptr<Storage>> lane_workspace_;
  // Arena byte ranges that the poison fill rewrites each run: all but graph inputs.
  std::vector<std::pair<std::size_t, std::size_t>> poison_ranges_;
  std::vector<Tensor> bound_;                  // per tensor (undefined when unplaced)
  std::vector<std::vector<Tensor>> reads_;     // per scheduled node
  std::vector<std::vector<Tensor>> writes_;
  std::size_t arena_bytes_ = 0;
  std::size_t unshared_bytes_ = 0;
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
  // capture_graph(), then keep the graph only where replay measures faster than
  // eager issue on this plan.  A replay costs a fixed host time per graph launch
  // on this runtime, a few microseconds, where eager issue costs a little per
  // node: replay pays for plans of many short nodes and loses on plans of a few.
  // So the choice is measured: `trials` back-to-back runs eagerly, then
  // `trials` replayed, twice in alternation, each block timed on the host from
  // its first enqueue to its last run's completion; the best block of each
  // decides.  A losing graph is released, and run_async() issues the plan's
  // launches as before.  Outputs are the same bits either way.
  [[nodiscard]] StatusOr<CaptureDecision> capture_if_faster(int trials = 50);
  [[nodiscard]] bool captured() const noexcept { return replay_ != nullptr; }
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
  // Waits for everything queued on the plan's streams, hands its storages back
  // to the allocator while those streams still exist, and forgets the plan.
  void drop_plan();
  void drop_replay();
  [[nodiscard]] Status run_program();                // one eager iteration
  [[nodiscard]] Status refill_poison(rt::Stream& s0);
  [[nodiscard]] Status launch(std::size_t i, rt::Stream& lane);   // scheduled node i's op
  [[nodiscard]] Status capture_lanes(void** out_exec);            // multi-stream capture
  struct GateOutcome;
  [[nodiscard]] Status gate_config(SchedulePolicy sp, MemoryPolicy mp, int repeats, GateOutcome* out);

  Graph graph_;
  DeviceAllocator& alloc_;
  DeviceInfo device_;
  ExecutorOptions opts_;
  ExecutionPlan plan_;
  Profiler profiler_;
  std::vector<NodeTiming> node_timings_;
  // Host copies of the graph inputs, kept for validate_numerics() to replan with.
  std::vector<std::pair<TensorId, std::vector<char>>> gate_inputs_;
  bool planned_ = false;
  void* replay_ = nullptr;             // hipGraphExec_t of the captured iteration
  // hipGraph_t of each node's capture (multi-stream plans), kept until the
  // executable graph assembled from them is released.
  std::vector<void*> replay_parts_;
};

}  // namespace mcke
