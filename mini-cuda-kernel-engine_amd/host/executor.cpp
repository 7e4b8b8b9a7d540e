// executor.cpp -- GraphExecutor: plan a graph onto HIP streams and one arena,
// replay it, time its nodes, capture it into a HIP graph, and gate it on
// bitwise-identical results across plans.
//
// Contract: reference include/mcke/graph/executor.hpp and
// src/graph/executor.cpp:39-619 (plan / set_input / run_async / synchronize /
// output / collect_timings / validate_numerics, ExecutionPlan's public view).
//
// plan() compiles one iteration into a list of host steps (ExecutionPlan::Step):
// the fork, then for each scheduled node its waits, timing stamps, launch and
// event record, then the join.  An eager run is the poison fill (when asked for)
// followed by a walk of that list; nothing in the list depends on the run except
// which stamp slot it writes, so the list is built once.  A captured replay
// turns the same schedule into graph edges instead of events.
#include "mcke/graph/executor.hpp"

#include <algorithm>
#include <chrono>
#include <cstring>
#include <sstream>

#include "mcke_amd.h"

namespace mcke {

namespace {

Status from_abi(int rc, const char* what) {
  if (rc == MCKE_STATUS_OK) return OkStatus();
  return Status(static_cast<StatusCode>(rc), std::string(what) + ": " + mcke_last_error());
}

const char* label(SchedulePolicy p) {
  switch (p) {
    case SchedulePolicy::kSequential: return "sequential";
    case SchedulePolicy::kLevelParallel: return "level-parallel";
    case SchedulePolicy::kChainGreedy: return "chain-greedy";
  }
  return "?";
}

const char* label(MemoryPolicy p) {
  switch (p) {
    case MemoryPolicy::kAllocPerTensor: return "per-tensor";
    case MemoryPolicy::kReuseTopoNaive: return "topo-naive";
    case MemoryPolicy::kReuseSameStream: return "same-stream";
    case MemoryPolicy::kReuseHappensBefore: return "happens-before";
  }
  return "?";
}

// Owns a hipGraph_t that is not instantiated.
class GraphRef {
 public:
  GraphRef() = default;
  GraphRef(const GraphRef&) = delete;
  GraphRef& operator=(const GraphRef&) = delete;
  ~GraphRef() {
    if (g_) (void)mcke_rt_graph_release(g_);
  }
  void** out() { return &g_; }
  void* get() const { return g_; }

 private:
  void* g_ = nullptr;
};

}  // namespace

GraphExecutor::GraphExecutor(Graph graph, DeviceAllocator& alloc, DeviceInfo device, ExecutorOptions opts)
    : graph_(std::move(graph)), alloc_(alloc), device_(std::move(device)), opts_(opts) {}

GraphExecutor::~GraphExecutor() { drop_plan(); }

void GraphExecutor::drop_plan() {
  for (rt::Stream& lane : plan_.lanes_) (void)lane.synchronize();
  drop_replay();
  // Tensors hold the storages; release every holder, then let the allocator
  // settle the parked frees while the streams they were used on still exist.
  plan_.reads_.clear();
  plan_.writes_.clear();
  plan_.bound_.clear();
  plan_.lane_workspace_.clear();
  plan_.arena_.reset();
  (void)alloc_.settle_pending();
  plan_ = ExecutionPlan{};
  planned_ = false;
}

void GraphExecutor::drop_replay() {
  if (replay_) (void)mcke_rt_graph_destroy(replay_);
  replay_ = nullptr;
  for (void* part : replay_parts_) (void)mcke_rt_graph_release(part);
  replay_parts_.clear();
}

Status GraphExecutor::plan() {
  MCKE_RETURN_IF_ERROR(graph_.finalize());
  drop_plan();
  ExecutionPlan& p = plan_;

  // Schedule, order, memory.  Streams are balanced by roofline time at the
  // device's HBM bandwidth and a nominal 1 TFLOP/s, which weighs GEMMs against
  // memory-bound ops the same way under every policy.
  Roofline rl;
  rl.peak_gb_s = device_.peak_dram_gb_s() > 0 ? device_.peak_dram_gb_s() : 1.0;
  rl.peak_tflops = 1.0;
  MCKE_ASSIGN_OR_RETURN(p.schedule_, plan_streams(graph_, opts_.schedule, opts_.num_streams, rl));
  MCKE_RETURN_IF_ERROR(verify_plan_ordering(graph_, p.schedule_));
  MCKE_ASSIGN_OR_RETURN(HappensBefore hb, p.schedule_.happens_before());
  MCKE_ASSIGN_OR_RETURN(p.memory_, plan_memory(graph_, p.schedule_, hb, opts_.memory));
  MCKE_RETURN_IF_ERROR(verify_no_buffer_races(graph_, p.schedule_, hb, p.memory_));
  const StreamAssignment& sa = p.schedule_;
  const MemoryPlan& mp = p.memory_;
  const std::size_t lanes = sa.num_streams_used;
  const std::size_t S = sa.nodes.size();

  // Streams and events: cross-stream events, fork, joins.
  for (std::size_t k = 0; k < lanes; ++k) {
    MCKE_ASSIGN_OR_RETURN(rt::Stream lane, rt::Stream::create());
    p.lanes_.push_back(std::move(lane));
  }
  const std::size_t n_signals = sa.num_events + (lanes > 1 ? lanes : 0);
  for (std::size_t e = 0; e < n_signals; ++e) {
    MCKE_ASSIGN_OR_RETURN(rt::Event ev, rt::Event::create(rt::Event::Purpose::kDependency));
    p.signals_.push_back(std::move(ev));
  }
  if (opts_.profile) {
    p.stamp_slots_ = std::max(1, opts_.profile_slots);
    for (std::size_t k = 0; k < S * static_cast<std::size_t>(p.stamp_slots_) * 2; ++k) {
      MCKE_ASSIGN_OR_RETURN(rt::Event ev, rt::Event::create(rt::Event::Purpose::kTiming));
      p.stamps_.push_back(std::move(ev));
    }
  }

  // Memory: the arena, one workspace per stream that needs one, bound tensors.
  const rt::StreamHandle s0 = p.lanes_.front().native();
  if (mp.arena_bytes) {
    MCKE_ASSIGN_OR_RETURN(p.arena_, Storage::create(alloc_, mp.arena_bytes, s0));
  }
  for (std::size_t w : mp.workspace_bytes) {
    std::shared_ptr<Storage> ws;
    if (w) {
      MCKE_ASSIGN_OR_RETURN(ws, Storage::create(alloc_, w, s0));
    }
    p.lane_workspace_.push_back(std::move(ws));
  }
  p.bound_.resize(graph_.num_tensors());
  std::vector<std::pair<std::size_t, std::size_t>> inputs;   // arena ranges of graph inputs
  for (std::size_t t = 0; t < graph_.num_tensors(); ++t) {
    if (mp.offset_of[t] == kNoOffset) continue;
    const TensorDesc& d = graph_.tensor(static_cast<TensorId>(t));
    MCKE_ASSIGN_OR_RETURN(p.bound_[t], Tensor::from_storage(p.arena_, mp.offset_of[t], d.shape, d.dtype));
    if (d.is_graph_input) inputs.emplace_back(mp.offset_of[t], mp.offset_of[t] + mp.bytes_of[t]);
  }
  // The poison ranges: the arena minus the graph inputs.
  std::sort(inputs.begin(), inputs.end());
  std::size_t cursor = 0;
  for (const auto& [lo, hi] : inputs) {
    if (lo > cursor) p.poison_ranges_.emplace_back(cursor, lo);
    cursor = std::max(cursor, hi);
  }
  if (mp.arena_bytes > cursor) p.poison_ranges_.emplace_back(cursor, mp.arena_bytes);

  // The public view of the schedule, and the step list of one iteration.
  using Step = ExecutionPlan::Step;
  const auto fork = static_cast<std::uint32_t>(sa.num_events);
  for (std::size_t k = 1; k < lanes; ++k) {
    if (k == 1) p.program_.push_back({Step::Kind::kRecord, 0, fork});
    p.program_.push_back({Step::Kind::kWait, static_cast<std::uint16_t>(k), fork});
  }
  p.sched_.resize(S);
  p.reads_.resize(S);
  p.writes_.resize(S);
  for (std::size_t i = 0; i < S; ++i) {
    const Node& nd = graph_.node(sa.nodes[i]);
    const auto lane = sa.stream_of[i];
    const auto idx = static_cast<std::uint32_t>(i);
    ScheduledNode& sn = p.sched_[i];
    sn.node = sa.nodes[i];
    sn.stream_idx = lane;
    sn.issue_index = static_cast<std::uint16_t>(sa.issue_of[i]);
    sn.wait_offset = static_cast<std::uint32_t>(p.wait_pool_.size());
    sn.wait_count = static_cast<std::uint32_t>(sa.waits_of[i].size());
    sn.record_event = sa.record_of[i];
    for (std::uint32_t e : sa.waits_of[i]) {
      p.wait_pool_.push_back(e);
      p.program_.push_back({Step::Kind::kWait, lane, e});
    }
    if (opts_.profile) p.program_.push_back({Step::Kind::kStampStart, lane, idx});
    p.program_.push_back({Step::Kind::kLaunch, lane, idx});
    if (opts_.profile) p.program_.push_back({Step::Kind::kStampStop, lane, idx});
    if (sn.record_event != kNoEvent) p.program_.push_back({Step::Kind::kRecord, lane, sn.record_event});
    for (TensorId t : nd.inputs) p.reads_[i].push_back(p.bound_[t]);
    for (TensorId t : nd.outputs) p.writes_[i].push_back(p.bound_[t]);
  }
  for (std::size_t k = 1; k < lanes; ++k) {
    const auto join = static_cast<std::uint32_t>(sa.num_events + k);
    p.program_.push_back({Step::Kind::kRecord, static_cast<std::uint16_t>(k), join});
    p.program_.push_back({Step::Kind::kWait, 0, join});
  }
  p.arena_bytes_ = mp.arena_bytes;
  p.unshared_bytes_ = mp.naive_bytes;
  planned_ = true;
  return OkStatus();
}

Status GraphExecutor::set_input(TensorId t, const void* host_data, std::size_t bytes) {
  if (!planned_) return FailedPreconditionError("set_input: plan() the graph first");
  if (t >= plan_.bound_.size() || !graph_.tensor(t).is_graph_input)
    return InvalidArgumentError("set_input: tensor " + std::to_string(t) + " is not an input of this graph");
  Tensor& dst = plan_.bound_[t];
  if (!dst.defined()) return FailedPreconditionError("set_input: input " + std::to_string(t) + " has no buffer");
  if (bytes != dst.nbytes())
    return InvalidArgumentError("set_input: input " + std::to_string(t) + " holds " +
                                std::to_string(dst.nbytes()) + " bytes, given " + std::to_string(bytes));
  MCKE_RETURN_IF_ERROR(dst.copy_from_host(host_data, bytes, plan_.lanes_.front().native()));
  if (opts_.validate_numerics) {
    const auto* src = static_cast<const char*>(host_data);
    auto it = std::find_if(gate_inputs_.begin(), gate_inputs_.end(),
                           [&](const auto& kv) { return kv.first == t; });
    if (it == gate_inputs_.end()) it = gate_inputs_.insert(gate_inputs_.end(), {t, {}});
    it->second.assign(src, src + bytes);
  }
  return OkStatus();
}

Status GraphExecutor::refill_poison(rt::Stream& s0) {
  if (!opts_.poison_buffers || !plan_.arena_) return OkStatus();
  // A finite pattern that differs from run to run: a node reading bytes that no
  // one wrote this run sees a changing value, which the gate reports as variance.
  const std::uint32_t pattern =
      opts_.poison_pattern ^ (static_cast<std::uint32_t>(plan_.runs_) * 0x01000193u);
  char* base = static_cast<char*>(plan_.arena_->data());
  for (const auto& [lo, hi] : plan_.poison_ranges_)
    MCKE_RETURN_IF_ERROR(
        from_abi(mcke_fill_u32_async(base + lo, pattern, (hi - lo) / 4, s0.native()), "poison fill"));
  return OkStatus();
}

Status GraphExecutor::launch(std::size_t i, rt::Stream& lane) {
  const ScheduledNode& sn = plan_.sched_[i];
  OpContext ctx;
  ctx.stream = lane.native();
  ctx.device = &device_;
  if (const auto& ws = plan_.lane_workspace_[sn.stream_idx]) {
    ctx.workspace = ws->data();
    ctx.workspace_bytes = ws->bytes();
  }
  NvtxRange marker(graph_.node(sn.node).name.c_str());
  return graph_.node_op(sn.node)->launch(ctx, plan_.reads_[i], plan_.writes_[i]);
}

Status GraphExecutor::run_program() {
  ExecutionPlan& p = plan_;
  MCKE_RETURN_IF_ERROR(refill_poison(p.lanes_.front()));
  const std::size_t slot = p.stamp_slots_ ? static_cast<std::size_t>(p.runs_ % p.stamp_slots_) : 0;
  auto stamp = [&](std::uint32_t node, std::size_t which) -> rt::Event& {
    return p.stamps_[(node * static_cast<std::size_t>(p.stamp_slots_) + slot) * 2 + which];
  };
  using Kind = ExecutionPlan::Step::Kind;
  for (const ExecutionPlan::Step& step : p.program_) {
    rt::Stream& lane = p.lanes_[step.lane];
    switch (step.kind) {
      case Kind::kWait: MCKE_RETURN_IF_ERROR(lane.wait(p.signals_[step.arg])); break;
      case Kind::kRecord: MCKE_RETURN_IF_ERROR(p.signals_[step.arg].record(lane)); break;
      case Kind::kStampStart: MCKE_RETURN_IF_ERROR(stamp(step.arg, 0).record(lane)); break;
      case Kind::kStampStop: MCKE_RETURN_IF_ERROR(stamp(step.arg, 1).record(lane)); break;
      case Kind::kLaunch: MCKE_RETURN_IF_ERROR(launch(step.arg, lane)); break;
    }
  }
  if (p.arena_) p.arena_->note_use(p.lanes_.front().native());
  ++p.runs_;
  return OkStatus();
}

Status GraphExecutor::run_async() {
  if (!planned_) return FailedPreconditionError("run_async: plan() the graph first");
  if (!replay_) return run_program();
  rt::Stream& s0 = plan_.lanes_.front();
  MCKE_RETURN_IF_ERROR(from_abi(mcke_rt_graph_launch(replay_, s0.native()), "run_async: graph launch"));
  if (plan_.arena_) plan_.arena_->note_use(s0.native());
  ++plan_.runs_;
  return OkStatus();
}

Status GraphExecutor::capture_graph() {
  if (!planned_) return FailedPreconditionError("capture_graph: plan() the graph first");
  if (opts_.profile)
    return FailedPreconditionError(
        "capture_graph: the timing stamps of profile = true would be frozen into the graph");
  for (const ScheduledNode& sn : plan_.sched_) {
    const auto* gemm = dynamic_cast<const GemmOp*>(graph_.node_op(sn.node));
    if (gemm && gemm->params().variant == kernels::GemmVariant::kCublasRef)
      return FailedPreconditionError("capture_graph: '" + graph_.node(sn.node).name +
                                     "' runs the vendor-library GEMM, which is not captured");
  }
  drop_replay();
  for (rt::Stream& lane : plan_.lanes_) MCKE_RETURN_IF_ERROR(lane.synchronize());
  void* exec = nullptr;
  if (plan_.lanes_.size() > 1) {
    MCKE_RETURN_IF_ERROR(capture_lanes(&exec));
  } else {
    // One stream: capture a whole eager iteration (its step list has no events).
    const rt::StreamHandle s0 = plan_.lanes_.front().native();
    MCKE_RETURN_IF_ERROR(from_abi(mcke_rt_stream_begin_capture(s0), "capture_graph: begin"));
    const int runs = plan_.runs_;
    const Status issued = run_program();
    plan_.runs_ = runs;   // the capture is not a run
    const Status ended = from_abi(mcke_rt_stream_end_capture(s0, &exec), "capture_graph: end");
    if (!issued.ok() && exec) (void)mcke_rt_graph_destroy(exec);
    MCKE_RETURN_IF_ERROR(issued);
    MCKE_RETURN_IF_ERROR(ended);
  }
  replay_ = exec;
  // Stage the graph's launch resources now, not on the first replay.
  MCKE_RETURN_IF_ERROR(from_abi(mcke_rt_graph_upload(replay_, plan_.lanes_.front().native()),
                                "capture_graph: upload"));
  return plan_.lanes_.front().synchronize();
}

StatusOr<CaptureDecision> GraphExecutor::capture_if_faster(int trials) {
  if (trials < 1) return InvalidArgumentError("capture_if_faster: trials must be >= 1");
  MCKE_RETURN_IF_ERROR(capture_graph());
  void* graph = replay_;
  // One block: `trials` runs back to back, host wall time per run from the first
  // enqueue to the completion of the last.
  auto block = [&](void* use) -> StatusOr<double> {
    replay_ = use;
    const auto t0 = std::chrono::steady_clock::now();
    for (int r = 0; r < trials; ++r) MCKE_RETURN_IF_ERROR(run_async());
    MCKE_RETURN_IF_ERROR(synchronize());
    const auto t1 = std::chrono::steady_clock::now();
    return std::chrono::duration<double, std::micro>(t1 - t0).count() / trials;
  };
  CaptureDecision d;
  d.trials = trials;
  d.eager_us_per_run = d.replay_us_per_run = 1e300;
  for (int round = 0; round < 2; ++round) {
    auto e = block(nullptr);
    if (!e.ok()) {
      replay_ = graph;
      return e.status();
    }
    auto g = block(graph);
    if (!g.ok()) return g.status();
    d.eager_us_per_run = std::min(d.eager_us_per_run, *e);
    d.replay_us_per_run = std::min(d.replay_us_per_run, *g);
  }
  replay_ = graph;
  d.captured = d.replay_us_per_run < d.eager_us_per_run;
  if (!d.captured) drop_replay();
  return d;
}

// Several streams: no capture may span two of them, so each node's launches are
// captured alone on its own stream and their kernel nodes are added to a parent
// graph whose edges stand for the schedule: a node depends on the previous node
// of its stream and on the recorders of the events it waits on.  The poison
// fills, when on, form a prologue that every node without another dependency
// follows.
Status GraphExecutor::capture_lanes(void** out_exec) {
  *out_exec = nullptr;
  GraphRef parent;
  MCKE_RETURN_IF_ERROR(from_abi(mcke_rt_graph_create(parent.out()), "capture_graph: create"));
  auto capture_into_parent = [&](rt::Stream& lane, const std::vector<void*>& after, auto&& enqueue,
                                 void** added) -> Status {
    MCKE_RETURN_IF_ERROR(from_abi(mcke_rt_stream_begin_capture(lane.native()), "capture_graph: begin"));
    const Status enqueued = enqueue();
    void* part = nullptr;
    const Status ended =
        from_abi(mcke_rt_stream_end_capture_graph(lane.native(), &part), "capture_graph: end");
    if (part) replay_parts_.push_back(part);
    MCKE_RETURN_IF_ERROR(enqueued);
    MCKE_RETURN_IF_ERROR(ended);
    return from_abi(mcke_rt_graph_add_child(parent.get(), part, after.data(), after.size(), added),
                    "capture_graph: add");
  };
  rt::Stream& s0 = plan_.lanes_.front();
  void* prologue = nullptr;
  if (opts_.poison_buffers && plan_.arena_)
    MCKE_RETURN_IF_ERROR(capture_into_parent(s0, {}, [&] { return refill_poison(s0); }, &prologue));
  std::vector<void*> tail(plan_.lanes_.size(), nullptr);            // last graph node per stream
  std::vector<void*> recorder(plan_.schedule_.num_events, nullptr);  // graph node per event
  for (std::size_t i = 0; i < plan_.sched_.size(); ++i) {
    const ScheduledNode& sn = plan_.sched_[i];
    std::vector<void*> after;
    auto need = [&](void* g) {
      if (g && std::find(after.begin(), after.end(), g) == after.end()) after.push_back(g);
    };
    need(tail[sn.stream_idx]);
    for (std::uint32_t k = 0; k < sn.wait_count; ++k) {
      const std::uint32_t e = plan_.wait_pool_[sn.wait_offset + k];
      if (!recorder[e])
        return InternalError("capture_graph: '" + graph_.node(sn.node).name + "' waits on event " +
                             std::to_string(e) + " before any node records it");
      need(recorder[e]);
    }
    if (after.empty()) need(prologue);
    rt::Stream& lane = plan_.lanes_[sn.stream_idx];
    void* added = nullptr;
    MCKE_RETURN_IF_ERROR(capture_into_parent(lane, after, [&] { return launch(i, lane); }, &added));
    tail[sn.stream_idx] = added;
    if (sn.record_event != kNoEvent) recorder[sn.record_event] = added;
  }
  return from_abi(mcke_rt_graph_instantiate(parent.get(), out_exec), "capture_graph: instantiate");
}

Status GraphExecutor::synchronize() {
  if (!planned_) return FailedPreconditionError("synchronize: plan() the graph first");
  for (rt::Stream& lane : plan_.lanes_) MCKE_RETURN_IF_ERROR(lane.synchronize());
  return OkStatus();
}

StatusOr<Tensor> GraphExecutor::output(TensorId t) const {
  if (!planned_) return FailedPreconditionError("output: plan() the graph first");
  if (t >= plan_.bound_.size() || !graph_.tensor(t).is_graph_output)
    return InvalidArgumentError("output: tensor " + std::to_string(t) + " is not an output of this graph");
  return plan_.bound_[t];
}

StatusOr<Tensor> GraphExecutor::any_bound_tensor(TensorId t) const {
  if (!planned_) return FailedPreconditionError("any_bound_tensor: plan() the graph first");
  if (t >= plan_.bound_.size() || !plan_.bound_[t].defined())
    return InvalidArgumentError("any_bound_tensor: tensor " + std::to_string(t) +
                                " is not placed in this plan's arena");
  return plan_.bound_[t];
}

Status GraphExecutor::collect_timings() {
  node_timings_.clear();
  if (!opts_.profile || !planned_) return OkStatus();
  const std::size_t slots = static_cast<std::size_t>(std::min(plan_.stamp_slots_, plan_.runs_));
  for (std::size_t i = 0; i < plan_.sched_.size(); ++i) {
    const ScheduledNode& sn = plan_.sched_[i];
    NodeTiming nt;
    nt.node = sn.node;
    nt.name = graph_.node(sn.node).name;
    nt.stream_idx = sn.stream_idx;
    if (const Op* op = graph_.node(sn.node).op.get()) {
      const OpCost c = op->cost(graph_.input_shapes(sn.node));
      nt.flops = c.flops;
      nt.bytes = c.bytes;
    }
    std::vector<double> ms;
    for (std::size_t s = 0; s < slots; ++s) {
      const std::size_t base = (i * static_cast<std::size_t>(plan_.stamp_slots_) + s) * 2;
      auto dt = rt::Event::elapsed_ms(plan_.stamps_[base], plan_.stamps_[base + 1]);
      if (dt.ok()) ms.push_back(*dt);
    }
    if (!ms.empty()) {
      std::nth_element(ms.begin(), ms.begin() + static_cast<std::ptrdiff_t>(ms.size() / 2), ms.end());
      nt.median_ms = ms[ms.size() / 2];
      nt.min_ms = *std::min_element(ms.begin(), ms.end());
      nt.samples = static_cast<int>(ms.size());
    }
    node_timings_.push_back(std::move(nt));
  }
  return OkStatus();
}

std::size_t first_bit_mismatch(const void* a, const void* b, std::size_t bytes) {
  const auto* x = static_cast<const unsigned char*>(a);
  const auto* y = static_cast<const unsigned char*>(b);
  const auto* hit = std::mismatch(x, x + bytes, y).first;
  // Report the start of the 32-bit word holding the first differing byte.
  const std::size_t at = static_cast<std::size_t>(hit - x);
  return at == bytes ? bytes : at & ~std::size_t{3};
}

// The outputs of a configuration's first run, or how its runs disagreed.
struct GraphExecutor::GateOutcome {
  std::vector<std::vector<char>> outputs;
  std::string variance;
};

Status GraphExecutor::gate_config(SchedulePolicy sp, MemoryPolicy mp, int repeats, GateOutcome* out) {
  opts_.schedule = sp;
  opts_.memory = mp;
  opts_.poison_buffers = true;
  MCKE_RETURN_IF_ERROR(plan());
  for (const auto& [t, bytes] : gate_inputs_) MCKE_RETURN_IF_ERROR(set_input(t, bytes.data(), bytes.size()));
  std::vector<TensorId> outs;
  for (std::size_t t = 0; t < graph_.num_tensors(); ++t)
    if (graph_.tensor(static_cast<TensorId>(t)).is_graph_output) outs.push_back(static_cast<TensorId>(t));
  const rt::StreamHandle s0 = plan_.lanes_.front().native();
  for (int r = 0; r < repeats; ++r) {
    MCKE_RETURN_IF_ERROR(run_async());
    std::vector<std::vector<char>> got(outs.size());
    for (std::size_t k = 0; k < outs.size(); ++k) {
      got[k].resize(plan_.bound_[outs[k]].nbytes());
      MCKE_RETURN_IF_ERROR(plan_.bound_[outs[k]].copy_to_host(got[k].data(), got[k].size(), s0));
    }
    MCKE_RETURN_IF_ERROR(synchronize());
    if (r == 0) {
      out->outputs = std::move(got);
      continue;
    }
    for (std::size_t k = 0; k < outs.size(); ++k) {
      const std::size_t at = first_bit_mismatch(out->outputs[k].data(), got[k].data(), got[k].size());
      if (at == got[k].size()) continue;
      std::uint32_t was = 0, now = 0;
      std::memcpy(&was, out->outputs[k].data() + at, std::min<std::size_t>(4, got[k].size() - at));
      std::memcpy(&now, got[k].data() + at, std::min<std::size_t>(4, got[k].size() - at));
      std::ostringstream os;
      os << "run " << r << " differs from run 0 in '" << graph_.tensor(outs[k]).name << "' at element "
         << at / 4 << " (0x" << std::hex << was << " then 0x" << now << ")";
      out->variance = os.str();
      return OkStatus();
    }
  }
  return OkStatus();
}

StatusOr<NumericsResult> GraphExecutor::validate_numerics(int repeats) {
  if (!opts_.validate_numerics)
    return FailedPreconditionError("validate_numerics: construct the executor with "
                                   "ExecutorOptions::validate_numerics = true");
  if (gate_inputs_.empty()) return FailedPreconditionError("validate_numerics: set_input() every input first");
  repeats = std::max(1, repeats);
  const ExecutorOptions user = opts_;
  NumericsResult res;
  res.repeats = repeats;

  // The sequential / per-tensor plan is the reference every plan is held to,
  // itself included (which also checks that it is stable over its repeats).
  std::vector<std::vector<char>> golden;
  std::string verdict;
  Status st = OkStatus();
  for (SchedulePolicy sp : {SchedulePolicy::kSequential, SchedulePolicy::kLevelParallel,
                            SchedulePolicy::kChainGreedy}) {
    for (MemoryPolicy mp : {MemoryPolicy::kAllocPerTensor, MemoryPolicy::kReuseSameStream,
                            MemoryPolicy::kReuseHappensBefore}) {
      opts_.num_streams = sp == SchedulePolicy::kSequential ? 1 : user.num_streams;
      GateOutcome got;
      st = gate_config(sp, mp, repeats, &got);
      if (!st.ok()) break;
      const std::string name = std::string(label(sp)) + " / " + label(mp);
      ++res.configs_compared;
      if (!got.variance.empty()) {
        verdict = name + ": " + got.variance;
        break;
      }
      if (golden.empty()) {
        golden = std::move(got.outputs);
        for (const auto& bytes : golden) res.elements_compared += bytes.size() / 4;
        continue;
      }
      for (std::size_t k = 0; k < golden.size() && verdict.empty(); ++k) {
        const std::size_t at = first_bit_mismatch(golden[k].data(), got.outputs[k].data(), golden[k].size());
        if (at < golden[k].size())
          verdict = name + " gives different bits from sequential / per-tensor in output " +
                    std::to_string(k) + " at element " + std::to_string(at / 4);
      }
      if (!verdict.empty()) break;
    }
    if (!st.ok() || !verdict.empty()) break;
  }

  // Back to the caller's plan and inputs.
  opts_ = user;
  if (!st.ok()) return st;
  MCKE_RETURN_IF_ERROR(plan());
  for (const auto& [t, bytes] : gate_inputs_) MCKE_RETURN_IF_ERROR(set_input(t, bytes.data(), bytes.size()));
  res.passed = verdict.empty();
  res.detail = res.passed ? "bitwise identical: " + std::to_string(res.configs_compared) +
                                " plans x " + std::to_string(repeats) + " runs each"
                          : verdict;
  return res;
}

std::string ExecutionPlan::describe() const {
  std::ostringstream os;
  os << sched_.size() << " node(s) on " << lanes_.size() << " stream(s), " << schedule_.num_events
     << " cross-stream event(s) + " << forkjoin_events() << " fork/join, " << program_.size()
     << " host steps per run\n"
     << schedule_.describe() << memory_.describe();
  return os.str();
}

}  // namespace mcke
