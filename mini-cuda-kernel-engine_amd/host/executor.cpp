// executor.cpp -- GraphExecutor: plan, replay, timing probes and the bitwise
// numerics gate (reference src/graph/executor.cpp:39-619).
#include "mcke/graph/executor.hpp"

#include <algorithm>
#include <cstring>
#include <sstream>

#include "mcke/graph/cost_model.hpp"
#include "mcke_amd.h"

namespace mcke {

namespace {
Status rc_status(int rc, const char* what) {
  if (rc == MCKE_STATUS_OK) return OkStatus();
  return Status(static_cast<StatusCode>(rc), std::string(what) + ": " + mcke_last_error());
}

const char* schedule_name(SchedulePolicy p) {
  switch (p) {
    case SchedulePolicy::kSequential: return "sequential";
    case SchedulePolicy::kLevelParallel: return "level_parallel";
    case SchedulePolicy::kChainGreedy: return "chain_greedy";
  }
  return "?";
}

const char* memory_name(MemoryPolicy p) {
  switch (p) {
    case MemoryPolicy::kAllocPerTensor: return "alloc_per_tensor";
    case MemoryPolicy::kReuseTopoNaive: return "reuse_topo_naive";
    case MemoryPolicy::kReuseSameStream: return "reuse_same_stream";
    case MemoryPolicy::kReuseHappensBefore: return "reuse_happens_before";
  }
  return "?";
}
}  // namespace

GraphExecutor::GraphExecutor(Graph graph, DeviceAllocator& alloc, DeviceInfo device, ExecutorOptions opts)
    : graph_(std::move(graph)), alloc_(alloc), device_(std::move(device)), opts_(opts) {}

GraphExecutor::~GraphExecutor() { release_plan(); }

void GraphExecutor::release_plan() {
  // Queued work may still touch the arena: drain the streams first.  The
  // storages go back to the allocator (stream-ordered, against stream 0) while
  // that stream still exists, and parked blocks are settled before the streams
  // are destroyed, so the allocator never holds a dead stream handle.
  for (rt::Stream& s : plan_.streams_) (void)s.synchronize();
  release_capture();
  plan_.node_inputs_.clear();
  plan_.node_outputs_.clear();
  plan_.bound_.clear();
  plan_.workspaces_.clear();
  plan_.arena_.reset();
  plan_.poison_src_.reset();
  (void)alloc_.settle_pending();
  plan_ = ExecutionPlan{};
  planned_ = false;
}

Status GraphExecutor::plan() {
  MCKE_RETURN_IF_ERROR(graph_.finalize());
  release_plan();
  // Streams are balanced by roofline time; 1 TFLOP/s keeps a GEMM's weight
  // comparable across policies without claiming a peak.
  Roofline rl;
  rl.peak_gb_s = device_.peak_dram_gb_s() > 0 ? device_.peak_dram_gb_s() : 1.0;
  rl.peak_tflops = 1.0;
  MCKE_ASSIGN_OR_RETURN(StreamAssignment sa, plan_streams(graph_, opts_.schedule, opts_.num_streams, rl));
  MCKE_RETURN_IF_ERROR(verify_plan_ordering(graph_, sa));
  MCKE_ASSIGN_OR_RETURN(HappensBefore hb, sa.happens_before());
  MCKE_ASSIGN_OR_RETURN(MemoryPlan mp, plan_memory(graph_, sa, hb, opts_.memory));
  MCKE_RETURN_IF_ERROR(verify_no_buffer_races(graph_, sa, hb, mp));

  plan_.streams_plan_ = sa;
  plan_.memory_plan_ = mp;
  const std::size_t K = sa.num_streams_used;
  for (std::size_t s = 0; s < K; ++s) {
    MCKE_ASSIGN_OR_RETURN(rt::Stream st, rt::Stream::create());
    plan_.streams_.push_back(std::move(st));
  }
  for (std::size_t e = 0; e < sa.num_events; ++e) {
    MCKE_ASSIGN_OR_RETURN(rt::Event ev, rt::Event::create(rt::Event::Purpose::kDependency));
    plan_.events_.push_back(std::move(ev));
  }
  if (K > 1) {
    MCKE_ASSIGN_OR_RETURN(rt::Event fk, rt::Event::create(rt::Event::Purpose::kDependency));
    plan_.fork_event_.push_back(std::move(fk));
    for (std::size_t s = 1; s < K; ++s) {
      MCKE_ASSIGN_OR_RETURN(rt::Event ev, rt::Event::create(rt::Event::Purpose::kDependency));
      plan_.join_events_.push_back(std::move(ev));
    }
  }
  const rt::StreamHandle s0 = plan_.streams_.front().native();
  if (mp.arena_bytes > 0) {
    MCKE_ASSIGN_OR_RETURN(plan_.arena_, Storage::create(alloc_, mp.arena_bytes, s0));
  }
  for (std::size_t s = 0; s < mp.workspace_bytes.size(); ++s) {
    if (mp.workspace_bytes[s] == 0) {
      plan_.workspaces_.emplace_back();
      continue;
    }
    MCKE_ASSIGN_OR_RETURN(std::shared_ptr<Storage> w, Storage::create(alloc_, mp.workspace_bytes[s], s0));
    plan_.workspaces_.push_back(std::move(w));
  }
  plan_.bound_.assign(graph_.num_tensors(), Tensor{});
  for (std::size_t t = 0; t < graph_.num_tensors(); ++t) {
    if (mp.offset_of[t] == kNoOffset) continue;
    const TensorDesc& d = graph_.tensor(static_cast<TensorId>(t));
    MCKE_ASSIGN_OR_RETURN(plan_.bound_[t], Tensor::from_storage(plan_.arena_, mp.offset_of[t], d.shape, d.dtype));
  }
  const std::size_t S = sa.nodes.size();
  plan_.sched_.resize(S);
  plan_.node_inputs_.resize(S);
  plan_.node_outputs_.resize(S);
  for (std::size_t i = 0; i < S; ++i) {
    ScheduledNode& sn = plan_.sched_[i];
    sn.node = sa.nodes[i];
    sn.stream_idx = sa.stream_of[i];
    sn.issue_index = static_cast<std::uint16_t>(sa.issue_of[i]);
    sn.wait_offset = static_cast<std::uint32_t>(plan_.wait_pool_.size());
    sn.wait_count = static_cast<std::uint32_t>(sa.waits_of[i].size());
    plan_.wait_pool_.insert(plan_.wait_pool_.end(), sa.waits_of[i].begin(), sa.waits_of[i].end());
    sn.record_event = sa.record_of[i];
    const Node& nd = graph_.node(sn.node);
    for (TensorId t : nd.inputs) plan_.node_inputs_[i].push_back(plan_.bound_[t]);
    for (TensorId t : nd.outputs) plan_.node_outputs_[i].push_back(plan_.bound_[t]);
  }
  // Byte ranges of graph inputs inside the arena (never poisoned), merged.
  for (std::size_t t = 0; t < graph_.num_tensors(); ++t)
    if (mp.offset_of[t] != kNoOffset && graph_.tensor(static_cast<TensorId>(t)).is_graph_input)
      plan_.input_byte_ranges_.emplace_back(mp.offset_of[t], mp.offset_of[t] + mp.bytes_of[t]);
  std::sort(plan_.input_byte_ranges_.begin(), plan_.input_byte_ranges_.end());
  std::vector<std::pair<std::size_t, std::size_t>> merged;
  for (const auto& r : plan_.input_byte_ranges_) {
    if (!merged.empty() && r.first <= merged.back().second)
      merged.back().second = std::max(merged.back().second, r.second);
    else
      merged.push_back(r);
  }
  plan_.input_byte_ranges_ = std::move(merged);
  plan_.peak_bytes_ = mp.arena_bytes;
  plan_.naive_bytes_ = mp.naive_bytes;
  if (opts_.profile) {
    plan_.probe_slots_ = std::max(1, opts_.profile_slots);
    const std::size_t n_probe = S * static_cast<std::size_t>(plan_.probe_slots_) * 2;
    plan_.probes_.reserve(n_probe);
    for (std::size_t k = 0; k < n_probe; ++k) {
      MCKE_ASSIGN_OR_RETURN(rt::Event ev, rt::Event::create(rt::Event::Purpose::kTiming));
      plan_.probes_.push_back(std::move(ev));
    }
  }
  planned_ = true;
  return OkStatus();
}

Status GraphExecutor::set_input(TensorId t, const void* host_data, std::size_t bytes) {
  if (!planned_) return FailedPreconditionError("set_input: call plan() first");
  if (t >= plan_.bound_.size()) return InvalidArgumentError("set_input: tensor out of range");
  if (!graph_.tensor(t).is_graph_input)
    return InvalidArgumentError("set_input: tensor " + std::to_string(t) + " is not a graph input");
  if (!plan_.bound_[t].defined()) return FailedPreconditionError("set_input: tensor is unbound");
  if (bytes != plan_.bound_[t].nbytes())
    return InvalidArgumentError("set_input: " + std::to_string(bytes) + " bytes for a tensor of " +
                                std::to_string(plan_.bound_[t].nbytes()));
  MCKE_RETURN_IF_ERROR(plan_.bound_[t].copy_from_host(host_data, bytes, plan_.streams_.front().native()));
  if (opts_.validate_numerics) {
    const auto* p = static_cast<const char*>(host_data);
    std::vector<char> copy(p, p + bytes);
    bool replaced = false;
    for (auto& kv : input_cache_)
      if (kv.first == t) {
        kv.second = copy;
        replaced = true;
      }
    if (!replaced) input_cache_.emplace_back(t, std::move(copy));
  }
  return OkStatus();
}

void GraphExecutor::release_capture() {
  if (graph_exec_) (void)mcke_rt_graph_destroy(graph_exec_);
  graph_exec_ = nullptr;
  for (void* g : capture_parts_) (void)mcke_rt_graph_release(g);
  capture_parts_.clear();
}

Status GraphExecutor::capture_graph() {
  if (!planned_) return FailedPreconditionError("capture_graph: call plan() first");
  if (opts_.profile)
    return FailedPreconditionError("capture_graph: per-node timing probes cannot be captured (profile = false)");
  for (const ScheduledNode& sn : plan_.sched_)
    if (const auto* g = dynamic_cast<const GemmOp*>(graph_.node_op(sn.node)))
      if (g->params().variant == kernels::GemmVariant::kCublasRef)
        return FailedPreconditionError("capture_graph: node '" + graph_.node(sn.node).name +
                                       "' uses the vendor-library GEMM, which is not captured");
  release_capture();
  // Nothing may still be queued on the plan's streams when capture starts.
  for (rt::Stream& st : plan_.streams_) MCKE_RETURN_IF_ERROR(st.synchronize());
  void* exec = nullptr;
  if (plan_.streams_.size() > 1) {
    MCKE_RETURN_IF_ERROR(assemble_across_streams(&exec));
  } else {
    rt::Stream& s0 = plan_.streams_.front();
    MCKE_RETURN_IF_ERROR(rc_status(mcke_rt_stream_begin_capture(s0.native()), "capture_graph: begin"));
    const Status issued = issue_plan();
    const Status ended = rc_status(mcke_rt_stream_end_capture(s0.native(), &exec), "capture_graph: end");
    if (!issued.ok() && exec) (void)mcke_rt_graph_destroy(exec);
    MCKE_RETURN_IF_ERROR(issued);
    MCKE_RETURN_IF_ERROR(ended);
  }
  graph_exec_ = exec;
  return OkStatus();
}

namespace {
// Owns a hipGraph_t that is not instantiated (the parent or a child).
struct GraphHolder {
  void* g = nullptr;
  GraphHolder() = default;
  GraphHolder(const GraphHolder&) = delete;
  GraphHolder& operator=(const GraphHolder&) = delete;
  ~GraphHolder() {
    if (g) (void)mcke_rt_graph_release(g);
  }
};
}  // namespace

Status GraphExecutor::assemble_across_streams(void** out_exec) {
  *out_exec = nullptr;
  // On failure the parts captured so far go with the next release_capture().
  GraphHolder parent;
  MCKE_RETURN_IF_ERROR(rc_status(mcke_rt_graph_create(&parent.g), "capture_graph: create"));
  // Captures what `issue` enqueues on `st` into a child graph and adds it to the
  // parent after `deps`; *node is the new parent node.
  auto add_captured = [&](rt::Stream& st, const std::vector<void*>& deps, auto&& issue,
                          void** node) -> Status {
    MCKE_RETURN_IF_ERROR(rc_status(mcke_rt_stream_begin_capture(st.native()), "capture_graph: begin"));
    const Status issued = issue();
    void* child = nullptr;
    const Status ended =
        rc_status(mcke_rt_stream_end_capture_graph(st.native(), &child), "capture_graph: end");
    if (child) capture_parts_.push_back(child);
    MCKE_RETURN_IF_ERROR(issued);
    MCKE_RETURN_IF_ERROR(ended);
    return rc_status(mcke_rt_graph_add_child(parent.g, child, deps.data(), deps.size(), node),
                     "capture_graph: add node");
  };
  rt::Stream& s0 = plan_.streams_.front();
  // The poison fills come first: every node without another dependency waits on them.
  void* prologue = nullptr;
  if (opts_.poison_buffers && plan_.arena_)
    MCKE_RETURN_IF_ERROR(add_captured(s0, {}, [&] { return issue_poison(s0); }, &prologue));
  std::vector<void*> last_on_stream(plan_.streams_.size(), nullptr);
  std::vector<void*> recorded_by(plan_.events_.size(), nullptr);
  for (std::size_t i = 0; i < plan_.sched_.size(); ++i) {
    const ScheduledNode& sn = plan_.sched_[i];
    std::vector<void*> deps;
    auto add_dep = [&](void* d) {
      if (d && std::find(deps.begin(), deps.end(), d) == deps.end()) deps.push_back(d);
    };
    add_dep(last_on_stream[sn.stream_idx]);
    for (std::uint32_t w = 0; w < sn.wait_count; ++w) {
      const std::size_t ev = plan_.wait_pool_[sn.wait_offset + w];
      // The plan was verified to record every event before its first wait in
      // issue order, so its recording node is already in the graph.
      if (ev >= recorded_by.size() || !recorded_by[ev])
        return InternalError("capture_graph: node '" + graph_.node(sn.node).name +
                             "' waits on an event no earlier node records");
      add_dep(recorded_by[ev]);
    }
    if (deps.empty()) add_dep(prologue);
    rt::Stream& st = plan_.streams_[sn.stream_idx];
    void* node = nullptr;
    MCKE_RETURN_IF_ERROR(add_captured(st, deps, [&] { return launch_node(i, st); }, &node));
    last_on_stream[sn.stream_idx] = node;
    if (sn.record_event != kNoEvent) recorded_by[sn.record_event] = node;
  }
  MCKE_RETURN_IF_ERROR(
      rc_status(mcke_rt_graph_instantiate(parent.g, out_exec), "capture_graph: instantiate"));
  return OkStatus();
}

Status GraphExecutor::run_async() {
  if (!planned_) return FailedPreconditionError("run_async: call plan() first");
  if (graph_exec_) {
    rt::Stream& s0 = plan_.streams_.front();
    MCKE_RETURN_IF_ERROR(rc_status(mcke_rt_graph_launch(graph_exec_, s0.native()), "run_async: graph launch"));
    if (plan_.arena_) plan_.arena_->note_use(s0.native());
    ++plan_.iteration_;
    return OkStatus();
  }
  return issue_plan();
}

Status GraphExecutor::issue_poison(rt::Stream& s0) {
  if (!opts_.poison_buffers || !plan_.arena_) return OkStatus();
  // A different finite pattern each iteration, everywhere but the inputs: a
  // node that reads bytes nobody wrote this iteration gets a changing value,
  // which the numerics gate sees as run-to-run variance.
  const std::uint32_t pat = opts_.poison_pattern + static_cast<std::uint32_t>(plan_.iteration_) * 0x9E3779B9u;
  char* base = static_cast<char*>(plan_.arena_->data());
  std::size_t cursor = 0;
  auto poison = [&](std::size_t lo, std::size_t hi) -> Status {
    if (hi <= lo) return OkStatus();
    return rc_status(mcke_fill_u32_async(base + lo, pat, (hi - lo) / 4, s0.native()), "poison");
  };
  for (const auto& r : plan_.input_byte_ranges_) {
    MCKE_RETURN_IF_ERROR(poison(cursor, r.first));
    cursor = r.second;
  }
  return poison(cursor, plan_.arena_->bytes());
}

Status GraphExecutor::launch_node(std::size_t i, rt::Stream& st) {
  const ScheduledNode& sn = plan_.sched_[i];
  OpContext ctx;
  ctx.stream = st.native();
  ctx.device = &device_;
  if (sn.stream_idx < plan_.workspaces_.size() && plan_.workspaces_[sn.stream_idx]) {
    ctx.workspace = plan_.workspaces_[sn.stream_idx]->data();
    ctx.workspace_bytes = plan_.workspaces_[sn.stream_idx]->bytes();
  }
  NvtxRange range(graph_.node(sn.node).name.c_str());
  return graph_.node_op(sn.node)->launch(ctx, plan_.node_inputs_[i], plan_.node_outputs_[i]);
}

Status GraphExecutor::issue_plan() {
  const std::size_t K = plan_.streams_.size();
  rt::Stream& s0 = plan_.streams_.front();
  MCKE_RETURN_IF_ERROR(issue_poison(s0));
  if (K > 1) {
    MCKE_RETURN_IF_ERROR(plan_.fork_event_[0].record(s0));
    for (std::size_t s = 1; s < K; ++s) MCKE_RETURN_IF_ERROR(plan_.streams_[s].wait(plan_.fork_event_[0]));
  }
  const int slot = plan_.probe_slots_ ? plan_.iteration_ % plan_.probe_slots_ : 0;
  for (std::size_t i = 0; i < plan_.sched_.size(); ++i) {
    const ScheduledNode& sn = plan_.sched_[i];
    rt::Stream& st = plan_.streams_[sn.stream_idx];
    for (std::uint32_t w = 0; w < sn.wait_count; ++w)
      MCKE_RETURN_IF_ERROR(st.wait(plan_.events_[plan_.wait_pool_[sn.wait_offset + w]]));
    const std::size_t p = (i * static_cast<std::size_t>(plan_.probe_slots_) + static_cast<std::size_t>(slot)) * 2;
    if (opts_.profile) MCKE_RETURN_IF_ERROR(plan_.probes_[p].record(st));
    MCKE_RETURN_IF_ERROR(launch_node(i, st));
    if (opts_.profile) MCKE_RETURN_IF_ERROR(plan_.probes_[p + 1].record(st));
    if (sn.record_event != kNoEvent) MCKE_RETURN_IF_ERROR(plan_.events_[sn.record_event].record(st));
  }
  if (K > 1) {
    for (std::size_t s = 1; s < K; ++s) {
      MCKE_RETURN_IF_ERROR(plan_.join_events_[s - 1].record(plan_.streams_[s]));
      MCKE_RETURN_IF_ERROR(s0.wait(plan_.join_events_[s - 1]));
    }
  }
  if (plan_.arena_) plan_.arena_->note_use(s0.native());
  ++plan_.iteration_;
  return OkStatus();
}

Status GraphExecutor::synchronize() {
  if (!planned_) return FailedPreconditionError("synchronize: call plan() first");
  for (rt::Stream& s : plan_.streams_) MCKE_RETURN_IF_ERROR(s.synchronize());
  return OkStatus();
}

StatusOr<Tensor> GraphExecutor::output(TensorId t) const {
  if (!planned_) return FailedPreconditionError("output: call plan() first");
  if (t >= plan_.bound_.size()) return InvalidArgumentError("output: tensor out of range");
  if (!graph_.tensor(t).is_graph_output)
    return InvalidArgumentError("output: tensor " + std::to_string(t) + " is not a graph output");
  return plan_.bound_[t];
}

StatusOr<Tensor> GraphExecutor::any_bound_tensor(TensorId t) const {
  if (!planned_) return FailedPreconditionError("any_bound_tensor: call plan() first");
  if (t >= plan_.bound_.size() || !plan_.bound_[t].defined())
    return InvalidArgumentError("any_bound_tensor: tensor " + std::to_string(t) + " has no buffer");
  return plan_.bound_[t];
}

Status GraphExecutor::collect_timings() {
  node_timings_.clear();
  if (!opts_.profile || !planned_) return OkStatus();
  const int slots = std::min(plan_.probe_slots_, plan_.iteration_);
  for (std::size_t i = 0; i < plan_.sched_.size(); ++i) {
    NodeTiming nt;
    nt.node = plan_.sched_[i].node;
    nt.name = graph_.node(nt.node).name;
    nt.stream_idx = plan_.sched_[i].stream_idx;
    if (const Op* op = graph_.node(nt.node).op.get()) {
      const OpCost c = op->cost(graph_.input_shapes(nt.node));
      nt.flops = c.flops;
      nt.bytes = c.bytes;
    }
    std::vector<double> ms;
    for (int s = 0; s < slots; ++s) {
      const std::size_t p = (i * static_cast<std::size_t>(plan_.probe_slots_) + static_cast<std::size_t>(s)) * 2;
      auto e = rt::Event::elapsed_ms(plan_.probes_[p], plan_.probes_[p + 1]);
      if (e.ok()) ms.push_back(*e);
    }
    if (!ms.empty()) {
      std::sort(ms.begin(), ms.end());
      nt.median_ms = ms[ms.size() / 2];
      nt.min_ms = ms.front();
      nt.samples = static_cast<int>(ms.size());
    }
    node_timings_.push_back(std::move(nt));
  }
  return OkStatus();
}

std::size_t first_bit_mismatch(const void* a, const void* b, std::size_t bytes) {
  const auto* x = static_cast<const unsigned char*>(a);
  const auto* y = static_cast<const unsigned char*>(b);
  std::size_t i = 0;
  for (; i + 4 <= bytes; i += 4)
    if (std::memcmp(x + i, y + i, 4) != 0) return i;
  for (; i < bytes; ++i)
    if (x[i] != y[i]) return i;
  return bytes;
}

StatusOr<NumericsResult> GraphExecutor::validate_numerics(int repeats) {
  if (!opts_.validate_numerics)
    return FailedPreconditionError("validate_numerics: set ExecutorOptions::validate_numerics before plan()");
  if (input_cache_.empty()) return FailedPreconditionError("validate_numerics: no inputs were set");
  repeats = std::max(1, repeats);
  std::vector<TensorId> outs;
  for (std::size_t t = 0; t < graph_.num_tensors(); ++t)
    if (graph_.tensor(static_cast<TensorId>(t)).is_graph_output) outs.push_back(static_cast<TensorId>(t));
  const ExecutorOptions saved = opts_;
  const auto cached = input_cache_;

  // Plans one configuration, runs it `repeats` times with poisoning and returns
  // the outputs of the first run; run-to-run differences are reported in *err.
  auto run_config = [&](SchedulePolicy sp, MemoryPolicy mpol, std::vector<std::vector<char>>* first,
                        std::string* err) -> Status {
    opts_ = saved;
    opts_.schedule = sp;
    opts_.memory = mpol;
    opts_.poison_buffers = true;
    opts_.num_streams = sp == SchedulePolicy::kSequential ? 1 : saved.num_streams;
    MCKE_RETURN_IF_ERROR(plan());
    for (const auto& kv : cached) MCKE_RETURN_IF_ERROR(set_input(kv.first, kv.second.data(), kv.second.size()));
    for (int r = 0; r < repeats; ++r) {
      MCKE_RETURN_IF_ERROR(run_async());
      MCKE_RETURN_IF_ERROR(synchronize());
      std::vector<std::vector<char>> got(outs.size());
      for (std::size_t k = 0; k < outs.size(); ++k) {
        MCKE_ASSIGN_OR_RETURN(Tensor t, output(outs[k]));
        got[k].resize(t.nbytes());
        MCKE_RETURN_IF_ERROR(t.copy_to_host(got[k].data(), got[k].size(), plan_.streams_.front().native()));
      }
      MCKE_RETURN_IF_ERROR(synchronize());
      if (r == 0) {
        *first = std::move(got);
        continue;
      }
      for (std::size_t k = 0; k < outs.size(); ++k) {
        const std::size_t off = first_bit_mismatch((*first)[k].data(), got[k].data(), got[k].size());
        if (off < got[k].size()) {
          std::uint32_t wa = 0, wb = 0;
          std::memcpy(&wa, (*first)[k].data() + (off & ~std::size_t{3}), 4);
          std::memcpy(&wb, got[k].data() + (off & ~std::size_t{3}), 4);
          std::ostringstream os;
          os << "run-to-run variance at repeat " << r << ", tensor " << outs[k] << " word " << off / 4
             << ": 0x" << std::hex << wa << " vs 0x" << wb;
          *err = os.str();
          return OkStatus();
        }
      }
    }
    return OkStatus();
  };

  NumericsResult res;
  res.repeats = repeats;
  std::vector<std::vector<char>> golden;
  std::string err;
  Status st = run_config(SchedulePolicy::kSequential, MemoryPolicy::kAllocPerTensor, &golden, &err);
  if (!st.ok() || !err.empty()) {
    opts_ = saved;
    if (!st.ok()) return st;
    res.detail = "the golden configuration is itself nondeterministic: " + err;
    return res;
  }
  for (const auto& b : golden) res.elements_compared += b.size() / 4;
  for (auto sp : {SchedulePolicy::kSequential, SchedulePolicy::kLevelParallel, SchedulePolicy::kChainGreedy}) {
    for (auto mpol : {MemoryPolicy::kAllocPerTensor, MemoryPolicy::kReuseSameStream, MemoryPolicy::kReuseHappensBefore}) {
      std::vector<std::vector<char>> got;
      err.clear();
      st = run_config(sp, mpol, &got, &err);
      if (!st.ok()) {
        opts_ = saved;
        return st;
      }
      ++res.configs_compared;
      const std::string cfg = std::string(schedule_name(sp)) + " x " + memory_name(mpol);
      if (!err.empty()) {
        opts_ = saved;
        res.detail = cfg + ": " + err;
        return res;
      }
      for (std::size_t k = 0; k < outs.size(); ++k) {
        const std::size_t off = first_bit_mismatch(golden[k].data(), got[k].data(), got[k].size());
        if (off < got[k].size()) {
          opts_ = saved;
          std::ostringstream os;
          os << cfg << " differs from the golden run in tensor " << outs[k] << " ('"
             << graph_.tensor(outs[k]).name << "') at word " << off / 4;
          res.detail = os.str();
          return res;
        }
      }
    }
  }
  opts_ = saved;
  MCKE_RETURN_IF_ERROR(plan());
  for (const auto& kv : cached) MCKE_RETURN_IF_ERROR(set_input(kv.first, kv.second.data(), kv.second.size()));
  res.passed = true;
  res.detail = "all " + std::to_string(res.configs_compared) + " configurations bitwise identical over " +
               std::to_string(repeats) + " repeats";
  return res;
}

std::string ExecutionPlan::describe() const {
  std::ostringstream os;
  os << "plan: " << sched_.size() << " nodes on " << streams_.size() << " stream(s); events "
     << streams_plan_.num_events << " + fork/join " << forkjoin_events() << "; waits "
     << streams_plan_.waits_dedup << "; arena " << peak_bytes_ << " B (naive " << naive_bytes_ << " B)\n"
     << streams_plan_.describe() << memory_plan_.describe();
  return os.str();
}

}  // namespace mcke
