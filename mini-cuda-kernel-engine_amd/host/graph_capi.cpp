// graph_capi.cpp -- the mcke_graph_* / mcke_executor_* C-ABI over the C++ graph
// layer (declared in include/mcke_graph.h).
#include <cstring>
#include <memory>
#include <string>

#include "mcke/graph/executor.hpp"
#include "mcke/memory/buddy_allocator.hpp"
#include "mcke/memory/freelist_allocator.hpp"
#include "mcke_graph.h"

struct mcke_graph {
  mcke::Graph g;
};

struct mcke_executor {
  std::unique_ptr<mcke::DeviceAllocator> alloc;
  std::unique_ptr<mcke::GraphExecutor> exec;
};

namespace {

thread_local std::string t_err;

int code(const mcke::Status& s) {
  if (s.ok()) return MCKE_STATUS_OK;
  t_err = s.message();
  return static_cast<int>(s.code());
}

int bad(const char* msg) {
  t_err = msg;
  return MCKE_STATUS_INVALID_ARGUMENT;
}

template <class T>
int add_op(mcke_graph* g, std::unique_ptr<mcke::Op> op, std::vector<mcke::TensorId> in, const char* name,
           uint32_t* out) {
  if (!g || !out) return bad("null graph or output handle");
  auto r = g->g.add_node(std::move(op), std::move(in), name ? name : "");
  if (!r.ok()) return code(r.status());
  *out = (*r)[0];
  return MCKE_STATUS_OK;
}

}  // namespace

extern "C" {

const char* mcke_graph_last_error(void) { return t_err.c_str(); }

mcke_graph* mcke_graph_create(void) { return new mcke_graph(); }

void mcke_graph_destroy(mcke_graph* g) { delete g; }

int mcke_graph_add_input(mcke_graph* g, const int64_t* dims, int rank, const char* name, uint32_t* out) {
  if (!g || !dims || !out) return bad("mcke_graph_add_input: null argument");
  if (rank < 1 || rank > mcke::kMaxRank) return bad("mcke_graph_add_input: rank must be 1..5");
  auto r = g->g.add_input(mcke::Shape(dims, rank), mcke::DType::kF32, name ? name : "");
  if (!r.ok()) return code(r.status());
  *out = *r;
  return MCKE_STATUS_OK;
}

int mcke_graph_add_input_typed(mcke_graph* g, const int64_t* dims, int rank, int dtype,
                               const char* name, uint32_t* out) {
  if (!g || !dims || !out) return bad("mcke_graph_add_input_typed: null argument");
  if (rank < 1 || rank > mcke::kMaxRank) return bad("mcke_graph_add_input_typed: rank must be 1..5");
  if (dtype != MCKE_DTYPE_F32 && dtype != MCKE_DTYPE_F16 && dtype != MCKE_DTYPE_BF16)
    return bad("mcke_graph_add_input_typed: dtype must be MCKE_DTYPE_F32, _F16 or _BF16");
  auto r = g->g.add_input(mcke::Shape(dims, rank), static_cast<mcke::DType>(dtype), name ? name : "");
  if (!r.ok()) return code(r.status());
  *out = *r;
  return MCKE_STATUS_OK;
}

int mcke_graph_add_gemm_lp(mcke_graph* g, uint32_t a, uint32_t b, float alpha, int out_dtype,
                           const mcke_gemm_tile* tile, const char* name, uint32_t* out) {
  if (!g || !out) return bad("mcke_graph_add_gemm_lp: null argument");
  if (a >= g->g.num_tensors()) return bad("mcke_graph_add_gemm_lp: tensor a is out of range");
  mcke::GemmParams p;
  p.alpha = alpha;
  p.beta = 0.0f;
  p.in_dtype = g->g.tensor(a).dtype;
  p.out_dtype = static_cast<mcke::DType>(out_dtype);
  if (p.in_dtype != mcke::DType::kBF16 && p.in_dtype != mcke::DType::kF16)
    return bad("mcke_graph_add_gemm_lp: tensor a must be bf16 or f16");
  if (tile) p.tile = mcke::kernels::GemmTile{tile->bm, tile->bn, tile->bk, tile->tm, tile->tn};
  else p.auto_tile = true;
  return add_op<mcke::GemmOp>(g, std::make_unique<mcke::GemmOp>(p), {a, b}, name, out);
}

int mcke_graph_add_gemm(mcke_graph* g, uint32_t a, uint32_t b, float alpha, int variant,
                        const mcke_gemm_tile* tile, const char* name, uint32_t* out) {
  mcke::GemmParams p;
  p.alpha = alpha;
  p.beta = 0.0f;
  p.variant = static_cast<mcke::kernels::GemmVariant>(variant);
  if (tile) {
    p.tile = mcke::kernels::GemmTile{tile->bm, tile->bn, tile->bk, tile->tm, tile->tn};
  } else {
    if (p.variant != mcke::kernels::GemmVariant::kMfmaF32)
      return bad("mcke_graph_add_gemm: a null tile (per-shape choice) needs the kMfmaF32 variant");
    p.auto_tile = true;
  }
  return add_op<mcke::GemmOp>(g, std::make_unique<mcke::GemmOp>(p), {a, b}, name, out);
}

int mcke_graph_add_gemm_bias_act(mcke_graph* g, uint32_t a, uint32_t b, uint32_t bias, float alpha,
                                 int act, const mcke_gemm_tile* tile, const char* name,
                                 uint32_t* out) {
  if (act < 0 || act > 3) return bad("mcke_graph_add_gemm_bias_act: unknown activation");
  mcke::GemmBiasActParams p;
  p.alpha = alpha;
  p.act = static_cast<mcke::BiasActParams::Act>(act);
  if (tile) {
    p.tile = mcke::kernels::GemmTile{tile->bm, tile->bn, tile->bk, tile->tm, tile->tn};
    p.auto_tile = false;
  }
  return add_op<mcke::GemmBiasActOp>(g, std::make_unique<mcke::GemmBiasActOp>(p), {a, b, bias},
                                     name, out);
}

int mcke_graph_add_bias_act_rows(mcke_graph* g, uint32_t x, uint32_t bias, int act,
                                 int vector_width, int max_row_blocks, const char* name,
                                 uint32_t* out) {
  if (act < 0 || act > 3) return bad("mcke_graph_add_bias_act: unknown activation");
  if (max_row_blocks < 0) return bad("mcke_graph_add_bias_act: negative max_row_blocks");
  mcke::BiasActParams p;
  p.act = static_cast<mcke::BiasActParams::Act>(act);
  p.vector_width = vector_width;
  p.max_row_blocks = max_row_blocks;
  return add_op<mcke::BiasActOp>(g, std::make_unique<mcke::BiasActOp>(p), {x, bias}, name, out);
}

int mcke_graph_add_bias_act(mcke_graph* g, uint32_t x, uint32_t bias, int act, int vector_width,
                            const char* name, uint32_t* out) {
  return mcke_graph_add_bias_act_rows(g, x, bias, act, vector_width, 0, name, out);
}

int mcke_graph_add_reduce(mcke_graph* g, uint32_t x, int kind, int variant, const char* name, uint32_t* out) {
  if (kind < 0 || kind > 2 || variant < 0 || variant > 2) return bad("mcke_graph_add_reduce: bad kind/variant");
  mcke::ReduceParams p;
  p.kind = static_cast<mcke::ReduceParams::Kind>(kind);
  p.variant = static_cast<mcke::ReduceParams::Variant>(variant);
  return add_op<mcke::ReduceOp>(g, std::make_unique<mcke::ReduceOp>(p), {x}, name, out);
}

int mcke_graph_add_softmax(mcke_graph* g, uint32_t x, int variant, const char* name, uint32_t* out) {
  if (variant < 0 || variant > 1) return bad("mcke_graph_add_softmax: bad variant");
  mcke::SoftmaxParams p;
  p.variant = static_cast<mcke::SoftmaxParams::Variant>(variant);
  return add_op<mcke::SoftmaxOp>(g, std::make_unique<mcke::SoftmaxOp>(p), {x}, name, out);
}

int mcke_graph_mark_output(mcke_graph* g, uint32_t t) {
  if (!g) return bad("null graph");
  return code(g->g.mark_output(t));
}

int mcke_graph_num_nodes(const mcke_graph* g, uint64_t* out) {
  if (!g || !out) return bad("null argument");
  *out = g->g.num_nodes();
  return MCKE_STATUS_OK;
}

int mcke_graph_tensor_shape(const mcke_graph* g, uint32_t t, int64_t* dims5, int* rank) {
  if (!g || !dims5 || !rank) return bad("null argument");
  if (t >= g->g.num_tensors()) return bad("tensor id out of range");
  const mcke::Shape& s = g->g.tensor(t).shape;
  *rank = s.rank();
  for (int i = 0; i < s.rank(); ++i) dims5[i] = s.dim(i);
  return MCKE_STATUS_OK;
}

int mcke_executor_create(mcke_graph* g, int allocator_kind, const mcke_executor_options* o, mcke_executor** out) {
  if (!g || !out) return bad("mcke_executor_create: null argument");
  *out = nullptr;
  auto dev = mcke::query_device(0);
  if (!dev.ok()) return code(dev.status());
  mcke::ExecutorOptions opts;
  if (o) {
    if (o->schedule < 0 || o->schedule > 2 || o->memory < 0 || o->memory > 3)
      return bad("mcke_executor_create: bad schedule/memory policy");
    opts.schedule = static_cast<mcke::SchedulePolicy>(o->schedule);
    opts.memory = static_cast<mcke::MemoryPolicy>(o->memory);
    opts.num_streams = o->num_streams;
    opts.profile = o->profile != 0;
    opts.profile_slots = o->profile_slots > 0 ? o->profile_slots : 32;
    opts.validate_numerics = o->validate_numerics != 0;
    opts.poison_buffers = o->poison_buffers != 0;
    opts.poison_pattern = o->poison_pattern ? o->poison_pattern : 0x7F7F7F7Fu;
  }
  auto e = std::make_unique<mcke_executor>();
  if (allocator_kind == MCKE_ALLOC_BUDDY)
    e->alloc = std::make_unique<mcke::BuddyAllocator>();
  else if (allocator_kind == MCKE_ALLOC_FREELIST)
    e->alloc = std::make_unique<mcke::FreeListAllocator>();
  else if (allocator_kind == MCKE_ALLOC_RAW)
    e->alloc = std::make_unique<mcke::RawDeviceAllocator>();
  else
    return bad("mcke_executor_create: unknown allocator kind");
  e->exec = std::make_unique<mcke::GraphExecutor>(std::move(g->g), *e->alloc, *dev, opts);
  delete g;
  *out = e.release();
  return MCKE_STATUS_OK;
}

void mcke_executor_destroy(mcke_executor* e) {
  if (!e) return;
  e->exec.reset();   // returns the arena before the allocator goes
  e->alloc.reset();
  delete e;
}

int mcke_executor_plan(mcke_executor* e) { return e ? code(e->exec->plan()) : bad("null executor"); }

int mcke_executor_set_input(mcke_executor* e, uint32_t t, const void* host, size_t bytes) {
  if (!e || !host) return bad("null argument");
  return code(e->exec->set_input(t, host, bytes));
}

int mcke_executor_run_async(mcke_executor* e) { return e ? code(e->exec->run_async()) : bad("null executor"); }

int mcke_executor_synchronize(mcke_executor* e) { return e ? code(e->exec->synchronize()) : bad("null executor"); }

int mcke_executor_capture(mcke_executor* e) { return e ? code(e->exec->capture_graph()) : bad("null executor"); }

int mcke_executor_capture_if_faster(mcke_executor* e, int trials, int* captured, double* eager_us,
                                    double* replay_us) {
  if (!e) return bad("null executor");
  auto d = e->exec->capture_if_faster(trials);
  if (!d.ok()) return code(d.status());
  if (captured) *captured = d->captured ? 1 : 0;
  if (eager_us) *eager_us = d->eager_us_per_run;
  if (replay_us) *replay_us = d->replay_us_per_run;
  return MCKE_STATUS_OK;
}

int mcke_executor_is_captured(mcke_executor* e, int* out) {
  if (!e || !out) return bad("mcke_executor_is_captured: null argument");
  *out = e->exec->captured() ? 1 : 0;
  return MCKE_STATUS_OK;
}

int mcke_executor_read_tensor(mcke_executor* e, uint32_t t, void* host, size_t bytes) {
  if (!e || !host) return bad("null argument");
  auto tr = e->exec->any_bound_tensor(t);
  if (!tr.ok()) return code(tr.status());
  const auto& plan = e->exec->plan_ref();
  if (int rc = code(tr->copy_to_host(host, bytes, plan.stream(0)))) return rc;
  return code(e->exec->synchronize());
}

int mcke_executor_plan_info(mcke_executor* e, mcke_plan_info* out) {
  if (!e || !out) return bad("null argument");
  const mcke::ExecutionPlan& p = e->exec->plan_ref();
  const auto& sa = p.stream_plan();
  const auto& mp = p.memory_plan();
  std::memset(out, 0, sizeof(*out));
  out->num_nodes = p.nodes().size();
  out->num_streams_used = sa.num_streams_used;
  out->num_streams_requested = sa.num_streams_requested;
  out->num_events = sa.num_events;
  out->waits_raw = sa.waits_raw;
  out->waits_dedup = sa.waits_dedup;
  out->forkjoin_events = p.forkjoin_events();
  out->arena_bytes = mp.arena_bytes;
  out->naive_bytes = mp.naive_bytes;
  out->buffers_used = mp.buffers_used;
  const mcke::OpCost c = e->exec->graph().total_cost();
  out->total_flops = c.flops;
  out->total_bytes = c.bytes;
  return MCKE_STATUS_OK;
}

int mcke_executor_collect_timings(mcke_executor* e, mcke_node_timing* out, size_t cap, size_t* count) {
  if (!e || !count) return bad("null argument");
  if (int rc = code(e->exec->collect_timings())) return rc;
  const auto& t = e->exec->node_timings();
  *count = t.size();
  for (size_t i = 0; i < t.size() && i < cap && out; ++i) {
    mcke_node_timing& o = out[i];
    std::memset(&o, 0, sizeof(o));
    o.node = t[i].node;
    o.stream_idx = t[i].stream_idx;
    o.median_ms = t[i].median_ms;
    o.min_ms = t[i].min_ms;
    o.flops = t[i].flops;
    o.bytes = t[i].bytes;
    o.samples = t[i].samples;
    std::strncpy(o.name, t[i].name.c_str(), sizeof(o.name) - 1);
  }
  return MCKE_STATUS_OK;
}

int mcke_executor_validate_numerics(mcke_executor* e, int repeats, int* passed, int* configs, char* detail,
                                    size_t cap) {
  if (!e || !passed) return bad("null argument");
  auto r = e->exec->validate_numerics(repeats);
  if (!r.ok()) return code(r.status());
  *passed = r->passed ? 1 : 0;
  if (configs) *configs = r->configs_compared;
  if (detail && cap) {
    std::strncpy(detail, r->detail.c_str(), cap - 1);
    detail[cap - 1] = '\0';
  }
  return MCKE_STATUS_OK;
}

int mcke_executor_allocator_stats(mcke_executor* e, mcke_allocator_stats* out) {
  if (!e || !out) return bad("null argument");
  const mcke::AllocatorStats s = e->alloc->stats();
  out->alloc_calls = s.alloc_calls;
  out->free_calls = s.free_calls;
  out->raw_malloc_calls = s.raw_malloc_calls;
  out->raw_free_calls = s.raw_free_calls;
  out->oom_events = s.oom_events;
  out->deferred_reuses = s.deferred_reuses;
  out->blocking_drains = s.blocking_drains;
  out->reuse_hits = s.reuse_hits;
  out->bytes_reserved = s.bytes_reserved;
  out->bytes_in_use = s.bytes_in_use;
  out->bytes_requested = s.bytes_requested;
  out->peak_bytes_in_use = s.peak_bytes_in_use;
  out->largest_free_block = s.largest_free_block;
  return MCKE_STATUS_OK;
}

int mcke_executor_stream(mcke_executor* e, void** out) {
  if (!e || !out) return bad("null argument");
  if (e->exec->plan_ref().num_streams() == 0) return bad("mcke_executor_stream: not planned");
  *out = e->exec->plan_ref().stream(0);
  return MCKE_STATUS_OK;
}

int mcke_executor_describe(mcke_executor* e, char* buf, size_t cap) {
  if (!e || !buf || !cap) return bad("null argument");
  const std::string s = e->exec->plan_ref().describe();
  std::strncpy(buf, s.c_str(), cap - 1);
  buf[cap - 1] = '\0';
  return MCKE_STATUS_OK;
}

}  // extern "C"
