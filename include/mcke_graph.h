/*
 * mcke_graph.h -- C-ABI of the graph layer (libmcke_host.so).
 *
 * Opaque handles over the C++ Graph / GraphExecutor / allocators of
 * include/mcke/graph/ (reference include/mcke/graph/graph.hpp, executor.hpp,
 * schedule.hpp, memory_plan.hpp and the src/graph sources), so that a non-C++ host
 * (Python/ctypes here) can build the reference's graphs, plan them onto streams
 * and an arena, replay them and read the plan statistics.  Return codes are the
 * mcke_status values of mcke_amd.h; messages via mcke_last_error() for kernel and
 * runtime failures, or mcke_graph_last_error() for failures of this layer.
 */
#ifndef MCKE_GRAPH_H_
#define MCKE_GRAPH_H_

#include <stddef.h>
#include <stdint.h>

#include "mcke_amd.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mcke_graph mcke_graph;
typedef struct mcke_executor mcke_executor;

/* SchedulePolicy (schedule.hpp:49) and MemoryPolicy (memory_plan.hpp) values. */
enum mcke_schedule_policy { MCKE_SCHED_SEQUENTIAL = 0, MCKE_SCHED_LEVEL_PARALLEL = 1, MCKE_SCHED_CHAIN_GREEDY = 2 };
enum mcke_memory_policy {
  MCKE_MEM_ALLOC_PER_TENSOR = 0,
  MCKE_MEM_REUSE_TOPO_NAIVE = 1,
  MCKE_MEM_REUSE_SAME_STREAM = 2,
  MCKE_MEM_REUSE_HAPPENS_BEFORE = 3
};
/* Allocator behind the executor's arena and workspaces: RawDeviceAllocator,
 * BuddyAllocator (buddy_allocator.hpp) or FreeListAllocator (freelist_allocator.hpp),
 * each with its default configuration. */
enum mcke_allocator_kind { MCKE_ALLOC_RAW = 0, MCKE_ALLOC_BUDDY = 1, MCKE_ALLOC_FREELIST = 2 };

/* ExecutorOptions (executor.hpp:115-134). */
typedef struct mcke_executor_options {
  int32_t schedule;
  int32_t memory;
  int32_t num_streams;
  int32_t profile;           /* per-node timing probes */
  int32_t profile_slots;
  int32_t validate_numerics; /* keep a host copy of inputs for validate_numerics */
  int32_t poison_buffers;
  uint32_t poison_pattern;
} mcke_executor_options;

typedef struct mcke_plan_info {
  uint64_t num_nodes;
  uint64_t num_streams_used;
  uint64_t num_streams_requested;
  uint64_t num_events;
  uint64_t waits_raw;
  uint64_t waits_dedup;
  uint64_t forkjoin_events;
  uint64_t arena_bytes;
  uint64_t naive_bytes;
  uint64_t buffers_used;
  uint64_t total_flops;      /* sum of live nodes' ideal flops */
  uint64_t total_bytes;      /* sum of live nodes' ideal bytes */
} mcke_plan_info;

typedef struct mcke_node_timing {
  uint32_t node;
  int32_t stream_idx;
  double median_ms;
  double min_ms;
  uint64_t flops;
  uint64_t bytes;
  int32_t samples;
  char name[64];
} mcke_node_timing;

/* AllocatorStats (allocator.hpp:128-158). */
typedef struct mcke_allocator_stats {
  uint64_t alloc_calls, free_calls, raw_malloc_calls, raw_free_calls, oom_events;
  uint64_t deferred_reuses, blocking_drains, reuse_hits;
  uint64_t bytes_reserved, bytes_in_use, bytes_requested, peak_bytes_in_use, largest_free_block;
} mcke_allocator_stats;

const char* mcke_graph_last_error(void);

/* ---- Graph (graph.hpp) ---------------------------------------------------- */
mcke_graph* mcke_graph_create(void);
void mcke_graph_destroy(mcke_graph* g);
int mcke_graph_add_input(mcke_graph* g, const int64_t* dims, int rank, const char* name, uint32_t* out_tensor);
/* GemmOp with beta = 0; tile == NULL means "pick per shape" (kMfmaF32 only). */
/* An input tensor of element type `dtype` (MCKE_DTYPE_F32, _F16 or _BF16; the
 * reference's graph is fp32 only, and mcke_graph_add_input makes fp32 inputs). */
int mcke_graph_add_input_typed(mcke_graph* g, const int64_t* dims, int rank, int dtype,
                               const char* name, uint32_t* out_tensor);

/* A GEMM node on 16-bit inputs (a and b bf16, or both f16): C = alpha * A B in
 * out_dtype (MCKE_DTYPE_F32 or the input type), through mcke_launch_gemm_lp.
 * NULL tile = the per-shape default.  The other operators take f32 tensors only;
 * a node given 16-bit inputs fails at build time. */
int mcke_graph_add_gemm_lp(mcke_graph* g, uint32_t a, uint32_t b, float alpha, int out_dtype,
                           const mcke_gemm_tile* tile, const char* name, uint32_t* out_tensor);

int mcke_graph_add_gemm(mcke_graph* g, uint32_t a, uint32_t b, float alpha, int variant,
                        const mcke_gemm_tile* tile, const char* name, uint32_t* out_tensor);
int mcke_graph_add_bias_act(mcke_graph* g, uint32_t x, uint32_t bias, int act, int vector_width,
                            const char* name, uint32_t* out_tensor);
/* The same node with BiasActParams::max_row_blocks (reference op.hpp BiasActParams,
 * ops_bias_act.cpp:102-130): caps the row dimension of the launch grid (0 =
 * automatic), as the reference graph bench's starved diamond uses. */
int mcke_graph_add_bias_act_rows(mcke_graph* g, uint32_t x, uint32_t bias, int act,
                                 int vector_width, int max_row_blocks, const char* name,
                                 uint32_t* out_tensor);
/* No reference counterpart: GemmOp (kMfmaF32, beta = 0) and BiasActOp fused into one
 * node, y = act(alpha * A B + bias[col]) through mcke_launch_gemm_bias_act_f32 --
 * the bits of the GemmOp -> BiasActOp pair, without C.  NULL tile = per-shape
 * choice. */
int mcke_graph_add_gemm_bias_act(mcke_graph* g, uint32_t a, uint32_t b, uint32_t bias, float alpha,
                                 int act, const mcke_gemm_tile* tile, const char* name,
                                 uint32_t* out_tensor);
int mcke_graph_add_reduce(mcke_graph* g, uint32_t x, int kind, int variant, const char* name,
                          uint32_t* out_tensor);
int mcke_graph_add_softmax(mcke_graph* g, uint32_t x, int variant, const char* name, uint32_t* out_tensor);
int mcke_graph_mark_output(mcke_graph* g, uint32_t t);
int mcke_graph_num_nodes(const mcke_graph* g, uint64_t* out);
/* Shape of tensor t: writes rank and up to 5 dims. */
int mcke_graph_tensor_shape(const mcke_graph* g, uint32_t t, int64_t* dims5, int* rank);

/* ---- GraphExecutor (executor.hpp) ------------------------------------------ */
/* On success takes ownership of the graph (the handle is consumed and must not be
 * reused); on failure the caller still owns it. */
int mcke_executor_create(mcke_graph* g, int allocator_kind, const mcke_executor_options* opts,
                         mcke_executor** out);
void mcke_executor_destroy(mcke_executor* e);
int mcke_executor_plan(mcke_executor* e);
int mcke_executor_set_input(mcke_executor* e, uint32_t t, const void* host, size_t bytes);
int mcke_executor_run_async(mcke_executor* e);
int mcke_executor_synchronize(mcke_executor* e);
/* Captures one iteration of the plan into a HIP graph; later run_async calls replay
 * it with one launch (GraphExecutor::capture_graph; the reference plans this as
 * capture_cuda_graph, executor.hpp:23-27).  A plan on several streams is
 * assembled from one single-stream capture per node, with the plan's stream order
 * and cross-stream events as the graph's edges.  FAILED_PRECONDITION with
 * per-node timing probes or a vendor-library GEMM node.  A new plan() drops the
 * capture. */
int mcke_executor_capture(mcke_executor* e);
/* No reference counterpart (the reference plans capture to cut per-launch host
 * cost, executor.hpp:23-27): captures as mcke_executor_capture, then keeps the
 * graph only if replay measures faster than eager issue on this plan -- `trials`
 * runs each way, twice in alternation, host wall time per run of the best block
 * (GraphExecutor::capture_if_faster).  *captured (may be NULL) is 1 when the graph
 * was kept; *eager_us and *replay_us (may be NULL) receive the two times. */
int mcke_executor_capture_if_faster(mcke_executor* e, int trials, int* captured, double* eager_us,
                                    double* replay_us);
int mcke_executor_is_captured(mcke_executor* e, int* out);
/* Copies tensor t (an output, or any tensor with a buffer) to host memory and waits. */
int mcke_executor_read_tensor(mcke_executor* e, uint32_t t, void* host, size_t bytes);
int mcke_executor_plan_info(mcke_executor* e, mcke_plan_info* out);
int mcke_executor_collect_timings(mcke_executor* e, mcke_node_timing* out, size_t cap, size_t* count);
int mcke_executor_validate_numerics(mcke_executor* e, int repeats, int* passed, int* configs_compared,
                                    char* detail, size_t detail_cap);
int mcke_executor_allocator_stats(mcke_executor* e, mcke_allocator_stats* out);
/* Stream 0 of the current plan (hipStream_t), for timing events around run_async. */
int mcke_executor_stream(mcke_executor* e, void** out_stream);
int mcke_executor_describe(mcke_executor* e, char* buf, size_t cap);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* MCKE_GRAPH_H_ */
