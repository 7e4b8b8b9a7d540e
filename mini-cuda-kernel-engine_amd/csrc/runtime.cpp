// runtime.cpp -- the mcke_rt_* C-ABI: streams, events, device memory and the
// device query, directly on the HIP runtime.
//
// Replaces the reference's L2 runtime and raw allocation:
//   rt::Stream / rt::Event and the raw-handle probes  stream.hpp:82-306
//   query_device / set_device / raw_device_malloc/free device.cpp:56-130
//   RawDeviceAllocator (one allocation per call)       allocator.cpp:44-73
//   async H2D/D2H copies                               tensor.cpp:108-138
// Streams are non-blocking and at default priority.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "common.hpp"

namespace mcke_amd {

namespace {
thread_local std::string t_last_error;
}

int fail(int code, const std::string& msg) {
  t_last_error = msg;
  return code;
}

int hip_fail(hipError_t e, const char* what, const char* file, int line) {
  std::string m = std::string(hipGetErrorName(e)) + " (" + hipGetErrorString(e) + ") in " +
                  what + " at " + file + ":" + std::to_string(line);
  if (e == hipErrorOutOfMemory) return fail(MCKE_STATUS_OUT_OF_MEMORY, m);
  return fail(MCKE_STATUS_DEVICE_ERROR, m);
}

const char* last_error_cstr() { return t_last_error.c_str(); }

}  // namespace mcke_amd

using namespace mcke_amd;

extern "C" {

const char* mcke_last_error(void) { return last_error_cstr(); }

int mcke_abi_version(void) { return MCKE_ABI_VERSION; }

int mcke_rt_get_device_count(int* count) {
  if (!count) return invalid("mcke_rt_get_device_count: null out");
  int n = 0;
  const hipError_t e = hipGetDeviceCount(&n);
  if (e == hipErrorNoDevice) {
    *count = 0;
    (void)hipGetLastError();
    return ok();
  }
  MCKE_HIP_TRY(e);
  *count = n;
  return ok();
}

int mcke_rt_set_device(int ordinal) {
  MCKE_HIP_TRY(hipSetDevice(ordinal));
  return ok();
}

int mcke_rt_get_device(int* ordinal) {
  if (!ordinal) return invalid("mcke_rt_get_device: null out");
  MCKE_HIP_TRY(hipGetDevice(ordinal));
  return ok();
}

// Spec HBM bandwidth of the part.  HIP reports the memory clock and bus width,
// but HBM3E's transfer rate per clock is not exposed in a form that the
// reference's DDR formula (device.hpp:101-104) gets right, so gfx950 parts use
// AMD's published figure and other parts fall back to 2 * clock * width.
static double peak_dram_gb_s(const hipDeviceProp_t& p) {
  if (std::strncmp(p.gcnArchName, "gfx950", 6) == 0) return 8000.0;
  return 2.0 * static_cast<double>(p.memoryClockRate) * 1e3 *
         (static_cast<double>(p.memoryBusWidth) / 8.0) / 1e9;
}

int mcke_rt_query_device(int ordinal, mcke_device_info* out) {
  if (!out) return invalid("mcke_rt_query_device: null out");
  hipDeviceProp_t p{};
  MCKE_HIP_TRY(hipGetDeviceProperties(&p, ordinal));
  std::memset(out, 0, sizeof(*out));
  out->ordinal = ordinal;
  std::snprintf(out->name, sizeof(out->name), "%s", p.name);
  std::snprintf(out->arch, sizeof(out->arch), "%s", p.gcnArchName);
  out->cc_major = p.major;
  out->cc_minor = p.minor;
  out->total_global_mem = p.totalGlobalMem;
  out->sm_count = p.multiProcessorCount;
  out->warp_size = p.warpSize;
  out->max_threads_per_block = p.maxThreadsPerBlock;
  out->max_threads_per_sm = p.maxThreadsPerMultiProcessor;
  out->max_blocks_per_sm = p.maxBlocksPerMultiProcessor;
  out->regs_per_block = p.regsPerBlock;
  out->regs_per_sm = p.regsPerMultiprocessor;
  out->shared_mem_per_block = p.sharedMemPerBlock;
  out->shared_mem_per_sm = p.maxSharedMemoryPerMultiProcessor;
  out->clock_khz = p.clockRate;
  out->memory_clock_khz = p.memoryClockRate;
  out->memory_bus_width_bits = p.memoryBusWidth;
  out->l2_cache_bytes = static_cast<uint64_t>(p.l2CacheSize);
  out->peak_dram_gb_s = peak_dram_gb_s(p);
  return ok();
}

int mcke_rt_device_synchronize(void) {
  MCKE_HIP_TRY(hipDeviceSynchronize());
  return ok();
}

int mcke_rt_stream_create(void** out_stream) {
  if (!out_stream) return invalid("mcke_rt_stream_create: null out");
  hipStream_t s = nullptr;
  MCKE_HIP_TRY(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *out_stream = s;
  return ok();
}

int mcke_rt_stream_destroy(void* stream) {
  if (!stream) return ok();
  MCKE_HIP_TRY(hipStreamDestroy(static_cast<hipStream_t>(stream)));
  return ok();
}

int mcke_rt_stream_synchronize(void* stream) {
  MCKE_HIP_TRY(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
  return ok();
}

int mcke_rt_stream_query(void* stream, int* done) {
  if (!done) return invalid("mcke_rt_stream_query: null out");
  const hipError_t e = hipStreamQuery(static_cast<hipStream_t>(stream));
  if (e == hipErrorNotReady) {
    *done = 0;
    return ok();
  }
  MCKE_HIP_TRY(e);
  *done = 1;
  return ok();
}

int mcke_rt_stream_wait_event(void* stream, void* event) {
  if (!event) return invalid("mcke_rt_stream_wait_event: null event");
  MCKE_HIP_TRY(hipStreamWaitEvent(static_cast<hipStream_t>(stream),
                                  static_cast<hipEvent_t>(event), 0));
  return ok();
}

// ---- stream capture into a HIP graph ---------------------------------------
int mcke_rt_stream_begin_capture(void* stream) {
  if (!stream) return invalid("mcke_rt_stream_begin_capture: the legacy default stream cannot be captured");
  MCKE_HIP_TRY(hipStreamBeginCapture(static_cast<hipStream_t>(stream), hipStreamCaptureModeThreadLocal));
  return ok();
}

int mcke_rt_stream_end_capture(void* stream, void** out_exec) {
  if (!stream || !out_exec) return invalid("mcke_rt_stream_end_capture: null argument");
  *out_exec = nullptr;
  hipGraph_t graph = nullptr;
  MCKE_HIP_TRY(hipStreamEndCapture(static_cast<hipStream_t>(stream), &graph));
  hipGraphExec_t exec = nullptr;
  const hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);   // the executable graph keeps what it needs
  MCKE_HIP_TRY(e);
  *out_exec = exec;
  return ok();
}

int mcke_rt_graph_launch(void* exec, void* stream) {
  if (!exec) return invalid("mcke_rt_graph_launch: null graph");
  MCKE_HIP_TRY(hipGraphLaunch(static_cast<hipGraphExec_t>(exec), static_cast<hipStream_t>(stream)));
  return ok();
}

int mcke_rt_graph_destroy(void* exec) {
  if (!exec) return ok();
  MCKE_HIP_TRY(hipGraphExecDestroy(static_cast<hipGraphExec_t>(exec)));
  return ok();
}

int mcke_rt_stream_end_capture_graph(void* stream, void** out_graph) {
  if (!stream || !out_graph) return invalid("mcke_rt_stream_end_capture_graph: null argument");
  *out_graph = nullptr;
  hipGraph_t graph = nullptr;
  MCKE_HIP_TRY(hipStreamEndCapture(static_cast<hipStream_t>(stream), &graph));
  *out_graph = graph;
  return ok();
}

int mcke_rt_graph_create(void** out_graph) {
  if (!out_graph) return invalid("mcke_rt_graph_create: null out");
  *out_graph = nullptr;
  hipGraph_t graph = nullptr;
  MCKE_HIP_TRY(hipGraphCreate(&graph, 0));
  *out_graph = graph;
  return ok();
}

int mcke_rt_graph_add_child(void* graph, void* child, void* const* deps, size_t n_deps,
                            void** out_node) {
  if (!graph || !child || !out_node || (n_deps > 0 && !deps))
    return invalid("mcke_rt_graph_add_child: null argument");
  *out_node = nullptr;
  std::vector<hipGraphNode_t> dep(n_deps);
  for (size_t i = 0; i < n_deps; ++i) {
    if (!deps[i]) return invalid("mcke_rt_graph_add_child: null dependency");
    dep[i] = static_cast<hipGraphNode_t>(deps[i]);
  }
  hipGraph_t parent = static_cast<hipGraph_t>(graph);
  hipGraph_t sub = static_cast<hipGraph_t>(child);
  size_t n_nodes = 0;
  MCKE_HIP_TRY(hipGraphGetNodes(sub, nullptr, &n_nodes));
  hipGraphNode_t node = nullptr;
  if (n_nodes == 0) {
    MCKE_HIP_TRY(hipGraphAddEmptyNode(&node, parent, dep.data(), n_deps));
    *out_node = node;
    return ok();
  }
  // A child captured from one stream is a chain of kernel nodes: walk it from its
  // root and add each kernel straight into the parent after the previous one, so
  // the parent holds plain kernel nodes.  Anything else is nested as a child
  // graph node.
  std::vector<hipGraphNode_t> chain;
  size_t n_roots = 0;
  MCKE_HIP_TRY(hipGraphGetRootNodes(sub, nullptr, &n_roots));
  if (n_roots == 1) {
    hipGraphNode_t cur = nullptr;
    MCKE_HIP_TRY(hipGraphGetRootNodes(sub, &cur, &n_roots));
    while (cur && chain.size() < n_nodes) {
      hipGraphNodeType type;
      MCKE_HIP_TRY(hipGraphNodeGetType(cur, &type));
      if (type != hipGraphNodeTypeKernel) break;
      chain.push_back(cur);
      size_t n_next = 0;
      MCKE_HIP_TRY(hipGraphNodeGetDependentNodes(cur, nullptr, &n_next));
      if (n_next > 1) break;
      hipGraphNode_t next = nullptr;
      if (n_next == 1) MCKE_HIP_TRY(hipGraphNodeGetDependentNodes(cur, &next, &n_next));
      cur = next;
    }
  }
  if (chain.size() == n_nodes) {
    const hipGraphNode_t* prev = dep.data();
    size_t n_prev = n_deps;
    for (hipGraphNode_t k : chain) {
      hipKernelNodeParams kp{};
      MCKE_HIP_TRY(hipGraphKernelNodeGetParams(k, &kp));
      MCKE_HIP_TRY(hipGraphAddKernelNode(&node, parent, prev, n_prev, &kp));
      prev = &node;
      n_prev = 1;
    }
  } else {
    MCKE_HIP_TRY(hipGraphAddChildGraphNode(&node, parent, dep.data(), n_deps, sub));
  }
  *out_node = node;
  return ok();
}

int mcke_rt_graph_instantiate(void* graph, void** out_exec) {
  if (!graph || !out_exec) return invalid("mcke_rt_graph_instantiate: null argument");
  *out_exec = nullptr;
  hipGraphExec_t exec = nullptr;
  MCKE_HIP_TRY(hipGraphInstantiate(&exec, static_cast<hipGraph_t>(graph), nullptr, nullptr, 0));
  *out_exec = exec;
  return ok();
}

int mcke_rt_graph_upload(void* exec, void* stream) {
  if (!exec) return invalid("mcke_rt_graph_upload: null graph");
  MCKE_HIP_TRY(hipGraphUpload(static_cast<hipGraphExec_t>(exec), static_cast<hipStream_t>(stream)));
  return ok();
}

int mcke_rt_graph_release(void* graph) {
  if (!graph) return ok();
  MCKE_HIP_TRY(hipGraphDestroy(static_cast<hipGraph_t>(graph)));
  return ok();
}

int mcke_rt_event_create(void** out_event, int timing) {
  if (!out_event) return invalid("mcke_rt_event_create: null out");
  hipEvent_t e = nullptr;
  MCKE_HIP_TRY(hipEventCreateWithFlags(&e, timing ? hipEventDefault : hipEventDisableTiming));
  *out_event = e;
  return ok();
}

int mcke_rt_event_destroy(void* event) {
  if (!event) return ok();
  MCKE_HIP_TRY(hipEventDestroy(static_cast<hipEvent_t>(event)));
  return ok();
}

int mcke_rt_event_record(void* event, void* stream) {
  if (!event) return invalid("mcke_rt_event_record: null event");
  MCKE_HIP_TRY(hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream)));
  return ok();
}

int mcke_rt_event_query(void* event, int* done) {
  if (!event || !done) return invalid("mcke_rt_event_query: null argument");
  const hipError_t e = hipEventQuery(static_cast<hipEvent_t>(event));
  if (e == hipErrorNotReady) {
    *done = 0;
    return ok();
  }
  MCKE_HIP_TRY(e);
  *done = 1;
  return ok();
}

int mcke_rt_event_synchronize(void* event) {
  if (!event) return invalid("mcke_rt_event_synchronize: null event");
  MCKE_HIP_TRY(hipEventSynchronize(static_cast<hipEvent_t>(event)));
  return ok();
}

int mcke_rt_event_elapsed_ms(void* start, void* stop, float* ms) {
  if (!start || !stop || !ms) return invalid("mcke_rt_event_elapsed_ms: null argument");
  MCKE_HIP_TRY(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start),
                                   static_cast<hipEvent_t>(stop)));
  return ok();
}

int mcke_rt_malloc(void** out_ptr, size_t bytes) {
  if (!out_ptr) return invalid("mcke_rt_malloc: null out");
  *out_ptr = nullptr;
  if (bytes == 0) return ok();
  void* p = nullptr;
  const hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess) {
    (void)hipGetLastError();  // an OOM is recoverable: do not leave it sticky
    return hip_fail(e, "hipMalloc", __FILE__, __LINE__);
  }
  *out_ptr = p;
  return ok();
}

int mcke_rt_free(void* ptr) {
  if (!ptr) return ok();
  MCKE_HIP_TRY(hipFree(ptr));
  return ok();
}

int mcke_rt_host_alloc(void** out_ptr, size_t bytes) {
  if (!out_ptr) return invalid("mcke_rt_host_alloc: null out");
  *out_ptr = nullptr;
  if (bytes == 0) return ok();
  void* p = nullptr;
  MCKE_HIP_TRY(hipHostMalloc(&p, bytes, hipHostMallocDefault));
  *out_ptr = p;
  return ok();
}

int mcke_rt_host_free(void* ptr) {
  if (!ptr) return ok();
  MCKE_HIP_TRY(hipHostFree(ptr));
  return ok();
}

int mcke_rt_memcpy_async(void* dst, const void* src, size_t bytes, int kind, void* stream) {
  if (bytes == 0) return ok();
  if (!dst || !src) return invalid("mcke_rt_memcpy_async: null pointer");
  hipMemcpyKind k;
  switch (kind) {
    case 0: k = hipMemcpyHostToDevice; break;
    case 1: k = hipMemcpyDeviceToHost; break;
    case 2: k = hipMemcpyDeviceToDevice; break;
    case 3: k = hipMemcpyDefault; break;
    default: return invalid("mcke_rt_memcpy_async: kind must be 0..3");
  }
  MCKE_HIP_TRY(hipMemcpyAsync(dst, src, bytes, k, static_cast<hipStream_t>(stream)));
  return ok();
}

int mcke_rt_memset_async(void* dst, int value, size_t bytes, void* stream) {
  if (bytes == 0) return ok();
  if (!dst) return invalid("mcke_rt_memset_async: null pointer");
  const hipStream_t st = static_cast<hipStream_t>(stream);
  // A memset recorded into a graph has given wrong results on replays after the
  // first on this stack; a fill kernel is the capturable way to clear memory.
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  MCKE_HIP_TRY(hipStreamIsCapturing(st, &cs));
  if (cs != hipStreamCaptureStatusNone)
    return invalid("mcke_rt_memset_async: the stream is being captured into a graph; "
                   "use mcke_fill_u32_async, which records a kernel node");
  MCKE_HIP_TRY(hipMemsetAsync(dst, value, bytes, st));
  return ok();
}

// ---- host data generators --------------------------------------------------
void mcke_fill_random_f32(float* host, size_t n, uint64_t seed, float lo, float hi) {
  if (!host) return;
  std::mt19937_64 eng(seed);
  const float span = hi - lo;
  for (size_t i = 0; i < n; ++i) {
    const double u = static_cast<double>(eng() >> 40) / static_cast<double>(1u << 24);
    host[i] = static_cast<float>(static_cast<double>(lo) + u * static_cast<double>(span));
  }
}

void mcke_fill_normal_f32(float* host, size_t n, uint64_t seed, float mu, float sigma) {
  if (!host) return;
  std::mt19937_64 eng(seed);
  const double two_pi = 6.283185307179586476925286766559;
  const double inv53 = 1.0 / 9007199254740992.0;
  for (size_t i = 0; i < n; i += 2) {
    const double u1 = (static_cast<double>(eng() >> 11) + 0.5) * inv53;
    const double u2 = static_cast<double>(eng() >> 11) * inv53;
    const double r = std::sqrt(-2.0 * std::log(u1));
    host[i] = static_cast<float>(static_cast<double>(mu) +
                                 static_cast<double>(sigma) * (r * std::cos(two_pi * u2)));
    if (i + 1 < n)
      host[i + 1] = static_cast<float>(static_cast<double>(mu) +
                                       static_cast<double>(sigma) * (r * std::sin(two_pi * u2)));
  }
}

}  // extern "C"
