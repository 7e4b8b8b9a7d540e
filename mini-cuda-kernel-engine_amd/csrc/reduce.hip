// reduce.hip -- per-row sum / max / mean, and the full-tensor reduction.
//
// Replaces kernels/reduce.cu (launchers reduce.cu:224-295, workspace query
// :213-218) and the combine operators of kernels/reduce_ops.cuh:38-119.
// HBM-bound: (rows*cols + rows) * 4 bytes per call.
//
// Variants keep the reference's meaning (kernels.hpp:162-180):
//   kSmemTree    one workgroup per row; per-thread partials combined by a
//                classic LDS tree (1 + log2(256) = 9 barriers);
//   kWarpShuffle one workgroup per row; wave64 butterfly, then one LDS stage
//                across the 4 waves (1 barrier);
//   kTwoPass     (rows x split) workgroups reduce column chunks of a row to
//                partials in the caller's workspace, then one workgroup per
//                row folds that row's partials in a fixed order (a second
//                launch, as reduce.cu:180-206).  Rows that need no split are
//                written out by the first launch, which is then the only one.
//                With rows == 1 this is the full-tensor reduction.
// Every variant is deterministic (nothing is combined atomically) and keeps no
// state between launches: the same input gives the same bits on every run, on
// any stream.
//
// The row sweep: 256 lanes walk the row in 16-byte (float4) steps when the row
// starts are 16-byte aligned, four loads in flight per lane before any add.
// Max uses -inf as its identity, so an all-(-inf) row reduces to -inf and NaN
// elements are ignored, as `std::max(m, v)` starting from -inf does.
#include <hip/hip_runtime.h>

#include <cmath>
#include <mutex>
#include <string>
#include <type_traits>

#include "common.hpp"
#include "device_math.hpp"

namespace mcke_amd {
namespace {

constexpr int kThreads = 256;
constexpr int kLoadUnroll = 4;      // loads in flight per lane, one-pass kernels
// kTwoPass sizing: one 512-lane workgroup per CU on a 256-CU part, each lane
// keeping 4 float4 loads in flight.  Measured on the full-tensor sum of 2^26
// floats, workgroups x lanes x loads: 256 x 512 x 4 40.6 us, 256 x 256 x 8
// 40.9 us, 256 x 1024 x 2 40.9 us, 256 x 1024 x 4 42.9 us, 512 x 256 x 8
// 42.5 us, 1024 x 256 x 8 44.9 us, 2048 x 256 x 8 50.3 us -- each workgroup
// ends with its partial's store, during which its slot issues no loads, so few,
// wide workgroups win.
constexpr int kSplitThreads = 512;
constexpr int kPass1Unroll = 4;
constexpr int64_t kTargetBlocks = 256;
constexpr int64_t kMinColsPerBlock = 4096;
constexpr int64_t kMaxSplit = 65535;

struct SumOp {
  static __device__ __forceinline__ float identity() { return 0.0f; }
  static __device__ __forceinline__ float apply(float a, float b) { return a + b; }
  static __device__ __forceinline__ float wave(float v) { return wave_sum(v); }
};

struct MaxOp {
  static __device__ __forceinline__ float identity() { return -INFINITY; }
  static __device__ __forceinline__ float apply(float a, float b) { return fmaxf(a, b); }
  static __device__ __forceinline__ float wave(float v) { return wave_max(v); }
};

template <class Op> __device__ __forceinline__ float fold4(f32x4 v) {
  return Op::apply(Op::apply(v[0], v[1]), Op::apply(v[2], v[3]));
}

// Partial of x[begin, end) for this thread, NT lanes striding through it.
// VEC: begin and end are multiples of 4 and x is 16-byte aligned.
template <class Op, bool VEC, int U = kLoadUnroll, int NT = kThreads>
__device__ __forceinline__ float thread_partial(const float* __restrict__ x, int64_t begin,
                                                int64_t end) {
  float acc = Op::identity();
  if constexpr (VEC) {
    const f32x4* __restrict__ xv = reinterpret_cast<const f32x4*>(x);
    const int64_t b4 = begin >> 2, e4 = end >> 2;
    for (int64_t i = b4 + threadIdx.x; i < e4; i += U * NT) {
      f32x4 a[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t j = i + u * NT;
        if (j < e4) a[u] = ld_stream(xv + j);
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (i + u * NT < e4) acc = Op::apply(acc, fold4<Op>(a[u]));
    }
  } else {
    for (int64_t i = begin + threadIdx.x; i < end; i += U * NT) {
      float a[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t j = i + u * NT;
        if (j < end) a[u] = ld_stream(x + j);
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (i + u * NT < end) acc = Op::apply(acc, a[u]);
    }
  }
  return acc;
}

// Workgroup combine (NT lanes), wave64 butterfly + one LDS stage.  Valid in every lane.
template <class Op, int NT = kThreads> __device__ __forceinline__ float block_combine_shfl(float v) {
  __shared__ float part[NT / kWave];
  v = Op::wave(v);
  const int w = threadIdx.x / kWave;
  if ((threadIdx.x % kWave) == 0) part[w] = v;
  __syncthreads();
  float r = part[0];
#pragma unroll
  for (int i = 1; i < NT / kWave; ++i) r = Op::apply(r, part[i]);
  return r;
}

// Workgroup combine through an LDS tree (sequential addressing).  Thread 0 only.
template <class Op> __device__ __forceinline__ float block_combine_tree(float v) {
  __shared__ float buf[kThreads];
  buf[threadIdx.x] = v;
  __syncthreads();
#pragma unroll
  for (int s = kThreads / 2; s > 0; s >>= 1) {
    if (static_cast<int>(threadIdx.x) < s)
      buf[threadIdx.x] = Op::apply(buf[threadIdx.x], buf[threadIdx.x + s]);
    __syncthreads();
  }
  return buf[0];
}

template <class Op, bool VEC, bool TREE, bool MEAN>
__global__ __launch_bounds__(kThreads) void row_reduce_kernel(const float* __restrict__ x,
                                                              float* __restrict__ out,
                                                              int64_t cols) {
  const int64_t r = blockIdx.x;
  const float* row = x + r * cols;
  float v = TREE ? thread_partial<Op, false>(row, 0, cols)
                 : thread_partial<Op, VEC>(row, 0, cols);
  v = TREE ? block_combine_tree<Op>(v) : block_combine_shfl<Op>(v);
  if (threadIdx.x == 0) out[r] = MEAN ? v / static_cast<float>(cols) : v;
}

// Folds the `split` partials p[0, split) of one row in a fixed order (lane-
// strided, then a wave64 butterfly, then the waves in order); the result is
// valid in thread 0.  Sums are carried in double: the partials are few and this
// stage should not add error on top of the first.
template <class Op, bool MEAN, int NT>
__device__ __forceinline__ float fold_partials(const float* __restrict__ p, int64_t split,
                                               int64_t cols) {
  const int w = threadIdx.x / kWave;
  if constexpr (std::is_same_v<Op, SumOp>) {
    __shared__ double part[NT / kWave];
    double acc = 0.0;
    for (int64_t i = threadIdx.x; i < split; i += NT) acc += static_cast<double>(p[i]);
#pragma unroll
    for (int m = kWave / 2; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
    if ((threadIdx.x % kWave) == 0) part[w] = acc;
    __syncthreads();
    double t = part[0];
#pragma unroll
    for (int i = 1; i < NT / kWave; ++i) t += part[i];
    return static_cast<float>(MEAN ? t / static_cast<double>(cols) : t);
  } else {
    float acc = Op::identity();
    for (int64_t i = threadIdx.x; i < split; i += NT) acc = Op::apply(acc, p[i]);
    return block_combine_shfl<Op, NT>(acc);
  }
}

// kTwoPass, first launch, workgroup (s, r): reduces columns
// [s*chunk, min(cols, (s+1)*chunk)) of row r.  With split == 1 the workgroup owns
// the row and writes out[r]; otherwise it stores its partial to
// part[r*split + s] for row_reduce_fold_kernel.
template <class Op, bool VEC, bool MEAN>
__global__ __launch_bounds__(kSplitThreads) void row_reduce_split_kernel(
    const float* __restrict__ x, float* __restrict__ part, float* __restrict__ out, int64_t cols,
    int64_t chunk, int64_t split) {
  const int64_t s = blockIdx.x;
  const int64_t r = blockIdx.y;
  const int64_t begin = s * chunk;
  int64_t end = begin + chunk;
  if (end > cols) end = cols;
  float v = Op::identity();
  if (begin < end) v = thread_partial<Op, VEC, kPass1Unroll, kSplitThreads>(x + r * cols, begin, end);
  v = block_combine_shfl<Op, kSplitThreads>(v);
  if (threadIdx.x != 0) return;
  if (split == 1)
    out[r] = MEAN ? v / static_cast<float>(cols) : v;
  else
    part[r * split + s] = v;
}

// kTwoPass, second launch: one workgroup per row folds that row's partials.
template <class Op, bool MEAN>
__global__ __launch_bounds__(kSplitThreads) void row_reduce_fold_kernel(
    const float* __restrict__ part, float* __restrict__ out, int64_t split, int64_t cols) {
  const int64_t r = blockIdx.x;
  const float t = fold_partials<Op, MEAN, kSplitThreads>(part + r * split, split, cols);
  if (threadIdx.x == 0) out[r] = t;
}

int64_t two_pass_split(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 1;
  int64_t s = (kTargetBlocks + rows - 1) / rows;
  int64_t cap = cols / kMinColsPerBlock;
  if (cap < 1) cap = 1;
  if (s > cap) s = cap;
  if (s > kMaxSplit) s = kMaxSplit;
  if (s < 1) s = 1;
  return s;
}

template <class Op, bool MEAN>
int launch_one_pass(const float* x, float* out, int64_t rows, int64_t cols, bool tree,
                    hipStream_t st) {
  const bool vec = (cols % 4 == 0) && aligned(x, 16);
  const unsigned g = static_cast<unsigned>(rows);
  if (tree)
    row_reduce_kernel<Op, false, true, MEAN><<<g, kThreads, 0, st>>>(x, out, cols);
  else if (vec)
    row_reduce_kernel<Op, true, false, MEAN><<<g, kThreads, 0, st>>>(x, out, cols);
  else
    row_reduce_kernel<Op, false, false, MEAN><<<g, kThreads, 0, st>>>(x, out, cols);
  MCKE_LAUNCH_CHECK("row_reduce_kernel");
  return ok();
}

// `part` holds at least rows * two_pass_split(rows, cols) floats; it is written
// before it is read, so its contents on entry do not matter.
template <class Op, bool MEAN>
int launch_two_pass(const float* x, float* out, int64_t rows, int64_t cols, float* part,
                    hipStream_t st) {
  const int64_t split = two_pass_split(rows, cols);
  // chunk is a multiple of 4 so each chunk keeps the row's 16-byte alignment.
  int64_t chunk = (cols + split - 1) / split;
  chunk = (chunk + 3) & ~static_cast<int64_t>(3);
  const bool vec = (cols % 4 == 0) && aligned(x, 16);
  const dim3 g1(static_cast<unsigned>(split), static_cast<unsigned>(rows), 1u);
  if (vec)
    row_reduce_split_kernel<Op, true, MEAN><<<g1, kSplitThreads, 0, st>>>(x, part, out, cols,
                                                                          chunk, split);
  else
    row_reduce_split_kernel<Op, false, MEAN><<<g1, kSplitThreads, 0, st>>>(x, part, out, cols,
                                                                           chunk, split);
  MCKE_LAUNCH_CHECK("row_reduce_split_kernel");
  if (split > 1) {
    row_reduce_fold_kernel<Op, MEAN><<<static_cast<unsigned>(rows), kSplitThreads, 0, st>>>(
        part, out, split, cols);
    MCKE_LAUNCH_CHECK("row_reduce_fold_kernel");
  }
  return ok();
}

int dispatch_two_pass(const float* x, float* out, int64_t rows, int64_t cols, int kind,
                      float* part, hipStream_t st) {
  switch (kind) {
    case MCKE_REDUCE_SUM: return launch_two_pass<SumOp, false>(x, out, rows, cols, part, st);
    case MCKE_REDUCE_MEAN: return launch_two_pass<SumOp, true>(x, out, rows, cols, part, st);
    default: return launch_two_pass<MaxOp, false>(x, out, rows, cols, part, st);
  }
}

// The partials of mcke_launch_row_reduce_noalloc_f32, for callers that cannot
// allocate: one array per GPU the library runs on, held until the process ends.
// 1024 floats (4 KiB); under two_pass_split a call needs at most
// rows * split <= 511 of them (rows <= 256 split into ceil(256 / rows) chunks,
// more rows are not split).  Every call on a GPU shares its array; the
// partials are written before they are read, so nothing in it has to start at
// zero, but calls that overlap on one GPU race.
constexpr int64_t kScratchFloats = 1024;
static __device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// This device's copy of `scratch`, as a device address.  Looked up once per
// device, with that device current: in host code the array's name is a host
// stand-in, not a device address.
int scratch_of_current_device(float** out) {
  int dev = -1;
  MCKE_HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices)
    return invalid("launch_row_reduce_noalloc_f32: device ordinal out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    MCKE_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return ok();
}

}  // namespace
}  // namespace mcke_amd

using namespace mcke_amd;

extern "C" {

size_t mcke_row_reduce_workspace_bytes(int64_t rows, int64_t cols, int variant) {
  if (variant != MCKE_REDUCE_TWO_PASS || rows <= 0) return 0;
  return static_cast<size_t>(rows * two_pass_split(rows, cols)) * sizeof(float);
}

int mcke_launch_row_reduce_ws_f32(const float* x, float* out, int64_t rows, int64_t cols,
                                  int kind, int variant, float* workspace,
                                  size_t workspace_bytes, void* stream) {
  if (rows == 0 || cols == 0) return ok();   // an empty grid is a launch error
  if (rows < 0 || cols < 0) return invalid("launch_row_reduce_f32: negative extent");
  if (!x || !out) return invalid("launch_row_reduce_f32: null pointer");
  if (kind < 0 || kind > 2) return invalid("launch_row_reduce_f32: unknown ReduceKind");
  if (variant < 0 || variant > 2) return invalid("launch_row_reduce_f32: unknown ReduceVariant");
  hipStream_t st = static_cast<hipStream_t>(stream);

  if (variant == MCKE_REDUCE_TWO_PASS) {
    if (rows > 65535)
      return invalid("launch_row_reduce_f32: kTwoPass rows exceed the grid's y limit (65535)");
    const size_t need = mcke_row_reduce_workspace_bytes(rows, cols, variant);
    if (workspace == nullptr || workspace_bytes < need)
      return invalid("launch_row_reduce_f32: kTwoPass needs " + std::to_string(need) +
                     " bytes of workspace (got " + std::to_string(workspace_bytes) +
                     "); query row_reduce_workspace_bytes() first");
    if (!aligned(workspace, 4)) return invalid("launch_row_reduce_f32: workspace not aligned");
    return dispatch_two_pass(x, out, rows, cols, kind, workspace, st);
  }

  if (rows > 2147483647LL)
    return invalid("launch_row_reduce_f32: rows exceeds the grid's x limit");
  const bool tree = (variant == MCKE_REDUCE_SMEM_TREE);
  switch (kind) {
    case MCKE_REDUCE_SUM: return launch_one_pass<SumOp, false>(x, out, rows, cols, tree, st);
    case MCKE_REDUCE_MEAN: return launch_one_pass<SumOp, true>(x, out, rows, cols, tree, st);
    default: return launch_one_pass<MaxOp, false>(x, out, rows, cols, tree, st);
  }
}

int mcke_launch_row_reduce_noalloc_f32(const float* x, float* out, int64_t rows, int64_t cols,
                                       int kind, void* stream) {
  if (rows == 0 || cols == 0) return ok();
  if (rows < 0 || cols < 0) return invalid("launch_row_reduce_noalloc_f32: negative extent");
  if (!x || !out) return invalid("launch_row_reduce_noalloc_f32: null pointer");
  if (kind < 0 || kind > 2) return invalid("launch_row_reduce_noalloc_f32: unknown ReduceKind");
  if (rows > 65535)
    return invalid("launch_row_reduce_noalloc_f32: rows exceed the grid's y limit (65535)");
  const int64_t split = two_pass_split(rows, cols);
  const int64_t partials = split > 1 ? rows * split : 0;
  if (partials > kScratchFloats)
    return invalid("launch_row_reduce_noalloc_f32: needs " + std::to_string(partials) +
                   " partials, more than the " + std::to_string(kScratchFloats) +
                   " its scratch holds; use launch_row_reduce_f32 with a workspace");
  float* part = nullptr;
  if (const int rc = scratch_of_current_device(&part)) return rc;
  return dispatch_two_pass(x, out, rows, cols, kind, part, static_cast<hipStream_t>(stream));
}

int mcke_launch_row_reduce_f32(const float* x, float* out, int64_t rows, int64_t cols, int kind,
                               int variant, void* stream) {
  if (variant == MCKE_REDUCE_TWO_PASS)
    return fail(MCKE_STATUS_UNIMPLEMENTED,
                "launch_row_reduce_f32: kTwoPass requires a workspace; call "
                "row_reduce_workspace_bytes() and use the 9-argument overload");
  return mcke_launch_row_reduce_ws_f32(x, out, rows, cols, kind, variant, nullptr, 0, stream);
}

}  // extern "C"
