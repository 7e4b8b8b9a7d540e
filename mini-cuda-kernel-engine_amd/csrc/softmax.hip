// softmax.hip -- numerically stable row softmax.
//
// Replaces kernels/softmax.cu (launcher softmax.cu:177-199, kernels :112-173,
// online combine :77-107) on top of the (m, d) algebra of
// include/mcke/kernels/softmax_online.hpp:73-112.
//
// kOnlineOnePass is the fast path and is HBM-bound at the compulsory traffic of
// one read and one write per element (2 * rows * cols * 4 bytes):
//   * rows whose float4 vectors fit in registers (cols <= 8192, cols % 4 == 0,
//     16-byte aligned) are held in VGPRs: a group of TPR lanes owns a row, each
//     lane loads VPT float4s, the group reduces the max and then sum(exp(x-m))
//     by wave64 butterflies (plus one LDS stage when a row spans several waves),
//     and the row is written from the same registers -- 1R + 1W;
//   * other rows fall back to the reference's online form: one traversal
//     carrying (m, d) per lane, a workgroup combine, and a write pass -- 2R + 1W.
// kThreePass is the baseline: max pass, sum pass, write pass (3R + 1W).
//
// exp(t) for t = x - m <= 0 is evaluated as 2^(t * log2 e) with the hardware
// exponential; the product's rounding perturbs the result by at most |t| * 2^-24
// relative, which is below 1e-9 in absolute terms wherever exp(t) is not already
// negligible.  The row's 1/d is one correctly rounded division per row.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <string>

#include "common.hpp"
#include "device_math.hpp"

namespace mcke_amd {
namespace {

constexpr int kThreads = 256;
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float exp_le0(float t) {
  return __builtin_amdgcn_exp2f(t * kLog2e);
}

// ---------------------------------------------------------------------------
// Register-resident rows.  NT-lane workgroups, TPR lanes per row (8 .. 1024), VPT
// float4 per lane.  A row wider than a wave spans TPR / 64 consecutive waves,
// combined through one LDS stage over that row's own waves.
// ---------------------------------------------------------------------------
template <int TPR> __device__ __forceinline__ float group_max(float v, float* lds) {
  if constexpr (TPR <= kWave) {
    return wave_max<TPR>(v);
  } else {
    v = wave_max<kWave>(v);
    const int w = threadIdx.x / kWave;
    const int first = (threadIdx.x / TPR) * (TPR / kWave);   // the row's first wave
    if ((threadIdx.x % kWave) == 0) lds[w] = v;
    __syncthreads();
    float r = lds[first];
#pragma unroll
    for (int i = 1; i < TPR / kWave; ++i) r = fmaxf(r, lds[first + i]);
    __syncthreads();   // lds is reused by group_sum
    return r;
  }
}

template <int TPR> __device__ __forceinline__ float group_sum(float v, float* lds) {
  if constexpr (TPR <= kWave) {
    return wave_sum<TPR>(v);
  } else {
    v = wave_sum<kWave>(v);
    const int w = threadIdx.x / kWave;
    const int first = (threadIdx.x / TPR) * (TPR / kWave);
    if ((threadIdx.x % kWave) == 0) lds[w] = v;
    __syncthreads();
    float r = lds[first];
#pragma unroll
    for (int i = 1; i < TPR / kWave; ++i) r += lds[first + i];
    return r;
  }
}

template <int TPR, int VPT, int NT = kThreads>
__global__ __launch_bounds__(NT) void softmax_regs_kernel(const float* __restrict__ x,
                                                          float* __restrict__ y, int64_t rows,
                                                          int64_t cols) {
  static_assert(NT % TPR == 0, "TPR must divide the workgroup");
  constexpr int kRowsPerBlock = NT / TPR;
  __shared__ float lds[NT / kWave];
  const int t = threadIdx.x % TPR;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / TPR;
  // Rows past the end still take part in the barriers of a multi-wave group,
  // so they only skip their loads and stores.  (With TPR <= 64 a whole group is
  // one wave and there are no barriers.)
  const bool live = r < rows;
  const int64_t cols_v = cols >> 2;
  const f32x4* __restrict__ xr = reinterpret_cast<const f32x4*>(x + (live ? r : 0) * cols);
  f32x4* __restrict__ yr = reinterpret_cast<f32x4*>(y + (live ? r : 0) * cols);

  f32x4 v[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int64_t j = static_cast<int64_t>(i) * TPR + t;
    if (live && j < cols_v) {
      v[i] = ld_stream(xr + j);
    } else {
      v[i] = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    }
  }
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < VPT; ++i)
    m = fmaxf(m, fmaxf(fmaxf(v[i][0], v[i][1]), fmaxf(v[i][2], v[i][3])));
  m = group_max<TPR>(m, lds);

  float d = 0.0f;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int64_t j = static_cast<int64_t>(i) * TPR + t;
    if (j < cols_v) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        v[i][c] = exp_le0(v[i][c] - m);
        d += v[i][c];
      }
    }
  }
  d = group_sum<TPR>(d, lds);
  const float inv = 1.0f / d;
  if (!live) return;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int64_t j = static_cast<int64_t>(i) * TPR + t;
    if (j < cols_v) st_stream(yr + j, v[i] * inv);
  }
}

// ---------------------------------------------------------------------------
// Online (m, d) fallback and the three-pass baseline: one workgroup per row.
// ---------------------------------------------------------------------------
struct OnlineState {
  float m, d;
};

__device__ __forceinline__ OnlineState online_identity() { return {-FLT_MAX, 0.0f}; }

__device__ __forceinline__ OnlineState online_update(OnlineState s, float x) {
  const float mn = fmaxf(s.m, x);
  return {mn, s.d * exp_le0(s.m - mn) + exp_le0(x - mn)};
}

__device__ __forceinline__ OnlineState online_combine(OnlineState a, OnlineState b) {
  if (b.d == 0.0f) return a;
  if (a.d == 0.0f) return b;
  const float mm = fmaxf(a.m, b.m);
  return {mm, a.d * exp_le0(a.m - mm) + b.d * exp_le0(b.m - mm)};
}

__device__ __forceinline__ OnlineState block_online(OnlineState s) {
  __shared__ float pm[kThreads / kWave], pd[kThreads / kWave];
#pragma unroll
  for (int k = kWave / 2; k >= 1; k >>= 1) {
    OnlineState o{__shfl_xor(s.m, k, 64), __shfl_xor(s.d, k, 64)};
    s = online_combine(s, o);
  }
  const int w = threadIdx.x / kWave;
  if ((threadIdx.x % kWave) == 0) {
    pm[w] = s.m;
    pd[w] = s.d;
  }
  __syncthreads();
  OnlineState r{pm[0], pd[0]};
#pragma unroll
  for (int i = 1; i < kThreads / kWave; ++i) r = online_combine(r, OnlineState{pm[i], pd[i]});
  return r;
}

__global__ __launch_bounds__(kThreads) void softmax_online_kernel(const float* __restrict__ x,
                                                                  float* __restrict__ y,
                                                                  int64_t cols) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * cols;
  OnlineState s = online_identity();
  for (int64_t c = threadIdx.x; c < cols; c += kThreads) s = online_update(s, x[base + c]);
  s = block_online(s);
  const float inv = 1.0f / s.d;
  for (int64_t c = threadIdx.x; c < cols; c += kThreads)
    y[base + c] = exp_le0(x[base + c] - s.m) * inv;
}

__device__ __forceinline__ float block_max(float v) {
  __shared__ float part[kThreads / kWave];
  v = wave_max(v);
  if ((threadIdx.x % kWave) == 0) part[threadIdx.x / kWave] = v;
  __syncthreads();
  float r = part[0];
#pragma unroll
  for (int i = 1; i < kThreads / kWave; ++i) r = fmaxf(r, part[i]);
  return r;
}

__device__ __forceinline__ float block_sum(float v) {
  __shared__ float part[kThreads / kWave];
  v = wave_sum(v);
  if ((threadIdx.x % kWave) == 0) part[threadIdx.x / kWave] = v;
  __syncthreads();
  float r = part[0];
#pragma unroll
  for (int i = 1; i < kThreads / kWave; ++i) r += part[i];
  return r;
}

__global__ __launch_bounds__(kThreads) void softmax_three_pass_kernel(
    const float* __restrict__ x, float* __restrict__ y, int64_t cols) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * cols;
  float m = -INFINITY;
  for (int64_t c = threadIdx.x; c < cols; c += kThreads) m = fmaxf(m, x[base + c]);
  m = block_max(m);
  float d = 0.0f;
  for (int64_t c = threadIdx.x; c < cols; c += kThreads) d += exp_le0(x[base + c] - m);
  d = block_sum(d);
  const float inv = 1.0f / d;
  for (int64_t c = threadIdx.x; c < cols; c += kThreads)
    y[base + c] = exp_le0(x[base + c] - m) * inv;
}

template <int TPR, int VPT, int NT = kThreads>
int launch_regs(const float* x, float* y, int64_t rows, int64_t cols, hipStream_t s) {
  constexpr int rpb = NT / TPR;
  const int64_t g = (rows + rpb - 1) / rpb;
  softmax_regs_kernel<TPR, VPT, NT><<<static_cast<unsigned>(g), NT, 0, s>>>(x, y, rows, cols);
  MCKE_LAUNCH_CHECK("softmax_regs_kernel");
  return ok();
}

// Register-resident configuration for a row of cols_v float4 vectors.
int launch_online(const float* x, float* y, int64_t rows, int64_t cols, hipStream_t s) {
  const bool vec = (cols % 4 == 0) && aligned(x, 16) && aligned(y, 16);
  const int64_t cv = cols / 4;
  if (vec && cv <= 2048) {
    // Short rows: fewer lanes per row and four float4s per lane, so a launch at
    // 32768 rows is one round of resident workgroups with 64 bytes per lane in
    // flight (measured 6.2 us vs 8.2 us for one float4 per lane at 128 columns).
    // Longer rows: two float4s per lane over more lanes.  At 32768 x 1024, 128
    // lanes x 2 took 42.9 us in 256-lane workgroups and 42.45 in 512-lane ones of
    // four rows (64 x 4: 43.4, 32 x 8: 44.5, 256 x 1: 45.1; a one-wave float4 copy
    // of the same bytes 41.1); at 32768 x 4096, 512-lane workgroups of one
    // row x 2 took 163.2 us (256 x 4: 172.9, 128 x 8: 178.0, 64 x 16: 181.4; the
    // copy 165.5); at 16384 x 8192, 1024-lane workgroups of one row x 2 took
    // 171.0 us (256 x 8: 176.5, 512 x 4: 187.2).
    if (cv <= 32) return launch_regs<8, 4>(x, y, rows, cols, s);
    if (cv <= 64) return launch_regs<16, 4>(x, y, rows, cols, s);
    if (cv <= 128) return launch_regs<64, 2>(x, y, rows, cols, s);
    if (cv <= 256) return launch_regs<128, 2, 512>(x, y, rows, cols, s);
    if (cv <= 512) return launch_regs<64, 8>(x, y, rows, cols, s);
    if (cv <= 1024) return launch_regs<512, 2, 512>(x, y, rows, cols, s);
    return launch_regs<1024, 2, 1024>(x, y, rows, cols, s);
  }
  softmax_online_kernel<<<static_cast<unsigned>(rows), kThreads, 0, s>>>(x, y, cols);
  MCKE_LAUNCH_CHECK("softmax_online_kernel");
  return ok();
}

}  // namespace
}  // namespace mcke_amd

using namespace mcke_amd;

extern "C" {

int mcke_launch_row_softmax_f32(const float* x, float* y, int64_t rows, int64_t cols,
                                int variant, void* stream) {
  if (rows == 0 || cols == 0) return ok();
  if (rows < 0 || cols < 0) return invalid("launch_row_softmax_f32: negative extent");
  if (!x || !y) return invalid("launch_row_softmax_f32: null pointer");
  if (x == y)
    return invalid("launch_row_softmax_f32: in-place (x == y) violates the __restrict__ contract");
  if (rows > 2147483647LL)
    return invalid("launch_row_softmax_f32: rows exceeds the grid's x limit");
  if (variant != MCKE_SOFTMAX_THREE_PASS && variant != MCKE_SOFTMAX_ONLINE_ONE_PASS)
    return invalid("launch_row_softmax_f32: unknown SoftmaxVariant");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (variant == MCKE_SOFTMAX_THREE_PASS) {
    softmax_three_pass_kernel<<<static_cast<unsigned>(rows), kThreads, 0, s>>>(x, y, cols);
    MCKE_LAUNCH_CHECK("softmax_three_pass_kernel");
    return ok();
  }
  return launch_online(x, y, rows, cols, s);
}

}  // extern "C"
