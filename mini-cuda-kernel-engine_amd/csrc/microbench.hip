// microbench.hip -- the measured denominators: an fp32 MFMA peak kernel and a
// STREAM triad, MI355X counterparts of the reference's bench/fma_peak.cu and
// bench/stream_triad.cu.
//
// The GEMM runs on the matrix cores, so its compute ceiling is the MFMA pipe's,
// not the vector FMA pipe's that the reference measures: each wave here keeps
// four independent v_mfma_f32_32x32x2_f32 accumulator chains in flight (a chain's
// result latency is covered by the other three) and touches memory only for its
// seed and one store, which keeps the result observable.  The sustained rate
// depends on how long the pipe stays busy (clock and power management), so the
// caller picks `iters` to match the duration of the kernel it divides.
//
// The triad a[i] = s * c[i] + b[i] moves 12 bytes per element (two reads, one
// write) through float4 non-temporal accesses, one float4 per lane per iteration
// of a grid-stride loop; a scalar tail covers n % 4.
#include <hip/hip_runtime.h>

#include "common.hpp"
#include "device_math.hpp"
#include "gemm_lp.hpp"

namespace mcke_amd {
namespace {

constexpr int kPeakThreads = 256;   // 4 waves per workgroup
constexpr int kChains = 4;          // independent accumulators per wave
constexpr uint64_t kFlopsPerMfma = 2ull * 32 * 32 * 2;

__global__ __launch_bounds__(kPeakThreads) void mfma_peak_f32_kernel(const float* __restrict__ seed,
                                                                     float* __restrict__ out,
                                                                     int64_t iters) {
  const float a = seed[threadIdx.x];
  const float b = seed[(threadIdx.x + 1) % kPeakThreads];
  f32x16 acc[kChains];
#pragma unroll
  for (int c = 0; c < kChains; ++c) {
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[c][r] = 0.0f;
  }
  for (int64_t i = 0; i < iters; ++i) {
#pragma unroll
    for (int c = 0; c < kChains; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[c], 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < kChains; ++c) {
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[c][r];
  }
  out[static_cast<int64_t>(blockIdx.x) * kPeakThreads + threadIdx.x] = s;
}

// The same four chains on the 16-bit MFMA (v_mfma_f32_32x32x16_{bf16,f16}),
// the ceiling of the 16-bit-input GEMM.  Operands are the seeds rounded to T.
constexpr uint64_t kFlopsPerMfmaLp = 2ull * 32 * 32 * 16;

template <typename T>
__global__ __launch_bounds__(kPeakThreads) void mfma_peak_lp_kernel(const float* __restrict__ seed,
                                                                    float* __restrict__ out,
                                                                    int64_t iters) {
  T av[8], bv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    av[e] = static_cast<T>(seed[(threadIdx.x + e) % kPeakThreads]);
    bv[e] = static_cast<T>(seed[(threadIdx.x + 8 + e) % kPeakThreads]);
  }
  const u32x4 a = __builtin_bit_cast(u32x4, av);
  const u32x4 b = __builtin_bit_cast(u32x4, bv);
  f32x16 acc[kChains];
#pragma unroll
  for (int c = 0; c < kChains; ++c) {
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[c][r] = 0.0f;
  }
  for (int64_t i = 0; i < iters; ++i) {
#pragma unroll
    for (int c = 0; c < kChains; ++c) acc[c] = LpMfma<T>::run(a, b, acc[c]);
  }
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < kChains; ++c) {
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[c][r];
  }
  out[static_cast<int64_t>(blockIdx.x) * kPeakThreads + threadIdx.x] = s;
}

constexpr int kTriadThreads = 256;

__global__ __launch_bounds__(kTriadThreads) void stream_triad_kernel(const float* __restrict__ b,
                                                                     const float* __restrict__ c,
                                                                     float* __restrict__ a, float s,
                                                                     int64_t n) {
  const int64_t n4 = n / 4;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kTriadThreads;
  const f32x4* b4 = reinterpret_cast<const f32x4*>(b);
  const f32x4* c4 = reinterpret_cast<const f32x4*>(c);
  f32x4* a4 = reinterpret_cast<f32x4*>(a);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kTriadThreads + threadIdx.x; i < n4; i += stride) {
    const f32x4 vb = ld_stream(b4 + i);
    const f32x4 vc = ld_stream(c4 + i);
    f32x4 r;
    r.x = fmaf(s, vc.x, vb.x);
    r.y = fmaf(s, vc.y, vb.y);
    r.z = fmaf(s, vc.z, vb.z);
    r.w = fmaf(s, vc.w, vb.w);
    st_stream(a4 + i, r);
  }
  const int64_t t = n4 * 4 + static_cast<int64_t>(blockIdx.x) * kTriadThreads + threadIdx.x;
  if (t < n) a[t] = fmaf(s, c[t], b[t]);
}

// The read+write ceiling for kernels that move one read and one write per
// element (softmax, bias+act): y = x, one float4 per lane, non-temporal both
// ways, one launch covering the array with no grid-stride loop, one wave per
// workgroup.  Of the copy shapes measured on MI355X (grid-stride loops at
// 256..16384 workgroups with 1..8 float4 per lane, contiguous chunks per
// workgroup, plain or non-temporal accesses, and this shape at 64..1024 lanes)
// this one moves the most: 2 x 256 MiB in 80.0 us against 82.5 us with
// 256-lane workgroups on the same box.
constexpr int kCopyThreads = 64;

__global__ __launch_bounds__(kCopyThreads) void stream_copy_kernel(const float* __restrict__ x,
                                                                   float* __restrict__ y,
                                                                   int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kCopyThreads + threadIdx.x;
  const int64_t n4 = n / 4;
  if (i < n4) {
    st_stream(reinterpret_cast<f32x4*>(y) + i, ld_stream(reinterpret_cast<const f32x4*>(x) + i));
  } else if (i == n4) {
    for (int64_t t = 4 * n4; t < n; ++t) y[t] = x[t];
  }
}

}  // namespace
}  // namespace mcke_amd

using namespace mcke_amd;

extern "C" {

uint64_t mcke_mfma_peak_flops(int64_t blocks, int64_t iters) {
  if (blocks <= 0 || iters <= 0) return 0;
  return static_cast<uint64_t>(blocks) * (kPeakThreads / kWave) * static_cast<uint64_t>(iters) *
         kChains * kFlopsPerMfma;
}

int mcke_launch_mfma_peak_f32(const float* seed, float* out, int64_t blocks, int64_t iters,
                              void* stream) {
  if (!seed || !out) return invalid("launch_mfma_peak_f32: null pointer");
  if (blocks <= 0 || blocks > 0x7fffffff) return invalid("launch_mfma_peak_f32: blocks out of range");
  if (iters <= 0) return invalid("launch_mfma_peak_f32: iters must be > 0");
  mfma_peak_f32_kernel<<<static_cast<unsigned>(blocks), kPeakThreads, 0,
                         static_cast<hipStream_t>(stream)>>>(seed, out, iters);
  MCKE_LAUNCH_CHECK("mfma_peak_f32_kernel");
  return ok();
}

uint64_t mcke_mfma_peak_lp_flops(int64_t blocks, int64_t iters) {
  if (blocks <= 0 || iters <= 0) return 0;
  return static_cast<uint64_t>(blocks) * (kPeakThreads / kWave) * static_cast<uint64_t>(iters) *
         kChains * kFlopsPerMfmaLp;
}

int mcke_launch_mfma_peak_lp(int ab_dtype, const float* seed, float* out, int64_t blocks,
                             int64_t iters, void* stream) {
  if (ab_dtype != MCKE_DTYPE_BF16 && ab_dtype != MCKE_DTYPE_F16)
    return invalid("launch_mfma_peak_lp: ab_dtype must be MCKE_DTYPE_BF16 or MCKE_DTYPE_F16");
  if (!seed || !out) return invalid("launch_mfma_peak_lp: null pointer");
  if (blocks <= 0 || blocks > 0x7fffffff) return invalid("launch_mfma_peak_lp: blocks out of range");
  if (iters <= 0) return invalid("launch_mfma_peak_lp: iters must be > 0");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (ab_dtype == MCKE_DTYPE_BF16)
    mfma_peak_lp_kernel<__bf16><<<static_cast<unsigned>(blocks), kPeakThreads, 0, s>>>(seed, out,
                                                                                       iters);
  else
    mfma_peak_lp_kernel<_Float16><<<static_cast<unsigned>(blocks), kPeakThreads, 0, s>>>(seed, out,
                                                                                         iters);
  MCKE_LAUNCH_CHECK("mfma_peak_lp_kernel");
  return ok();
}

int mcke_launch_stream_triad_f32(const float* b, const float* c, float* a, float scalar, int64_t n,
                                 void* stream) {
  if (n == 0) return ok();
  if (n < 0) return invalid("launch_stream_triad_f32: negative n");
  if (!a || !b || !c) return invalid("launch_stream_triad_f32: null pointer");
  if (!aligned(a, 16) || !aligned(b, 16) || !aligned(c, 16))
    return invalid("launch_stream_triad_f32: pointers must be 16-byte aligned");
  if (a == b || a == c) return invalid("launch_stream_triad_f32: output aliases an input");
  const int64_t n4 = n / 4;
  int64_t blocks = (n4 + kTriadThreads - 1) / kTriadThreads;
  if (blocks < 1) blocks = 1;           // the tail alone (n < 4) still needs one block
  if (blocks > 65536) blocks = 65536;
  // The scalar tail is indexed by blockIdx.x * 256 + lane, so it needs n % 4 < 256 lanes: always true.
  stream_triad_kernel<<<static_cast<unsigned>(blocks), kTriadThreads, 0,
                        static_cast<hipStream_t>(stream)>>>(b, c, a, scalar, n);
  MCKE_LAUNCH_CHECK("stream_triad_kernel");
  return ok();
}

int mcke_launch_stream_copy_f32(const float* x, float* y, int64_t n, void* stream) {
  if (n == 0) return ok();
  if (n < 0) return invalid("launch_stream_copy_f32: negative n");
  if (!x || !y) return invalid("launch_stream_copy_f32: null pointer");
  if (!aligned(x, 16) || !aligned(y, 16))
    return invalid("launch_stream_copy_f32: pointers must be 16-byte aligned");
  if (x == y) return invalid("launch_stream_copy_f32: output aliases the input");
  // One lane per float4 plus one lane for the tail (n % 4 elements).
  const int64_t lanes = n / 4 + 1;
  const int64_t blocks = (lanes + kCopyThreads - 1) / kCopyThreads;
  if (blocks > 0x7fffffff) return invalid("launch_stream_copy_f32: n too large for one launch");
  stream_copy_kernel<<<static_cast<unsigned>(blocks), kCopyThreads, 0,
                       static_cast<hipStream_t>(stream)>>>(x, y, n);
  MCKE_LAUNCH_CHECK("stream_copy_kernel");
  return ok();
}

}  // extern "C"
