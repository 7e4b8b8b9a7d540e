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

// Engine-clock probe for the 16-bit matrix pipe.  The peak kernel above feeds
// every MFMA the same operands; a GEMM's change with every instruction, and with
// random operands the pipe draws more power and the clock management lowers the
// engine clock.  Here each lane holds eight operand registers of random 16-bit
// values (`bits`, 8 x 16 bytes per lane of the workgroup) and every MFMA takes a
// different pair.  SHAPE 0 runs 4 chains of v_mfma_f32_32x32x16, SHAPE 1 8 chains of
// v_mfma_f32_16x16x32: the same flops per iteration (8 x 32768).  The chains are
// inline asm so that the compiler keeps them independent (it merges chains whose
// inputs it can prove equal); each chain's next MFMA is at least three
// instructions later, and the s_nops cover the result latency before the sums.
// Lane 0 of each workgroup records its s_memtime (engine clock) and
// s_memrealtime (100 MHz) spans in ticks[2 b], ticks[2 b + 1].
template <bool BF16, int SHAPE>
__global__ __launch_bounds__(kPeakThreads) void mfma_clock_lp_kernel(
    const u32x4* __restrict__ bits, float* __restrict__ out, uint64_t* __restrict__ ticks,
    int64_t iters) {
  const uint64_t c0 = __builtin_amdgcn_s_memtime();
  const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
  const u32x4* b = bits + threadIdx.x * 8;
  const u32x4 o0 = b[0], o1 = b[1], o2 = b[2], o3 = b[3], o4 = b[4], o5 = b[5], o6 = b[6],
              o7 = b[7];
  float s = 0.0f;
  if constexpr (SHAPE == 0) {
    f32x16 x0 = {}, x1 = {}, x2 = {}, x3 = {};
    for (int64_t it = 0; it < iters; ++it) {
      if constexpr (BF16)
        asm volatile(
            "v_mfma_f32_32x32x16_bf16 %0, %4, %5, %0\n\t"
            "v_mfma_f32_32x32x16_bf16 %1, %6, %7, %1\n\t"
            "v_mfma_f32_32x32x16_bf16 %2, %8, %9, %2\n\t"
            "v_mfma_f32_32x32x16_bf16 %3, %10, %11, %3\n\t"
            "v_mfma_f32_32x32x16_bf16 %0, %5, %6, %0\n\t"
            "v_mfma_f32_32x32x16_bf16 %1, %7, %8, %1\n\t"
            "v_mfma_f32_32x32x16_bf16 %2, %9, %10, %2\n\t"
            "v_mfma_f32_32x32x16_bf16 %3, %11, %4, %3\n\t"
            "s_nop 7"
            : "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3)
            : "v"(o0), "v"(o1), "v"(o2), "v"(o3), "v"(o4), "v"(o5), "v"(o6), "v"(o7));
      else
        asm volatile(
            "v_mfma_f32_32x32x16_f16 %0, %4, %5, %0\n\t"
            "v_mfma_f32_32x32x16_f16 %1, %6, %7, %1\n\t"
            "v_mfma_f32_32x32x16_f16 %2, %8, %9, %2\n\t"
            "v_mfma_f32_32x32x16_f16 %3, %10, %11, %3\n\t"
            "v_mfma_f32_32x32x16_f16 %0, %5, %6, %0\n\t"
            "v_mfma_f32_32x32x16_f16 %1, %7, %8, %1\n\t"
            "v_mfma_f32_32x32x16_f16 %2, %9, %10, %2\n\t"
            "v_mfma_f32_32x32x16_f16 %3, %11, %4, %3\n\t"
            "s_nop 7"
            : "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3)
            : "v"(o0), "v"(o1), "v"(o2), "v"(o3), "v"(o4), "v"(o5), "v"(o6), "v"(o7));
    }
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
    for (int r = 0; r < 16; ++r) s += x0[r] + x1[r] + x2[r] + x3[r];
  } else {
    f32x4 x0 = {}, x1 = {}, x2 = {}, x3 = {}, x4 = {}, x5 = {}, x6 = {}, x7 = {};
    for (int64_t it = 0; it < iters; ++it) {
      if constexpr (BF16)
        asm volatile(
            "v_mfma_f32_16x16x32_bf16 %0, %8, %9, %0\n\t"
            "v_mfma_f32_16x16x32_bf16 %1, %10, %11, %1\n\t"
            "v_mfma_f32_16x16x32_bf16 %2, %12, %13, %2\n\t"
            "v_mfma_f32_16x16x32_bf16 %3, %14, %15, %3\n\t"
            "v_mfma_f32_16x16x32_bf16 %4, %9, %10, %4\n\t"
            "v_mfma_f32_16x16x32_bf16 %5, %11, %12, %5\n\t"
            "v_mfma_f32_16x16x32_bf16 %6, %13, %14, %6\n\t"
            "v_mfma_f32_16x16x32_bf16 %7, %15, %8, %7\n\t"
            "v_mfma_f32_16x16x32_bf16 %0, %10, %13, %0\n\t"
            "v_mfma_f32_16x16x32_bf16 %1, %12, %15, %1\n\t"
            "v_mfma_f32_16x16x32_bf16 %2, %14, %9, %2\n\t"
            "v_mfma_f32_16x16x32_bf16 %3, %8, %11, %3\n\t"
            "v_mfma_f32_16x16x32_bf16 %4, %11, %14, %4\n\t"
            "v_mfma_f32_16x16x32_bf16 %5, %13, %8, %5\n\t"
            "v_mfma_f32_16x16x32_bf16 %6, %15, %10, %6\n\t"
            "v_mfma_f32_16x16x32_bf16 %7, %9, %12, %7\n\t"
            "s_nop 7"
            : "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3), "+v"(x4), "+v"(x5), "+v"(x6), "+v"(x7)
            : "v"(o0), "v"(o1), "v"(o2), "v"(o3), "v"(o4), "v"(o5), "v"(o6), "v"(o7));
      else
        asm volatile(
            "v_mfma_f32_16x16x32_f16 %0, %8, %9, %0\n\t"
            "v_mfma_f32_16x16x32_f16 %1, %10, %11, %1\n\t"
            "v_mfma_f32_16x16x32_f16 %2, %12, %13, %2\n\t"
            "v_mfma_f32_16x16x32_f16 %3, %14, %15, %3\n\t"
            "v_mfma_f32_16x16x32_f16 %4, %9, %10, %4\n\t"
            "v_mfma_f32_16x16x32_f16 %5, %11, %12, %5\n\t"
            "v_mfma_f32_16x16x32_f16 %6, %13, %14, %6\n\t"
            "v_mfma_f32_16x16x32_f16 %7, %15, %8, %7\n\t"
            "v_mfma_f32_16x16x32_f16 %0, %10, %13, %0\n\t"
            "v_mfma_f32_16x16x32_f16 %1, %12, %15, %1\n\t"
            "v_mfma_f32_16x16x32_f16 %2, %14, %9, %2\n\t"
            "v_mfma_f32_16x16x32_f16 %3, %8, %11, %3\n\t"
            "v_mfma_f32_16x16x32_f16 %4, %11, %14, %4\n\t"
            "v_mfma_f32_16x16x32_f16 %5, %13, %8, %5\n\t"
            "v_mfma_f32_16x16x32_f16 %6, %15, %10, %6\n\t"
            "v_mfma_f32_16x16x32_f16 %7, %9, %12, %7\n\t"
            "s_nop 7"
            : "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3), "+v"(x4), "+v"(x5), "+v"(x6), "+v"(x7)
            : "v"(o0), "v"(o1), "v"(o2), "v"(o3), "v"(o4), "v"(o5), "v"(o6), "v"(o7));
    }
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
    for (int r = 0; r < 4; ++r) s += x0[r] + x1[r] + x2[r] + x3[r] + x4[r] + x5[r] + x6[r] + x7[r];
  }
  out[static_cast<int64_t>(blockIdx.x) * kPeakThreads + threadIdx.x] = s;
  if (threadIdx.x == 0) {
    ticks[2 * static_cast<int64_t>(blockIdx.x)] = __builtin_amdgcn_s_memtime() - c0;
    ticks[2 * static_cast<int64_t>(blockIdx.x) + 1] = __builtin_amdgcn_s_memrealtime() - r0;
  }
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

uint64_t mcke_mfma_clock_lp_flops(int64_t blocks, int64_t iters) {
  if (blocks <= 0 || iters <= 0) return 0;
  return static_cast<uint64_t>(blocks) * (kPeakThreads / kWave) * static_cast<uint64_t>(iters) * 8 *
         kFlopsPerMfmaLp;
}

int mcke_launch_mfma_clock_lp(int ab_dtype, int shape, const void* operand_bits, float* out,
                              uint64_t* ticks, int64_t blocks, int64_t iters, void* stream) {
  if (ab_dtype != MCKE_DTYPE_BF16 && ab_dtype != MCKE_DTYPE_F16)
    return invalid("launch_mfma_clock_lp: ab_dtype must be MCKE_DTYPE_BF16 or MCKE_DTYPE_F16");
  if (shape != 0 && shape != 1)
    return invalid("launch_mfma_clock_lp: shape must be 0 (32x32x16) or 1 (16x16x32)");
  if (!operand_bits || !out || !ticks) return invalid("launch_mfma_clock_lp: null pointer");
  if (!aligned(operand_bits, 16)) return invalid("launch_mfma_clock_lp: operand_bits not 16-byte aligned");
  if (blocks <= 0 || blocks > 0x7fffffff) return invalid("launch_mfma_clock_lp: blocks out of range");
  if (iters <= 0) return invalid("launch_mfma_clock_lp: iters must be > 0");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const auto* bits = static_cast<const u32x4*>(operand_bits);
  const dim3 g(static_cast<unsigned>(blocks)), t(kPeakThreads);
  const bool bf16 = ab_dtype == MCKE_DTYPE_BF16;
  if (bf16 && shape == 0) mfma_clock_lp_kernel<true, 0><<<g, t, 0, s>>>(bits, out, ticks, iters);
  else if (bf16) mfma_clock_lp_kernel<true, 1><<<g, t, 0, s>>>(bits, out, ticks, iters);
  else if (shape == 0) mfma_clock_lp_kernel<false, 0><<<g, t, 0, s>>>(bits, out, ticks, iters);
  else mfma_clock_lp_kernel<false, 1><<<g, t, 0, s>>>(bits, out, ticks, iters);
  MCKE_LAUNCH_CHECK("mfma_clock_lp_kernel");
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
