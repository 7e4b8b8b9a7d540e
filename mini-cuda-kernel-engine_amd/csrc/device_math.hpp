// device_math.hpp -- device-side building blocks shared by the kernels:
// vector loads/stores, wave64 reductions, and the activation functions.
#pragma once

#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

namespace mcke_amd {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int VW> struct VecT;
template <> struct VecT<1> { using type = float; };
template <> struct VecT<2> { using type = f32x2; };
template <> struct VecT<4> { using type = f32x4; };
template <int VW> using Vec = typename VecT<VW>::type;

template <int VW> __device__ __forceinline__ float lane(const Vec<VW>& v, int i);
template <> __device__ __forceinline__ float lane<1>(const float& v, int) { return v; }
template <> __device__ __forceinline__ float lane<2>(const f32x2& v, int i) { return v[i]; }
template <> __device__ __forceinline__ float lane<4>(const f32x4& v, int i) { return v[i]; }

// Streaming (non-temporal) accesses: data touched exactly once should not evict
// what the caches hold for other work.
template <class T> __device__ __forceinline__ T ld_stream(const T* p) {
  return __builtin_nontemporal_load(p);
}
template <class T> __device__ __forceinline__ void st_stream(T* p, T v) {
  __builtin_nontemporal_store(v, p);
}

// ---------------------------------------------------------------------------
// Wave64 group reductions over WIDTH consecutive lanes (WIDTH a power of two).
// The steps inside 16-lane rows use DPP lane permutations (a few cycles each)
// instead of ds_bpermute (an LDS-pipe round trip each):
//   pairs        quad_perm [1,0,3,2]
//   quads        quad_perm [2,3,0,1]
//   8 lanes      row_half_mirror (lane i <-> 7 - i: pairs the two quads)
//   16 lanes     row_mirror      (lane i <-> 15 - i: pairs the two halves)
// and the steps across rows use __shfl_xor 16 / 32.  Every lane ends with the
// same bits: each step combines a lane with a partner holding the same partial
// set, op(a, b) on one side and op(b, a) on the other, and both ops commute.
// ---------------------------------------------------------------------------
template <int CTRL> __device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL,
                                                            0xF, 0xF, true));
}

template <int WIDTH, class Op> __device__ __forceinline__ float wave_reduce(float v, Op op) {
  static_assert(WIDTH >= 1 && WIDTH <= 64 && (WIDTH & (WIDTH - 1)) == 0, "power of two");
  if constexpr (WIDTH >= 2) v = op(v, dpp_mov<0xB1>(v));    // quad_perm [1,0,3,2]
  if constexpr (WIDTH >= 4) v = op(v, dpp_mov<0x4E>(v));    // quad_perm [2,3,0,1]
  if constexpr (WIDTH >= 8) v = op(v, dpp_mov<0x141>(v));   // row_half_mirror
  if constexpr (WIDTH >= 16) v = op(v, dpp_mov<0x140>(v));  // row_mirror
  if constexpr (WIDTH >= 32) v = op(v, __shfl_xor(v, 16, 64));
  if constexpr (WIDTH >= 64) v = op(v, __shfl_xor(v, 32, 64));
  return v;
}

template <int WIDTH = 64> __device__ __forceinline__ float wave_sum(float v) {
  return wave_reduce<WIDTH>(v, [](float a, float b) { return a + b; });
}

template <int WIDTH = 64> __device__ __forceinline__ float wave_max(float v) {
  return wave_reduce<WIDTH>(v, [](float a, float b) { return fmaxf(a, b); });
}

// ---------------------------------------------------------------------------
// Activations (reference tests/reference.hpp:116-136 and bias_act.cu:95-117).
//
// Each takes x and the bias separately.  GELU_tanh is the hot one and is kept
// cheap (see gelu_tanh_xb).  GELU_erf carries v = x + b exactly as (vh, vl) with
// vh = fl(x + b) (Knuth's TwoSum), matching the reference's double sum, and is
// evaluated through erfc so that the cancellation in (1 + erf) near -1 never
// happens:
//   GELU_erf(v) = 0.5 v (1 + erf(v / sqrt 2)) = 0.5 v erfc(-v / sqrt 2)
//     v >= 0 :  y = vh + (vl - 0.5 vh erfc(v / sqrt 2))
//     v <  0 :  y = 0.5 vh erfc(-v / sqrt 2)
// ---------------------------------------------------------------------------
enum : int { kActNone = 0, kActRelu = 1, kActGeluErf = 2, kActGeluTanh = 3 };

__device__ __forceinline__ void two_sum(float a, float b, float& s, float& e) {
  s = a + b;
  const float bb = s - a;
  e = (a - (s - bb)) + (b - bb);
}

// GELU_tanh(v) = 0.5 v (1 + tanh(z)), z = sqrt(2/pi) (v + 0.044715 v^3), evaluated
// through 0.5 (1 + tanh z) = 1 / (1 + exp(-2z)) with the hardware base-2
// exponential and reciprocal:  y = v * rcp(1 + 2^(v (c1 + c2 v^2))),
// c1 = -2 log2(e) sqrt(2/pi), c2 = 0.044715 c1.  Seven VALU operations and two
// transcendentals per element, so the kernel stays HBM-bound.  The limits come out
// as the reference's formula gives them: v -> +inf gives +inf, v -> -inf gives
// -inf * 0 = NaN, -0 gives -0, NaN propagates.  Against the double-precision
// formula on float(x) + float(b) (v itself rounded once, as the reference kernel
// rounds it) the error stays within a fifth of abs 1e-6 + rel 1e-6 over
// |v| <= 30, also with the exponential and the reciprocal one ulp off.
__device__ __forceinline__ float gelu_tanh_xb(float x, float b) {
  constexpr float c1 = -2.30220818520f;    // -2 * log2(e) * sqrt(2/pi)
  constexpr float c2 = -0.102943241596f;  // c1 * 0.044715
  const float v = x + b;
  const float a = v * __builtin_fmaf(c2, v * v, c1);
  return v * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(a));
}

// erfc(s) for s >= 0 by Abramowitz & Stegun 7.1.26 (Hastings' approximation):
// t = 1 / (1 + p s), erfc(s) ~= t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) exp(-s^2),
// absolute error <= 1.5e-7 in exact arithmetic.  Branch-free: one reciprocal,
// five FMAs and one base-2 exponential, where the library erfcf branches over
// several ranges.  In GELU_erf on float inputs, evaluated in f32 with the
// hardware exponential and reciprocal each one ulp off, the error stays within
// 0.22 of abs 1e-6 + rel 1e-6 against the double formula over |v| <= 14.
__device__ __forceinline__ float erfc_nonneg(float s) {
  constexpr float kLog2eF = 1.4426950408889634f;
  const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.3275911f, s, 1.0f));
  float p = 1.061405429f;
  p = __builtin_fmaf(p, t, -1.453152027f);
  p = __builtin_fmaf(p, t, 1.421413741f);
  p = __builtin_fmaf(p, t, -0.284496736f);
  p = __builtin_fmaf(p, t, 0.254829592f);
  return (p * t) * __builtin_amdgcn_exp2f(-(s * s) * kLog2eF);
}

__device__ __forceinline__ float gelu_erf_xb(float x, float b) {
  float v, vl;
  two_sum(x, b, v, vl);
  const float e = erfc_nonneg(__builtin_fabsf(v) * 0.70710678118654752440f);
  const float half = 0.5f * v;
  float y = (v >= 0.0f) ? v + __builtin_fmaf(-half, e, vl) : half * e;
  if (__builtin_isinf(v)) y = (v > 0.0f) ? v : __builtin_nanf("");
  return y;
}

template <int ACT> __device__ __forceinline__ float act_xb(float x, float b) {
  if constexpr (ACT == kActNone) {
    return x + b;
  } else if constexpr (ACT == kActRelu) {
    const float v = x + b;
    return v > 0.0f ? v : 0.0f;   // NaN and -0 map to +0, as `v > 0.0 ? v : 0.0` does
  } else if constexpr (ACT == kActGeluErf) {
    return gelu_erf_xb(x, b);
  } else {
    return gelu_tanh_xb(x, b);
  }
}

}  // namespace mcke_amd
