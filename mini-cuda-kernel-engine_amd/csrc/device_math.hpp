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
// Wave64 butterfly reductions.  Every lane ends with the same bits: at each step
// lane i forms op(v_i, v_{i^m}) and lane i^m forms op(v_{i^m}, v_i), and both
// ops are commutative.
// ---------------------------------------------------------------------------
template <int WIDTH = 64> __device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = WIDTH / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

template <int WIDTH = 64> __device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = WIDTH / 2; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

// ---------------------------------------------------------------------------
// Activations (reference tests/reference.hpp:116-136 and bias_act.cu:95-117).
//
// Each takes x and the bias separately so that v = x + b is carried exactly as
// (vh, vl) with vh = fl(x + b) (Knuth's TwoSum), matching the reference's double
// sum, and the GELUs are evaluated in forms that keep the absolute error near
// half an ulp of the result:
//
//   GELU_tanh(v) = 0.5 v (1 + tanh(z)),  z = sqrt(2/pi) (v + 0.044715 v^3)
//                = v * sigmoid(2z)                    [0.5(1+tanh z) = sigmoid(2z)]
//   with r = sigmoid(-2|z|) = e / (1 + e), e = exp(-2|z|) in (0, 1]:
//     v >= 0 :  y = v (1 - r) = vh + (vl - vh r)      (small correction term)
//     v <  0 :  y = v r                               (small result)
//
//   GELU_erf(v) = 0.5 v (1 + erf(v / sqrt 2)) = 0.5 v erfc(-v / sqrt 2)
//     v >= 0 :  y = vh + (vl - 0.5 vh erfc(v / sqrt 2))
//     v <  0 :  y = 0.5 (vh + vl) erfc(-v / sqrt 2)
//
// so that the cancellation in (1 + tanh) or (1 + erf) near -1 never happens and
// for large positive v the result is vh plus a tiny correction.
// ---------------------------------------------------------------------------
enum : int { kActNone = 0, kActRelu = 1, kActGeluErf = 2, kActGeluTanh = 3 };

__device__ __forceinline__ void two_sum(float a, float b, float& s, float& e) {
  s = a + b;
  const float bb = s - a;
  e = (a - (s - bb)) + (b - bb);
}

__device__ __forceinline__ float gelu_tanh_xb(float x, float b) {
  float v, vl;
  two_sum(x, b, v, vl);
  const float u = v * v;
  const float z = 0.7978845608028654f * __builtin_fmaf(0.044715f * v, u, v);
  // e = exp(-2|z|) via the hardware base-2 exponential.
  const float e = __builtin_amdgcn_exp2f(-2.8853900817779268f * __builtin_fabsf(z));
  const float r = e * __builtin_amdgcn_rcpf(1.0f + e);
  float y = (v >= 0.0f) ? v + __builtin_fmaf(-v, r, vl) : __builtin_fmaf(v, r, vl * r);
  // Infinite v: TwoSum's error term is NaN there; the limits are +inf -> +inf and
  // -inf -> 0 * inf = NaN, which is what the reference's formula gives.
  if (__builtin_isinf(v)) y = (v > 0.0f) ? v : __builtin_nanf("");
  return y;
}

__device__ __forceinline__ float gelu_erf_xb(float x, float b) {
  float v, vl;
  two_sum(x, b, v, vl);
  const float t = v * 0.70710678118654752440f;
  float y;
  if (v >= 0.0f) {
    y = v + __builtin_fmaf(-0.5f * v, erfcf(t), vl);
  } else {
    y = 0.5f * erfcf(-t) * (v + vl);
  }
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
