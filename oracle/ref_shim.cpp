// ref_shim.cpp -- TEST INFRASTRUCTURE ONLY.
//
// C-linkage wrappers around the reference's own header-only CPU oracle
// (tests/reference.hpp and include/mcke/kernels/softmax_online.hpp), compiled
// straight from the reference tree by oracle/Makefile into oracle/_ref/.  This
// file contains no reference code: it includes the reference headers where they
// lie and forwards plain pointers to them, so the restatement in mcke_oracle.c
// can be checked against the original, bit for bit, and so the benchmark's CPU
// baseline can time the reference's own loops ("kind": "reference").
#include <cstddef>
#include <cstdint>
#include <random>

#include "mcke/kernels/softmax_online.hpp"
#include "reference.hpp"

namespace T = mcke::testing;
namespace K = mcke::kernels;

extern "C" {

__attribute__((visibility("default"))) std::uint64_t ref_mt64_nth(std::uint64_t seed,
                                                                  std::uint64_t n) {
  std::mt19937_64 g(seed);
  std::uint64_t v = 0;
  for (std::uint64_t i = 0; i < n; ++i) v = g();
  return v;
}

__attribute__((visibility("default"))) void ref_fill_random(float* p, std::size_t n,
                                                            std::uint64_t seed, float lo,
                                                            float hi) {
  T::fill_random(p, n, seed, lo, hi);
}

__attribute__((visibility("default"))) void ref_bias_act(const float* x, const float* bias,
                                                         float* y, std::int64_t rows,
                                                         std::int64_t cols, int act) {
  T::reference_bias_act(x, bias, y, rows, cols, static_cast<K::Activation>(act));
}

__attribute__((visibility("default"))) void ref_row_reduce(const float* x, float* out,
                                                           std::int64_t rows,
                                                           std::int64_t cols, int kind) {
  T::reference_row_reduce(x, out, rows, cols, static_cast<K::ReduceKind>(kind));
}

__attribute__((visibility("default"))) void ref_row_softmax(const float* x, float* y,
                                                            std::int64_t rows,
                                                            std::int64_t cols) {
  T::reference_row_softmax(x, y, rows, cols);
}

__attribute__((visibility("default"))) void ref_gemm(const float* a, const float* b, float* c,
                                                     std::int64_t m, std::int64_t n,
                                                     std::int64_t k, float alpha, float beta) {
  T::reference_gemm(a, b, c, m, n, k, alpha, beta);
}

// Compare result flattened into doubles: n, mismatches, max_abs, max_rel,
// worst_index, worst_got, worst_want, any_nan, any_inf.
__attribute__((visibility("default"))) void ref_compare(const float* got, const float* want,
                                                        std::size_t n, double rel_tol,
                                                        double abs_tol, double* out9) {
  const T::CompareResult r = T::compare(got, want, n, rel_tol, abs_tol);
  out9[0] = static_cast<double>(r.n);
  out9[1] = static_cast<double>(r.mismatches);
  out9[2] = r.max_abs_err;
  out9[3] = r.max_rel_err;
  out9[4] = static_cast<double>(r.worst_index);
  out9[5] = r.worst_got;
  out9[6] = r.worst_want;
  out9[7] = r.any_nan ? 1.0 : 0.0;
  out9[8] = r.any_inf ? 1.0 : 0.0;
}

__attribute__((visibility("default"))) double ref_tol_gemm(std::int64_t k) {
  return T::tol_gemm(k);
}

__attribute__((visibility("default"))) double ref_abs_tol_gemm(std::int64_t k, double amax) {
  return T::abs_tol_gemm(k, amax);
}

// Spot-check result flattened: checked, mismatches, max_abs, max_rel.
__attribute__((visibility("default"))) void ref_spot_check_gemm(
    const float* a, const float* b, const float* got, std::int64_t m, std::int64_t n,
    std::int64_t k, float alpha, std::size_t samples, std::uint64_t seed, double rel_tol,
    double abs_tol, double* out4) {
  const T::SpotCheckResult r =
      T::spot_check_gemm(a, b, got, m, n, k, alpha, samples, seed, rel_tol, abs_tol);
  out4[0] = static_cast<double>(r.checked);
  out4[1] = static_cast<double>(r.mismatches);
  out4[2] = r.max_abs_err;
  out4[3] = r.max_rel_err;
}

__attribute__((visibility("default"))) void ref_online_update(float m, float d, float x,
                                                              float* om, float* od) {
  const K::OnlineState s = K::online_update(K::OnlineState{m, d}, x);
  *om = s.m;
  *od = s.d;
}

__attribute__((visibility("default"))) void ref_online_combine(float am, float ad, float bm,
                                                               float bd, float* om,
                                                               float* od) {
  const K::OnlineState s = K::online_combine(K::OnlineState{am, ad}, K::OnlineState{bm, bd});
  *om = s.m;
  *od = s.d;
}

}  // extern "C"
