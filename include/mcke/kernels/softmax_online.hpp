// mcke/kernels/softmax_online.hpp -- the online-softmax running state (m, d).
//
// Same API as the reference's include/mcke/kernels/softmax_online.hpp:73-112:
//   update:  m' = max(m, x),      d' = d * exp(m - m') + exp(x - m')
//   combine: m  = max(ma, mb),    d  = da * exp(ma - m) + db * exp(mb - m)
// The combine is associative and commutative, so partial states can be merged
// in any tree order (lane, wave, workgroup).  The identity is (-FLT_MAX, 0), not
// -inf, so that combining two empty states gives 0 * exp(0) = 0 rather than NaN;
// combine also returns the other operand when one side is empty (d == 0).
#pragma once

#include <cfloat>
#include <cmath>

#include "mcke/core/config.hpp"

namespace mcke::kernels {

struct OnlineState {
  float m;
  float d;
};

[[nodiscard]] MCKE_HOST_DEVICE inline OnlineState online_identity() { return OnlineState{-FLT_MAX, 0.0f}; }

[[nodiscard]] MCKE_HOST_DEVICE inline OnlineState online_update(OnlineState s, float x) {
  const float mn = fmaxf(s.m, x);
  return OnlineState{mn, s.d * expf(s.m - mn) + expf(x - mn)};
}

[[nodiscard]] MCKE_HOST_DEVICE inline OnlineState online_combine(OnlineState a, OnlineState b) {
  if (b.d == 0.0f) return a;
  if (a.d == 0.0f) return b;
  const float m = fmaxf(a.m, b.m);
  return OnlineState{m, a.d * expf(a.m - m) + b.d * expf(b.m - m)};
}

}  // namespace mcke::kernels
