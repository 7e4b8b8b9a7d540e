// mcke/profiling/host_timer.hpp -- steady-clock host timing and latency stats
// (the API of the reference's include/mcke/profiling/host_timer.hpp:102-217).
#pragma once

#include <algorithm>
#include <chrono>
#include <cstddef>
#include <vector>

namespace mcke {

class HostTimer {
 public:
  HostTimer() : t0_(std::chrono::steady_clock::now()) {}
  void reset() { t0_ = std::chrono::steady_clock::now(); }
  [[nodiscard]] double elapsed_ms() const {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0_).count();
  }
  [[nodiscard]] double elapsed_us() const { return elapsed_ms() * 1e3; }

 private:
  std::chrono::steady_clock::time_point t0_;
};

struct LatencyStats {
  std::size_t count = 0;
  double min = 0, median = 0, p99 = 0, max = 0, mean = 0;
  [[nodiscard]] static LatencyStats from(std::vector<double> v) {
    LatencyStats s;
    if (v.empty()) return s;
    std::sort(v.begin(), v.end());
    s.count = v.size();
    s.min = v.front();
    s.max = v.back();
    s.median = v[v.size() / 2];
    s.p99 = v[std::min(v.size() - 1, static_cast<std::size_t>(0.99 * static_cast<double>(v.size())))];
    double sum = 0;
    for (double x : v) sum += x;
    s.mean = sum / static_cast<double>(v.size());
    return s;
  }
};

}  // namespace mcke
