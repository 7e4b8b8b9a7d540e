// mcke/profiling/host_timer.hpp -- host-side latency measurement: a steady-clock
// bracket, a self-measured clock resolution, and a retained sample of durations
// with exact percentiles.  The API of the reference's
// include/mcke/profiling/host_timer.hpp:102-217 (HostTimer, ClockCalibration,
// LatencyStats), implemented here; pure host code, no GPU needed.
#pragma once

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace mcke {

// Brackets one host operation on the monotonic clock (never the wall clock,
// which NTP may step while a measurement runs).
class HostTimer {
 public:
  void start() noexcept { t0_ = std::chrono::steady_clock::now(); }
  // Nanoseconds since the last start().
  [[nodiscard]] std::uint64_t stop_ns() const noexcept {
    return static_cast<std::uint64_t>(
        std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now() - t0_)
            .count());
  }

 private:
  std::chrono::steady_clock::time_point t0_{};
};

// What this machine's clock resolves, measured with the clock itself: pairs of
// start() / stop_ns() with nothing between them.
struct ClockCalibration {
  std::uint64_t tick_ns = 0;           // smallest nonzero paired delta
  std::uint64_t paired_median_ns = 0;  // median paired delta (call overhead)
  std::uint64_t floor_ns = 0;          // max(tick_ns, paired_median_ns)

  [[nodiscard]] static ClockCalibration measure(int samples = 100000);
  // A duration within two floors of zero says more about the clock than about
  // the operation timed.
  [[nodiscard]] bool is_below_floor(std::uint64_t ns) const { return floor_ns > 0 && ns <= 2 * floor_ns; }
  [[nodiscard]] std::string describe() const;
};

// Every sample kept (reserved up front, so add() does not allocate inside a timed
// region), sorted once by finalize(); percentiles are nearest-rank: the smallest
// sample with at least p% of the samples at or below it, index ceil(p/100 * n) - 1
// clamped to [0, n - 1].  Every query of an empty sample returns 0.
class LatencyStats {
 public:
  explicit LatencyStats(std::size_t expected_count) { samples_.reserve(expected_count); }
  void add(std::uint64_t ns) { samples_.push_back(ns); }
  void finalize() {
    std::sort(samples_.begin(), samples_.end());
    finalized_ = true;
  }
  [[nodiscard]] std::size_t count() const { return samples_.size(); }
  [[nodiscard]] bool empty() const { return samples_.empty(); }
  [[nodiscard]] bool is_finalized() const { return finalized_; }

  // Needs finalize() first (the order statistics read the sorted sample).
  [[nodiscard]] std::uint64_t percentile(double p) const {
    if (samples_.empty()) return 0;
    const auto n = static_cast<double>(samples_.size());
    const double rank = std::ceil(p / 100.0 * n);
    const double idx = std::clamp(rank - 1.0, 0.0, n - 1.0);
    return samples_[static_cast<std::size_t>(idx)];
  }
  [[nodiscard]] std::uint64_t median() const { return percentile(50.0); }
  [[nodiscard]] std::uint64_t p90() const { return percentile(90.0); }
  [[nodiscard]] std::uint64_t p99() const { return percentile(99.0); }
  [[nodiscard]] std::uint64_t p999() const { return percentile(99.9); }
  [[nodiscard]] std::uint64_t min() const { return samples_.empty() ? 0 : samples_.front(); }
  [[nodiscard]] std::uint64_t max() const { return samples_.empty() ? 0 : samples_.back(); }
  [[nodiscard]] double mean_ns() const {
    if (samples_.empty()) return 0.0;
    double sum = 0.0;
    for (std::uint64_t v : samples_) sum += static_cast<double>(v);
    return sum / static_cast<double>(samples_.size());
  }
  // Counts per power-of-two bucket above the clock's floor: [0, floor], then
  // (floor, 2 floor], (2 floor, 4 floor], ...; one line per non-empty bucket,
  // "<= edge ns: count".  A floor of 0 is taken as 1 ns.
  [[nodiscard]] std::string log2_histogram(std::uint64_t floor_ns) const;

 private:
  std::vector<std::uint64_t> samples_;
  bool finalized_ = false;
};

}  // namespace mcke
