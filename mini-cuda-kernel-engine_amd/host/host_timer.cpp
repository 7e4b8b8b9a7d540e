// host_timer.cpp -- clock self-calibration and the latency histogram
// (API of the reference's src/core/host_timer.cpp).
#include "mcke/profiling/host_timer.hpp"

#include <sstream>

namespace mcke {

ClockCalibration ClockCalibration::measure(int samples) {
  const std::size_t n = samples > 0 ? static_cast<std::size_t>(samples) : 1;
  std::vector<std::uint64_t> d(n);
  HostTimer t;
  for (std::size_t i = 0; i < n; ++i) {
    t.start();
    d[i] = t.stop_ns();
  }
  std::sort(d.begin(), d.end());
  ClockCalibration c;
  // A pair can read 0 when the clock did not tick between the two reads; the
  // first nonzero delta is the granularity.
  const auto first_tick = std::upper_bound(d.begin(), d.end(), std::uint64_t{0});
  c.tick_ns = first_tick == d.end() ? 0 : *first_tick;
  c.paired_median_ns = d[n / 2];
  c.floor_ns = std::max(c.tick_ns, c.paired_median_ns);
  return c;
}

std::string ClockCalibration::describe() const {
  std::ostringstream os;
  os << "clock tick " << tick_ns << " ns, back-to-back reads " << paired_median_ns
     << " ns (median): floor " << floor_ns << " ns; durations up to " << 2 * floor_ns
     << " ns are at the clock's resolution";
  return os.str();
}

std::string LatencyStats::log2_histogram(std::uint64_t floor_ns) const {
  if (samples_.empty()) return "  (no samples)\n";
  const std::uint64_t floor = floor_ns ? floor_ns : 1;
  // Bucket of v: 0 for v <= floor, else the smallest b with v <= floor << b.
  auto bucket_of = [&](std::uint64_t v) {
    std::size_t b = 0;
    while (b < 63 && v > (floor << b) && (floor << b) <= (UINT64_MAX >> 1)) ++b;
    return b;
  };
  std::vector<std::size_t> counts;
  for (std::uint64_t v : samples_) {
    const std::size_t b = bucket_of(v);
    if (b >= counts.size()) counts.resize(b + 1, 0);
    ++counts[b];
  }
  std::ostringstream os;
  for (std::size_t b = 0; b < counts.size(); ++b)
    if (counts[b]) os << "    <= " << (floor << b) << " ns: " << counts[b] << '\n';
  return os.str();
}

}  // namespace mcke
