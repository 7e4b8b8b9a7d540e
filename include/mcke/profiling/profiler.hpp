// mcke/profiling/profiler.hpp -- event-bracketed kernel timing and the roofline.
//
// Same API as the reference's include/mcke/profiling/profiler.hpp:67-265:
// KernelRecord (ideal flops/bytes + median/min ms), Roofline (ridge point,
// attainable TFLOP/s, efficiency), Profiler::time_op (warmup, then `iters`
// launches each bracketed by its own timing-event pair on the stream, one host
// synchronisation at the end) and the 13-column CSV / summary table.  NvtxRange
// becomes a ROCTX range marker when built with MCKE_USE_ROCTX (no-op otherwise).
#pragma once

#include <algorithm>
#include <cstdint>
#include <string>
#include <utility>
#include <vector>

#include "mcke/core/device.hpp"
#include "mcke/core/status.hpp"
#include "mcke/runtime/stream.hpp"

#if defined(MCKE_USE_ROCTX)
#include <roctracer/roctx.h>
#endif

namespace mcke {

class NvtxRange {
 public:
  explicit NvtxRange([[maybe_unused]] const char* name) {
#if defined(MCKE_USE_ROCTX)
    roctxRangePushA(name);
#endif
  }
  ~NvtxRange() {
#if defined(MCKE_USE_ROCTX)
    roctxRangePop();
#endif
  }
  NvtxRange(const NvtxRange&) = delete;
  NvtxRange& operator=(const NvtxRange&) = delete;
};

struct KernelRecord {
  std::string name;
  std::string variant;
  double median_ms = 0.0;
  double min_ms = 0.0;
  std::uint64_t flops = 0;   // ideal (algorithmic)
  std::uint64_t bytes = 0;   // ideal (compulsory)
  int iterations = 1;
  int stream_idx = 0;
  [[nodiscard]] double seconds() const { return median_ms * 1e-3; }
  [[nodiscard]] double tflops() const {
    return seconds() > 0 ? static_cast<double>(flops) / seconds() / 1e12 : 0.0;
  }
  [[nodiscard]] double gb_per_s() const {
    return seconds() > 0 ? static_cast<double>(bytes) / seconds() / 1e9 : 0.0;
  }
  [[nodiscard]] double arithmetic_intensity() const {
    return bytes ? static_cast<double>(flops) / static_cast<double>(bytes) : 0.0;
  }
};

struct Roofline {
  double peak_tflops = 0.0;
  double peak_gb_s = 0.0;
  [[nodiscard]] double ridge_point_ai() const {
    return peak_gb_s > 0 ? (peak_tflops * 1e12) / (peak_gb_s * 1e9) : 0.0;
  }
  [[nodiscard]] double attainable_tflops(double ai) const {
    const double bw_bound = ai * peak_gb_s * 1e9 / 1e12;
    return bw_bound < peak_tflops ? bw_bound : peak_tflops;
  }
  [[nodiscard]] bool memory_bound(double ai) const { return ai < ridge_point_ai(); }
  [[nodiscard]] double efficiency(const KernelRecord& r) const {
    const double att = attainable_tflops(r.arithmetic_intensity());
    return att > 0 ? r.tflops() / att : 0.0;
  }
};

// Dense fp32 peak of a CDNA part: CUs x clock x 256 flops per clock per CU (the
// fp32 matrix rate, equal to the packed-fp32 vector rate); 157.3 TFLOP/s on
// MI355X at 2.4 GHz.
[[nodiscard]] double theoretical_peak_f32_tflops(const DeviceInfo& d);

// The roofline of an MI355X from AMD's published figures.
[[nodiscard]] inline Roofline mi355x_roofline() { return Roofline{157.3, 8000.0}; }

class Profiler {
 public:
  template <typename EnqueueFn>
  [[nodiscard]] StatusOr<KernelRecord> time_op(const std::string& name, const std::string& variant,
                                               const rt::Stream& stream, std::uint64_t flops,
                                               std::uint64_t bytes, int warmup, int iters,
                                               EnqueueFn&& fn);
  void add(KernelRecord r) { records_.push_back(std::move(r)); }
  [[nodiscard]] const std::vector<KernelRecord>& records() const { return records_; }
  [[nodiscard]] Status write_csv(const std::string& path, const Roofline& rl) const;
  [[nodiscard]] std::string summary_table(const Roofline& rl) const;

 private:
  std::vector<KernelRecord> records_;
};

template <typename EnqueueFn>
StatusOr<KernelRecord> Profiler::time_op(const std::string& name, const std::string& variant,
                                         const rt::Stream& stream, std::uint64_t flops,
                                         std::uint64_t bytes, int warmup, int iters,
                                         EnqueueFn&& fn) {
  if (iters <= 0) return InvalidArgumentError("time_op: iters must be > 0");
  for (int i = 0; i < warmup; ++i) MCKE_RETURN_IF_ERROR(fn(stream));
  std::vector<rt::Event> marks;
  marks.reserve(static_cast<std::size_t>(iters) * 2);
  for (int i = 0; i < 2 * iters; ++i) {
    MCKE_ASSIGN_OR_RETURN(rt::Event e, rt::Event::create(rt::Event::Purpose::kTiming));
    marks.push_back(std::move(e));
  }
  for (int i = 0; i < iters; ++i) {
    MCKE_RETURN_IF_ERROR(marks[2 * i].record(stream));
    MCKE_RETURN_IF_ERROR(fn(stream));
    MCKE_RETURN_IF_ERROR(marks[2 * i + 1].record(stream));
  }
  MCKE_RETURN_IF_ERROR(stream.synchronize());
  std::vector<double> ms;
  ms.reserve(static_cast<std::size_t>(iters));
  for (int i = 0; i < iters; ++i) {
    MCKE_ASSIGN_OR_RETURN(float t, rt::Event::elapsed_ms(marks[2 * i], marks[2 * i + 1]));
    ms.push_back(static_cast<double>(t));
  }
  std::sort(ms.begin(), ms.end());
  KernelRecord r;
  r.name = name;
  r.variant = variant;
  r.median_ms = ms[ms.size() / 2];
  r.min_ms = ms.front();
  r.flops = flops;
  r.bytes = bytes;
  r.iterations = iters;
  records_.push_back(r);
  return r;
}

}  // namespace mcke
