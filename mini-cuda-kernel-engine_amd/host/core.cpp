// core.cpp -- device query and raw memory over the C-ABI, the raw allocator,
// the profiler's table/CSV output and the CDNA peak formula.
// Reference counterparts: src/core/device.cpp:56-168, src/memory/allocator.cpp:44-73,
// src/core/profiler.cpp:47-113.
#include <fstream>
#include <iomanip>
#include <sstream>

#include "mcke/core/device.hpp"
#include "mcke/memory/allocator.hpp"
#include "mcke/profiling/profiler.hpp"
#include "mcke_amd.h"

namespace mcke {

namespace {
Status from_rc(int rc, const char* what) {
  if (rc == MCKE_STATUS_OK) return OkStatus();
  return Status(static_cast<StatusCode>(rc), std::string(what) + ": " + mcke_last_error());
}
}  // namespace

std::string DeviceInfo::describe() const {
  std::ostringstream os;
  os << "device " << index << ": " << (name.empty() ? arch : name) << " (" << arch << ")  CUs "
     << sm_count << "  lanes/CU " << max_threads_per_sm << "  LDS/CU " << shared_mem_per_sm
     << " B  HBM " << (global_mem_bytes >> 30) << " GiB  peak " << peak_dram_gb_s() << " GB/s";
  return os.str();
}

DeviceInfo mi355x_device_info() {
  DeviceInfo d;
  d.index = 0;
  d.name = "AMD Instinct MI355X";
  d.arch = "gfx950";
  d.cc_major = 9;
  d.cc_minor = 5;
  d.sm_count = 256;
  d.max_threads_per_sm = 2048;
  d.max_threads_per_block = 1024;
  d.warps_per_sm = 2048 / kWarpSize;
  d.regs_per_sm = 4 * 512 * kWarpSize;
  d.regs_per_block = 512 * kWarpSize * 4;
  d.max_blocks_per_sm = 32;
  d.global_mem_bytes = std::size_t{288} << 30;
  d.shared_mem_per_block = 160 * 1024;
  d.shared_mem_per_block_optin = 160 * 1024;
  d.shared_mem_per_sm = 160 * 1024;
  d.l2_cache_bytes = 4 << 20;
  d.memory_bus_width_bits = 8192;
  d.clock_khz = 2400000;
  d.published_peak_dram_gb_s = 8000.0;
  return d;
}

int device_count() {
  int n = 0;
  if (mcke_rt_get_device_count(&n) != MCKE_STATUS_OK) return 0;
  return n;
}

StatusOr<DeviceInfo> query_device(int index) {
  mcke_device_info c{};
  MCKE_RETURN_IF_ERROR(from_rc(mcke_rt_query_device(index, &c), "query_device"));
  DeviceInfo d;
  d.index = c.ordinal;
  d.name = c.name;
  d.arch = c.arch;
  d.cc_major = c.cc_major;
  d.cc_minor = c.cc_minor;
  d.sm_count = c.sm_count;
  d.max_threads_per_sm = c.max_threads_per_sm;
  d.max_threads_per_block = c.max_threads_per_block;
  d.warps_per_sm = c.warp_size > 0 ? c.max_threads_per_sm / c.warp_size : 0;
  d.regs_per_sm = c.regs_per_sm;
  d.regs_per_block = c.regs_per_block;
  d.max_blocks_per_sm = c.max_blocks_per_sm;
  d.global_mem_bytes = c.total_global_mem;
  d.shared_mem_per_block = c.shared_mem_per_block;
  d.shared_mem_per_block_optin = c.shared_mem_per_block;
  d.shared_mem_per_sm = c.shared_mem_per_sm;
  d.l2_cache_bytes = static_cast<int>(c.l2_cache_bytes);
  d.memory_bus_width_bits = c.memory_bus_width_bits;
  d.memory_clock_khz = c.memory_clock_khz;
  d.clock_khz = c.clock_khz;
  d.published_peak_dram_gb_s = c.peak_dram_gb_s;
  return d;
}

Status set_device(int index) { return from_rc(mcke_rt_set_device(index), "set_device"); }

StatusOr<void*> raw_device_malloc(std::size_t bytes) {
  void* p = nullptr;
  MCKE_RETURN_IF_ERROR(from_rc(mcke_rt_malloc(&p, bytes), "raw_device_malloc"));
  return p;
}

Status raw_device_free(void* ptr) { return from_rc(mcke_rt_free(ptr), "raw_device_free"); }

std::string AllocatorStats::to_string() const {
  std::ostringstream os;
  os << "allocs " << alloc_calls << "  frees " << free_calls << "  hipMalloc " << raw_malloc_calls
     << "  hipFree " << raw_free_calls << "  reuse_hits " << reuse_hits << "  deferred "
     << deferred_reuses << "  drains " << blocking_drains << "  oom " << oom_events
     << "  reserved " << bytes_reserved << " B  in_use " << bytes_in_use << " B  peak "
     << peak_bytes_in_use << " B  largest_free " << largest_free_block << " B";
  return os.str();
}

StatusOr<Allocation> RawDeviceAllocator::allocate(std::size_t bytes, rt::StreamHandle stream) {
  (void)stream;
  ++stats_.alloc_calls;
  if (bytes == 0) return InvalidArgumentError("RawDeviceAllocator::allocate: zero bytes");
  auto p = raw_device_malloc(bytes);
  if (!p.ok()) {
    ++stats_.oom_events;
    return p.status();
  }
  ++stats_.raw_malloc_calls;
  Allocation a;
  a.ptr = *p;
  a.bytes = bytes;
  a.requested_bytes = bytes;
  a.slab_id = kBypassSlabId;
  stats_.bytes_reserved += bytes;
  stats_.bytes_in_use += bytes;
  stats_.bytes_requested += bytes;
  stats_.peak_bytes_in_use = std::max(stats_.peak_bytes_in_use, stats_.bytes_in_use);
  return a;
}

Status RawDeviceAllocator::deallocate(const Allocation& a, rt::StreamHandle stream) {
  (void)stream;
  if (!a.ptr) return OkStatus();
  ++stats_.free_calls;
  // hipFree waits for the device, so no stream-ordered hazard remains afterwards.
  MCKE_RETURN_IF_ERROR(raw_device_free(a.ptr));
  ++stats_.raw_free_calls;
  stats_.bytes_reserved -= a.bytes;
  stats_.bytes_in_use -= a.bytes;
  stats_.bytes_requested -= a.requested_bytes;
  return OkStatus();
}

double theoretical_peak_f32_tflops(const DeviceInfo& d) {
  return static_cast<double>(d.sm_count) * static_cast<double>(d.clock_khz) * 1e3 * 256.0 / 1e12;
}

std::string Profiler::summary_table(const Roofline& rl) const {
  std::ostringstream os;
  os << std::left << std::setw(22) << "kernel" << std::setw(30) << "variant" << std::right
     << std::setw(10) << "med_ms" << std::setw(10) << "min_ms" << std::setw(10) << "GB/s"
     << std::setw(10) << "TFLOP/s" << std::setw(8) << "AI" << std::setw(10) << "%peak"
     << "  bound\n"
     << std::string(117, '-') << '\n'
     << std::fixed;
  for (const auto& r : records_) {
    const double ai = r.arithmetic_intensity();
    os << std::left << std::setw(22) << r.name << std::setw(30) << r.variant << std::right
       << std::setprecision(3) << std::setw(10) << r.median_ms << std::setw(10) << r.min_ms
       << std::setw(10) << std::setprecision(1) << r.gb_per_s() << std::setw(10)
       << std::setprecision(3) << r.tflops() << std::setw(8) << std::setprecision(2) << ai
       << std::setw(9) << std::setprecision(1) << rl.efficiency(r) * 100.0 << "%"
       << "  " << (rl.memory_bound(ai) ? "memory" : "compute") << '\n';
  }
  return os.str();
}

Status Profiler::write_csv(const std::string& path, const Roofline& rl) const {
  std::ofstream f(path);
  if (!f) return InternalError("write_csv: cannot open " + path);
  f << "kernel,variant,median_ms,min_ms,iterations,ideal_flops,ideal_bytes,achieved_gb_s,"
       "achieved_tflops,arithmetic_intensity,attainable_tflops,efficiency_pct,bound\n";
  for (const auto& r : records_) {
    const double ai = r.arithmetic_intensity();
    f << r.name << ',' << r.variant << ',' << r.median_ms << ',' << r.min_ms << ',' << r.iterations
      << ',' << r.flops << ',' << r.bytes << ',' << r.gb_per_s() << ',' << r.tflops() << ',' << ai
      << ',' << rl.attainable_tflops(ai) << ',' << rl.efficiency(r) * 100.0 << ','
      << (rl.memory_bound(ai) ? "memory" : "compute") << '\n';
  }
  return OkStatus();
}

}  // namespace mcke
