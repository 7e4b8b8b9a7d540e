// mcke/core/device.hpp -- device snapshot, selection and raw device memory.
//
// Mirrors the reference's include/mcke/core/device.hpp:29-136 and
// src/core/device.cpp:56-168 on the C-ABI (mcke_rt_query_device, mcke_rt_malloc,
// ...).  Field names follow the reference; the values are CDNA's: sm_count is
// the number of compute units, warps_per_sm counts 64-lane wavefronts, and
// peak_dram_gb_s() is the part's published HBM figure rather than the reference's
// DDR formula (which does not describe HBM3E).
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>

#include "mcke/core/config.hpp"
#include "mcke/core/status.hpp"

namespace mcke {

struct DeviceInfo {
  int index = 0;
  std::string name = "unknown";
  std::string arch;                 // gcnArchName, e.g. "gfx950:sramecc+:xnack-"
  int cc_major = 0;
  int cc_minor = 0;
  int sm_count = 0;                 // compute units
  int max_threads_per_sm = 0;
  int max_threads_per_block = 0;
  int warps_per_sm = 0;             // max_threads_per_sm / kWarpSize
  int regs_per_sm = 0;
  int regs_per_block = 0;
  int max_blocks_per_sm = 0;
  std::size_t global_mem_bytes = 0;
  std::size_t shared_mem_per_block = 0;
  std::size_t shared_mem_per_block_optin = 0;
  std::size_t shared_mem_per_sm = 0;   // LDS per CU
  int l2_cache_bytes = 0;
  int memory_bus_width_bits = 0;
  int memory_clock_khz = 0;
  int clock_khz = 0;
  double published_peak_dram_gb_s = 0.0;

  [[nodiscard]] double peak_dram_gb_s() const { return published_peak_dram_gb_s; }
  [[nodiscard]] int compute_capability() const { return cc_major * 10 + cc_minor; }
  [[nodiscard]] std::string describe() const;
};

// A gfx950 (MI355X) description for host-only planning and tests: 256 CUs,
// 2048 lanes and 160 KiB LDS per CU, 512 unified VGPRs per lane, 8 TB/s HBM.
[[nodiscard]] DeviceInfo mi355x_device_info();

[[nodiscard]] int device_count();
[[nodiscard]] StatusOr<DeviceInfo> query_device(int index = 0);
Status set_device(int index);
[[nodiscard]] StatusOr<void*> raw_device_malloc(std::size_t bytes);
Status raw_device_free(void* ptr);

}  // namespace mcke
