// mcke/memory/allocator.hpp -- device allocator interface and the raw allocator.
//
// Same API as the reference's include/mcke/memory/allocator.hpp:107-230:
// Allocation, AllocatorStats, the abstract DeviceAllocator (stream-ordered
// allocate/deallocate, trim, settle_pending, stats, validate) and
// RawDeviceAllocator, which makes one hipMalloc per allocation and one hipFree
// per deallocation.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <string_view>

#include "mcke/core/config.hpp"
#include "mcke/core/status.hpp"
#include "mcke/runtime/stream.hpp"

namespace mcke {

inline constexpr std::uint32_t kBypassSlabId = 0xFFFFFFFFu;

struct Allocation {
  void* ptr = nullptr;
  std::size_t bytes = 0;            // usable size of the block
  std::size_t requested_bytes = 0;  // what the caller asked for
  std::uint32_t slab_id = 0;
  std::uint32_t block_id = 0;
  [[nodiscard]] bool valid() const noexcept { return ptr != nullptr; }
  [[nodiscard]] std::size_t internal_waste() const noexcept { return bytes - requested_bytes; }
};

struct AllocatorStats {
  std::uint64_t alloc_calls = 0;
  std::uint64_t free_calls = 0;
  std::uint64_t raw_malloc_calls = 0;   // hipMalloc calls actually made
  std::uint64_t raw_free_calls = 0;
  std::uint64_t oom_events = 0;
  std::uint64_t deferred_reuses = 0;    // frees parked until their stream/event completes
  std::uint64_t blocking_drains = 0;    // host waits taken to reclaim parked blocks
  std::uint64_t reuse_hits = 0;         // allocations served from previously freed blocks
  std::size_t bytes_reserved = 0;
  std::size_t bytes_in_use = 0;
  std::size_t bytes_requested = 0;
  std::size_t peak_bytes_in_use = 0;
  std::size_t largest_free_block = 0;
  [[nodiscard]] std::size_t internal_waste() const noexcept {
    return bytes_in_use >= bytes_requested ? bytes_in_use - bytes_requested : 0;
  }
  [[nodiscard]] double utilisation() const noexcept {
    return bytes_reserved ? static_cast<double>(bytes_requested) / static_cast<double>(bytes_reserved) : 0.0;
  }
  [[nodiscard]] std::string to_string() const;
};

class DeviceAllocator {
 public:
  virtual ~DeviceAllocator() = default;
  [[nodiscard]] virtual StatusOr<Allocation> allocate(std::size_t bytes, rt::StreamHandle stream) = 0;
  virtual Status deallocate(const Allocation& a, rt::StreamHandle stream) = 0;
  virtual Status trim() { return OkStatus(); }
  virtual Status settle_pending() { return OkStatus(); }
  [[nodiscard]] virtual AllocatorStats stats() const = 0;
  [[nodiscard]] virtual std::string_view name() const = 0;
  [[nodiscard]] virtual Status validate() const { return OkStatus(); }
};

class RawDeviceAllocator final : public DeviceAllocator {
 public:
  StatusOr<Allocation> allocate(std::size_t bytes, rt::StreamHandle stream) override;
  Status deallocate(const Allocation& a, rt::StreamHandle stream) override;
  [[nodiscard]] AllocatorStats stats() const override { return stats_; }
  [[nodiscard]] std::string_view name() const override { return "raw(hipMalloc)"; }

 private:
  AllocatorStats stats_{};
};

}  // namespace mcke
