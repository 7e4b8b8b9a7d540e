// mcke/memory/buddy_allocator.hpp -- binary buddy sub-allocator over large slabs,
// with stream-ordered reuse.
//
// Same API as the reference's include/mcke/memory/buddy_allocator.hpp:114-313
// (BuddyConfig, reserve, allocate/deallocate, trim, settle_pending, stats,
// validate, dump_free_map, and the overridable stream/event completion seams),
// written here as:
//   * a slab is one hipMalloc of a power-of-two size; blocks are power-of-two
//     pieces of it, identified by (slab, byte offset, order); free blocks sit in
//     one ordered set per order, and a freed block merges with its buddy
//     (offset ^ size) as long as the buddy is free at the same order;
//   * requests above large_alloc_threshold bypass the slabs (one hipMalloc each);
//   * a block freed on stream S is parked until it is safe for the requesting
//     stream (ReusePolicy); allocate() first reclaims parked blocks that are safe,
//     then splits, then waits for parked blocks (a counted blocking drain), then
//     grows by a new slab (growth_factor, capped by max_total_bytes), then fails
//     with OutOfMemory.
#pragma once

#include <cstdint>
#include <map>
#include <set>
#include <string>
#include <unordered_map>
#include <vector>

#include "mcke/memory/allocator.hpp"
#include "mcke/memory/reuse_policy.hpp"

namespace mcke {

// Defaults sized for a 288 GB MI355X: 1 GiB first slab, doubling growth, and only
// requests above 4 GiB bypass the slabs.
struct BuddyConfig {
  std::size_t initial_slab_bytes = std::size_t{1} << 30;
  std::size_t max_total_bytes = 0;   // cap on the slabs' bytes (0 = unlimited); bypass allocations do not count
  std::size_t min_block_bytes = kMinBlockBytes;
  double growth_factor = 2.0;
  std::size_t large_alloc_threshold = std::size_t{4} << 30;
  ReusePolicy reuse_policy = ReusePolicy::kCoarseStreamPoll;
};

class BuddyAllocator : public DeviceAllocator {
 public:
  explicit BuddyAllocator(BuddyConfig cfg = {});
  ~BuddyAllocator() override;
  BuddyAllocator(const BuddyAllocator&) = delete;
  BuddyAllocator& operator=(const BuddyAllocator&) = delete;

  [[nodiscard]] Status reserve(std::size_t bytes);
  StatusOr<Allocation> allocate(std::size_t bytes, rt::StreamHandle stream) override;
  Status deallocate(const Allocation& a, rt::StreamHandle stream) override;
  Status trim() override;
  Status settle_pending() override;
  [[nodiscard]] AllocatorStats stats() const override;
  [[nodiscard]] std::string_view name() const override { return "buddy"; }
  [[nodiscard]] Status validate() const override;
  [[nodiscard]] std::string dump_free_map() const;
  [[nodiscard]] const BuddyConfig& config() const noexcept { return cfg_; }
  // Freed blocks still waiting for their stream or event before reuse.
  [[nodiscard]] std::size_t parked_count() const noexcept { return parked_.size(); }

 protected:
  // Completion seams (tests substitute fake streams through these).
  [[nodiscard]] virtual bool stream_completed(rt::StreamHandle stream) const {
    return rt::stream_query(stream);
  }
  [[nodiscard]] virtual bool event_completed(std::uint32_t event_slot) const;
  virtual void wait_stream(rt::StreamHandle stream) const;
  // Memory seams (tests substitute host memory through these).
  [[nodiscard]] virtual StatusOr<void*> raw_alloc(std::size_t bytes);
  virtual void raw_free(void* p);
  // Waits for the streams of parked blocks, then returns every slab and bypass
  // allocation through raw_free; idempotent.  The destructor calls it, but a
  // virtual call from a base destructor reaches the base's own seams, so a
  // subclass that overrides wait_stream or raw_free must call release_all() from
  // its own destructor.
  void release_all() noexcept;

 private:
  struct Slab {
    void* base = nullptr;
    std::size_t bytes = 0;      // power of two
    unsigned top_order = 0;     // log2(bytes)
    std::vector<std::set<std::size_t>> free_at;   // free_at[order] = offsets
    std::size_t used_bytes = 0;
  };
  struct Live {
    std::uint32_t slab = 0;
    std::size_t offset = 0;
    unsigned order = 0;
    std::size_t requested = 0;
  };
  struct Parked {
    std::uint32_t slab = 0;
    std::size_t offset = 0;
    unsigned order = 0;
    rt::StreamHandle stream{};
    std::uint32_t event_slot = kNoEventSlot;
  };

  [[nodiscard]] unsigned order_for(std::size_t bytes) const;
  [[nodiscard]] std::uint32_t node_id(std::uint32_t slab, std::size_t offset, unsigned order) const;
  [[nodiscard]] StatusOr<std::uint32_t> add_slab(std::size_t min_bytes);
  [[nodiscard]] bool try_take(unsigned order, std::uint32_t* slab, std::size_t* offset);
  void release_block(std::uint32_t slab, std::size_t offset, unsigned order);
  void reclaim(rt::StreamHandle for_stream);
  void drain_all_blocking();
  [[nodiscard]] std::size_t largest_free() const;

  BuddyConfig cfg_;
  unsigned min_order_ = 8;
  std::vector<Slab> slabs_;
  std::unordered_map<void*, Live> live_;
  std::unordered_map<void*, std::size_t> bypassed_;
  std::vector<Parked> parked_;
  std::vector<rt::Event> event_pool_;
  std::vector<std::uint32_t> free_event_slots_;
  AllocatorStats stats_{};
};

}  // namespace mcke
