// mcke/memory/freelist_allocator.hpp -- size-class caching allocator over
// bump-carved slabs, with stream-ordered reuse.
//
// Same API as the reference's include/mcke/memory/freelist_allocator.hpp
// (FreeListConfig, reserve, allocate/deallocate, trim, settle_pending, stats,
// validate, size_class_of, class_block_bytes, num_classes, dump_free_map, and the
// overridable completion seams), written here as:
//   * size classes: linear classes of `small_class_granularity` bytes up to
//     `small_large_split`, then one class per power of two up to
//     `large_alloc_threshold`; a request is rounded up to its class's block size;
//   * a block is carved once from a slab (a bump pointer per slab) and is never
//     coalesced: freed blocks are cached per class (LIFO) and handed out again to
//     requests of that class; with `split_large_blocks` a request may cut its block
//     from the head of a cached block of a larger class when the tail is exactly
//     one block of another class;
//   * requests above `large_alloc_threshold` bypass the slabs (one hipMalloc each);
//   * a block freed on stream S is parked until it is safe for the requesting
//     stream (ReusePolicy), exactly as in the buddy allocator; allocate() reclaims
//     safe parked blocks first, then takes a cached block, then splits (if
//     enabled), then carves, then adds a slab, then waits for the parked blocks (a
//     counted blocking drain) and retries the cache, then fails with OutOfMemory;
//   * trim() waits for parked blocks and releases every slab that holds no live
//     block (its cached blocks are dropped with it).
// Trade-off against the buddy allocator: O(1) allocate/free with no splitting or
// merging on the hot path, at the price of internal rounding waste and
// fragmentation across classes (a block freed in one class cannot serve another).
#pragma once

#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "mcke/memory/allocator.hpp"
#include "mcke/memory/reuse_policy.hpp"

namespace mcke {

// Defaults sized for a 288 GB MI355X: 1 GiB slabs, 512-byte classes up to 1 MiB,
// powers of two up to 1 GiB, and only requests above 1 GiB bypass the slabs.
struct FreeListConfig {
  std::size_t slab_bytes = std::size_t{1} << 30;
  std::size_t max_total_bytes = 0;   // cap on the slabs' bytes (0 = unlimited); bypass allocations do not count
  std::size_t small_class_granularity = 512;
  std::size_t small_large_split = std::size_t{1} << 20;
  std::size_t large_alloc_threshold = std::size_t{1} << 30;
  bool split_large_blocks = false;
  ReusePolicy reuse_policy = ReusePolicy::kCoarseStreamPoll;
};

class FreeListAllocator : public DeviceAllocator {
 public:
  explicit FreeListAllocator(FreeListConfig cfg = {});
  ~FreeListAllocator() override;
  FreeListAllocator(const FreeListAllocator&) = delete;
  FreeListAllocator& operator=(const FreeListAllocator&) = delete;

  // Makes sure one slab of at least `bytes` exists (adds one if not).
  [[nodiscard]] Status reserve(std::size_t bytes);
  StatusOr<Allocation> allocate(std::size_t bytes, rt::StreamHandle stream) override;
  Status deallocate(const Allocation& a, rt::StreamHandle stream) override;
  Status trim() override;
  Status settle_pending() override;
  [[nodiscard]] AllocatorStats stats() const override;
  [[nodiscard]] std::string_view name() const override { return "freelist"; }
  [[nodiscard]] Status validate() const override;

  // Class index of a request of `bytes` (bytes <= large_alloc_threshold), and
  // the block size every request of class `cls` receives.
  [[nodiscard]] std::size_t size_class_of(std::size_t bytes) const;
  [[nodiscard]] std::size_t class_block_bytes(std::size_t cls) const;
  [[nodiscard]] std::size_t num_classes() const { return cache_.size(); }
  [[nodiscard]] std::string dump_free_map() const;
  [[nodiscard]] const FreeListConfig& config() const noexcept { return cfg_; }
  // Freed blocks still waiting for their stream or event before reuse.
  [[nodiscard]] std::size_t parked_count() const noexcept { return parked_.size(); }
  // Status of the configuration (every call fails with it when it is invalid).
  [[nodiscard]] Status config_status() const { return config_status_; }

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
    char* base = nullptr;        // nullptr: released by trim(); the index stays reserved
    std::size_t bytes = 0;
    std::size_t carved = 0;      // bump pointer: [0, carved) has been handed out as blocks
    std::size_t live_blocks = 0;
  };
  struct Block {
    char* ptr = nullptr;
    std::uint32_t slab = 0;
  };
  struct LiveBlock {
    std::uint32_t slab = 0;
    std::size_t block_bytes = 0;
    std::size_t requested = 0;
  };
  struct Parked {
    Block block;
    std::size_t block_bytes = 0;
    rt::StreamHandle stream{};
    std::uint32_t event_slot = kNoEventSlot;
  };

  [[nodiscard]] Status check_config() const;
  [[nodiscard]] StatusOr<std::uint32_t> add_slab(std::size_t bytes);
  [[nodiscard]] bool take_cached(std::size_t cls, Block* out);
  [[nodiscard]] bool take_split(std::size_t cls, Block* out);
  [[nodiscard]] bool carve(std::size_t block_bytes, Block* out);
  void cache(const Block& b, std::size_t block_bytes);
  void reclaim(rt::StreamHandle for_stream);
  void drain_all_blocking();
  [[nodiscard]] std::uint32_t record_free_event(rt::StreamHandle stream);
  [[nodiscard]] std::size_t largest_free() const;
  [[nodiscard]] StatusOr<Allocation> allocate_bypass(std::size_t bytes);

  FreeListConfig cfg_;
  Status config_status_;
  std::size_t n_linear_ = 0;      // number of linear classes
  unsigned split_log2_ = 0;       // log2(small_large_split)
  std::vector<Slab> slabs_;
  std::vector<std::vector<Block>> cache_;                  // per class, LIFO
  std::unordered_map<void*, LiveBlock> live_;
  std::unordered_map<void*, std::size_t> bypassed_;
  std::vector<Parked> parked_;
  std::vector<rt::Event> event_pool_;
  std::vector<std::uint32_t> free_event_slots_;
  AllocatorStats stats_{};
};

}  // namespace mcke
