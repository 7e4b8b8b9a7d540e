// buddy_allocator.cpp -- binary buddy sub-allocation over hipMalloc'd slabs with
// stream-ordered reuse (API of the reference's src/memory/buddy_allocator.cpp;
// the data structures here are this build's own: one ordered free set per order).
#include "mcke/memory/buddy_allocator.hpp"

#include <algorithm>
#include <bit>
#include <sstream>
#include <string>

#include "mcke/core/device.hpp"
#include "mcke/memory/buddy_math.hpp"

namespace mcke {

namespace {
unsigned log2_ceil(std::size_t v) {
  unsigned l = 0;
  while ((std::size_t{1} << l) < v) ++l;
  return l;
}
}  // namespace

BuddyAllocator::BuddyAllocator(BuddyConfig cfg) : cfg_(cfg) {
  if (cfg_.min_block_bytes < kMinBlockBytes) cfg_.min_block_bytes = kMinBlockBytes;
  min_order_ = log2_ceil(cfg_.min_block_bytes);
  if (cfg_.growth_factor < 1.0) cfg_.growth_factor = 1.0;
}

BuddyAllocator::~BuddyAllocator() { release_all(); }

void BuddyAllocator::release_all() noexcept {
  // Work that still uses parked blocks must finish before the slabs go away.
  for (const Parked& p : parked_) wait_stream(p.stream);
  parked_.clear();
  for (auto& kv : bypassed_) raw_free(kv.first);
  bypassed_.clear();
  for (Slab& s : slabs_)
    if (s.base) raw_free(s.base);
  slabs_.clear();
}

StatusOr<void*> BuddyAllocator::raw_alloc(std::size_t bytes) { return raw_device_malloc(bytes); }

void BuddyAllocator::raw_free(void* p) { (void)raw_device_free(p); }

bool BuddyAllocator::event_completed(std::uint32_t event_slot) const {
  if (event_slot >= event_pool_.size()) return true;
  return event_pool_[event_slot].query();
}

void BuddyAllocator::wait_stream(rt::StreamHandle stream) const {
  (void)mcke_rt_stream_synchronize(stream);
}

unsigned BuddyAllocator::order_for(std::size_t bytes) const {
  return std::max(min_order_, log2_ceil(bytes));
}

StatusOr<std::uint32_t> BuddyAllocator::add_slab(std::size_t min_bytes) {
  std::size_t want = slabs_.empty() ? cfg_.initial_slab_bytes : 0;
  if (!slabs_.empty()) {
    std::size_t last = 0;
    for (const Slab& s : slabs_)
      if (s.base) last = std::max(last, s.bytes);
    want = static_cast<std::size_t>(static_cast<double>(last ? last : cfg_.initial_slab_bytes) * cfg_.growth_factor);
  }
  want = std::max(want, min_bytes);
  std::size_t bytes = std::size_t{1} << log2_ceil(std::max(want, cfg_.min_block_bytes));
  if (cfg_.max_total_bytes) {
    // The cap bounds the pool's slabs; allocations that bypass the pool are the
    // caller's own and do not count (reference buddy_allocator.cpp:185-195).
    std::size_t in_slabs = 0;
    for (const Slab& s : slabs_)
      if (s.base) in_slabs += s.bytes;
    if (in_slabs + (std::size_t{1} << log2_ceil(min_bytes)) > cfg_.max_total_bytes)
      return OutOfMemoryError("BuddyAllocator: max_total_bytes (" + std::to_string(cfg_.max_total_bytes) +
                              ") would be exceeded by the pool's slabs (" + std::to_string(in_slabs) +
                              " B reserved in slabs)");
    while (bytes > min_bytes && in_slabs + bytes > cfg_.max_total_bytes) bytes >>= 1;
    if (bytes < min_bytes) bytes = std::size_t{1} << log2_ceil(min_bytes);
  }
  MCKE_ASSIGN_OR_RETURN(void* base, raw_alloc(bytes));
  ++stats_.raw_malloc_calls;
  stats_.bytes_reserved += bytes;
  Slab s;
  s.base = base;
  s.bytes = bytes;
  s.top_order = log2_ceil(bytes);
  s.free_at.resize(s.top_order + 1);
  s.free_at[s.top_order].insert(0);
  // Reuse a dead slot (left by trim) if there is one.
  for (std::size_t i = 0; i < slabs_.size(); ++i)
    if (!slabs_[i].base) {
      slabs_[i] = std::move(s);
      return static_cast<std::uint32_t>(i);
    }
  slabs_.push_back(std::move(s));
  return static_cast<std::uint32_t>(slabs_.size() - 1);
}

Status BuddyAllocator::reserve(std::size_t bytes) {
  MCKE_ASSIGN_OR_RETURN(std::uint32_t id, add_slab(bytes));
  (void)id;
  return OkStatus();
}

// Takes a free block of exactly `order`, splitting a larger one if needed.
bool BuddyAllocator::try_take(unsigned order, std::uint32_t* slab, std::size_t* offset) {
  for (std::uint32_t si = 0; si < slabs_.size(); ++si) {
    Slab& s = slabs_[si];
    if (!s.base || order > s.top_order) continue;
    unsigned o = order;
    while (o <= s.top_order && s.free_at[o].empty()) ++o;
    if (o > s.top_order) continue;
    std::size_t off = *s.free_at[o].begin();   // lowest address first: keeps the top of the slab free
    s.free_at[o].erase(s.free_at[o].begin());
    while (o > order) {
      --o;
      s.free_at[o].insert(off + (std::size_t{1} << o));   // upper half stays free
    }
    s.used_bytes += std::size_t{1} << order;
    *slab = si;
    *offset = off;
    return true;
  }
  return false;
}

void BuddyAllocator::release_block(std::uint32_t slab, std::size_t offset, unsigned order) {
  Slab& s = slabs_[slab];
  s.used_bytes -= std::size_t{1} << order;
  while (order < s.top_order) {
    const std::size_t buddy = offset ^ (std::size_t{1} << order);
    auto it = s.free_at[order].find(buddy);
    if (it == s.free_at[order].end()) break;
    s.free_at[order].erase(it);
    offset = std::min(offset, buddy);
    ++order;
  }
  s.free_at[order].insert(offset);
}

void BuddyAllocator::reclaim(rt::StreamHandle for_stream) {
  auto safe = [&](const Parked& p) {
    return pending_reusable(
        cfg_.reuse_policy, p.stream, p.event_slot, for_stream,
        [&](rt::StreamHandle h) { return stream_completed(h); },
        [&](std::uint32_t e) { return event_completed(e); });
  };
  std::vector<Parked> keep;
  for (const Parked& p : parked_) {
    if (safe(p)) {
      release_block(p.slab, p.offset, p.order);
      if (p.event_slot != kNoEventSlot) free_event_slots_.push_back(p.event_slot);
    } else {
      keep.push_back(p);
    }
  }
  parked_ = std::move(keep);
}

void BuddyAllocator::drain_all_blocking() {
  if (parked_.empty()) return;
  ++stats_.blocking_drains;
  for (const Parked& p : parked_) {
    wait_stream(p.stream);
    release_block(p.slab, p.offset, p.order);
    if (p.event_slot != kNoEventSlot) free_event_slots_.push_back(p.event_slot);
  }
  parked_.clear();
}

// The block's node in heap order over its slab's tree (buddy_math.hpp): level
// top_order - order, index offset >> order within the level.
std::uint32_t BuddyAllocator::node_id(std::uint32_t slab, std::size_t offset, unsigned order) const {
  const unsigned top = slabs_[slab].top_order;
  return static_cast<std::uint32_t>(buddy::node_at(offset, top - order, top));
}

StatusOr<Allocation> BuddyAllocator::allocate(std::size_t bytes, rt::StreamHandle stream) {
  ++stats_.alloc_calls;
  if (bytes == 0) return InvalidArgumentError("BuddyAllocator::allocate: zero bytes");
  if (bytes > cfg_.large_alloc_threshold) {
    auto p = raw_alloc(bytes);
    if (!p.ok()) {
      ++stats_.oom_events;
      return p.status();
    }
    ++stats_.raw_malloc_calls;
    bypassed_[*p] = bytes;
    stats_.bytes_reserved += bytes;
    stats_.bytes_in_use += bytes;
    stats_.bytes_requested += bytes;
    stats_.peak_bytes_in_use = std::max(stats_.peak_bytes_in_use, stats_.bytes_in_use);
    Allocation a;
    a.ptr = *p;
    a.bytes = bytes;
    a.requested_bytes = bytes;
    a.slab_id = kBypassSlabId;
    return a;
  }
  const unsigned order = order_for(bytes);
  const bool had_parked = !parked_.empty();
  reclaim(stream);
  std::uint32_t slab = 0;
  std::size_t off = 0;
  bool ok = try_take(order, &slab, &off);
  if (!ok && !parked_.empty()) {
    drain_all_blocking();
    ok = try_take(order, &slab, &off);
  }
  if (!ok) {
    auto id = add_slab(std::size_t{1} << order);
    if (!id.ok()) {
      ++stats_.oom_events;
      return id.status();
    }
    ok = try_take(order, &slab, &off);
    if (!ok) return InternalError("BuddyAllocator: a fresh slab could not serve the request");
  } else if (had_parked || stats_.free_calls > 0) {
    ++stats_.reuse_hits;
  }
  void* ptr = static_cast<char*>(slabs_[slab].base) + off;
  live_[ptr] = Live{slab, off, order, bytes};
  const std::size_t block = std::size_t{1} << order;
  stats_.bytes_in_use += block;
  stats_.bytes_requested += bytes;
  stats_.peak_bytes_in_use = std::max(stats_.peak_bytes_in_use, stats_.bytes_in_use);
  Allocation a;
  a.ptr = ptr;
  a.bytes = block;
  a.requested_bytes = bytes;
  a.slab_id = slab;
  a.block_id = node_id(slab, off, order);
  return a;
}

Status BuddyAllocator::deallocate(const Allocation& a, rt::StreamHandle stream) {
  if (!a.ptr) return OkStatus();
  ++stats_.free_calls;
  if (auto b = bypassed_.find(a.ptr); b != bypassed_.end()) {
    wait_stream(stream);   // the direct free must not race queued work
    raw_free(a.ptr);
    ++stats_.raw_free_calls;
    stats_.bytes_reserved -= b->second;
    stats_.bytes_in_use -= b->second;
    stats_.bytes_requested -= b->second;
    bypassed_.erase(b);
    return OkStatus();
  }
  // Error codes as the reference's (buddy_allocator.cpp:557-576): a handle that
  // names no live block of this allocator is an invalid argument, a block of one
  // of its slabs that is not live (a double free) a failed precondition.
  auto it = live_.find(a.ptr);
  if (it == live_.end()) {
    const auto p = reinterpret_cast<std::uintptr_t>(a.ptr);
    for (const Slab& s : slabs_) {
      const auto base = reinterpret_cast<std::uintptr_t>(s.base);
      if (s.base && p >= base && p < base + s.bytes)
        return FailedPreconditionError(
            "BuddyAllocator::deallocate: the block at this pointer is not live (double free)");
    }
    return InvalidArgumentError("BuddyAllocator::deallocate: pointer was not allocated here");
  }
  const Live l = it->second;
  if (a.slab_id != l.slab || a.block_id != node_id(l.slab, l.offset, l.order))
    return InvalidArgumentError("BuddyAllocator::deallocate: slab_id " + std::to_string(a.slab_id) +
                                " / block_id " + std::to_string(a.block_id) +
                                " do not name the live block at this pointer");
  live_.erase(it);
  stats_.bytes_in_use -= std::size_t{1} << l.order;
  stats_.bytes_requested -= l.requested;
  Parked p{l.slab, l.offset, l.order, stream, kNoEventSlot};
  if (cfg_.reuse_policy == ReusePolicy::kPerFreeEvent) {
    std::uint32_t slot;
    if (!free_event_slots_.empty()) {
      slot = free_event_slots_.back();
      free_event_slots_.pop_back();
    } else {
      MCKE_ASSIGN_OR_RETURN(rt::Event ev, rt::Event::create(rt::Event::Purpose::kDependency));
      event_pool_.push_back(std::move(ev));
      slot = static_cast<std::uint32_t>(event_pool_.size() - 1);
    }
    MCKE_RETURN_IF_ERROR(event_pool_[slot].record(stream));
    p.event_slot = slot;
  }
  parked_.push_back(p);
  ++stats_.deferred_reuses;
  return OkStatus();
}

Status BuddyAllocator::settle_pending() {
  drain_all_blocking();
  return OkStatus();
}

Status BuddyAllocator::trim() {
  drain_all_blocking();
  for (Slab& s : slabs_) {
    if (!s.base || s.used_bytes != 0) continue;
    raw_free(s.base);
    ++stats_.raw_free_calls;
    stats_.bytes_reserved -= s.bytes;
    s = Slab{};
  }
  return OkStatus();
}

std::size_t BuddyAllocator::largest_free() const {
  std::size_t best = 0;
  for (const Slab& s : slabs_) {
    if (!s.base) continue;
    for (unsigned o = s.top_order + 1; o-- > 0;)
      if (!s.free_at[o].empty()) {
        best = std::max(best, std::size_t{1} << o);
        break;
      }
  }
  return best;
}

AllocatorStats BuddyAllocator::stats() const {
  AllocatorStats s = stats_;
  s.largest_free_block = largest_free();
  return s;
}

Status BuddyAllocator::validate() const {
  for (std::size_t si = 0; si < slabs_.size(); ++si) {
    const Slab& s = slabs_[si];
    if (!s.base) continue;
    // Free blocks + live blocks + parked blocks tile the slab exactly once.
    std::vector<std::pair<std::size_t, std::size_t>> pieces;
    for (unsigned o = 0; o <= s.top_order; ++o)
      for (std::size_t off : s.free_at[o]) {
        if (off % (std::size_t{1} << o) != 0)
          return InternalError("BuddyAllocator::validate: free block misaligned in slab " + std::to_string(si));
        pieces.emplace_back(off, std::size_t{1} << o);
      }
    std::size_t live_bytes = 0;
    for (const auto& kv : live_)
      if (kv.second.slab == si) {
        pieces.emplace_back(kv.second.offset, std::size_t{1} << kv.second.order);
        live_bytes += std::size_t{1} << kv.second.order;
      }
    for (const Parked& p : parked_)
      if (p.slab == si) {
        pieces.emplace_back(p.offset, std::size_t{1} << p.order);
        live_bytes += std::size_t{1} << p.order;
      }
    std::sort(pieces.begin(), pieces.end());
    std::size_t cursor = 0;
    for (const auto& [off, len] : pieces) {
      if (off != cursor)
        return InternalError("BuddyAllocator::validate: slab " + std::to_string(si) + " has a gap or overlap at " +
                             std::to_string(off));
      cursor = off + len;
    }
    if (cursor != s.bytes) return InternalError("BuddyAllocator::validate: slab " + std::to_string(si) + " not covered");
    if (live_bytes != s.used_bytes)
      return InternalError("BuddyAllocator::validate: slab " + std::to_string(si) + " used-byte count drifted");
    // No two free buddies at the same order (they would have merged).
    for (unsigned o = 0; o < s.top_order; ++o)
      for (std::size_t off : s.free_at[o])
        if (s.free_at[o].count(off ^ (std::size_t{1} << o)))
          return InternalError("BuddyAllocator::validate: unmerged free buddies in slab " + std::to_string(si));
  }
  return OkStatus();
}

std::string BuddyAllocator::dump_free_map() const {
  std::ostringstream os;
  for (std::size_t si = 0; si < slabs_.size(); ++si) {
    const Slab& s = slabs_[si];
    if (!s.base) continue;
    os << "slab " << si << " (" << s.bytes << " B, used " << s.used_bytes << " B):";
    for (unsigned o = 0; o <= s.top_order; ++o)
      if (!s.free_at[o].empty()) os << " [2^" << o << " x" << s.free_at[o].size() << "]";
    os << "\n";
  }
  os << "parked " << parked_.size() << ", bypassed " << bypassed_.size() << "\n";
  return os.str();
}

}  // namespace mcke
