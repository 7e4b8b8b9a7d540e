// freelist_allocator.cpp -- size-class caching over bump-carved hipMalloc'd slabs
// with stream-ordered reuse (API of the reference's src/memory/freelist_allocator.cpp;
// the bookkeeping here is this build's own: per-slab live counts, one LIFO cache per
// class, parked frees shared in form with the buddy allocator).
#include "mcke/memory/freelist_allocator.hpp"

#include <algorithm>
#include <sstream>

#include "mcke/core/device.hpp"

namespace mcke {

namespace {
bool pow2(std::size_t v) { return v != 0 && (v & (v - 1)) == 0; }
unsigned log2_ceil(std::size_t v) {
  unsigned l = 0;
  while ((std::size_t{1} << l) < v) ++l;
  return l;
}
}  // namespace

FreeListAllocator::FreeListAllocator(FreeListConfig cfg) : cfg_(cfg) {
  config_status_ = check_config();
  if (!config_status_.ok()) return;
  n_linear_ = cfg_.small_large_split / cfg_.small_class_granularity;
  split_log2_ = log2_ceil(cfg_.small_large_split);
  cache_.resize(size_class_of(cfg_.large_alloc_threshold) + 1);
}

FreeListAllocator::~FreeListAllocator() { release_all(); }

void FreeListAllocator::release_all() noexcept {
  // Work that still uses parked blocks must finish before the slabs go away.
  for (const Parked& p : parked_) wait_stream(p.stream);
  parked_.clear();
  for (auto& kv : bypassed_) raw_free(kv.first);
  bypassed_.clear();
  for (Slab& s : slabs_)
    if (s.base) raw_free(s.base);
  slabs_.clear();
}

Status FreeListAllocator::check_config() const {
  const std::size_t g = cfg_.small_class_granularity, split = cfg_.small_large_split;
  if (!pow2(g) || g < kDeviceAlignment)
    return InvalidArgumentError("FreeListAllocator: small_class_granularity must be a power of two >= " +
                                std::to_string(kDeviceAlignment) + ", got " + std::to_string(g));
  if (!pow2(split) || split < g)
    return InvalidArgumentError("FreeListAllocator: small_large_split must be a power of two >= the "
                                "granularity, got " + std::to_string(split));
  if (cfg_.large_alloc_threshold < split)
    return InvalidArgumentError("FreeListAllocator: large_alloc_threshold must be >= small_large_split");
  if (cfg_.slab_bytes < g) return InvalidArgumentError("FreeListAllocator: slab_bytes smaller than one class");
  return OkStatus();
}

StatusOr<void*> FreeListAllocator::raw_alloc(std::size_t bytes) { return raw_device_malloc(bytes); }

void FreeListAllocator::raw_free(void* p) { (void)raw_device_free(p); }

bool FreeListAllocator::event_completed(std::uint32_t event_slot) const {
  if (event_slot >= event_pool_.size()) return true;
  return event_pool_[event_slot].query();
}

void FreeListAllocator::wait_stream(rt::StreamHandle stream) const {
  (void)mcke_rt_stream_synchronize(stream);
}

std::size_t FreeListAllocator::size_class_of(std::size_t bytes) const {
  if (bytes == 0) return 0;
  if (bytes <= cfg_.small_large_split)
    return (bytes + cfg_.small_class_granularity - 1) / cfg_.small_class_granularity - 1;
  // Powers of two above the split: 2^(split_log2 + 1) is class n_linear_.
  return n_linear_ + (log2_ceil(bytes) - (split_log2_ + 1));
}

std::size_t FreeListAllocator::class_block_bytes(std::size_t cls) const {
  if (cls < n_linear_) return (cls + 1) * cfg_.small_class_granularity;
  return std::size_t{1} << (split_log2_ + 1 + (cls - n_linear_));
}

StatusOr<std::uint32_t> FreeListAllocator::add_slab(std::size_t bytes) {
  // The cap bounds the pool's slabs; bypass allocations do not count (reference
  // freelist_allocator.cpp:134-143).
  std::size_t in_slabs = 0;
  for (const Slab& s : slabs_)
    if (s.base) in_slabs += s.bytes;
  if (cfg_.max_total_bytes && in_slabs + bytes > cfg_.max_total_bytes)
    return OutOfMemoryError("FreeListAllocator: a slab of " + std::to_string(bytes) +
                            " B would exceed max_total_bytes (" + std::to_string(cfg_.max_total_bytes) +
                            ") with " + std::to_string(in_slabs) + " B already in slabs");
  MCKE_ASSIGN_OR_RETURN(void* base, raw_alloc(bytes));
  ++stats_.raw_malloc_calls;
  stats_.bytes_reserved += bytes;
  Slab s;
  s.base = static_cast<char*>(base);
  s.bytes = bytes;
  for (std::size_t i = 0; i < slabs_.size(); ++i)   // reuse a slot released by trim()
    if (!slabs_[i].base) {
      slabs_[i] = s;
      return static_cast<std::uint32_t>(i);
    }
  slabs_.push_back(s);
  return static_cast<std::uint32_t>(slabs_.size() - 1);
}

Status FreeListAllocator::reserve(std::size_t bytes) {
  MCKE_RETURN_IF_ERROR(config_status_);
  if (bytes == 0) return InvalidArgumentError("FreeListAllocator::reserve: zero bytes");
  for (const Slab& s : slabs_)
    if (s.base && s.bytes >= bytes) return OkStatus();
  MCKE_ASSIGN_OR_RETURN(std::uint32_t id, add_slab(std::max(bytes, cfg_.slab_bytes)));
  (void)id;
  return OkStatus();
}

bool FreeListAllocator::take_cached(std::size_t cls, Block* out) {
  auto& lst = cache_[cls];
  if (lst.empty()) return false;
  *out = lst.back();
  lst.pop_back();
  return true;
}

// Head of a cached block of a larger class (at most 8 classes up), when the
// remainder is exactly one block of some class, which is cached in turn.
bool FreeListAllocator::take_split(std::size_t cls, Block* out) {
  const std::size_t need = class_block_bytes(cls);
  const std::size_t last = std::min(cache_.size(), cls + 9);
  for (std::size_t c = cls + 1; c < last; ++c) {
    if (cache_[c].empty()) continue;
    const std::size_t rest = class_block_bytes(c) - need;
    if (rest == 0 || class_block_bytes(size_class_of(rest)) != rest) continue;
    const Block whole = cache_[c].back();
    cache_[c].pop_back();
    cache(Block{whole.ptr + need, whole.slab}, rest);
    *out = whole;
    return true;
  }
  return false;
}

bool FreeListAllocator::carve(std::size_t block_bytes, Block* out) {
  for (std::uint32_t si = 0; si < slabs_.size(); ++si) {
    Slab& s = slabs_[si];
    if (!s.base || s.bytes - s.carved < block_bytes) continue;
    *out = Block{s.base + s.carved, si};
    s.carved += block_bytes;
    return true;
  }
  return false;
}

void FreeListAllocator::cache(const Block& b, std::size_t block_bytes) {
  cache_[size_class_of(block_bytes)].push_back(b);
}

void FreeListAllocator::reclaim(rt::StreamHandle for_stream) {
  std::size_t keep = 0;
  for (const Parked& p : parked_) {
    const bool safe = pending_reusable(
        cfg_.reuse_policy, p.stream, p.event_slot, for_stream,
        [&](rt::StreamHandle h) { return stream_completed(h); },
        [&](std::uint32_t e) { return event_completed(e); });
    if (safe) {
      cache(p.block, p.block_bytes);
      if (p.event_slot != kNoEventSlot) free_event_slots_.push_back(p.event_slot);
    } else {
      parked_[keep++] = p;
    }
  }
  parked_.resize(keep);
}

void FreeListAllocator::drain_all_blocking() {
  if (parked_.empty()) return;
  ++stats_.blocking_drains;
  for (const Parked& p : parked_) {
    wait_stream(p.stream);
    cache(p.block, p.block_bytes);
    if (p.event_slot != kNoEventSlot) free_event_slots_.push_back(p.event_slot);
  }
  parked_.clear();
}

StatusOr<Allocation> FreeListAllocator::allocate_bypass(std::size_t bytes) {
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

StatusOr<Allocation> FreeListAllocator::allocate(std::size_t bytes, rt::StreamHandle stream) {
  ++stats_.alloc_calls;
  MCKE_RETURN_IF_ERROR(config_status_);
  if (bytes == 0) return InvalidArgumentError("FreeListAllocator::allocate: zero bytes");
  if (bytes > cfg_.large_alloc_threshold) return allocate_bypass(bytes);
  const std::size_t cls = size_class_of(bytes);
  const std::size_t block_bytes = class_block_bytes(cls);
  reclaim(stream);
  Block b;
  bool reused = take_cached(cls, &b) || (cfg_.split_large_blocks && take_split(cls, &b));
  bool ok = reused || carve(block_bytes, &b);
  if (!ok) {
    auto id = add_slab(std::max(cfg_.slab_bytes, block_bytes));
    if (id.ok()) {
      ok = carve(block_bytes, &b);
    } else if (!parked_.empty()) {
      // No memory left to grow into: wait for the parked blocks, then retry the cache.
      drain_all_blocking();
      reused = take_cached(cls, &b) || (cfg_.split_large_blocks && take_split(cls, &b));
      ok = reused;
    }
    if (!ok) {
      ++stats_.oom_events;
      const Status why = id.ok() ? InternalError("FreeListAllocator: a fresh slab could not serve the request")
                                 : id.status();
      return OutOfMemoryError("FreeListAllocator: no block of " + std::to_string(block_bytes) + " B for a " +
                              std::to_string(bytes) + " B request (" + std::string(why.message()) +
                              "); largest free block " + std::to_string(largest_free()) + " B");
    }
  }
  if (reused) ++stats_.reuse_hits;
  ++slabs_[b.slab].live_blocks;
  live_[b.ptr] = LiveBlock{b.slab, block_bytes, bytes};
  stats_.bytes_in_use += block_bytes;
  stats_.bytes_requested += bytes;
  stats_.peak_bytes_in_use = std::max(stats_.peak_bytes_in_use, stats_.bytes_in_use);
  Allocation a;
  a.ptr = b.ptr;
  a.bytes = block_bytes;
  a.requested_bytes = bytes;
  a.slab_id = b.slab;
  a.block_id = static_cast<std::uint32_t>(cls);
  return a;
}

std::uint32_t FreeListAllocator::record_free_event(rt::StreamHandle stream) {
  std::uint32_t slot;
  if (!free_event_slots_.empty()) {
    slot = free_event_slots_.back();
    free_event_slots_.pop_back();
  } else {
    auto ev = rt::Event::create(rt::Event::Purpose::kDependency);
    if (!ev.ok()) return kNoEventSlot;
    event_pool_.push_back(std::move(*ev));
    slot = static_cast<std::uint32_t>(event_pool_.size() - 1);
  }
  if (!event_pool_[slot].record(stream).ok()) {
    free_event_slots_.push_back(slot);
    return kNoEventSlot;
  }
  return slot;
}

Status FreeListAllocator::deallocate(const Allocation& a, rt::StreamHandle stream) {
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
  auto it = live_.find(a.ptr);
  if (it == live_.end())
    return FailedPreconditionError("FreeListAllocator::deallocate: pointer is not live here "
                                   "(double free, or never allocated by this allocator)");
  const LiveBlock l = it->second;
  live_.erase(it);
  --slabs_[l.slab].live_blocks;
  stats_.bytes_in_use -= l.block_bytes;
  stats_.bytes_requested -= l.requested;
  const Block blk{static_cast<char*>(a.ptr), l.slab};
  std::uint32_t slot = kNoEventSlot;
  if (cfg_.reuse_policy == ReusePolicy::kPerFreeEvent) {
    slot = record_free_event(stream);
    if (slot == kNoEventSlot) {
      // No event to watch: wait for the stream here rather than guess.
      wait_stream(stream);
      ++stats_.blocking_drains;
      cache(blk, l.block_bytes);
      return OkStatus();
    }
  }
  parked_.push_back(Parked{blk, l.block_bytes, stream, slot});
  ++stats_.deferred_reuses;
  return OkStatus();
}

Status FreeListAllocator::settle_pending() {
  drain_all_blocking();
  return OkStatus();
}

Status FreeListAllocator::trim() {
  drain_all_blocking();
  for (std::uint32_t si = 0; si < slabs_.size(); ++si) {
    Slab& s = slabs_[si];
    if (!s.base || s.live_blocks != 0) continue;
    for (auto& lst : cache_)
      lst.erase(std::remove_if(lst.begin(), lst.end(), [&](const Block& b) { return b.slab == si; }),
                lst.end());
    raw_free(s.base);
    ++stats_.raw_free_calls;
    stats_.bytes_reserved -= s.bytes;
    s = Slab{};
  }
  return OkStatus();
}

std::size_t FreeListAllocator::largest_free() const {
  std::size_t best = 0;
  for (std::size_t c = cache_.size(); c-- > 0;)
    if (!cache_[c].empty()) {
      best = class_block_bytes(c);
      break;
    }
  for (const Slab& s : slabs_) {
    if (!s.base) continue;
    const std::size_t tail = s.bytes - s.carved;
    // The largest class block the uncarved tail can still hold.
    for (std::size_t c = cache_.size(); c-- > 0;)
      if (class_block_bytes(c) <= tail) {
        best = std::max(best, class_block_bytes(c));
        break;
      }
  }
  return best;
}

AllocatorStats FreeListAllocator::stats() const {
  AllocatorStats s = stats_;
  s.largest_free_block = config_status_.ok() ? largest_free() : 0;
  return s;
}

Status FreeListAllocator::validate() const {
  MCKE_RETURN_IF_ERROR(config_status_);
  // Every live, cached and parked block lies in the carved part of a live slab,
  // no two overlap, and the carved bytes of each slab are exactly accounted for.
  struct Piece {
    std::uint32_t slab;
    std::size_t off, len;
  };
  std::vector<Piece> pieces;
  std::vector<std::size_t> live_count(slabs_.size(), 0);
  std::size_t live_bytes = 0;
  auto add = [&](std::uint32_t si, const void* p, std::size_t len, const char* what) -> Status {
    if (si >= slabs_.size() || !slabs_[si].base)
      return InternalError(std::string("FreeListAllocator::validate: ") + what + " block in a released slab");
    const Slab& s = slabs_[si];
    const auto off = static_cast<std::size_t>(static_cast<const char*>(p) - s.base);
    if (static_cast<const char*>(p) < s.base || off + len > s.carved)
      return InternalError(std::string("FreeListAllocator::validate: ") + what + " block outside the carved part of slab " +
                           std::to_string(si));
    pieces.push_back(Piece{si, off, len});
    return OkStatus();
  };
  for (const auto& [ptr, l] : live_) {
    MCKE_RETURN_IF_ERROR(add(l.slab, ptr, l.block_bytes, "live"));
    ++live_count[l.slab];
    live_bytes += l.block_bytes;
  }
  for (std::size_t c = 0; c < cache_.size(); ++c)
    for (const Block& b : cache_[c]) MCKE_RETURN_IF_ERROR(add(b.slab, b.ptr, class_block_bytes(c), "cached"));
  for (const Parked& p : parked_) MCKE_RETURN_IF_ERROR(add(p.block.slab, p.block.ptr, p.block_bytes, "parked"));
  std::sort(pieces.begin(), pieces.end(), [](const Piece& a, const Piece& b) {
    return a.slab != b.slab ? a.slab < b.slab : a.off < b.off;
  });
  std::vector<std::size_t> covered(slabs_.size(), 0);
  for (std::size_t i = 0; i < pieces.size(); ++i) {
    if (i > 0 && pieces[i].slab == pieces[i - 1].slab && pieces[i - 1].off + pieces[i - 1].len > pieces[i].off)
      return InternalError("FreeListAllocator::validate: overlapping blocks in slab " + std::to_string(pieces[i].slab));
    covered[pieces[i].slab] += pieces[i].len;
  }
  std::size_t bypass_bytes = 0;
  for (const auto& kv : bypassed_) bypass_bytes += kv.second;
  for (std::size_t si = 0; si < slabs_.size(); ++si) {
    if (!slabs_[si].base) continue;
    if (covered[si] != slabs_[si].carved)
      return InternalError("FreeListAllocator::validate: carved bytes of slab " + std::to_string(si) +
                           " are not all accounted for");
    if (live_count[si] != slabs_[si].live_blocks)
      return InternalError("FreeListAllocator::validate: live-block count of slab " + std::to_string(si) + " drifted");
  }
  if (live_bytes + bypass_bytes != stats_.bytes_in_use)
    return InternalError("FreeListAllocator::validate: bytes_in_use drifted");
  return OkStatus();
}

std::string FreeListAllocator::dump_free_map() const {
  std::ostringstream os;
  os << "freelist: " << n_linear_ << " classes of " << cfg_.small_class_granularity << " B up to "
     << cfg_.small_large_split << " B, then powers of two; " << cache_.size() << " classes\n";
  for (std::size_t si = 0; si < slabs_.size(); ++si) {
    const Slab& s = slabs_[si];
    if (!s.base) {
      os << "slab " << si << ": released\n";
      continue;
    }
    os << "slab " << si << " (" << s.bytes << " B): carved " << s.carved << " B, " << s.live_blocks
       << " live blocks\n";
  }
  for (std::size_t c = 0; c < cache_.size(); ++c)
    if (!cache_[c].empty()) os << "class " << c << " (" << class_block_bytes(c) << " B): " << cache_[c].size() << " cached\n";
  os << "live " << live_.size() << ", parked " << parked_.size() << ", bypassed " << bypassed_.size() << "\n";
  return os.str();
}

}  // namespace mcke
