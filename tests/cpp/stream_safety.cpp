// stream_safety.cpp -- GPU race test of stream-ordered reuse in the allocators:
// the MI355X counterpart of the reference's tests/test_stream_safety.cu, with its
// own HIP kernels (stream_safety_kernels.hip).
//
// One trial: block B1 is allocated on stream s1 and filled with 1.0; a reader on
// s1 then waits for a flag the host sets later (a bounded poll), and counts the
// elements of B1 that are not 1.0.  While the reader waits, the host frees B1
// (stream-ordered, on s1), allocates B2 of the same size on s2, fills B2 with
// -7.0 on s2, waits for s2, and only then releases the flag.  If the allocator
// handed B1's bytes to s2 while s1 still used them, the reader counts -7.0s:
// CORRUPT.  Arms:
//   naive_pool              a pool that always returns its one block: must come
//                           out CORRUPT (proves the harness can see the race);
//   buddy / freelist x {same_stream_only, coarse_poll, per_free_event}:
//                           must come out CLEAN, with the freed block parked and
//                           not reclaimed by the s2 allocation, and, after s1
//                           drains, reclaimed by the next s2 allocation except
//                           under same_stream_only;
//   buddy same-stream control  B2 on s1: the same bytes (aliased) and still CLEAN,
//                           because s1's queue orders the reader before the fill;
// plus a check that RawDeviceAllocator's hipFree leaves the stream idle.
//
// Built into tests/cpp/bin/libstream_safety.so with its kernels and run in-process
// by tests/test_gpu_stream_safety.py through mcke_test_stream_safety(): 0 when every
// arm met its expectation in every trial, 1 when one did not, 2 on a harness
// error, 77 without a GPU; the report is written to the caller's buffer.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <functional>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "mcke/core/device.hpp"
#include "mcke/memory/allocator.hpp"
#include "mcke/memory/buddy_allocator.hpp"
#include "mcke/memory/freelist_allocator.hpp"
#include "mcke/runtime/stream.hpp"
#include "mcke_amd.h"

extern "C" {
int ss_fill_f32(float* buf, int n, float v, void* stream);
int ss_gated_read_f32(const float* buf, int n, const int* gate_dev, unsigned* bad_out, int* gate_seen_out,
                      void* stream);
int ss_gate_create(int** host_ptr, int** dev_ptr);
int ss_gate_destroy(int* host_ptr);
}

using namespace mcke;

namespace {

constexpr int kElems = 512 * 1024;   // 2 MiB of f32
constexpr std::size_t kBytes = kElems * sizeof(float);
constexpr std::size_t kSlabBytes = std::size_t{32} << 20;
constexpr int kTrials = 10;

[[noreturn]] void die(const char* what) {
  throw std::runtime_error(std::string("harness error: ") + what + " (" + mcke_last_error() + ")");
}

std::string g_report;
void out(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void out(const char* fmt, ...) {
  char line[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(line, sizeof line, fmt, ap);
  va_end(ap);
  g_report += line;
}

class NaivePool final : public DeviceAllocator {
 public:
  explicit NaivePool(std::size_t bytes) : bytes_(bytes) {
    if (mcke_rt_malloc(&block_, bytes)) die("naive pool malloc");
  }
  ~NaivePool() override { (void)mcke_rt_free(block_); }
  StatusOr<Allocation> allocate(std::size_t bytes, rt::StreamHandle) override {
    if (held_ || bytes > bytes_) return OutOfMemoryError("naive_pool: busy");
    held_ = true;
    Allocation a;
    a.ptr = block_;
    a.bytes = bytes_;
    a.requested_bytes = bytes;
    return a;
  }
  Status deallocate(const Allocation&, rt::StreamHandle) override {
    held_ = false;   // no stream ordering at all: the bug under test
    return OkStatus();
  }
  [[nodiscard]] AllocatorStats stats() const override { return {}; }
  [[nodiscard]] std::string_view name() const override { return "naive_pool"; }

 private:
  void* block_ = nullptr;
  std::size_t bytes_ = 0;
  bool held_ = false;
};

struct Gate {
  int* host = nullptr;
  int* dev = nullptr;
  void arm() { __atomic_store_n(host, 0, __ATOMIC_SEQ_CST); }
  void release() { __atomic_store_n(host, 1, __ATOMIC_SEQ_CST); }
};

struct Arm {
  std::string name;
  bool expect_corrupt = false;
  bool control = false;                         // allocate B2 on s1
  std::function<std::unique_ptr<DeviceAllocator>()> make;
  std::function<std::size_t(const DeviceAllocator&)> parked;   // null: not a pool
  ReusePolicy policy = ReusePolicy::kCoarseStreamPoll;
};

struct Trial {
  bool corrupt = false, harness_bug = false, aliased = false;
  bool refused = false, reclaimed_after_drain = false;
};

Trial run_trial(const Arm& arm, rt::Stream& s1, rt::Stream& s2, Gate& gate, unsigned* d_bad, int* d_seen) {
  Trial r;
  auto alloc = arm.make();
  // Warm-up: one block through each stream, then everything settled.
  for (rt::Stream* s : {&s1, &s2}) {
    auto w = alloc->allocate(kBytes, s->native());
    if (w.ok()) (void)alloc->deallocate(*w, s->native());
    if (!s->synchronize().ok()) die("warm-up sync");
  }
  (void)alloc->settle_pending();

  gate.arm();
  const unsigned zero_u = 0;
  const int zero = 0;
  if (mcke_rt_memcpy_async(d_bad, &zero_u, sizeof zero_u, 0, s1.native()) ||
      mcke_rt_memcpy_async(d_seen, &zero, sizeof zero, 0, s1.native()))
    die("reset counters");
  auto b1 = alloc->allocate(kBytes, s1.native());
  if (!b1.ok()) die("allocate B1");
  if (ss_fill_f32(static_cast<float*>(b1->ptr), kElems, 1.0f, s1.native())) die("fill B1");
  if (ss_gated_read_f32(static_cast<const float*>(b1->ptr), kElems, gate.dev, d_bad, d_seen, s1.native()))
    die("gated read");
  const std::size_t parked_before = arm.parked ? arm.parked(*alloc) : 0;
  if (!alloc->deallocate(*b1, s1.native()).ok()) die("free B1");
  const std::size_t parked_after_free = arm.parked ? arm.parked(*alloc) : 0;
  rt::Stream& reuse_on = arm.control ? s1 : s2;
  auto b2 = alloc->allocate(kBytes, reuse_on.native());
  if (!b2.ok()) die("allocate B2");
  const std::size_t parked_after_alloc = arm.parked ? arm.parked(*alloc) : 0;
  r.aliased = b2->ptr == b1->ptr;
  r.refused = arm.parked && !arm.control && parked_after_free == parked_before + 1 &&
              parked_after_alloc == parked_after_free;
  if (ss_fill_f32(static_cast<float*>(b2->ptr), kElems, -7.0f, reuse_on.native())) die("fill B2");
  if (!arm.control && !s2.synchronize().ok()) die("sync s2");
  gate.release();
  if (!s1.synchronize().ok()) die("sync s1");
  unsigned bad = 0;
  int seen = 0;
  if (mcke_rt_memcpy_async(&bad, d_bad, sizeof bad, 1, nullptr) ||
      mcke_rt_memcpy_async(&seen, d_seen, sizeof seen, 1, nullptr) || mcke_rt_device_synchronize())
    die("read counters");
  r.harness_bug = seen == 0;   // the reader gave up waiting: no race window was observed
  r.corrupt = bad != 0;
  if (arm.parked && !arm.control) {
    const std::size_t before = arm.parked(*alloc);
    auto b3 = alloc->allocate(kBytes, s2.native());
    if (b3.ok()) {
      r.reclaimed_after_drain = arm.parked(*alloc) < before;
      (void)alloc->deallocate(*b3, s2.native());
    }
  }
  (void)alloc->deallocate(*b2, reuse_on.native());
  if (!s1.synchronize().ok() || !s2.synchronize().ok()) die("final sync");
  return r;
}

bool raw_free_leaves_stream_idle(rt::Stream& s1, Gate& gate, unsigned* d_bad, int* d_seen) {
  RawDeviceAllocator alloc;
  gate.arm();
  auto b = alloc.allocate(kBytes, s1.native());
  if (!b.ok()) die("raw allocate");
  if (ss_fill_f32(static_cast<float*>(b->ptr), kElems, 1.0f, s1.native())) die("raw fill");
  if (ss_gated_read_f32(static_cast<const float*>(b->ptr), kElems, gate.dev, d_bad, d_seen, s1.native()))
    die("raw gated read");
  gate.release();
  if (!alloc.deallocate(*b, s1.native()).ok()) die("raw free");
  const bool idle = rt::stream_query(s1.native());
  if (!s1.synchronize().ok()) die("raw sync");
  return idle;
}

int run_all() {
  if (device_count() == 0) {
    out("no HIP device: skipped\n");
    return 77;
  }
  if (!set_device(0).ok()) die("set_device");
  auto s1r = rt::Stream::create();
  auto s2r = rt::Stream::create();
  if (!s1r.ok() || !s2r.ok()) die("stream create");
  rt::Stream s1 = std::move(*s1r), s2 = std::move(*s2r);
  Gate gate;
  if (ss_gate_create(&gate.host, &gate.dev)) die("gate create");
  void* d_bad = nullptr;
  void* d_seen = nullptr;
  if (mcke_rt_malloc(&d_bad, 256) || mcke_rt_malloc(&d_seen, 256)) die("counter malloc");

  auto buddy_with = [](ReusePolicy p) {
    return [p]() -> std::unique_ptr<DeviceAllocator> {
      BuddyConfig c;
      c.initial_slab_bytes = kSlabBytes;
      c.max_total_bytes = kSlabBytes;
      c.large_alloc_threshold = SIZE_MAX;
      c.reuse_policy = p;
      auto a = std::make_unique<BuddyAllocator>(c);
      if (!a->reserve(kSlabBytes).ok()) die("buddy reserve");
      return a;
    };
  };
  auto freelist_with = [](ReusePolicy p) {
    return [p]() -> std::unique_ptr<DeviceAllocator> {
      FreeListConfig c;
      c.slab_bytes = kSlabBytes;
      c.max_total_bytes = kSlabBytes;
      c.large_alloc_threshold = std::size_t{16} << 20;
      c.reuse_policy = p;
      auto a = std::make_unique<FreeListAllocator>(c);
      if (!a->reserve(kSlabBytes).ok()) die("freelist reserve");
      return a;
    };
  };
  auto buddy_parked = [](const DeviceAllocator& a) { return static_cast<const BuddyAllocator&>(a).parked_count(); };
  auto fl_parked = [](const DeviceAllocator& a) { return static_cast<const FreeListAllocator&>(a).parked_count(); };

  std::vector<Arm> arms;
  arms.push_back({"naive_pool", true, false, [] { return std::unique_ptr<DeviceAllocator>(new NaivePool(kBytes)); },
                  nullptr, ReusePolicy::kCoarseStreamPoll});
  const std::pair<const char*, ReusePolicy> pols[] = {{"same_stream_only", ReusePolicy::kSameStreamOnly},
                                                      {"coarse_poll", ReusePolicy::kCoarseStreamPoll},
                                                      {"per_free_event", ReusePolicy::kPerFreeEvent}};
  for (const auto& [pn, pv] : pols) arms.push_back({std::string("buddy/") + pn, false, false, buddy_with(pv), buddy_parked, pv});
  for (const auto& [pn, pv] : pols)
    arms.push_back({std::string("freelist/") + pn, false, false, freelist_with(pv), fl_parked, pv});
  arms.push_back({"buddy/same_stream_control", false, true, buddy_with(ReusePolicy::kCoarseStreamPoll), buddy_parked,
                  ReusePolicy::kCoarseStreamPoll});

  bool all_ok = true;
  out("%-28s %-8s %8s %8s %8s %8s %s\n", "arm", "expect", "corrupt", "aliased", "refused", "reclaim", "result");
  for (const Arm& arm : arms) {
    int corrupt = 0, aliased = 0, refused = 0, reclaimed = 0, harness = 0;
    for (int t = 0; t < kTrials; ++t) {
      const Trial r = run_trial(arm, s1, s2, gate, static_cast<unsigned*>(d_bad), static_cast<int*>(d_seen));
      corrupt += r.corrupt;
      aliased += r.aliased;
      refused += r.refused;
      reclaimed += r.reclaimed_after_drain;
      harness += r.harness_bug;
    }
    bool ok = harness == 0;
    if (arm.expect_corrupt) {
      ok = ok && corrupt == kTrials;
    } else {
      ok = ok && corrupt == 0;
      if (arm.control) ok = ok && aliased == kTrials;
      if (arm.parked && !arm.control) {
        ok = ok && refused == kTrials && aliased == 0;
        if (arm.policy == ReusePolicy::kSameStreamOnly)
          ok = ok && reclaimed == 0;
        else
          ok = ok && reclaimed == kTrials;
      }
    }
    all_ok = all_ok && ok;
    out("%-28s %-8s %5d/%-2d %5d/%-2d %5d/%-2d %5d/%-2d %s%s\n", arm.name.c_str(),
                arm.expect_corrupt ? "CORRUPT" : "CLEAN", corrupt, kTrials, aliased, kTrials, refused, kTrials,
                reclaimed, kTrials, ok ? "PASS" : "FAIL", harness ? " (reader gave up waiting)" : "");
  }
  const bool raw_idle = raw_free_leaves_stream_idle(s1, gate, static_cast<unsigned*>(d_bad), static_cast<int*>(d_seen));
  out("%-28s %-8s %s\n", "raw/hipFree_synchronises", "IDLE", raw_idle ? "PASS" : "FAIL");
  all_ok = all_ok && raw_idle;

  (void)mcke_rt_free(d_bad);
  (void)mcke_rt_free(d_seen);
  (void)ss_gate_destroy(gate.host);
  out("%s\n", all_ok ? "stream safety: all arms PASS" : "stream safety: FAILED");
  return all_ok ? 0 : 1;
}

}  // namespace

extern "C" int mcke_test_stream_safety(char* report, size_t cap) {
  g_report.clear();
  int rc;
  try {
    rc = run_all();
  } catch (const std::exception& e) {
    g_report += std::string(e.what()) + "\n";
    rc = 2;
  }
  if (report && cap) {
    std::strncpy(report, g_report.c_str(), cap - 1);
    report[cap - 1] = '\0';
  }
  return rc;
}
