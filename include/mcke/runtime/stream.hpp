// mcke/runtime/stream.hpp -- rt::Stream / rt::Event over the HIP runtime.
//
// Mirrors the reference's include/mcke/runtime/stream.hpp:82-306 (RAII streams
// and events, raw-handle probes) on the C-ABI's mcke_rt_* entry points, so this
// header needs no HIP headers.  StreamHandle and EventHandle are the HIP handle
// types (hipStream_t is `ihipStream_t*`, hipEvent_t is `ihipEvent_t*`), so they
// pass straight through to HIP code.
//
// Streams are created non-blocking and always at the default priority: the
// StreamPriority argument of Stream::create is accepted for source compatibility
// and ignored, because work on streams of different priorities has been seen to
// hang on this platform.
#pragma once

#include <utility>

#include "mcke/core/status.hpp"
#include "mcke_amd.h"

struct ihipStream_t;
struct ihipEvent_t;

namespace mcke::rt {

using StreamHandle = ihipStream_t*;
using EventHandle = ihipEvent_t*;

namespace detail {
inline Status from_rc(int rc, const char* what) {
  if (rc == MCKE_STATUS_OK) return OkStatus();
  return Status(static_cast<StatusCode>(rc), std::string(what) + ": " + mcke_last_error());
}
}  // namespace detail

enum class StreamPriority { kHigh, kNormal, kLow };

// Raw-handle probes (stream.hpp:82-113): true when all work is complete.
[[nodiscard]] inline bool stream_query(StreamHandle h) {
  int done = 0;
  return mcke_rt_stream_query(h, &done) == MCKE_STATUS_OK && done != 0;
}
[[nodiscard]] inline bool event_record(EventHandle e, StreamHandle s) {
  return mcke_rt_event_record(e, s) == MCKE_STATUS_OK;
}
[[nodiscard]] inline bool event_query(EventHandle e) {
  int done = 0;
  return mcke_rt_event_query(e, &done) == MCKE_STATUS_OK && done != 0;
}
inline void event_synchronize(EventHandle e) { (void)mcke_rt_event_synchronize(e); }

class Event;

class Stream {
 public:
  static Stream default_stream() { return Stream(StreamHandle{}, false); }
  [[nodiscard]] static StatusOr<Stream> create(StreamPriority prio = StreamPriority::kNormal) {
    (void)prio;
    void* h = nullptr;
    MCKE_RETURN_IF_ERROR(detail::from_rc(mcke_rt_stream_create(&h), "Stream::create"));
    return Stream(static_cast<StreamHandle>(h), true);
  }
  Stream(const Stream&) = delete;
  Stream& operator=(const Stream&) = delete;
  Stream(Stream&& o) noexcept : handle_(o.handle_), owned_(o.owned_) { o.owned_ = false; }
  Stream& operator=(Stream&& o) noexcept {
    if (this != &o) {
      destroy();
      handle_ = o.handle_;
      owned_ = o.owned_;
      o.owned_ = false;
    }
    return *this;
  }
  ~Stream() { destroy(); }

  [[nodiscard]] StreamHandle native() const noexcept { return handle_; }
  Status synchronize() const {
    return detail::from_rc(mcke_rt_stream_synchronize(handle_), "Stream::synchronize");
  }
  [[nodiscard]] bool query() const { return stream_query(handle_); }
  Status wait(const Event& e);

 private:
  Stream(StreamHandle h, bool owned) : handle_(h), owned_(owned) {}
  void destroy() {
    if (owned_ && handle_) (void)mcke_rt_stream_destroy(handle_);
    owned_ = false;
  }
  StreamHandle handle_{};
  bool owned_ = false;
};

class Event {
 public:
  enum class Purpose { kDependency, kTiming };
  [[nodiscard]] static StatusOr<Event> create(Purpose purpose = Purpose::kDependency) {
    void* h = nullptr;
    MCKE_RETURN_IF_ERROR(detail::from_rc(
        mcke_rt_event_create(&h, purpose == Purpose::kTiming ? 1 : 0), "Event::create"));
    return Event(static_cast<EventHandle>(h));
  }
  Event(const Event&) = delete;
  Event& operator=(const Event&) = delete;
  Event(Event&& o) noexcept : handle_(o.handle_) { o.handle_ = EventHandle{}; }
  Event& operator=(Event&& o) noexcept {
    if (this != &o) {
      destroy();
      handle_ = o.handle_;
      o.handle_ = EventHandle{};
    }
    return *this;
  }
  ~Event() { destroy(); }

  [[nodiscard]] EventHandle native() const noexcept { return handle_; }
  Status record(const Stream& s) { return record(s.native()); }
  Status record(StreamHandle s) {
    return detail::from_rc(mcke_rt_event_record(handle_, s), "Event::record");
  }
  Status synchronize() const {
    return detail::from_rc(mcke_rt_event_synchronize(handle_), "Event::synchronize");
  }
  [[nodiscard]] bool query() const { return event_query(handle_); }
  [[nodiscard]] static StatusOr<float> elapsed_ms(const Event& start, const Event& stop) {
    float ms = 0.f;
    MCKE_RETURN_IF_ERROR(detail::from_rc(
        mcke_rt_event_elapsed_ms(start.native(), stop.native(), &ms), "Event::elapsed_ms"));
    return ms;
  }

 private:
  explicit Event(EventHandle h) : handle_(h) {}
  void destroy() {
    if (handle_) (void)mcke_rt_event_destroy(handle_);
    handle_ = EventHandle{};
  }
  EventHandle handle_{};
};

inline Status Stream::wait(const Event& e) {
  return detail::from_rc(mcke_rt_stream_wait_event(handle_, e.native()), "Stream::wait");
}

}  // namespace mcke::rt
