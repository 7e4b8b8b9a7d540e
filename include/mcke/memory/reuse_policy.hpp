// mcke/memory/reuse_policy.hpp -- when may a block freed on one stream be handed
// to an allocation on another?  Same rule and enumerators as the reference's
// include/mcke/memory/reuse_policy.hpp:52-124:
//   same stream            always (stream order already serialises the uses);
//   kSameStreamOnly        never across streams;
//   kCoarseStreamPoll      once the freeing stream has drained (stream query);
//   kPerFreeEvent          once an event recorded at the free has completed.
#pragma once

#include <cstdint>

#include "mcke/runtime/stream.hpp"

namespace mcke {

inline constexpr std::uint32_t kNoEventSlot = 0xFFFFFFFFu;

enum class ReusePolicy : std::uint8_t { kSameStreamOnly, kCoarseStreamPoll, kPerFreeEvent };

[[nodiscard]] constexpr const char* to_string(ReusePolicy p) noexcept {
  switch (p) {
    case ReusePolicy::kSameStreamOnly: return "same_stream_only";
    case ReusePolicy::kCoarseStreamPoll: return "coarse_stream_poll";
    case ReusePolicy::kPerFreeEvent: return "per_free_event";
  }
  return "unknown";
}

template <typename StreamProbe, typename EventProbe>
[[nodiscard]] bool pending_reusable(ReusePolicy policy, rt::StreamHandle entry_stream,
                                    std::uint32_t event_slot, rt::StreamHandle for_stream,
                                    StreamProbe&& stream_probe, EventProbe&& event_probe) {
  if (entry_stream == for_stream) return true;
  switch (policy) {
    case ReusePolicy::kSameStreamOnly: return false;
    case ReusePolicy::kCoarseStreamPoll: return stream_probe(entry_stream);
    case ReusePolicy::kPerFreeEvent: return event_probe(event_slot);
  }
  return false;
}

}  // namespace mcke
