// mcke/graph/happens_before.hpp -- the happens-before relation of a multi-stream
// schedule, by vector clocks.
//
// Same API as the reference's include/mcke/graph/happens_before.hpp:108-153.
// Node v's clock has one entry per stream: the highest issue index on that
// stream known to have completed before v starts.  A node inherits the clock of
// its predecessor on its own stream and of the recorders of every event it
// waits on, then sets its own stream's entry to its issue index.  u precedes v
// iff clock[v][stream(u)] >= issue(u).
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "mcke/core/status.hpp"

namespace mcke {

inline constexpr std::uint32_t kNoEventId = 0xFFFFFFFFu;

class HappensBefore {
 public:
  [[nodiscard]] static StatusOr<HappensBefore> build(
      std::size_t num_streams, const std::vector<std::uint16_t>& stream_of,
      const std::vector<std::uint32_t>& issue_of, const std::vector<std::uint32_t>& record_of,
      const std::vector<std::vector<std::uint32_t>>& waits_of,
      const std::vector<std::uint32_t>& order);

  [[nodiscard]] bool precedes(std::uint32_t u, std::uint32_t v) const {
    if (u == v) return false;
    return clock_[static_cast<std::size_t>(v) * num_streams_ + stream_of_[u]] >=
           static_cast<std::int64_t>(issue_of_[u]);
  }
  [[nodiscard]] bool concurrent(std::uint32_t u, std::uint32_t v) const {
    return u != v && !precedes(u, v) && !precedes(v, u);
  }
  [[nodiscard]] std::size_t num_nodes() const noexcept { return issue_of_.size(); }
  [[nodiscard]] std::size_t num_streams() const noexcept { return num_streams_; }
  [[nodiscard]] std::string describe_pair(std::uint32_t u, std::uint32_t v) const;

 private:
  HappensBefore() = default;
  std::size_t num_streams_ = 0;
  std::vector<std::uint16_t> stream_of_;
  std::vector<std::uint32_t> issue_of_;
  std::vector<std::int64_t> clock_;
};

}  // namespace mcke
