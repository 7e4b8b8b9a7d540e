// happens_before.cpp -- vector clocks over a stream schedule
// (reference src/graph/happens_before.cpp:20-137).
#include "mcke/graph/happens_before.hpp"

#include <algorithm>
#include <sstream>

namespace mcke {

StatusOr<HappensBefore> HappensBefore::build(std::size_t num_streams,
                                             const std::vector<std::uint16_t>& stream_of,
                                             const std::vector<std::uint32_t>& issue_of,
                                             const std::vector<std::uint32_t>& record_of,
                                             const std::vector<std::vector<std::uint32_t>>& waits_of,
                                             const std::vector<std::uint32_t>& order) {
  const std::size_t n = stream_of.size();
  if (num_streams == 0) return InvalidArgumentError("HappensBefore::build: num_streams must be > 0");
  if (issue_of.size() != n || record_of.size() != n || waits_of.size() != n)
    return InvalidArgumentError("HappensBefore::build: per-node arrays disagree in length");
  if (order.size() != n) return InvalidArgumentError("HappensBefore::build: order length != node count");

  // Which node records each event (exactly one).
  std::vector<std::uint32_t> recorder;
  for (std::size_t i = 0; i < n; ++i) {
    if (stream_of[i] >= num_streams)
      return InvalidArgumentError("HappensBefore::build: node " + std::to_string(i) + " is on stream " +
                                  std::to_string(stream_of[i]) + " of " + std::to_string(num_streams));
    const std::uint32_t e = record_of[i];
    if (e == kNoEventId) continue;
    if (e >= recorder.size()) recorder.resize(e + 1, kNoEventId);
    if (recorder[e] != kNoEventId)
      return InvalidArgumentError("HappensBefore::build: event " + std::to_string(e) +
                                  " is recorded by nodes " + std::to_string(recorder[e]) + " and " +
                                  std::to_string(i));
    recorder[e] = static_cast<std::uint32_t>(i);
  }

  // Per stream: node at each issue index (must be dense).
  std::vector<std::vector<std::uint32_t>> at(num_streams);
  for (std::size_t i = 0; i < n; ++i) {
    auto& col = at[stream_of[i]];
    if (col.size() <= issue_of[i]) col.resize(issue_of[i] + 1, kNoEventId);
    if (col[issue_of[i]] != kNoEventId)
      return InvalidArgumentError("HappensBefore::build: nodes " + std::to_string(col[issue_of[i]]) +
                                  " and " + std::to_string(i) + " share issue index " +
                                  std::to_string(issue_of[i]) + " on stream " + std::to_string(stream_of[i]));
    col[issue_of[i]] = static_cast<std::uint32_t>(i);
  }
  for (std::size_t s = 0; s < num_streams; ++s)
    for (std::size_t k = 0; k < at[s].size(); ++k)
      if (at[s][k] == kNoEventId)
        return InvalidArgumentError("HappensBefore::build: stream " + std::to_string(s) +
                                    " has no node at issue index " + std::to_string(k));

  HappensBefore hb;
  hb.num_streams_ = num_streams;
  hb.stream_of_ = stream_of;
  hb.issue_of_ = issue_of;
  hb.clock_.assign(n * num_streams, -1);
  std::vector<bool> done(n, false);
  for (std::uint32_t v : order) {
    if (v >= n) return InvalidArgumentError("HappensBefore::build: order names node " + std::to_string(v));
    std::int64_t* cv = &hb.clock_[static_cast<std::size_t>(v) * num_streams];
    auto join = [&](std::uint32_t u) -> Status {
      if (!done[u])
        return InvalidArgumentError("HappensBefore::build: node " + std::to_string(v) +
                                    " depends on node " + std::to_string(u) + " which is issued later");
      const std::int64_t* cu = &hb.clock_[static_cast<std::size_t>(u) * num_streams];
      for (std::size_t s = 0; s < num_streams; ++s) cv[s] = std::max(cv[s], cu[s]);
      return OkStatus();
    };
    if (issue_of[v] > 0) MCKE_RETURN_IF_ERROR(join(at[stream_of[v]][issue_of[v] - 1]));
    for (std::uint32_t e : waits_of[v]) {
      if (e >= recorder.size() || recorder[e] == kNoEventId)
        return InvalidArgumentError("HappensBefore::build: node " + std::to_string(v) + " waits on event " +
                                    std::to_string(e) + " which no node records");
      MCKE_RETURN_IF_ERROR(join(recorder[e]));
    }
    cv[stream_of[v]] = static_cast<std::int64_t>(issue_of[v]);
    done[v] = true;
  }
  return hb;
}

std::string HappensBefore::describe_pair(std::uint32_t u, std::uint32_t v) const {
  std::ostringstream os;
  os << "node " << u << " (stream " << stream_of_[u] << ", issue " << issue_of_[u] << ") and node " << v
     << " (stream " << stream_of_[v] << ", issue " << issue_of_[v] << "): ";
  if (precedes(u, v)) os << u << " happens-before " << v;
  else if (precedes(v, u)) os << v << " happens-before " << u;
  else os << "CONCURRENT";
  os << "; clock[" << v << "][s" << stream_of_[u] << "] = "
     << clock_[static_cast<std::size_t>(v) * num_streams_ + stream_of_[u]] << " vs issue[" << u
     << "] = " << issue_of_[u];
  return os.str();
}

}  // namespace mcke
