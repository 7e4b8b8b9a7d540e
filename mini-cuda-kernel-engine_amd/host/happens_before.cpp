// happens_before.cpp -- vector clocks over a multi-stream schedule.
//
// Contract: reference include/mcke/graph/happens_before.hpp:108-153 (built from
// a schedule's stream, issue index, recorded event and waited events per node,
// and an issue order; precedes() answers in O(1)).
//
// Construction here is two passes.  The first checks the schedule's shape: every
// stream's issue indices, sorted, must be exactly 0, 1, 2, ... (so each node has
// one predecessor on its stream, or none), and every event has at most one
// recorder.  The second walks the issue order once; a node's clock is the
// element-wise maximum of the clocks of its stream predecessor and of the
// recorders of the events it waits on, with its own stream's entry then set to
// its issue index.  Every node a clock is taken from must already have been
// walked, which is what makes the issue order executable.
#include "mcke/graph/happens_before.hpp"

#include <algorithm>
#include <sstream>
#include <utility>

namespace mcke {

namespace {

Status malformed(const std::string& why) {
  return InvalidArgumentError("HappensBefore: malformed schedule: " + why);
}

}  // namespace

StatusOr<HappensBefore> HappensBefore::build(std::size_t num_streams,
                                             const std::vector<std::uint16_t>& stream_of,
                                             const std::vector<std::uint32_t>& issue_of,
                                             const std::vector<std::uint32_t>& record_of,
                                             const std::vector<std::vector<std::uint32_t>>& waits_of,
                                             const std::vector<std::uint32_t>& order) {
  const std::size_t n = stream_of.size();
  if (num_streams == 0) return malformed("zero streams");
  if (issue_of.size() != n || record_of.size() != n || waits_of.size() != n || order.size() != n) {
    std::ostringstream os;
    os << "expected " << n << " entries per node, got issue " << issue_of.size() << ", record "
       << record_of.size() << ", waits " << waits_of.size() << ", order " << order.size();
    return malformed(os.str());
  }

  // Pass 1a: each stream's (issue index, node) pairs, sorted, must be dense.
  std::vector<std::vector<std::pair<std::uint32_t, std::uint32_t>>> lane(num_streams);
  for (std::uint32_t v = 0; v < n; ++v) {
    if (stream_of[v] >= num_streams) {
      std::ostringstream os;
      os << "node " << v << " names stream " << stream_of[v] << " (have " << num_streams << ")";
      return malformed(os.str());
    }
    lane[stream_of[v]].emplace_back(issue_of[v], v);
  }
  // prev_on_lane[v]: the node issued just before v on v's stream, or v itself.
  std::vector<std::uint32_t> prev_on_lane(n);
  for (std::size_t s = 0; s < num_streams; ++s) {
    auto& members = lane[s];
    std::sort(members.begin(), members.end());
    for (std::size_t k = 0; k < members.size(); ++k) {
      if (members[k].first != k) {
        std::ostringstream os;
        os << "stream " << s << " expects issue index " << k << " next but node "
           << members[k].second << " has " << members[k].first
           << (k > 0 && members[k].first == members[k - 1].first ? " (a duplicate)" : " (a gap)");
        return malformed(os.str());
      }
      prev_on_lane[members[k].second] = k ? members[k - 1].second : members[k].second;
    }
  }

  // Pass 1b: one recorder per event.
  std::uint32_t max_event = 0;
  for (std::uint32_t e : record_of)
    if (e != kNoEventId) max_event = std::max(max_event, e + 1);
  std::vector<std::uint32_t> recorder(max_event, kNoEventId);
  for (std::uint32_t v = 0; v < n; ++v) {
    const std::uint32_t e = record_of[v];
    if (e == kNoEventId) continue;
    if (recorder[e] != kNoEventId) {
      std::ostringstream os;
      os << "event " << e << " has two recorders, nodes " << recorder[e] << " and " << v;
      return malformed(os.str());
    }
    recorder[e] = v;
  }

  // Pass 2: clocks along the issue order.
  HappensBefore hb;
  hb.num_streams_ = num_streams;
  hb.stream_of_ = stream_of;
  hb.issue_of_ = issue_of;
  hb.clock_.assign(n * num_streams, -1);
  std::vector<char> walked(n, 0);
  for (std::uint32_t v : order) {
    if (v >= n || walked[v]) {
      std::ostringstream os;
      os << "issue order lists node " << v << (v < n ? " twice" : ", which does not exist");
      return malformed(os.str());
    }
    std::int64_t* mine = &hb.clock_[static_cast<std::size_t>(v) * num_streams];
    auto absorb = [&](std::uint32_t src, const char* via) -> Status {
      if (!walked[src]) {
        std::ostringstream os;
        os << "node " << v << " needs node " << src << " (" << via << ") but comes first in the "
           << "issue order";
        return malformed(os.str());
      }
      const std::int64_t* theirs = &hb.clock_[static_cast<std::size_t>(src) * num_streams];
      for (std::size_t s = 0; s < num_streams; ++s) mine[s] = std::max(mine[s], theirs[s]);
      return OkStatus();
    };
    if (prev_on_lane[v] != v) MCKE_RETURN_IF_ERROR(absorb(prev_on_lane[v], "stream order"));
    for (std::uint32_t e : waits_of[v]) {
      if (e >= recorder.size() || recorder[e] == kNoEventId) {
        std::ostringstream os;
        os << "node " << v << " waits on event " << e << ", which nothing records";
        return malformed(os.str());
      }
      MCKE_RETURN_IF_ERROR(absorb(recorder[e], "event wait"));
    }
    mine[stream_of[v]] = static_cast<std::int64_t>(issue_of[v]);
    walked[v] = 1;
  }
  return hb;
}

std::string HappensBefore::describe_pair(std::uint32_t u, std::uint32_t v) const {
  const char* rel = precedes(u, v) ? "before" : precedes(v, u) ? "after" : "unordered with";
  std::ostringstream os;
  os << "#" << u << "@s" << stream_of_[u] << "." << issue_of_[u] << " is " << rel << " #" << v << "@s"
     << stream_of_[v] << "." << issue_of_[v] << " (#" << v << " has seen s" << stream_of_[u]
     << " up to issue " << clock_[static_cast<std::size_t>(v) * num_streams_ + stream_of_[u]] << ")";
  return os.str();
}

}  // namespace mcke
