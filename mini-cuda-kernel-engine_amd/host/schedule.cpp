// schedule.cpp -- stream assignment policies and cross-stream events
// (reference src/graph/schedule.cpp:27-301).
#include "mcke/graph/schedule.hpp"

#include <algorithm>
#include <sstream>

#include "mcke/graph/cost_model.hpp"

namespace mcke {

StatusOr<StreamAssignment> plan_streams(const Graph& g, SchedulePolicy policy, int num_streams,
                                        const Roofline& rl) {
  if (num_streams < 1)
    return InvalidArgumentError("plan_streams: num_streams must be >= 1, got " + std::to_string(num_streams));
  if (!g.finalized()) return FailedPreconditionError("plan_streams: call Graph::finalize() first");
  MCKE_ASSIGN_OR_RETURN(std::vector<NodeId> topo, g.topological_order());

  StreamAssignment sa;
  std::vector<std::uint32_t> idx_of(g.num_nodes(), kNoEventId);   // NodeId -> scheduled index
  for (NodeId n : topo) {
    if (g.node(n).is_dead) continue;
    idx_of[n] = static_cast<std::uint32_t>(sa.nodes.size());
    sa.nodes.push_back(n);
  }
  const std::size_t S = sa.nodes.size();
  if (S == 0) return InvalidArgumentError("plan_streams: every node is dead");
  sa.num_streams_requested = static_cast<std::size_t>(num_streams);
  sa.stream_of.assign(S, 0);
  sa.issue_of.assign(S, 0);
  sa.record_of.assign(S, kNoEventId);
  sa.waits_of.assign(S, {});
  sa.order.resize(S);
  for (std::size_t i = 0; i < S; ++i) sa.order[i] = static_cast<std::uint32_t>(i);

  std::vector<double> cost_ms(S, 0.0);
  for (std::size_t i = 0; i < S; ++i) {
    const Node& nd = g.node(sa.nodes[i]);
    if (nd.op) cost_ms[i] = plan_cost_ms(nd.op->cost(g.input_shapes(sa.nodes[i])), rl);
  }

  // dep[i]: scheduled indices that node i must wait for (same stream or not).
  std::vector<std::vector<std::uint32_t>> dep(S);
  const int K = std::min<int>(num_streams, static_cast<int>(S));
  switch (policy) {
    case SchedulePolicy::kSequential:
      break;   // one stream: stream order is the topological order
    case SchedulePolicy::kLevelParallel: {
      MCKE_ASSIGN_OR_RETURN(std::vector<std::vector<NodeId>> lv, g.levels());
      std::vector<std::vector<std::uint32_t>> levels;
      for (const auto& l : lv) {
        std::vector<std::uint32_t> live;
        for (NodeId n : l)
          if (idx_of[n] != kNoEventId) live.push_back(idx_of[n]);
        std::sort(live.begin(), live.end());
        if (!live.empty()) levels.push_back(std::move(live));
      }
      for (const auto& l : levels)
        for (std::size_t j = 0; j < l.size(); ++j) sa.stream_of[l[j]] = static_cast<std::uint16_t>(j % K);
      // Barrier between consecutive levels: the first node of level d+1 on each
      // stream waits for the last node of level d on every other stream.
      for (std::size_t d = 0; d + 1 < levels.size(); ++d) {
        std::vector<std::uint32_t> last(K, kNoEventId), first(K, kNoEventId);
        for (std::uint32_t i : levels[d]) {
          auto& x = last[sa.stream_of[i]];
          if (x == kNoEventId || i > x) x = i;
        }
        for (std::uint32_t i : levels[d + 1]) {
          auto& x = first[sa.stream_of[i]];
          if (x == kNoEventId || i < x) x = i;
        }
        for (int t = 0; t < K; ++t) {
          if (first[t] == kNoEventId) continue;
          for (int s = 0; s < K; ++s)
            if (s != t && last[s] != kNoEventId) dep[first[t]].push_back(last[s]);
        }
      }
      break;
    }
    case SchedulePolicy::kChainGreedy: {
      std::vector<double> load(K, 0.0);
      std::vector<bool> continued(S, false);
      for (std::size_t i = 0; i < S; ++i) {
        std::vector<std::uint32_t> preds;
        for (NodeId p : g.node(sa.nodes[i]).preds)
          if (idx_of[p] != kNoEventId) preds.push_back(idx_of[p]);
        if (preds.size() == 1 && !continued[preds[0]]) {
          sa.stream_of[i] = sa.stream_of[preds[0]];
          continued[preds[0]] = true;
        } else {
          sa.stream_of[i] = static_cast<std::uint16_t>(std::min_element(load.begin(), load.end()) - load.begin());
        }
        load[sa.stream_of[i]] += cost_ms[i];
        dep[i] = preds;
      }
      sa.stream_load_ms = load;
      break;
    }
  }

  // Issue indices; renumber streams densely if some were never used.
  {
    std::vector<std::uint32_t> next(K, 0);
    std::vector<int> remap(K, -1);
    int used = 0;
    for (std::size_t i = 0; i < S; ++i)
      if (remap[sa.stream_of[i]] < 0) remap[sa.stream_of[i]] = used++;
    std::vector<double> load(used, 0.0);
    for (std::size_t i = 0; i < S; ++i) {
      const int s = remap[sa.stream_of[i]];
      sa.stream_of[i] = static_cast<std::uint16_t>(s);
      sa.issue_of[i] = next[s]++;
      load[s] += cost_ms[i];
    }
    sa.num_streams_used = static_cast<std::size_t>(used);
    sa.stream_load_ms = load;
  }

  // Events: one per producer that another stream waits on; waits deduplicated
  // per consuming stream.
  std::vector<bool> recorded(S, false);
  for (std::size_t i = 0; i < S; ++i)
    for (std::uint32_t p : dep[i])
      if (sa.stream_of[p] != sa.stream_of[i]) recorded[p] = true;
  std::uint32_t next_event = 0;
  for (std::size_t i = 0; i < S; ++i)
    if (recorded[i]) sa.record_of[i] = next_event++;
  sa.num_events = next_event;
  std::vector<std::vector<std::uint32_t>> seen(sa.num_streams_used);
  for (std::size_t i = 0; i < S; ++i) {
    const std::uint16_t t = sa.stream_of[i];
    for (std::uint32_t p : dep[i]) {
      if (sa.stream_of[p] == t) continue;
      ++sa.waits_raw;
      const std::uint32_t e = sa.record_of[p];
      if (std::find(seen[t].begin(), seen[t].end(), e) != seen[t].end()) continue;
      seen[t].push_back(e);
      sa.waits_of[i].push_back(e);
      ++sa.waits_dedup;
    }
  }
  return sa;
}

StatusOr<HappensBefore> StreamAssignment::happens_before() const {
  return HappensBefore::build(num_streams_used, stream_of, issue_of, record_of, waits_of, order);
}

std::string StreamAssignment::describe() const {
  std::ostringstream os;
  os << "streams " << num_streams_used << "/" << num_streams_requested << "  events " << num_events
     << "  waits " << waits_dedup << "/" << waits_raw << " (dedup/raw)\n";
  for (std::size_t i = 0; i < nodes.size(); ++i) {
    os << "  [" << i << "] node " << nodes[i] << "  stream " << stream_of[i] << " issue " << issue_of[i];
    if (!waits_of[i].empty()) {
      os << "  waits {";
      for (std::size_t k = 0; k < waits_of[i].size(); ++k) os << (k ? "," : "") << waits_of[i][k];
      os << "}";
    }
    if (record_of[i] != kNoEventId) os << "  records " << record_of[i];
    os << "\n";
  }
  for (std::size_t s = 0; s < stream_load_ms.size(); ++s)
    os << "  stream " << s << " estimated load " << stream_load_ms[s] << " ms\n";
  return os.str();
}

Status verify_plan_ordering(const Graph& g, const StreamAssignment& sa) {
  MCKE_ASSIGN_OR_RETURN(HappensBefore hb, sa.happens_before());
  std::vector<std::uint32_t> idx_of(g.num_nodes(), kNoEventId);
  for (std::size_t i = 0; i < sa.nodes.size(); ++i) idx_of[sa.nodes[i]] = static_cast<std::uint32_t>(i);
  for (std::size_t i = 0; i < sa.nodes.size(); ++i)
    for (NodeId p : g.node(sa.nodes[i]).preds) {
      const std::uint32_t pi = idx_of[p];
      if (pi == kNoEventId)
        return InternalError("verify_plan_ordering: node " + std::to_string(sa.nodes[i]) +
                             " depends on unscheduled node " + std::to_string(p));
      if (!hb.precedes(pi, static_cast<std::uint32_t>(i)))
        return InternalError("verify_plan_ordering: dependency " + std::to_string(p) + " -> " +
                             std::to_string(sa.nodes[i]) + " is not ordered by the schedule; " +
                             hb.describe_pair(pi, static_cast<std::uint32_t>(i)));
    }
  return OkStatus();
}

}  // namespace mcke
