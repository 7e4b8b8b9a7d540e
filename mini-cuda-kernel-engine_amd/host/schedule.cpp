// schedule.cpp -- nodes onto streams, and the events that order them.
//
// Contract: reference include/mcke/graph/schedule.hpp:49-108 and
// src/graph/schedule.cpp:27-301 (three policies, the StreamAssignment record,
// verify_plan_ordering).  Structure here:
//
//   1. Topology: the live nodes in topological order get scheduled indices 0..S-1
//      (that order is also the issue order), each with its live predecessors
//      and its roofline time (its ideal cost at the planning roofline).
//   2. A policy function assigns a stream to every node and lists the nodes each
//      node must start after ("needs"): its graph predecessors, or for the
//      level-parallel policy the level barrier.
//   3. Streams are renumbered densely in order of first use; issue indices count
//      up per stream.
//   4. Waits: the cross-stream needs of each node, latest first, are checked
//      against the node's vector clock as built so far (its stream predecessor's
//      clock merged with those of the producers it already waits on); a need the
//      clock already covers is implied by an earlier wait or by stream order and
//      gets no wait of its own.  Producers left with a waiter record one event
//      each, numbered in issue order.
#include "mcke/graph/schedule.hpp"

#include <algorithm>
#include <numeric>
#include <sstream>

#include "mcke/graph/cost_model.hpp"

namespace mcke {

namespace {

constexpr std::uint32_t kUnscheduled = 0xFFFFFFFFu;

struct Topology {
  std::vector<NodeId> node_at;                        // scheduled index -> node
  std::vector<std::uint32_t> index_of;                // node -> scheduled index
  std::vector<std::vector<std::uint32_t>> preds;      // live predecessors, scheduled
  std::vector<double> cost_ms;
};

StatusOr<Topology> live_topology(const Graph& g, const Roofline& rl) {
  MCKE_ASSIGN_OR_RETURN(std::vector<NodeId> topo, g.topological_order());
  Topology t;
  t.index_of.assign(g.num_nodes(), kUnscheduled);
  for (NodeId n : topo)
    if (!g.node(n).is_dead) {
      t.index_of[n] = static_cast<std::uint32_t>(t.node_at.size());
      t.node_at.push_back(n);
    }
  for (NodeId n : t.node_at) {
    std::vector<std::uint32_t> p;
    for (NodeId q : g.node(n).preds)
      if (t.index_of[q] != kUnscheduled) p.push_back(t.index_of[q]);
    std::sort(p.begin(), p.end());
    t.preds.push_back(std::move(p));
    const Op* op = g.node(n).op.get();
    t.cost_ms.push_back(op ? plan_cost_ms(op->cost(g.input_shapes(n)), rl) : 0.0);
  }
  return t;
}

struct Assignment {
  std::vector<std::uint16_t> stream;
  std::vector<std::vector<std::uint32_t>> needs;
};

Assignment assign_sequential(const Topology& t) {
  return {std::vector<std::uint16_t>(t.node_at.size(), 0), t.preds};
}

// Level d's nodes are dealt round-robin over the streams in scheduled order.
// Between levels d and d+1 a barrier: on each stream, the first node of level d+1
// needs the last node of level d of every other stream (stream order covers its
// own).  Graph edges never span less than one level, so the barrier orders them.
StatusOr<Assignment> assign_levels(const Graph& g, const Topology& t, int lanes) {
  MCKE_ASSIGN_OR_RETURN(std::vector<std::vector<NodeId>> by_depth, g.levels());
  Assignment a;
  a.stream.assign(t.node_at.size(), 0);
  a.needs.assign(t.node_at.size(), {});
  std::vector<std::uint32_t> tail(static_cast<std::size_t>(lanes), kUnscheduled);   // previous level
  for (const auto& nodes : by_depth) {
    std::vector<std::uint32_t> level;
    for (NodeId n : nodes)
      if (t.index_of[n] != kUnscheduled) level.push_back(t.index_of[n]);
    if (level.empty()) continue;
    std::sort(level.begin(), level.end());
    std::vector<std::uint32_t> head(static_cast<std::size_t>(lanes), kUnscheduled);
    std::vector<std::uint32_t> last(static_cast<std::size_t>(lanes), kUnscheduled);
    for (std::size_t k = 0; k < level.size(); ++k) {
      const auto s = static_cast<std::size_t>(k % static_cast<std::size_t>(lanes));
      a.stream[level[k]] = static_cast<std::uint16_t>(s);
      if (head[s] == kUnscheduled) head[s] = level[k];
      last[s] = level[k];
    }
    for (std::size_t s = 0; s < head.size(); ++s) {
      if (head[s] == kUnscheduled) continue;
      for (std::size_t o = 0; o < tail.size(); ++o)
        if (o != s && tail[o] != kUnscheduled) a.needs[head[s]].push_back(tail[o]);
    }
    tail = last;
  }
  return a;
}

// A node whose only live predecessor p has not yet passed its stream on (p's
// heir: the first node in scheduled order whose single predecessor is p) takes
// p's stream; every other node takes the stream with the least roofline time
// assigned so far (the lowest-numbered one on a tie).  Needs are the graph edges.
Assignment assign_chains(const Topology& t, int lanes) {
  const std::size_t S = t.node_at.size();
  std::vector<std::uint32_t> heir(S, kUnscheduled);
  for (std::uint32_t i = 0; i < S; ++i)
    if (t.preds[i].size() == 1 && heir[t.preds[i][0]] == kUnscheduled) heir[t.preds[i][0]] = i;
  Assignment a{std::vector<std::uint16_t>(S, 0), t.preds};
  std::vector<double> load(static_cast<std::size_t>(lanes), 0.0);
  for (std::uint32_t i = 0; i < S; ++i) {
    std::size_t s;
    if (t.preds[i].size() == 1 && heir[t.preds[i][0]] == i)
      s = a.stream[t.preds[i][0]];
    else
      s = static_cast<std::size_t>(std::min_element(load.begin(), load.end()) - load.begin());
    a.stream[i] = static_cast<std::uint16_t>(s);
    load[s] += t.cost_ms[i];
  }
  return a;
}

}  // namespace

StatusOr<StreamAssignment> plan_streams(const Graph& g, SchedulePolicy policy, int num_streams,
                                        const Roofline& rl) {
  if (num_streams < 1)
    return InvalidArgumentError("plan_streams: asked for " + std::to_string(num_streams) +
                                " streams; at least one is needed");
  if (!g.finalized()) return FailedPreconditionError("plan_streams: the graph is not finalized");
  MCKE_ASSIGN_OR_RETURN(Topology topo, live_topology(g, rl));
  const std::size_t S = topo.node_at.size();
  if (S == 0) return InvalidArgumentError("plan_streams: no node reaches a graph output");
  const int lanes = static_cast<int>(std::min<std::size_t>(static_cast<std::size_t>(num_streams), S));

  Assignment asg;
  switch (policy) {
    case SchedulePolicy::kSequential: asg = assign_sequential(topo); break;
    case SchedulePolicy::kLevelParallel: {
      MCKE_ASSIGN_OR_RETURN(asg, assign_levels(g, topo, lanes));
      break;
    }
    case SchedulePolicy::kChainGreedy: asg = assign_chains(topo, lanes); break;
  }

  StreamAssignment sa;
  sa.nodes = topo.node_at;
  sa.num_streams_requested = static_cast<std::size_t>(num_streams);
  sa.order.resize(S);
  std::iota(sa.order.begin(), sa.order.end(), 0u);

  // Dense stream numbers in order of first use, then issue indices.
  std::vector<int> renumber(static_cast<std::size_t>(lanes), -1);
  std::vector<std::uint32_t> count;
  sa.stream_of.resize(S);
  sa.issue_of.resize(S);
  for (std::size_t i = 0; i < S; ++i) {
    int& s = renumber[asg.stream[i]];
    if (s < 0) {
      s = static_cast<int>(count.size());
      count.push_back(0);
      sa.stream_load_ms.push_back(0.0);
    }
    sa.stream_of[i] = static_cast<std::uint16_t>(s);
    sa.issue_of[i] = count[static_cast<std::size_t>(s)]++;
    sa.stream_load_ms[static_cast<std::size_t>(s)] += topo.cost_ms[i];
  }
  sa.num_streams_used = count.size();
  const std::size_t K = sa.num_streams_used;

  // Waits, pruned by the vector clock each node has accumulated so far.
  std::vector<std::int64_t> clock(S * K, -1);
  std::vector<std::int64_t> lane_clock(K * K, -1);   // clock of the last node on each stream
  std::vector<std::vector<std::uint32_t>> waits_on(S);   // producers each node waits on
  std::vector<char> waited(S, 0);
  for (std::size_t i = 0; i < S; ++i) {
    const std::size_t s = sa.stream_of[i];
    std::int64_t* c = &clock[i * K];
    std::copy_n(&lane_clock[s * K], K, c);
    std::vector<std::uint32_t> cross;
    for (std::uint32_t p : asg.needs[i])
      if (sa.stream_of[p] != s) cross.push_back(p);
    sa.waits_raw += cross.size();
    std::sort(cross.rbegin(), cross.rend());
    cross.erase(std::unique(cross.begin(), cross.end()), cross.end());
    for (std::uint32_t p : cross) {
      if (c[sa.stream_of[p]] >= static_cast<std::int64_t>(sa.issue_of[p])) continue;   // implied
      const std::int64_t* cp = &clock[static_cast<std::size_t>(p) * K];
      for (std::size_t k = 0; k < K; ++k) c[k] = std::max(c[k], cp[k]);
      waits_on[i].push_back(p);
      waited[p] = 1;
    }
    c[s] = static_cast<std::int64_t>(sa.issue_of[i]);
    std::copy_n(c, K, &lane_clock[s * K]);
  }
  sa.record_of.assign(S, kNoEventId);
  for (std::size_t i = 0; i < S; ++i)
    if (waited[i]) sa.record_of[i] = static_cast<std::uint32_t>(sa.num_events++);
  sa.waits_of.resize(S);
  for (std::size_t i = 0; i < S; ++i) {
    for (std::uint32_t p : waits_on[i]) sa.waits_of[i].push_back(sa.record_of[p]);
    sa.waits_dedup += waits_on[i].size();
  }
  return sa;
}

StatusOr<HappensBefore> StreamAssignment::happens_before() const {
  return HappensBefore::build(num_streams_used, stream_of, issue_of, record_of, waits_of, order);
}

std::string StreamAssignment::describe() const {
  std::ostringstream os;
  os << "schedule over " << num_streams_used << " of " << num_streams_requested
     << " requested stream(s): " << num_events << " event(s), " << waits_dedup << " wait(s) kept of "
     << waits_raw << " cross-stream dependencies\n";
  for (std::size_t s = 0; s < num_streams_used; ++s) {
    os << "  s" << s << " (" << (s < stream_load_ms.size() ? stream_load_ms[s] : 0.0)
       << " ms roofline):";
    for (std::size_t i = 0; i < nodes.size(); ++i) {
      if (stream_of[i] != s) continue;
      os << " n" << nodes[i];
      for (std::uint32_t e : waits_of[i]) os << " <e" << e;
      if (record_of[i] != kNoEventId) os << " >e" << record_of[i];
    }
    os << "\n";
  }
  return os.str();
}

Status verify_plan_ordering(const Graph& g, const StreamAssignment& sa) {
  MCKE_ASSIGN_OR_RETURN(HappensBefore hb, sa.happens_before());
  std::vector<std::uint32_t> at(g.num_nodes(), kUnscheduled);
  for (std::size_t i = 0; i < sa.nodes.size(); ++i) at[sa.nodes[i]] = static_cast<std::uint32_t>(i);
  for (std::size_t i = 0; i < sa.nodes.size(); ++i) {
    const NodeId n = sa.nodes[i];
    for (NodeId p : g.node(n).preds) {
      if (at[p] == kUnscheduled)
        return InternalError("verify_plan_ordering: '" + g.node(n).name + "' reads from '" +
                             g.node(p).name + "', which the schedule leaves out");
      if (!hb.precedes(at[p], static_cast<std::uint32_t>(i)))
        return InternalError("verify_plan_ordering: '" + g.node(n).name + "' may start before '" +
                             g.node(p).name + "' ends: " +
                             hb.describe_pair(at[p], static_cast<std::uint32_t>(i)));
    }
  }
  return OkStatus();
}

}  // namespace mcke
