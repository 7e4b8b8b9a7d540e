// memory_plan.cpp -- every tensor of a schedule placed in one arena, and the
// check that no two tensors sharing bytes can be live at the same time.
//
// Contract: reference include/mcke/graph/memory_plan.hpp and
// src/graph/memory_plan.cpp:40-267 (four sharing policies, the MemoryPlan
// record, verify_no_buffer_races).  Structure here:
//
//   * Lifetimes.  For each tensor: the scheduled index of its producer and of
//     every node that reads it.  Tensor b may reuse tensor a's bytes when both
//     are intermediates and every access of a is over before b's producer runs,
//     where "over before" is the policy's notion: never (per-tensor), earlier in
//     the issue order (topo-naive, which ignores streams and is unsafe -- kept to
//     show what the race check catches), happens-before on one stream
//     (same-stream), or happens-before across streams (happens-before).
//   * Placement.  Largest tensors first (ties by id).  Each goes into the
//     smallest gap between the already placed tensors it may not share with
//     that holds it (best fit, gaps at 256-byte aligned offsets), or past the
//     end of them when no gap does.  The arena is the highest end placed, so it
//     never exceeds the sum of the sizes.
//   * Race check.  The placed byte ranges are swept in offset order; every pair
//     that overlaps must be ordered by happens-before, one way or the other.
#include "mcke/graph/memory_plan.hpp"

#include <algorithm>
#include <sstream>

namespace mcke {

namespace {

constexpr std::uint32_t kNone = 0xFFFFFFFFu;

std::size_t round_up(std::size_t v) {
  return (v + kDeviceAlignment - 1) / kDeviceAlignment * kDeviceAlignment;
}

struct Lifetime {
  std::uint32_t producer = kNone;        // scheduled index
  std::vector<std::uint32_t> touches;    // producer (if scheduled) and readers
};

std::vector<Lifetime> lifetimes(const Graph& g, const StreamAssignment& sa) {
  std::vector<std::uint32_t> at(g.num_nodes(), kNone);
  for (std::size_t i = 0; i < sa.nodes.size(); ++i) at[sa.nodes[i]] = static_cast<std::uint32_t>(i);
  std::vector<Lifetime> life(g.num_tensors());
  for (std::size_t t = 0; t < life.size(); ++t) {
    const TensorDesc& d = g.tensor(static_cast<TensorId>(t));
    if (d.producer != kInvalidNode && at[d.producer] != kNone) {
      life[t].producer = at[d.producer];
      life[t].touches.push_back(life[t].producer);
    }
    for (NodeId c : d.consumers)
      if (at[c] != kNone) life[t].touches.push_back(at[c]);
  }
  return life;
}

// Is every access of tensor a over before tensor b is produced, under `policy`?
bool over_before(MemoryPolicy policy, const Graph& g, const StreamAssignment& sa,
                 const HappensBefore& hb, const std::vector<Lifetime>& life, TensorId a, TensorId b) {
  if (policy == MemoryPolicy::kAllocPerTensor) return false;
  if (!g.tensor(a).reusable() || !g.tensor(b).reusable()) return false;
  const std::uint32_t pb = life[b].producer;
  if (pb == kNone || life[a].touches.empty()) return false;
  const auto& ta = life[a].touches;
  switch (policy) {
    case MemoryPolicy::kReuseTopoNaive:
      return *std::max_element(ta.begin(), ta.end()) < pb;
    case MemoryPolicy::kReuseSameStream:
      return std::all_of(ta.begin(), ta.end(), [&](std::uint32_t u) {
        return sa.stream_of[u] == sa.stream_of[pb] && hb.precedes(u, pb);
      });
    case MemoryPolicy::kReuseHappensBefore:
      return std::all_of(ta.begin(), ta.end(), [&](std::uint32_t u) { return hb.precedes(u, pb); });
    case MemoryPolicy::kAllocPerTensor:
      break;
  }
  return false;
}

const char* policy_label(MemoryPolicy p) {
  switch (p) {
    case MemoryPolicy::kAllocPerTensor: return "one buffer per tensor";
    case MemoryPolicy::kReuseTopoNaive: return "reuse by issue position (unsafe across streams)";
    case MemoryPolicy::kReuseSameStream: return "reuse within a stream";
    case MemoryPolicy::kReuseHappensBefore: return "reuse under happens-before";
  }
  return "?";
}

}  // namespace

StatusOr<MemoryPlan> plan_memory(const Graph& g, const StreamAssignment& sa, const HappensBefore& hb,
                                 MemoryPolicy policy) {
  const std::vector<Lifetime> life = lifetimes(g, sa);
  MemoryPlan mp;
  mp.policy = policy;
  mp.offset_of.assign(g.num_tensors(), kNoOffset);
  mp.bytes_of.assign(g.num_tensors(), 0);

  std::vector<TensorId> todo;
  for (std::size_t t = 0; t < g.num_tensors(); ++t) {
    const TensorDesc& d = g.tensor(static_cast<TensorId>(t));
    const bool dead_producer = d.producer != kInvalidNode && life[t].producer == kNone;
    const std::size_t bytes = round_up(d.shape.bytes(d.dtype));
    if (dead_producer || bytes == 0) continue;
    mp.bytes_of[t] = bytes;
    mp.naive_bytes += bytes;
    if (d.is_graph_input) mp.input_bytes += bytes;
    else if (d.is_graph_output) mp.output_bytes += bytes;
    else mp.intermediate_bytes += bytes;
    todo.push_back(static_cast<TensorId>(t));
  }
  std::stable_sort(todo.begin(), todo.end(),
                   [&](TensorId x, TensorId y) { return mp.bytes_of[x] > mp.bytes_of[y]; });

  std::vector<TensorId> placed;
  for (TensorId t : todo) {
    const std::size_t need = mp.bytes_of[t];
    // Byte ranges of the placed tensors t may not share with, in offset order.
    std::vector<std::pair<std::size_t, std::size_t>> taken;
    for (TensorId o : placed)
      if (!over_before(policy, g, sa, hb, life, o, t) && !over_before(policy, g, sa, hb, life, t, o))
        taken.emplace_back(mp.offset_of[o], mp.offset_of[o] + mp.bytes_of[o]);
    std::sort(taken.begin(), taken.end());
    std::size_t best = kNoOffset, best_gap = kNoOffset, cursor = 0;
    for (const auto& [lo, hi] : taken) {
      if (lo >= cursor && lo - cursor >= need && lo - cursor < best_gap) {
        best = cursor;
        best_gap = lo - cursor;
      }
      cursor = std::max(cursor, round_up(hi));
    }
    if (best == kNoOffset) best = cursor;   // past every conflicting tensor
    mp.offset_of[t] = best;
    mp.arena_bytes = std::max(mp.arena_bytes, best + need);
    placed.push_back(t);
  }

  std::vector<std::size_t> starts;
  for (TensorId t : placed) starts.push_back(mp.offset_of[t]);
  std::sort(starts.begin(), starts.end());
  mp.buffers_used = static_cast<std::size_t>(std::unique(starts.begin(), starts.end()) - starts.begin());

  // One workspace per stream, as large as the largest need of its nodes.
  mp.workspace_bytes.assign(sa.num_streams_used, 0);
  for (std::size_t i = 0; i < sa.nodes.size(); ++i)
    if (const Op* op = g.node(sa.nodes[i]).op.get()) {
      std::size_t& w = mp.workspace_bytes[sa.stream_of[i]];
      w = std::max(w, round_up(op->workspace_bytes(g.input_shapes(sa.nodes[i]))));
    }
  return mp;
}

Status verify_no_buffer_races(const Graph& g, const StreamAssignment& sa, const HappensBefore& hb,
                              const MemoryPlan& mp) {
  const std::vector<Lifetime> life = lifetimes(g, sa);
  // Is every access of `a` over before b's producer?  If not, *late is an access
  // of `a` that is not (kNone when b has no producer or a no access at all).
  auto finished_before = [&](std::size_t a, std::size_t b, std::uint32_t* late) -> bool {
    *late = kNone;
    const std::uint32_t pb = life[b].producer;
    if (pb == kNone || life[a].touches.empty()) return false;
    for (std::uint32_t u : life[a].touches)
      if (!hb.precedes(u, pb)) {
        *late = u;
        return false;
      }
    return true;
  };
  std::vector<std::size_t> by_offset;
  for (std::size_t t = 0; t < mp.offset_of.size(); ++t)
    if (mp.offset_of[t] != kNoOffset) by_offset.push_back(t);
  std::sort(by_offset.begin(), by_offset.end(),
            [&](std::size_t x, std::size_t y) { return mp.offset_of[x] < mp.offset_of[y]; });
  for (std::size_t i = 0; i < by_offset.size(); ++i) {
    const std::size_t a = by_offset[i];
    const std::size_t a_end = mp.offset_of[a] + mp.bytes_of[a];
    for (std::size_t j = i + 1; j < by_offset.size() && mp.offset_of[by_offset[j]] < a_end; ++j) {
      const std::size_t b = by_offset[j];
      std::uint32_t ab = kNone, ba = kNone;
      if (finished_before(a, b, &ab) || finished_before(b, a, &ba)) continue;
      std::ostringstream os;
      os << "verify_no_buffer_races: '" << g.tensor(static_cast<TensorId>(a)).name << "' (tensor " << a
         << ") and '" << g.tensor(static_cast<TensorId>(b)).name << "' (tensor " << b
         << ") overlap at bytes [" << mp.offset_of[b] << ", "
         << std::min(a_end, mp.offset_of[b] + mp.bytes_of[b]) << ") with neither finished before the other "
         << "is written";
      if (ab != kNone && ab != life[b].producer) os << "; " << hb.describe_pair(ab, life[b].producer);
      return InternalError(os.str());
    }
  }
  return OkStatus();
}

std::string MemoryPlan::describe() const {
  std::ostringstream os;
  os << "arena (" << policy_label(policy) << "): " << arena_bytes << " B in " << buffers_used
     << " buffer(s), against " << naive_bytes << " B with no sharing";
  if (arena_bytes) os << " (" << static_cast<double>(naive_bytes) / static_cast<double>(arena_bytes) << "x)";
  os << "\n  graph inputs " << input_bytes << " B, intermediates " << intermediate_bytes
     << " B, graph outputs " << output_bytes << " B";
  for (std::size_t s = 0; s < workspace_bytes.size(); ++s)
    if (workspace_bytes[s]) os << "\n  workspace s" << s << ": " << workspace_bytes[s] << " B";
  os << "\n";
  return os.str();
}

}  // namespace mcke
