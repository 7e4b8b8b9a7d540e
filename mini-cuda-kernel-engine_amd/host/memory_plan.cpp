// memory_plan.cpp -- arena placement with happens-before sharing and the race
// verifier (reference src/graph/memory_plan.cpp:40-267).
#include "mcke/graph/memory_plan.hpp"

#include <algorithm>
#include <sstream>

namespace mcke {

namespace {

std::size_t align_up(std::size_t v, std::size_t a) { return (v + a - 1) / a * a; }

const char* policy_name(MemoryPolicy p) {
  switch (p) {
    case MemoryPolicy::kAllocPerTensor: return "alloc_per_tensor";
    case MemoryPolicy::kReuseTopoNaive: return "reuse_topo_naive(UNSAFE)";
    case MemoryPolicy::kReuseSameStream: return "reuse_same_stream";
    case MemoryPolicy::kReuseHappensBefore: return "reuse_happens_before";
  }
  return "?";
}

// Scheduled indices of the nodes touching each tensor (producer first).
struct Uses {
  std::uint32_t producer = kNoEventId;
  std::vector<std::uint32_t> all;
};

std::vector<Uses> collect_uses(const Graph& g, const std::vector<std::uint32_t>& idx_of) {
  std::vector<Uses> u(g.num_tensors());
  for (std::size_t t = 0; t < g.num_tensors(); ++t) {
    const TensorDesc& d = g.tensor(static_cast<TensorId>(t));
    if (d.producer != kInvalidNode && idx_of[d.producer] != kNoEventId) {
      u[t].producer = idx_of[d.producer];
      u[t].all.push_back(u[t].producer);
    }
    for (NodeId c : d.consumers)
      if (idx_of[c] != kNoEventId) u[t].all.push_back(idx_of[c]);
  }
  return u;
}

}  // namespace

StatusOr<MemoryPlan> plan_memory(const Graph& g, const StreamAssignment& sa, const HappensBefore& hb,
                                 MemoryPolicy policy) {
  MemoryPlan mp;
  mp.policy = policy;
  const std::size_t T = g.num_tensors();
  mp.offset_of.assign(T, kNoOffset);
  mp.bytes_of.assign(T, 0);
  std::vector<std::uint32_t> idx_of(g.num_nodes(), kNoEventId);
  for (std::size_t i = 0; i < sa.nodes.size(); ++i) idx_of[sa.nodes[i]] = static_cast<std::uint32_t>(i);
  const std::vector<Uses> uses = collect_uses(g, idx_of);

  std::vector<TensorId> placed;
  for (std::size_t t = 0; t < T; ++t) {
    const TensorDesc& d = g.tensor(static_cast<TensorId>(t));
    if (d.producer != kInvalidNode && idx_of[d.producer] == kNoEventId) continue;   // dead producer
    const std::size_t bytes = align_up(d.shape.bytes(d.dtype), kDeviceAlignment);
    if (bytes == 0) continue;
    mp.bytes_of[t] = bytes;
    placed.push_back(static_cast<TensorId>(t));
    (d.is_graph_input ? mp.input_bytes : d.is_graph_output ? mp.output_bytes : mp.intermediate_bytes) += bytes;
    mp.naive_bytes += bytes;
  }

  // May tensor b take bytes that tensor a used?  Only if every use of a is over
  // before b's producer starts.
  auto a_before_b = [&](TensorId a, TensorId b) -> bool {
    if (!g.tensor(a).reusable() || !g.tensor(b).reusable()) return false;
    const std::uint32_t pb = uses[b].producer;
    if (pb == kNoEventId || uses[a].all.empty()) return false;
    switch (policy) {
      case MemoryPolicy::kAllocPerTensor:
        return false;
      case MemoryPolicy::kReuseTopoNaive: {
        std::uint32_t last = 0;
        for (std::uint32_t n : uses[a].all) last = std::max(last, n);
        return last < pb;
      }
      case MemoryPolicy::kReuseSameStream:
        for (std::uint32_t n : uses[a].all)
          if (sa.stream_of[n] != sa.stream_of[pb] || !hb.precedes(n, pb)) return false;
        return true;
      case MemoryPolicy::kReuseHappensBefore:
        for (std::uint32_t n : uses[a].all)
          if (!hb.precedes(n, pb)) return false;
        return true;
    }
    return false;
  };

  std::vector<TensorId> by_size = placed;
  std::sort(by_size.begin(), by_size.end(), [&](TensorId x, TensorId y) {
    return mp.bytes_of[x] != mp.bytes_of[y] ? mp.bytes_of[x] > mp.bytes_of[y] : x < y;
  });
  std::vector<TensorId> done;
  for (TensorId t : by_size) {
    std::vector<std::pair<std::size_t, std::size_t>> busy;
    for (TensorId u : done)
      if (!a_before_b(u, t) && !a_before_b(t, u)) busy.emplace_back(mp.offset_of[u], mp.offset_of[u] + mp.bytes_of[u]);
    std::sort(busy.begin(), busy.end());
    std::size_t off = 0;
    for (const auto& [lo, hi] : busy) {
      if (off + mp.bytes_of[t] <= lo) break;
      off = std::max(off, align_up(hi, kDeviceAlignment));
    }
    mp.offset_of[t] = off;
    mp.arena_bytes = std::max(mp.arena_bytes, off + mp.bytes_of[t]);
    done.push_back(t);
  }
  std::vector<std::size_t> offs;
  for (TensorId t : placed) offs.push_back(mp.offset_of[t]);
  std::sort(offs.begin(), offs.end());
  mp.buffers_used = static_cast<std::size_t>(std::unique(offs.begin(), offs.end()) - offs.begin());

  mp.workspace_bytes.assign(sa.num_streams_used, 0);
  for (std::size_t i = 0; i < sa.nodes.size(); ++i) {
    const Node& nd = g.node(sa.nodes[i]);
    if (!nd.op) continue;
    const std::size_t w = nd.op->workspace_bytes(g.input_shapes(sa.nodes[i]));
    auto& slot = mp.workspace_bytes[sa.stream_of[i]];
    slot = std::max(slot, align_up(w, kDeviceAlignment));
  }
  return mp;
}

Status verify_no_buffer_races(const Graph& g, const StreamAssignment& sa, const HappensBefore& hb,
                              const MemoryPlan& mp) {
  std::vector<std::uint32_t> idx_of(g.num_nodes(), kNoEventId);
  for (std::size_t i = 0; i < sa.nodes.size(); ++i) idx_of[sa.nodes[i]] = static_cast<std::uint32_t>(i);
  const std::vector<Uses> uses = collect_uses(g, idx_of);
  // All uses of `a` precede the producer of `b`?
  auto ordered = [&](std::size_t a, std::size_t b, std::uint32_t* bad_u, std::uint32_t* bad_v) {
    const std::uint32_t pb = uses[b].producer;
    if (pb == kNoEventId || uses[a].all.empty()) return false;
    for (std::uint32_t u : uses[a].all)
      if (!hb.precedes(u, pb)) {
        *bad_u = u;
        *bad_v = pb;
        return false;
      }
    return true;
  };
  const std::size_t T = g.num_tensors();
  for (std::size_t a = 0; a < T; ++a) {
    if (mp.offset_of[a] == kNoOffset) continue;
    for (std::size_t b = a + 1; b < T; ++b) {
      if (mp.offset_of[b] == kNoOffset) continue;
      const std::size_t a0 = mp.offset_of[a], a1 = a0 + mp.bytes_of[a];
      const std::size_t b0 = mp.offset_of[b], b1 = b0 + mp.bytes_of[b];
      if (a1 <= b0 || b1 <= a0) continue;
      std::uint32_t u = 0, v = 0;
      if (ordered(a, b, &u, &v) || ordered(b, a, &u, &v)) continue;
      std::ostringstream os;
      os << "verify_no_buffer_races: tensors " << a << " ('" << g.tensor(static_cast<TensorId>(a)).name
         << "') and " << b << " ('" << g.tensor(static_cast<TensorId>(b)).name << "') share bytes ["
         << std::max(a0, b0) << "," << std::min(a1, b1) << ") but neither's uses are ordered before the "
         << "other's producer";
      if (u != v) os << "; " << hb.describe_pair(u, v);
      return InternalError(os.str());
    }
  }
  return OkStatus();
}

std::string MemoryPlan::describe() const {
  std::ostringstream os;
  os << "memory " << policy_name(policy) << ": arena " << arena_bytes << " B ("
     << arena_bytes / 1048576.0 << " MiB) vs naive " << naive_bytes << " B (" << naive_bytes / 1048576.0
     << " MiB)";
  if (arena_bytes) os << "  ratio " << static_cast<double>(naive_bytes) / static_cast<double>(arena_bytes) << "x";
  os << "\n  buffers " << buffers_used << "  inputs " << input_bytes << " B, intermediates "
     << intermediate_bytes << " B, outputs " << output_bytes << " B\n";
  for (std::size_t s = 0; s < workspace_bytes.size(); ++s)
    os << "  stream " << s << " workspace " << workspace_bytes[s] << " B\n";
  return os.str();
}

}  // namespace mcke
