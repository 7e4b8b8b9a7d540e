// graph.cpp -- building a graph of ops over SSA tensors, finalising it, and the
// queries the scheduler and memory planner use.
//
// Contract: reference include/mcke/graph/graph.hpp and src/graph/graph.cpp:59-441
// (add_input / add_node with shape inference / mark_output / finalize; depths,
// slack, dead nodes, levels, live ranges, total cost, DOT).  Structure here:
//
//   finalize()  wires consumers, predecessors (deduplicated, ascending) and
//               successors; runs a three-colour depth-first search from every
//               node that both finds a cycle (reported as the path around it)
//               and yields a reverse postorder; computes ASAP depths along that
//               order and heights against it; then marks liveness in one sweep
//               from the sinks back (a node is live if it writes a graph output
//               or feeds a live node).
//   topological_order() is level-major: nodes by ASAP depth, then by id.  Every
//               edge goes from a lower depth to a higher one, so this is a
//               topological order, and it hands the scheduler each level's
//               independent nodes together.
#include "mcke/graph/graph.hpp"

#include <algorithm>
#include <limits>
#include <numeric>
#include <sstream>

namespace mcke {

namespace {

Status validate_extents(const Shape& s, const std::string& who) {
  if (s.rank() < 1)
    return InvalidArgumentError(who + ": a tensor needs rank >= 1 (a scalar is shape {1})");
  dim_t count = 1;
  for (int i = 0; i < s.rank(); ++i) {
    const dim_t d = s.dim(i);
    if (d < 1) {
      std::ostringstream os;
      os << who << ": extent " << d << " in dimension " << i << " of " << s.to_string()
         << " (extents start at 1)";
      return InvalidArgumentError(os.str());
    }
    if (count > std::numeric_limits<dim_t>::max() / d)
      return InvalidArgumentError(who + ": " + s.to_string() + " has more elements than int64 counts");
    count *= d;
  }
  if (!s.is_contiguous())
    return InvalidArgumentError(who + ": " + s.to_string() + " is strided; graph tensors are dense");
  return OkStatus();
}

}  // namespace

std::string Graph::describe(NodeId n) const {
  if (n >= nodes_.size()) return "<no node " + std::to_string(n) + ">";
  const Node& nd = nodes_[n];
  return "'" + nd.name + "' [" + (nd.op ? std::string(nd.op->type_name()) : std::string("no op")) +
         " #" + std::to_string(n) + "]";
}

std::string Graph::describe_tensor(TensorId t) const {
  if (t >= tensors_.size()) return "<no tensor " + std::to_string(t) + ">";
  return "'" + tensors_[t].name + "' " + tensors_[t].shape.to_string() + " [#" + std::to_string(t) + "]";
}

StatusOr<TensorId> Graph::add_input(Shape shape, DType dtype, std::string name) {
  if (finalized_) return FailedPreconditionError("add_input: the graph is finalized; build a new one");
  MCKE_RETURN_IF_ERROR(validate_extents(shape, "add_input '" + name + "'"));
  TensorDesc d;
  d.shape = shape;
  d.dtype = dtype;
  d.name = std::move(name);
  d.is_graph_input = true;
  tensors_.push_back(std::move(d));
  return static_cast<TensorId>(tensors_.size() - 1);
}

StatusOr<std::vector<TensorId>> Graph::add_node(OpPtr op, std::vector<TensorId> inputs, std::string name) {
  if (finalized_) return FailedPreconditionError("add_node: the graph is finalized; build a new one");
  if (!op) return InvalidArgumentError("add_node '" + name + "': the op is null");
  const std::string who = "add_node '" + name + "' (" + std::string(op->type_name()) + ")";
  std::vector<Shape> in_shapes;
  std::vector<DType> in_types;
  for (std::size_t i = 0; i < inputs.size(); ++i) {
    if (inputs[i] >= tensors_.size()) {
      std::ostringstream os;
      os << who << ": operand " << i << " is tensor id " << inputs[i] << ", but the graph holds "
         << tensors_.size() << " tensors";
      return InvalidArgumentError(os.str());
    }
    in_shapes.push_back(tensors_[inputs[i]].shape);
    in_types.push_back(tensors_[inputs[i]].dtype);
  }
  MCKE_ASSIGN_OR_RETURN(std::vector<Shape> out_shapes, op->infer_shapes(in_shapes));
  if (out_shapes.empty()) return InvalidArgumentError(who + ": the op infers no outputs");
  StatusOr<DType> out_type = op->infer_dtype(in_types);
  if (!out_type.ok()) return Status(out_type.status().code(), who + ": " + out_type.status().message());
  for (std::size_t k = 0; k < out_shapes.size(); ++k)
    MCKE_RETURN_IF_ERROR(validate_extents(out_shapes[k], who + " result " + std::to_string(k)));

  const auto id = static_cast<NodeId>(nodes_.size());
  Node node;
  node.op = std::move(op);
  node.inputs = std::move(inputs);
  node.name = name;
  for (std::size_t k = 0; k < out_shapes.size(); ++k) {
    TensorDesc d;
    d.shape = out_shapes[k];
    d.dtype = *out_type;
    d.producer = id;
    d.name = out_shapes.size() == 1 ? name : name + ":" + std::to_string(k);
    node.outputs.push_back(static_cast<TensorId>(tensors_.size()));
    tensors_.push_back(std::move(d));
  }
  nodes_.push_back(std::move(node));
  return nodes_.back().outputs;
}

Status Graph::mark_output(TensorId t) {
  if (finalized_) return FailedPreconditionError("mark_output: the graph is finalized; build a new one");
  if (t >= tensors_.size())
    return InvalidArgumentError("mark_output: there is no tensor " + std::to_string(t));
  tensors_[t].is_graph_output = true;
  return OkStatus();
}

std::vector<NodeId> Graph::level_major_order() const {
  std::vector<NodeId> order(nodes_.size());
  std::iota(order.begin(), order.end(), 0u);
  std::stable_sort(order.begin(), order.end(),
                   [&](NodeId a, NodeId b) { return nodes_[a].depth < nodes_[b].depth; });
  return order;
}

Status Graph::finalize() {
  if (finalized_) return OkStatus();
  if (nodes_.empty()) return FailedPreconditionError("finalize: the graph has no nodes to run");
  bool any_output = false;
  for (const TensorDesc& d : tensors_) any_output = any_output || d.is_graph_output;
  if (!any_output) return InvalidArgumentError("finalize: no tensor is marked as a graph output");

  // Wiring.
  for (TensorDesc& d : tensors_) d.consumers.clear();
  for (std::size_t n = 0; n < nodes_.size(); ++n) {
    Node& nd = nodes_[n];
    nd.preds.clear();
    nd.succs.clear();
    for (std::size_t i = 0; i < nd.inputs.size(); ++i) {
      TensorDesc& d = tensors_[nd.inputs[i]];
      if (d.producer == kInvalidNode && !d.is_graph_input)
        return InvalidArgumentError("finalize: " + describe(static_cast<NodeId>(n)) + " reads " +
                                    describe_tensor(nd.inputs[i]) + ", which nothing produces");
      d.consumers.push_back(static_cast<NodeId>(n));
      if (d.producer != kInvalidNode) nd.preds.push_back(d.producer);
    }
    std::sort(nd.preds.begin(), nd.preds.end());
    nd.preds.erase(std::unique(nd.preds.begin(), nd.preds.end()), nd.preds.end());
  }
  for (std::size_t n = 0; n < nodes_.size(); ++n)
    for (NodeId p : nodes_[n].preds) nodes_[p].succs.push_back(static_cast<NodeId>(n));

  // Three-colour DFS over successor edges: a grey node met again closes a cycle.
  enum : char { kWhite, kGrey, kBlack };
  std::vector<char> colour(nodes_.size(), kWhite);
  std::vector<NodeId> postorder;
  postorder.reserve(nodes_.size());
  std::vector<std::pair<NodeId, std::size_t>> path;   // node, next successor to try
  for (std::size_t root = 0; root < nodes_.size(); ++root) {
    if (colour[root] != kWhite) continue;
    path.emplace_back(static_cast<NodeId>(root), 0);
    colour[root] = kGrey;
    while (!path.empty()) {
      auto& [n, next] = path.back();
      if (next == nodes_[n].succs.size()) {
        colour[n] = kBlack;
        postorder.push_back(n);
        path.pop_back();
        continue;
      }
      const NodeId s = nodes_[n].succs[next++];
      if (colour[s] == kGrey) {
        std::string ring;
        bool on = false;
        for (const auto& [m, unused] : path) {
          (void)unused;
          on = on || m == s;
          if (on) ring += describe(m) + " -> ";
        }
        return InternalError("finalize: the graph has a cycle: " + ring + describe(s));
      }
      if (colour[s] == kWhite) {
        colour[s] = kGrey;
        path.emplace_back(s, 0);
      }
    }
  }

  // Depths along the reverse postorder (a topological order), heights against it.
  std::vector<int> height(nodes_.size(), 0);
  for (Node& nd : nodes_) nd.depth = 0;
  for (auto it = postorder.rbegin(); it != postorder.rend(); ++it)
    for (NodeId s : nodes_[*it].succs) nodes_[s].depth = std::max(nodes_[s].depth, nodes_[*it].depth + 1);
  for (NodeId n : postorder)
    for (NodeId s : nodes_[n].succs) height[n] = std::max(height[n], height[s] + 1);
  int last_level = 0;
  for (const Node& nd : nodes_) last_level = std::max(last_level, nd.depth);
  for (std::size_t n = 0; n < nodes_.size(); ++n) {
    nodes_[n].alap_depth = last_level - height[n];
    nodes_[n].slack = nodes_[n].alap_depth - nodes_[n].depth;
  }

  // Liveness: the postorder visits every node after all of its successors.
  for (NodeId n : postorder) {
    Node& nd = nodes_[n];
    bool live = false;
    for (TensorId t : nd.outputs) live = live || tensors_[t].is_graph_output;
    for (NodeId s : nd.succs) live = live || !nodes_[s].is_dead;
    nd.is_dead = !live;
  }
  finalized_ = true;
  return OkStatus();
}

StatusOr<std::vector<NodeId>> Graph::topological_order() const {
  if (!finalized_) return FailedPreconditionError("topological_order: finalize() the graph first");
  return level_major_order();
}

StatusOr<std::vector<std::vector<NodeId>>> Graph::levels() const {
  if (!finalized_) return FailedPreconditionError("levels: finalize() the graph first");
  std::vector<std::vector<NodeId>> by_depth;
  for (NodeId n : level_major_order()) {
    const auto d = static_cast<std::size_t>(nodes_[n].depth);
    if (by_depth.size() <= d) by_depth.resize(d + 1);
    by_depth[d].push_back(n);
  }
  return by_depth;
}

StatusOr<std::size_t> Graph::max_level_width() const {
  MCKE_ASSIGN_OR_RETURN(std::vector<std::vector<NodeId>> by_depth, levels());
  std::size_t widest = 0;
  for (const auto& level : by_depth) widest = std::max(widest, level.size());
  return widest;
}

std::vector<NodeId> Graph::dead_nodes() const {
  std::vector<NodeId> dead;
  for (std::size_t n = 0; n < nodes_.size(); ++n)
    if (nodes_[n].is_dead) dead.push_back(static_cast<NodeId>(n));
  return dead;
}

// def_pos: position of the producer in `order` (-1 for graph inputs); last_use_pos:
// position of the last reader, never below def_pos, and order.size() for graph inputs
// and outputs, which live through the whole run: an input is filled by set_input()
// outside the plan and read again on every run (reference graph.hpp:71-81).
std::vector<Graph::LiveRange> Graph::compute_live_ranges(const std::vector<NodeId>& order) const {
  std::vector<LiveRange> ranges(tensors_.size());
  for (int pos = 0; pos < static_cast<int>(order.size()); ++pos) {
    const NodeId n = order[static_cast<std::size_t>(pos)];
    if (n >= nodes_.size()) continue;
    for (TensorId t : nodes_[n].outputs)
      if (ranges[t].def_pos < 0) ranges[t].def_pos = pos;
    for (TensorId t : nodes_[n].inputs) ranges[t].last_use_pos = std::max(ranges[t].last_use_pos, pos);
  }
  for (std::size_t t = 0; t < tensors_.size(); ++t) {
    LiveRange& r = ranges[t];
    if (tensors_[t].is_graph_input) r.def_pos = -1;
    if (tensors_[t].is_graph_input || tensors_[t].is_graph_output)
      r.last_use_pos = static_cast<int>(order.size());
    r.last_use_pos = std::max(r.last_use_pos, r.def_pos);
  }
  return ranges;
}

std::vector<Shape> Graph::input_shapes(NodeId n) const {
  std::vector<Shape> shapes;
  shapes.reserve(nodes_[n].inputs.size());
  for (TensorId t : nodes_[n].inputs) shapes.push_back(tensors_[t].shape);
  return shapes;
}

OpCost Graph::total_cost() const {
  OpCost sum;
  for (std::size_t n = 0; n < nodes_.size(); ++n) {
    const Node& nd = nodes_[n];
    if (nd.is_dead || !nd.op) continue;
    const OpCost c = nd.op->cost(input_shapes(static_cast<NodeId>(n)));
    sum.flops += c.flops;
    sum.bytes += c.bytes;
  }
  return sum;
}

// Nodes as boxes, tensors as edges labelled with name and shape; graph inputs
// come from one "inputs" point and graph outputs go to one "outputs" point.
std::string Graph::to_dot() const {
  std::ostringstream os;
  os << "digraph G {\n  node [fontname=monospace];\n  inputs [shape=point];\n  outputs [shape=point];\n";
  for (std::size_t n = 0; n < nodes_.size(); ++n) {
    const Node& nd = nodes_[n];
    os << "  op" << n << " [shape=box,label=\"" << nd.name << " : "
       << (nd.op ? std::string(nd.op->type_name()) : std::string("?")) << "\""
       << (nd.is_dead ? ",color=gray" : "") << "];\n";
  }
  auto edge = [&](const std::string& from, const std::string& to, TensorId t) {
    os << "  " << from << " -> " << to << " [label=\"" << tensors_[t].name << " "
       << tensors_[t].shape.to_string() << "\"];\n";
  };
  for (std::size_t t = 0; t < tensors_.size(); ++t) {
    const TensorDesc& d = tensors_[t];
    const std::string src = d.producer == kInvalidNode ? "inputs" : "op" + std::to_string(d.producer);
    for (NodeId c : d.consumers) edge(src, "op" + std::to_string(c), static_cast<TensorId>(t));
    if (d.is_graph_output) edge(src, "outputs", static_cast<TensorId>(t));
  }
  os << "}\n";
  return os.str();
}

}  // namespace mcke
