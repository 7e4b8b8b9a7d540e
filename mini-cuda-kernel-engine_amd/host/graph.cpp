// graph.cpp -- DAG construction, finalisation and queries
// (reference src/graph/graph.cpp:59-441).
#include "mcke/graph/graph.hpp"

#include <algorithm>
#include <deque>
#include <limits>
#include <sstream>

namespace mcke {

namespace {

Status check_shape(const Shape& s, const std::string& what) {
  if (s.rank() < 1) return InvalidArgumentError(what + ": rank 0 (use rank 1 with dim 1 for a scalar)");
  dim_t n = 1;
  for (int i = 0; i < s.rank(); ++i) {
    const dim_t d = s.dim(i);
    if (d <= 0)
      return InvalidArgumentError(what + ": dim " + std::to_string(i) + " is " + std::to_string(d) +
                                  "; extents must be positive");
    if (d > std::numeric_limits<dim_t>::max() / n)
      return InvalidArgumentError(what + ": element count overflows int64");
    n *= d;
  }
  if (!s.is_contiguous()) return InvalidArgumentError(what + ": strides are not row-major contiguous");
  return OkStatus();
}

}  // namespace

std::string Graph::describe(NodeId n) const {
  if (n >= nodes_.size()) return "node#" + std::to_string(n);
  const Node& nd = nodes_[n];
  return "node " + std::to_string(n) + " '" + nd.name + "' (" +
         (nd.op ? std::string(nd.op->type_name()) : std::string("?")) + ")";
}

std::string Graph::describe_tensor(TensorId t) const {
  if (t >= tensors_.size()) return "tensor#" + std::to_string(t);
  return "tensor " + std::to_string(t) + " '" + tensors_[t].name + "' " + tensors_[t].shape.to_string();
}

StatusOr<TensorId> Graph::add_input(Shape shape, DType dtype, std::string name) {
  if (finalized_) return FailedPreconditionError("add_input: graph is already finalized");
  MCKE_RETURN_IF_ERROR(check_shape(shape, "add_input('" + name + "')"));
  TensorDesc d;
  d.shape = shape;
  d.dtype = dtype;
  d.name = std::move(name);
  d.is_graph_input = true;
  tensors_.push_back(std::move(d));
  return static_cast<TensorId>(tensors_.size() - 1);
}

StatusOr<std::vector<TensorId>> Graph::add_node(OpPtr op, std::vector<TensorId> inputs, std::string name) {
  if (finalized_) return FailedPreconditionError("add_node: graph is already finalized");
  if (!op) return InvalidArgumentError("add_node('" + name + "'): null op");
  const std::string where = "add_node('" + name + "', " + std::string(op->type_name()) + ")";
  std::vector<Shape> shapes;
  shapes.reserve(inputs.size());
  for (std::size_t i = 0; i < inputs.size(); ++i) {
    if (inputs[i] >= tensors_.size())
      return InvalidArgumentError(where + ": input " + std::to_string(i) + " is tensor " +
                                  std::to_string(inputs[i]) + " but the graph has " +
                                  std::to_string(tensors_.size()) + " tensors");
    shapes.push_back(tensors_[inputs[i]].shape);
  }
  MCKE_ASSIGN_OR_RETURN(std::vector<Shape> outs, op->infer_shapes(shapes));
  if (outs.empty()) return InvalidArgumentError(where + ": the op produced no outputs");
  std::vector<DType> dtypes;
  dtypes.reserve(inputs.size());
  for (TensorId t : inputs) dtypes.push_back(tensors_[t].dtype);
  auto out_dtype = op->infer_dtype(dtypes);
  if (!out_dtype.ok())
    return Status(out_dtype.status().code(), where + ": " + out_dtype.status().message());
  const auto nid = static_cast<NodeId>(nodes_.size());
  std::vector<TensorId> out_ids;
  for (std::size_t k = 0; k < outs.size(); ++k) {
    MCKE_RETURN_IF_ERROR(check_shape(outs[k], where + " output " + std::to_string(k)));
    TensorDesc d;
    d.shape = outs[k];
    d.dtype = *out_dtype;
    d.producer = nid;
    d.name = outs.size() > 1 ? name + ":" + std::to_string(k) : name;
    tensors_.push_back(std::move(d));
    out_ids.push_back(static_cast<TensorId>(tensors_.size() - 1));
  }
  Node n;
  n.op = std::move(op);
  n.inputs = std::move(inputs);
  n.outputs = out_ids;
  n.name = std::move(name);
  nodes_.push_back(std::move(n));
  return out_ids;
}

Status Graph::mark_output(TensorId t) {
  if (finalized_) return FailedPreconditionError("mark_output: graph is already finalized");
  if (t >= tensors_.size())
    return InvalidArgumentError("mark_output: tensor " + std::to_string(t) + " is out of range");
  tensors_[t].is_graph_output = true;
  return OkStatus();
}

std::vector<NodeId> Graph::kahn_order() const {
  std::vector<std::size_t> indeg(nodes_.size());
  std::deque<NodeId> ready;
  for (std::size_t n = 0; n < nodes_.size(); ++n) {
    indeg[n] = nodes_[n].preds.size();
    if (indeg[n] == 0) ready.push_back(static_cast<NodeId>(n));
  }
  std::vector<NodeId> order;
  order.reserve(nodes_.size());
  while (!ready.empty()) {
    const NodeId n = ready.front();
    ready.pop_front();
    order.push_back(n);
    for (NodeId s : nodes_[n].succs)
      if (--indeg[s] == 0) ready.push_back(s);
  }
  return order;   // shorter than nodes_ means a cycle
}

Status Graph::finalize() {
  if (finalized_) return OkStatus();
  if (nodes_.empty()) return FailedPreconditionError("finalize: graph has no nodes");
  if (std::none_of(tensors_.begin(), tensors_.end(), [](const TensorDesc& t) { return t.is_graph_output; }))
    return InvalidArgumentError("finalize: graph has no outputs; call mark_output()");
  for (std::size_t n = 0; n < nodes_.size(); ++n)
    for (std::size_t i = 0; i < nodes_[n].inputs.size(); ++i) {
      const TensorDesc& d = tensors_[nodes_[n].inputs[i]];
      if (d.producer == kInvalidNode && !d.is_graph_input)
        return InvalidArgumentError("finalize: " + describe(static_cast<NodeId>(n)) + " input " +
                                    std::to_string(i) + " has no producer and is not a graph input");
    }

  for (TensorDesc& d : tensors_) d.consumers.clear();
  for (Node& nd : nodes_) {
    nd.preds.clear();
    nd.succs.clear();
  }
  for (std::size_t n = 0; n < nodes_.size(); ++n)
    for (TensorId t : nodes_[n].inputs) tensors_[t].consumers.push_back(static_cast<NodeId>(n));
  for (std::size_t n = 0; n < nodes_.size(); ++n) {
    auto& p = nodes_[n].preds;
    for (TensorId t : nodes_[n].inputs)
      if (tensors_[t].producer != kInvalidNode) p.push_back(tensors_[t].producer);
    std::sort(p.begin(), p.end());
    p.erase(std::unique(p.begin(), p.end()), p.end());
  }
  for (std::size_t n = 0; n < nodes_.size(); ++n)
    for (NodeId p : nodes_[n].preds) nodes_[p].succs.push_back(static_cast<NodeId>(n));

  const std::vector<NodeId> order = kahn_order();
  if (order.size() != nodes_.size()) {
    std::vector<bool> placed(nodes_.size(), false);
    for (NodeId n : order) placed[n] = true;
    std::string cyc;
    for (std::size_t n = 0; n < nodes_.size(); ++n)
      if (!placed[n]) cyc += (cyc.empty() ? "" : ", ") + describe(static_cast<NodeId>(n));
    return InternalError("finalize: graph has a cycle through [" + cyc + "]");
  }

  // ASAP depth, height, ALAP depth and slack.
  for (Node& nd : nodes_) nd.depth = 0;
  for (NodeId n : order)
    for (NodeId p : nodes_[n].preds) nodes_[n].depth = std::max(nodes_[n].depth, nodes_[p].depth + 1);
  int critical = 0;
  for (const Node& nd : nodes_) critical = std::max(critical, nd.depth);
  std::vector<int> height(nodes_.size(), 0);
  for (auto it = order.rbegin(); it != order.rend(); ++it)
    for (NodeId s : nodes_[*it].succs) height[*it] = std::max(height[*it], height[s] + 1);
  for (std::size_t n = 0; n < nodes_.size(); ++n) {
    nodes_[n].alap_depth = critical - height[n];
    nodes_[n].slack = nodes_[n].alap_depth - nodes_[n].depth;
  }

  // Dead nodes: those from which no graph output is reachable.
  std::vector<bool> alive(nodes_.size(), false);
  std::vector<NodeId> stack;
  for (const TensorDesc& t : tensors_)
    if (t.is_graph_output && t.producer != kInvalidNode && !alive[t.producer]) {
      alive[t.producer] = true;
      stack.push_back(t.producer);
    }
  while (!stack.empty()) {
    const NodeId n = stack.back();
    stack.pop_back();
    for (NodeId p : nodes_[n].preds)
      if (!alive[p]) {
        alive[p] = true;
        stack.push_back(p);
      }
  }
  for (std::size_t n = 0; n < nodes_.size(); ++n) nodes_[n].is_dead = !alive[n];
  finalized_ = true;
  return OkStatus();
}

StatusOr<std::vector<NodeId>> Graph::topological_order() const {
  if (!finalized_) return FailedPreconditionError("topological_order: call finalize() first");
  return kahn_order();
}

StatusOr<std::vector<std::vector<NodeId>>> Graph::levels() const {
  if (!finalized_) return FailedPreconditionError("levels: call finalize() first");
  int critical = 0;
  for (const Node& nd : nodes_) critical = std::max(critical, nd.depth);
  std::vector<std::vector<NodeId>> out(static_cast<std::size_t>(critical) + 1);
  for (std::size_t n = 0; n < nodes_.size(); ++n)
    out[static_cast<std::size_t>(nodes_[n].depth)].push_back(static_cast<NodeId>(n));
  return out;
}

StatusOr<std::size_t> Graph::max_level_width() const {
  MCKE_ASSIGN_OR_RETURN(std::vector<std::vector<NodeId>> lv, levels());
  std::size_t w = 0;
  for (const auto& l : lv) w = std::max(w, l.size());
  return w;
}

std::vector<NodeId> Graph::dead_nodes() const {
  std::vector<NodeId> out;
  for (std::size_t n = 0; n < nodes_.size(); ++n)
    if (nodes_[n].is_dead) out.push_back(static_cast<NodeId>(n));
  return out;
}

std::vector<Graph::LiveRange> Graph::compute_live_ranges(const std::vector<NodeId>& order) const {
  std::vector<LiveRange> lr(tensors_.size());
  for (std::size_t i = 0; i < order.size(); ++i) {
    const NodeId n = order[i];
    if (n >= nodes_.size()) continue;
    for (TensorId t : nodes_[n].outputs)
      if (lr[t].def_pos < 0) lr[t].def_pos = static_cast<int>(i);
    for (TensorId t : nodes_[n].inputs) lr[t].last_use_pos = std::max(lr[t].last_use_pos, static_cast<int>(i));
  }
  for (std::size_t t = 0; t < tensors_.size(); ++t) {
    if (tensors_[t].is_graph_input) lr[t].def_pos = -1;
    if (tensors_[t].is_graph_output) lr[t].last_use_pos = static_cast<int>(order.size());
    if (lr[t].last_use_pos < lr[t].def_pos) lr[t].last_use_pos = lr[t].def_pos;
  }
  return lr;
}

std::vector<Shape> Graph::input_shapes(NodeId n) const {
  std::vector<Shape> in;
  for (TensorId t : nodes_[n].inputs) in.push_back(tensors_[t].shape);
  return in;
}

OpCost Graph::total_cost() const {
  OpCost c;
  for (std::size_t n = 0; n < nodes_.size(); ++n) {
    if (!nodes_[n].op || nodes_[n].is_dead) continue;
    const OpCost k = nodes_[n].op->cost(input_shapes(static_cast<NodeId>(n)));
    c.flops += k.flops;
    c.bytes += k.bytes;
  }
  return c;
}

std::string Graph::to_dot() const {
  std::ostringstream os;
  os << "digraph mcke {\n  rankdir=TB;\n";
  for (std::size_t t = 0; t < tensors_.size(); ++t) {
    const TensorDesc& d = tensors_[t];
    os << "  t" << t << " [shape=box,label=\"" << d.name << "\\n" << d.shape.to_string() << "\""
       << (d.is_graph_output ? ",style=bold" : "") << "];\n";
  }
  for (std::size_t n = 0; n < nodes_.size(); ++n) {
    const Node& nd = nodes_[n];
    os << "  n" << n << " [shape=ellipse,label=\"" << nd.name << "\\n"
       << (nd.op ? std::string(nd.op->type_name()) : std::string("?")) << "\""
       << (nd.is_dead ? ",style=dashed" : "") << "];\n";
    for (TensorId t : nd.inputs) os << "  t" << t << " -> n" << n << ";\n";
    for (TensorId t : nd.outputs) os << "  n" << n << " -> t" << t << ";\n";
  }
  os << "}\n";
  return os.str();
}

}  // namespace mcke
