// mcke/graph/graph.hpp -- a DAG of Ops over SSA tensors.
//
// Same API as the reference's include/mcke/graph/graph.hpp (and graph.cpp:59-441):
// add_input / add_node (shapes inferred by the op) / mark_output / finalize
// (consumers, preds and succs, cycle detection, ASAP depth, ALAP depth and slack,
// and dead nodes that reach no output), plus a topological order, levels, live
// ranges over an order, the total ideal cost and a DOT dump.
#pragma once

#include <cassert>
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "mcke/core/status.hpp"
#include "mcke/graph/op.hpp"
#include "mcke/tensor/shape.hpp"

namespace mcke {

struct TensorDesc {
  Shape shape{};
  DType dtype = DType::kF32;
  NodeId producer = kInvalidNode;   // kInvalidNode: a graph input
  std::vector<NodeId> consumers;    // filled by finalize()
  std::string name;
  bool is_graph_input = false;
  bool is_graph_output = false;
  [[nodiscard]] bool reusable() const noexcept {
    return producer != kInvalidNode && !is_graph_input && !is_graph_output;
  }
};

struct Node {
  OpPtr op;
  std::vector<TensorId> inputs;
  std::vector<TensorId> outputs;
  std::string name;
  std::vector<NodeId> preds;
  std::vector<NodeId> succs;
  int depth = 0;
  int alap_depth = 0;
  int slack = 0;
  bool is_dead = false;
};

class Graph {
 public:
  Graph() = default;
  Graph(const Graph&) = delete;
  Graph& operator=(const Graph&) = delete;
  Graph(Graph&&) = default;
  Graph& operator=(Graph&&) = default;

  [[nodiscard]] StatusOr<TensorId> add_input(Shape shape, DType dtype, std::string name);
  [[nodiscard]] StatusOr<std::vector<TensorId>> add_node(OpPtr op, std::vector<TensorId> inputs,
                                                         std::string name);
  [[nodiscard]] Status mark_output(TensorId t);
  [[nodiscard]] Status finalize();
  [[nodiscard]] bool finalized() const noexcept { return finalized_; }

  [[nodiscard]] Op* node_op(NodeId n) {
    assert(n < nodes_.size());
    return nodes_[n].op.get();
  }
  [[nodiscard]] std::size_t num_nodes() const noexcept { return nodes_.size(); }
  [[nodiscard]] std::size_t num_tensors() const noexcept { return tensors_.size(); }
  [[nodiscard]] const Node& node(NodeId n) const {
    assert(n < nodes_.size());
    return nodes_[n];
  }
  [[nodiscard]] const TensorDesc& tensor(TensorId t) const {
    assert(t < tensors_.size());
    return tensors_[t];
  }

  [[nodiscard]] StatusOr<std::vector<NodeId>> topological_order() const;
  [[nodiscard]] StatusOr<std::vector<std::vector<NodeId>>> levels() const;
  [[nodiscard]] StatusOr<std::size_t> max_level_width() const;
  [[nodiscard]] std::vector<NodeId> dead_nodes() const;

  struct LiveRange {
    int def_pos = -1;
    int last_use_pos = -1;
  };
  [[nodiscard]] std::vector<LiveRange> compute_live_ranges(const std::vector<NodeId>& order) const;
  [[nodiscard]] OpCost total_cost() const;
  [[nodiscard]] std::string to_dot() const;
  // Input shapes of node n (for cost and workspace queries).
  [[nodiscard]] std::vector<Shape> input_shapes(NodeId n) const;

 private:
  [[nodiscard]] std::vector<NodeId> level_major_order() const;   // ASAP depth, then id
  [[nodiscard]] std::string describe(NodeId n) const;
  [[nodiscard]] std::string describe_tensor(TensorId t) const;

  std::vector<Node> nodes_;
  std::vector<TensorDesc> tensors_;
  bool finalized_ = false;
};

}  // namespace mcke
