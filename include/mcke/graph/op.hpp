// mcke/graph/op.hpp -- the operator interface of the graph layer and the four
// kernel-backed operators.
//
// Same API as the reference's include/mcke/graph/op.hpp:72-303: an Op infers its
// output shapes, states its ideal cost (the algorithmic flops and compulsory
// bytes that every roofline number in this tree divides by), declares its
// workspace, and launches its kernel on the stream and workspace in OpContext.
// GemmParams gains `auto_tile`: with kMfmaF32 the tile is then chosen per shape
// at launch (kernels::mfma_default_tile).
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <string_view>
#include <vector>

#include "mcke/core/device.hpp"
#include "mcke/core/status.hpp"
#include "mcke/kernels/kernels.hpp"
#include "mcke/runtime/stream.hpp"
#include "mcke/tensor/tensor.hpp"

namespace mcke {

using TensorId = std::uint32_t;
using NodeId = std::uint32_t;
inline constexpr TensorId kInvalidTensor = 0xFFFFFFFFu;
inline constexpr NodeId kInvalidNode = 0xFFFFFFFFu;

struct OpContext {
  rt::StreamHandle stream = {};
  const DeviceInfo* device = nullptr;
  void* workspace = nullptr;
  std::size_t workspace_bytes = 0;
};

struct OpCost {
  std::uint64_t flops = 0;   // useful floating-point operations
  std::uint64_t bytes = 0;   // inputs read once + outputs written once
  [[nodiscard]] double arithmetic_intensity() const {
    return bytes ? static_cast<double>(flops) / static_cast<double>(bytes) : 0.0;
  }
};

class Op {
 public:
  virtual ~Op() = default;
  [[nodiscard]] virtual std::string_view type_name() const = 0;
  [[nodiscard]] virtual Status launch(const OpContext& ctx, const std::vector<Tensor>& inputs,
                                      const std::vector<Tensor>& outputs) = 0;
  [[nodiscard]] virtual StatusOr<std::vector<Shape>> infer_shapes(
      const std::vector<Shape>& input_shapes) const = 0;
  [[nodiscard]] virtual OpCost cost(const std::vector<Shape>& input_shapes) const = 0;
  [[nodiscard]] virtual std::size_t workspace_bytes(const std::vector<Shape>&) const { return 0; }
  // Element type of the outputs from those of the inputs (no reference
  // counterpart: the reference's graph is fp32 throughout).  The default accepts
  // fp32 inputs only and produces fp32; GemmOp also takes 16-bit inputs.
  [[nodiscard]] virtual StatusOr<DType> infer_dtype(const std::vector<DType>& input_dtypes) const;
};

using OpPtr = std::unique_ptr<Op>;

struct GemmParams {
  float alpha = 1.f;
  float beta = 0.f;
  using Variant = kernels::GemmVariant;
  Variant variant = Variant::kTiledRegBlock;
  kernels::GemmTile tile{};
  bool auto_tile = false;   // kMfmaF32 (or 16-bit inputs): pick the tile per shape at launch
  // Element types (this build's addition).  kF32 inputs run `variant`;
  // kBF16 / kF16 inputs run the 16-bit MFMA GEMM (kernels::launch_gemm_lp, whose
  // tiles are gemm_lp_tile_is_supported's), with C in out_dtype (kF32 or the
  // input type).
  DType in_dtype = DType::kF32;
  DType out_dtype = DType::kF32;
};

class GemmOp final : public Op {
 public:
  explicit GemmOp(GemmParams p) : p_(p) {}
  [[nodiscard]] std::string_view type_name() const override { return "Gemm"; }
  [[nodiscard]] Status launch(const OpContext&, const std::vector<Tensor>&,
                              const std::vector<Tensor>&) override;
  [[nodiscard]] StatusOr<std::vector<Shape>> infer_shapes(const std::vector<Shape>&) const override;
  [[nodiscard]] OpCost cost(const std::vector<Shape>&) const override;
  [[nodiscard]] StatusOr<DType> infer_dtype(const std::vector<DType>&) const override;
  [[nodiscard]] const GemmParams& params() const noexcept { return p_; }

 private:
  GemmParams p_;
};

struct BiasActParams {
  enum class Act { kNone, kRelu, kGeluErf, kGeluTanh } act = Act::kGeluErf;
  int vector_width = 0;     // 0 = widest legal width at launch
  int max_row_blocks = 0;
};

class BiasActOp final : public Op {
 public:
  explicit BiasActOp(BiasActParams p) : p_(p) {}
  [[nodiscard]] std::string_view type_name() const override { return "BiasAct"; }
  [[nodiscard]] Status launch(const OpContext&, const std::vector<Tensor>&,
                              const std::vector<Tensor>&) override;
  [[nodiscard]] StatusOr<std::vector<Shape>> infer_shapes(const std::vector<Shape>&) const override;
  [[nodiscard]] OpCost cost(const std::vector<Shape>&) const override;

 private:
  BiasActParams p_;
};

// GEMM with the bias + activation in its epilogue (no reference counterpart: the
// reference chains GemmOp and BiasActOp).  Inputs A [m,k], B [k,n] and bias [n],
// all fp32; y = act(alpha * A B + bias[col]) through
// kernels::launch_gemm_bias_act_f32 (kMfmaF32), with the bits of the GemmOp ->
// BiasActOp pair it replaces.  C never reaches memory, so the op costs the pair's
// flops and the GEMM's bytes plus the bias.
struct GemmBiasActParams {
  float alpha = 1.f;
  BiasActParams::Act act = BiasActParams::Act::kGeluTanh;
  kernels::GemmTile tile{};
  bool auto_tile = true;    // pick the kMfmaF32 tile per shape at launch
};

class GemmBiasActOp final : public Op {
 public:
  explicit GemmBiasActOp(GemmBiasActParams p) : p_(p) {}
  [[nodiscard]] std::string_view type_name() const override { return "GemmBiasAct"; }
  [[nodiscard]] Status launch(const OpContext&, const std::vector<Tensor>&,
                              const std::vector<Tensor>&) override;
  [[nodiscard]] StatusOr<std::vector<Shape>> infer_shapes(const std::vector<Shape>&) const override;
  [[nodiscard]] OpCost cost(const std::vector<Shape>&) const override;
  [[nodiscard]] const GemmBiasActParams& params() const noexcept { return p_; }

 private:
  GemmBiasActParams p_;
};

struct ReduceParams {
  enum class Kind { kSum, kMax, kMean } kind = Kind::kSum;
  int axis = -1;
  enum class Variant { kSmemTree, kWarpShuffle, kTwoPass } variant = Variant::kWarpShuffle;
};

class ReduceOp final : public Op {
 public:
  explicit ReduceOp(ReduceParams p) : p_(p) {}
  [[nodiscard]] std::string_view type_name() const override { return "Reduce"; }
  [[nodiscard]] Status launch(const OpContext&, const std::vector<Tensor>&,
                              const std::vector<Tensor>&) override;
  [[nodiscard]] StatusOr<std::vector<Shape>> infer_shapes(const std::vector<Shape>&) const override;
  [[nodiscard]] OpCost cost(const std::vector<Shape>&) const override;
  [[nodiscard]] std::size_t workspace_bytes(const std::vector<Shape>&) const override;

 private:
  ReduceParams p_;
};

struct SoftmaxParams {
  int axis = -1;
  bool numerically_stable = true;
  enum class Variant { kThreePass, kOnlineOnePass } variant = Variant::kOnlineOnePass;
};

class SoftmaxOp final : public Op {
 public:
  explicit SoftmaxOp(SoftmaxParams p) : p_(p) {}
  [[nodiscard]] std::string_view type_name() const override { return "Softmax"; }
  [[nodiscard]] Status launch(const OpContext&, const std::vector<Tensor>&,
                              const std::vector<Tensor>&) override;
  [[nodiscard]] StatusOr<std::vector<Shape>> infer_shapes(const std::vector<Shape>&) const override;
  [[nodiscard]] OpCost cost(const std::vector<Shape>&) const override;

 private:
  SoftmaxParams p_;
};

}  // namespace mcke
