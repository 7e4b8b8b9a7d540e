// ops.cpp -- the four kernel-backed operators: shape inference, ideal cost and
// launch.  Reference counterparts: src/graph/ops_gemm.cpp:15-96,
// ops_bias_act.cpp:30-130, ops_reduce.cpp:18-133, ops_softmax.cpp:11-83.
//
// Ideal costs (the roofline numerators, kept identical to the reference's):
//   Gemm     flops 2mnk,                     bytes (mk + kn + mn) * 4
//   BiasAct  flops n * {1, 2, 22, 10} for {none, relu, gelu_erf, gelu_tanh},
//            bytes (2n + cols) * 4
//   Reduce   flops rows * (cols - 1) (0 for max), bytes (rows * cols + rows) * 4
//   Softmax  flops 5n,                       bytes 2n * 4
#include <algorithm>
#include <string>

#include "mcke/graph/op.hpp"

namespace mcke {

namespace {

static_assert(static_cast<int>(BiasActParams::Act::kNone) == static_cast<int>(kernels::Activation::kNone));
static_assert(static_cast<int>(BiasActParams::Act::kRelu) == static_cast<int>(kernels::Activation::kRelu));
static_assert(static_cast<int>(BiasActParams::Act::kGeluErf) == static_cast<int>(kernels::Activation::kGeluErf));
static_assert(static_cast<int>(BiasActParams::Act::kGeluTanh) == static_cast<int>(kernels::Activation::kGeluTanh));
static_assert(static_cast<int>(ReduceParams::Kind::kSum) == static_cast<int>(kernels::ReduceKind::kSum));
static_assert(static_cast<int>(ReduceParams::Kind::kMax) == static_cast<int>(kernels::ReduceKind::kMax));
static_assert(static_cast<int>(ReduceParams::Kind::kMean) == static_cast<int>(kernels::ReduceKind::kMean));
static_assert(static_cast<int>(ReduceParams::Variant::kSmemTree) == static_cast<int>(kernels::ReduceVariant::kSmemTree));
static_assert(static_cast<int>(ReduceParams::Variant::kWarpShuffle) == static_cast<int>(kernels::ReduceVariant::kWarpShuffle));
static_assert(static_cast<int>(ReduceParams::Variant::kTwoPass) == static_cast<int>(kernels::ReduceVariant::kTwoPass));
static_assert(static_cast<int>(SoftmaxParams::Variant::kThreePass) == static_cast<int>(kernels::SoftmaxVariant::kThreePass));
static_assert(static_cast<int>(SoftmaxParams::Variant::kOnlineOnePass) == static_cast<int>(kernels::SoftmaxVariant::kOnlineOnePass));

std::uint64_t act_flops_per_elem(BiasActParams::Act a) {
  switch (a) {
    case BiasActParams::Act::kNone: return 1;
    case BiasActParams::Act::kRelu: return 2;
    case BiasActParams::Act::kGeluTanh: return 10;
    case BiasActParams::Act::kGeluErf: return 22;
  }
  return 0;
}

bool last_axis(int axis, int rank) { return axis == -1 || axis == rank - 1; }

std::string tile_str(const kernels::GemmTile& t) {
  return "(" + std::to_string(t.bm) + "," + std::to_string(t.bn) + "," + std::to_string(t.bk) + "," +
         std::to_string(t.tm) + "," + std::to_string(t.tn) + ")";
}

bool lp_dtype(DType t) { return t == DType::kBF16 || t == DType::kF16; }

}  // namespace

StatusOr<DType> Op::infer_dtype(const std::vector<DType>& in) const {
  for (std::size_t i = 0; i < in.size(); ++i)
    if (in[i] != DType::kF32)
      return InvalidArgumentError(std::string(type_name()) + ": input " + std::to_string(i) +
                                  " is " + std::string(dtype_name(in[i])) +
                                  "; this operator runs on f32 tensors only");
  return DType::kF32;
}

// ---------------------------------------------------------------------------
StatusOr<DType> GemmOp::infer_dtype(const std::vector<DType>& in) const {
  if (in.size() != 2)
    return InvalidArgumentError("GemmOp: expects 2 inputs (A, B), got " + std::to_string(in.size()));
  if (in[0] != p_.in_dtype || in[1] != p_.in_dtype)
    return InvalidArgumentError("GemmOp: inputs are " + std::string(dtype_name(in[0])) + " and " +
                                std::string(dtype_name(in[1])) + " but the op was built for " +
                                std::string(dtype_name(p_.in_dtype)));
  if (p_.in_dtype == DType::kF32) {
    if (p_.out_dtype != DType::kF32)
      return InvalidArgumentError("GemmOp: f32 inputs produce f32 C");
    return DType::kF32;
  }
  if (!lp_dtype(p_.in_dtype))
    return InvalidArgumentError("GemmOp: inputs must be f32, bf16 or f16");
  if (p_.out_dtype != DType::kF32 && p_.out_dtype != p_.in_dtype)
    return InvalidArgumentError("GemmOp: 16-bit inputs produce C in f32 or the input type");
  return p_.out_dtype;
}

StatusOr<std::vector<Shape>> GemmOp::infer_shapes(const std::vector<Shape>& in) const {
  if (in.size() != 2)
    return InvalidArgumentError("GemmOp: expects 2 inputs (A, B), got " + std::to_string(in.size()));
  if (in[0].rank() != 2 || in[1].rank() != 2)
    return InvalidArgumentError("GemmOp: both inputs must be rank 2, got ranks " +
                                std::to_string(in[0].rank()) + " and " + std::to_string(in[1].rank()));
  const dim_t m = in[0].dim(0), k = in[0].dim(1), k2 = in[1].dim(0), n = in[1].dim(1);
  if (k != k2)
    return InvalidArgumentError("GemmOp: inner dimensions disagree: A is [" + std::to_string(m) + "," +
                                std::to_string(k) + "], B is [" + std::to_string(k2) + "," +
                                std::to_string(n) + "]");
  if (p_.beta != 0.0f)
    return UnimplementedError("GemmOp: beta != 0 reads C, which the graph does not model as an "
                              "input; add the term with a separate node");
  if (lp_dtype(p_.in_dtype)) {
    if (!p_.auto_tile && !kernels::gemm_lp_tile_is_supported(p_.tile))
      return InvalidArgumentError("GemmOp: tile " + tile_str(p_.tile) +
                                  " is not instantiated for the 16-bit GEMM ((256,256,64,16,16), "
                                  "(128,128,64,8,8), (64,64,64,4,4))");
    return std::vector<Shape>{Shape{m, n}};
  }
  const bool auto_mfma = p_.auto_tile && p_.variant == kernels::GemmVariant::kMfmaF32;
  if (!auto_mfma && !kernels::gemm_tile_is_supported(p_.variant, p_.tile))
    return InvalidArgumentError("GemmOp: tile " + tile_str(p_.tile) +
                                " is not instantiated for this variant (kTiledSmem: (32,32,32,1,1); "
                                "register-blocked variants: (128,128,8,8,8); kMfmaF32: "
                                "(256,256,32|16,16,16), (128,128,32|16,8,8), (64,64,32,4,4))");
  return std::vector<Shape>{Shape{m, n}};
}

OpCost GemmOp::cost(const std::vector<Shape>& in) const {
  OpCost c;
  if (in.size() != 2 || in[0].rank() != 2 || in[1].rank() != 2) return c;
  const auto m = static_cast<std::uint64_t>(in[0].dim(0));
  const auto k = static_cast<std::uint64_t>(in[0].dim(1));
  const auto n = static_cast<std::uint64_t>(in[1].dim(1));
  c.flops = 2ull * m * n * k;
  c.bytes = (m * k + k * n) * dtype_size(p_.in_dtype) + m * n * dtype_size(p_.out_dtype);
  return c;
}

Status GemmOp::launch(const OpContext& ctx, const std::vector<Tensor>& inputs,
                      const std::vector<Tensor>& outputs) {
  if (inputs.size() != 2 || outputs.size() != 1)
    return InvalidArgumentError("GemmOp::launch: expects 2 inputs and 1 output");
  if (lp_dtype(p_.in_dtype)) {
    if (inputs[0].dtype() != p_.in_dtype || inputs[1].dtype() != p_.in_dtype ||
        outputs[0].dtype() != p_.out_dtype)
      return InvalidArgumentError("GemmOp::launch: tensor types do not match the op's");
    const dim_t m = inputs[0].shape().dim(0), k = inputs[0].shape().dim(1),
                n = inputs[1].shape().dim(1);
    const kernels::GemmTile tile = p_.auto_tile ? kernels::lp_default_tile(m, n, k) : p_.tile;
    return kernels::launch_gemm_lp(inputs[0].data_ptr(), inputs[1].data_ptr(), outputs[0].data_ptr(),
                                   p_.in_dtype, p_.out_dtype, m, n, k, p_.alpha, p_.beta, tile,
                                   ctx.stream);
  }
  const float* a = inputs[0].data_as<float>();
  const float* b = inputs[1].data_as<float>();
  float* c = outputs[0].data_as<float>();
  if (!a || !b || !c) return InvalidArgumentError("GemmOp::launch: a tensor is undefined or not f32");
  const dim_t m = inputs[0].shape().dim(0), k = inputs[0].shape().dim(1), n = inputs[1].shape().dim(1);
  kernels::GemmTile tile = p_.tile;
  if (p_.auto_tile && p_.variant == kernels::GemmVariant::kMfmaF32) tile = kernels::mfma_default_tile(m, n, k);
  return kernels::launch_gemm_f32(a, b, c, m, n, k, p_.alpha, p_.beta, p_.variant, tile, ctx.stream);
}

// ---------------------------------------------------------------------------
StatusOr<std::vector<Shape>> BiasActOp::infer_shapes(const std::vector<Shape>& in) const {
  if (in.size() != 2)
    return InvalidArgumentError("BiasActOp: expects 2 inputs (x, bias), got " + std::to_string(in.size()));
  if (in[1].rank() != 1)
    return InvalidArgumentError("BiasActOp: bias must be rank 1, got rank " + std::to_string(in[1].rank()));
  if (in[1].dim(0) != in[0].cols())
    return InvalidArgumentError("BiasActOp: bias length " + std::to_string(in[1].dim(0)) +
                                " does not match x's last dimension " + std::to_string(in[0].cols()));
  if (p_.vector_width != 0 && p_.vector_width != 1 && p_.vector_width != 2 && p_.vector_width != 4)
    return InvalidArgumentError("BiasActOp: vector_width must be 0 (auto), 1, 2 or 4");
  if (p_.vector_width > 1 && in[0].cols() % p_.vector_width != 0)
    return InvalidArgumentError("BiasActOp: cols " + std::to_string(in[0].cols()) +
                                " is not a multiple of vector_width " + std::to_string(p_.vector_width));
  return std::vector<Shape>{in[0]};
}

OpCost BiasActOp::cost(const std::vector<Shape>& in) const {
  OpCost c;
  if (in.empty()) return c;
  const auto n = static_cast<std::uint64_t>(in[0].numel());
  const auto cols = static_cast<std::uint64_t>(in[0].cols());
  c.flops = n * act_flops_per_elem(p_.act);
  c.bytes = (2ull * n + cols) * sizeof(float);
  return c;
}

Status BiasActOp::launch(const OpContext& ctx, const std::vector<Tensor>& inputs,
                         const std::vector<Tensor>& outputs) {
  if (inputs.size() != 2 || outputs.size() != 1)
    return InvalidArgumentError("BiasActOp::launch: expects 2 inputs and 1 output");
  const float* x = inputs[0].data_as<float>();
  const float* bias = inputs[1].data_as<float>();
  float* y = outputs[0].data_as<float>();
  if (!x || !bias || !y) return InvalidArgumentError("BiasActOp::launch: a tensor is undefined or not f32");
  const dim_t rows = inputs[0].shape().rows(), cols = inputs[0].shape().cols();
  const int vw = p_.vector_width != 0
                     ? p_.vector_width
                     : std::min({kernels::max_vector_width_f32(x, cols), kernels::max_vector_width_f32(y, cols),
                                 kernels::max_vector_width_f32(bias, cols)});
  return kernels::launch_bias_act_f32(x, bias, y, rows, cols, static_cast<kernels::Activation>(p_.act), vw,
                                      ctx.stream, p_.max_row_blocks);
}

// ---------------------------------------------------------------------------
StatusOr<std::vector<Shape>> GemmBiasActOp::infer_shapes(const std::vector<Shape>& in) const {
  if (in.size() != 3)
    return InvalidArgumentError("GemmBiasActOp: expects 3 inputs (A, B, bias), got " +
                                std::to_string(in.size()));
  if (in[0].rank() != 2 || in[1].rank() != 2 || in[2].rank() != 1)
    return InvalidArgumentError("GemmBiasActOp: A and B must be rank 2 and the bias rank 1");
  const dim_t m = in[0].dim(0), k = in[0].dim(1), k2 = in[1].dim(0), n = in[1].dim(1);
  if (k != k2)
    return InvalidArgumentError("GemmBiasActOp: inner dimensions disagree: A is [" +
                                std::to_string(m) + "," + std::to_string(k) + "], B is [" +
                                std::to_string(k2) + "," + std::to_string(n) + "]");
  if (in[2].dim(0) != n)
    return InvalidArgumentError("GemmBiasActOp: bias length " + std::to_string(in[2].dim(0)) +
                                " does not match B's columns " + std::to_string(n));
  if (!p_.auto_tile && !kernels::gemm_tile_is_supported(kernels::GemmVariant::kMfmaF32, p_.tile))
    return InvalidArgumentError("GemmBiasActOp: tile " + tile_str(p_.tile) +
                                " is not a kMfmaF32 tile ((256,256,32|16,16,16), "
                                "(128,128,32|16,8,8), (64,64,32,4,4), (32,32,32,2,2))");
  return std::vector<Shape>{Shape{m, n}};
}

OpCost GemmBiasActOp::cost(const std::vector<Shape>& in) const {
  OpCost c;
  if (in.size() != 3 || in[0].rank() != 2 || in[1].rank() != 2) return c;
  const auto m = static_cast<std::uint64_t>(in[0].dim(0));
  const auto k = static_cast<std::uint64_t>(in[0].dim(1));
  const auto n = static_cast<std::uint64_t>(in[1].dim(1));
  c.flops = 2ull * m * n * k + m * n * act_flops_per_elem(p_.act);
  c.bytes = (m * k + k * n + n + m * n) * sizeof(float);
  return c;
}

Status GemmBiasActOp::launch(const OpContext& ctx, const std::vector<Tensor>& inputs,
                             const std::vector<Tensor>& outputs) {
  if (inputs.size() != 3 || outputs.size() != 1)
    return InvalidArgumentError("GemmBiasActOp::launch: expects 3 inputs and 1 output");
  const float* a = inputs[0].data_as<float>();
  const float* b = inputs[1].data_as<float>();
  const float* bias = inputs[2].data_as<float>();
  float* y = outputs[0].data_as<float>();
  if (!a || !b || !bias || !y)
    return InvalidArgumentError("GemmBiasActOp::launch: a tensor is undefined or not f32");
  const dim_t m = inputs[0].shape().dim(0), k = inputs[0].shape().dim(1), n = inputs[1].shape().dim(1);
  const kernels::GemmTile tile = p_.auto_tile ? kernels::mfma_default_tile(m, n, k) : p_.tile;
  return kernels::launch_gemm_bias_act_f32(a, b, bias, y, m, n, k, p_.alpha,
                                           static_cast<kernels::Activation>(p_.act), tile,
                                           ctx.stream);
}

// ---------------------------------------------------------------------------
StatusOr<std::vector<Shape>> ReduceOp::infer_shapes(const std::vector<Shape>& in) const {
  if (in.size() != 1)
    return InvalidArgumentError("ReduceOp: expects 1 input, got " + std::to_string(in.size()));
  if (!last_axis(p_.axis, in[0].rank()))
    return InvalidArgumentError("ReduceOp: axis " + std::to_string(p_.axis) +
                                " is not the last axis of a rank-" + std::to_string(in[0].rank()) +
                                " tensor; the kernels reduce rows only");
  const int r = in[0].rank();
  if (r <= 1) return std::vector<Shape>{Shape{1}};
  dim_t dims[kMaxRank]{};
  for (int i = 0; i < r - 1; ++i) dims[i] = in[0].dim(i);
  return std::vector<Shape>{Shape(dims, r - 1)};
}

OpCost ReduceOp::cost(const std::vector<Shape>& in) const {
  OpCost c;
  if (in.empty()) return c;
  const auto rows = static_cast<std::uint64_t>(in[0].rows());
  const auto cols = static_cast<std::uint64_t>(in[0].cols());
  c.flops = (p_.kind == ReduceParams::Kind::kMax) ? 0ull : rows * (cols > 0 ? cols - 1 : 0);
  c.bytes = (rows * cols + rows) * sizeof(float);
  return c;
}

std::size_t ReduceOp::workspace_bytes(const std::vector<Shape>& in) const {
  if (in.empty()) return 0;
  return kernels::row_reduce_workspace_bytes(in[0].rows(), in[0].cols(),
                                             static_cast<kernels::ReduceVariant>(p_.variant));
}

Status ReduceOp::launch(const OpContext& ctx, const std::vector<Tensor>& inputs,
                        const std::vector<Tensor>& outputs) {
  if (inputs.size() != 1 || outputs.size() != 1)
    return InvalidArgumentError("ReduceOp::launch: expects 1 input and 1 output");
  const float* x = inputs[0].data_as<float>();
  float* out = outputs[0].data_as<float>();
  if (!x || !out) return InvalidArgumentError("ReduceOp::launch: a tensor is undefined or not f32");
  return kernels::launch_row_reduce_f32(x, out, inputs[0].shape().rows(), inputs[0].shape().cols(),
                                        static_cast<kernels::ReduceKind>(p_.kind),
                                        static_cast<kernels::ReduceVariant>(p_.variant),
                                        static_cast<float*>(ctx.workspace), ctx.workspace_bytes, ctx.stream);
}

// ---------------------------------------------------------------------------
StatusOr<std::vector<Shape>> SoftmaxOp::infer_shapes(const std::vector<Shape>& in) const {
  if (in.size() != 1)
    return InvalidArgumentError("SoftmaxOp: expects 1 input, got " + std::to_string(in.size()));
  if (!last_axis(p_.axis, in[0].rank()))
    return InvalidArgumentError("SoftmaxOp: axis " + std::to_string(p_.axis) +
                                " is not the last axis; the kernels are row-wise only");
  if (!p_.numerically_stable)
    return UnimplementedError("SoftmaxOp: numerically_stable = false is not implemented; every "
                              "kernel subtracts the row max");
  return std::vector<Shape>{in[0]};
}

OpCost SoftmaxOp::cost(const std::vector<Shape>& in) const {
  OpCost c;
  if (in.empty()) return c;
  const auto n = static_cast<std::uint64_t>(in[0].numel());
  c.flops = n * 5ull;
  c.bytes = 2ull * n * sizeof(float);
  return c;
}

Status SoftmaxOp::launch(const OpContext& ctx, const std::vector<Tensor>& inputs,
                         const std::vector<Tensor>& outputs) {
  if (inputs.size() != 1 || outputs.size() != 1)
    return InvalidArgumentError("SoftmaxOp::launch: expects 1 input and 1 output");
  const float* x = inputs[0].data_as<float>();
  float* y = outputs[0].data_as<float>();
  if (!x || !y) return InvalidArgumentError("SoftmaxOp::launch: a tensor is undefined or not f32");
  return kernels::launch_row_softmax_f32(x, y, inputs[0].shape().rows(), inputs[0].shape().cols(),
                                         static_cast<kernels::SoftmaxVariant>(p_.variant), ctx.stream);
}

}  // namespace mcke
