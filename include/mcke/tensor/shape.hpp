// mcke/tensor/shape.hpp -- rank <= 5 shapes with row-major contiguous strides.
// Same API as the reference's include/mcke/tensor/shape.hpp:38-178 (rows() is
// the product of every dimension but the last, cols() the last).
#pragma once

#include <cassert>
#include <cstddef>
#include <cstdint>
#include <initializer_list>
#include <string>

#include "mcke/core/config.hpp"
#include "mcke/core/dtype.hpp"

namespace mcke {

inline constexpr int kMaxRank = 5;
using dim_t = std::int64_t;

class Shape {
 public:
  Shape() = default;
  Shape(std::initializer_list<dim_t> dims) {
    assert(dims.size() <= static_cast<std::size_t>(kMaxRank) && "Shape: rank exceeds kMaxRank");
    for (dim_t d : dims) {
      if (rank_ >= kMaxRank) break;
      dims_[rank_++] = d;
    }
    make_strides();
  }
  Shape(const dim_t* dims, int rank) {
    assert(rank >= 0 && rank <= kMaxRank && "Shape: rank out of range");
    rank_ = rank < 0 ? 0 : (rank > kMaxRank ? kMaxRank : rank);
    for (int i = 0; i < rank_; ++i) dims_[i] = dims[i];
    make_strides();
  }
  [[nodiscard]] static bool rank_is_representable(std::size_t rank) noexcept {
    return rank <= static_cast<std::size_t>(kMaxRank);
  }
  MCKE_HOST_DEVICE int rank() const noexcept { return rank_; }
  MCKE_HOST_DEVICE dim_t dim(int i) const noexcept { return dims_[i]; }
  MCKE_HOST_DEVICE dim_t stride(int i) const noexcept { return strides_[i]; }
  MCKE_HOST_DEVICE dim_t numel() const noexcept {
    dim_t n = 1;
    for (int i = 0; i < rank_; ++i) n *= dims_[i];
    return n;
  }
  MCKE_HOST_DEVICE std::size_t bytes(DType t) const noexcept {
    return static_cast<std::size_t>(numel()) * dtype_size(t);
  }
  MCKE_HOST_DEVICE bool is_contiguous() const noexcept {
    dim_t expect = 1;
    for (int i = rank_ - 1; i >= 0; --i) {
      if (strides_[i] != expect) return false;
      expect *= dims_[i];
    }
    return true;
  }
  MCKE_HOST_DEVICE dim_t offset_of(const dim_t* idx) const noexcept {
    dim_t off = 0;
    for (int i = 0; i < rank_; ++i) off += idx[i] * strides_[i];
    return off;
  }
  MCKE_HOST_DEVICE dim_t rows() const noexcept {
    dim_t r = 1;
    for (int i = 0; i + 1 < rank_; ++i) r *= dims_[i];
    return r;
  }
  MCKE_HOST_DEVICE dim_t cols() const noexcept { return rank_ > 0 ? dims_[rank_ - 1] : 0; }
  [[nodiscard]] bool operator==(const Shape& o) const noexcept {
    if (rank_ != o.rank_) return false;
    for (int i = 0; i < rank_; ++i)
      if (dims_[i] != o.dims_[i] || strides_[i] != o.strides_[i]) return false;
    return true;
  }
  [[nodiscard]] std::string to_string() const {
    std::string s = "[";
    for (int i = 0; i < rank_; ++i) s += std::to_string(dims_[i]) + (i + 1 < rank_ ? "," : "");
    return s + "]";
  }

 private:
  MCKE_HOST_DEVICE void make_strides() noexcept {
    dim_t acc = 1;
    for (int i = rank_ - 1; i >= 0; --i) {
      strides_[i] = acc;
      acc *= dims_[i];
    }
  }
  dim_t dims_[kMaxRank]{};
  dim_t strides_[kMaxRank]{};
  int rank_ = 0;
};

}  // namespace mcke
