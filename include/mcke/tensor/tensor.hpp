// mcke/tensor/tensor.hpp -- owning device Storage and Tensor views over it.
// Same API as the reference's include/mcke/tensor/tensor.hpp:64-186; copies go
// through the C-ABI's async memcpy on the given stream.
#pragma once

#include <cstddef>
#include <memory>
#include <string>
#include <utility>

#include "mcke/core/dtype.hpp"
#include "mcke/core/status.hpp"
#include "mcke/memory/allocator.hpp"
#include "mcke/runtime/stream.hpp"
#include "mcke/tensor/shape.hpp"

namespace mcke {

class Storage {
 public:
  [[nodiscard]] static StatusOr<std::shared_ptr<Storage>> create(DeviceAllocator& alloc,
                                                                 std::size_t bytes,
                                                                 rt::StreamHandle stream);
  Storage(const Storage&) = delete;
  Storage& operator=(const Storage&) = delete;
  ~Storage();
  [[nodiscard]] void* data() noexcept { return alloc_.ptr; }
  [[nodiscard]] const void* data() const noexcept { return alloc_.ptr; }
  [[nodiscard]] std::size_t bytes() const noexcept { return alloc_.bytes; }
  void note_use(rt::StreamHandle s) noexcept { last_use_stream_ = s; }
  [[nodiscard]] rt::StreamHandle last_use_stream() const noexcept { return last_use_stream_; }

 private:
  Storage(DeviceAllocator& a, Allocation alloc, rt::StreamHandle s)
      : allocator_(a), alloc_(alloc), last_use_stream_(s) {}
  DeviceAllocator& allocator_;
  Allocation alloc_{};
  rt::StreamHandle last_use_stream_{};
};

template <typename T>
struct TensorRef {
  T* data = nullptr;
  Shape shape{};
  MCKE_HOST_DEVICE dim_t numel() const noexcept { return shape.numel(); }
  MCKE_HOST_DEVICE dim_t rows() const noexcept { return shape.rows(); }
  MCKE_HOST_DEVICE dim_t cols() const noexcept { return shape.cols(); }
};

class Tensor {
 public:
  Tensor() = default;
  [[nodiscard]] static StatusOr<Tensor> empty(DeviceAllocator& alloc, Shape shape, DType dtype,
                                              rt::StreamHandle stream);
  [[nodiscard]] StatusOr<Tensor> reshape(Shape new_shape) const;
  [[nodiscard]] StatusOr<Tensor> slice(dim_t elem_offset, Shape shape) const;
  [[nodiscard]] static StatusOr<Tensor> from_storage(std::shared_ptr<Storage> s,
                                                     std::size_t byte_offset, Shape shape,
                                                     DType dtype);
  [[nodiscard]] const Shape& shape() const noexcept { return shape_; }
  [[nodiscard]] DType dtype() const noexcept { return dtype_; }
  [[nodiscard]] dim_t numel() const noexcept { return shape_.numel(); }
  [[nodiscard]] std::size_t nbytes() const noexcept { return shape_.bytes(dtype_); }
  [[nodiscard]] bool defined() const noexcept { return storage_ != nullptr; }
  [[nodiscard]] void* data_ptr() const noexcept {
    return storage_ ? static_cast<char*>(storage_->data()) + byte_offset_ : nullptr;
  }
  template <typename T>
  [[nodiscard]] T* data_as() const {
    if (dtype_ != kDTypeOf<T>) return nullptr;
    return static_cast<T*>(data_ptr());
  }
  template <typename T>
  [[nodiscard]] TensorRef<T> ref() const {
    return TensorRef<T>{data_as<T>(), shape_};
  }
  void note_use(rt::StreamHandle s) const {
    if (storage_) storage_->note_use(s);
  }
  [[nodiscard]] const std::shared_ptr<Storage>& storage() const noexcept { return storage_; }
  [[nodiscard]] std::size_t byte_offset() const noexcept { return byte_offset_; }
  [[nodiscard]] std::string to_string() const;
  [[nodiscard]] Status copy_from_host(const void* src, std::size_t bytes, rt::StreamHandle stream);
  [[nodiscard]] Status copy_to_host(void* dst, std::size_t bytes, rt::StreamHandle stream) const;

 private:
  Tensor(std::shared_ptr<Storage> s, std::size_t byte_offset, Shape shape, DType dt)
      : storage_(std::move(s)), byte_offset_(byte_offset), shape_(shape), dtype_(dt) {}
  std::shared_ptr<Storage> storage_;
  std::size_t byte_offset_ = 0;
  Shape shape_{};
  DType dtype_ = DType::kF32;
};

}  // namespace mcke
