// tensor.cpp -- Storage and Tensor (reference src/tensor/tensor.cpp:22-138).
#include "mcke/tensor/tensor.hpp"

#include <sstream>

#include "mcke_amd.h"

namespace mcke {

StatusOr<std::shared_ptr<Storage>> Storage::create(DeviceAllocator& alloc, std::size_t bytes,
                                                   rt::StreamHandle stream) {
  if (bytes == 0) return InvalidArgumentError("Storage::create: zero bytes");
  MCKE_ASSIGN_OR_RETURN(Allocation a, alloc.allocate(bytes, stream));
  return std::shared_ptr<Storage>(new Storage(alloc, a, stream));
}

Storage::~Storage() {
  // Stream-ordered release: the allocator parks the block until work already
  // queued on the last stream that used it has finished.
  if (alloc_.ptr) (void)allocator_.deallocate(alloc_, last_use_stream_);
}

StatusOr<Tensor> Tensor::empty(DeviceAllocator& alloc, Shape shape, DType dtype,
                               rt::StreamHandle stream) {
  const std::size_t bytes = shape.bytes(dtype);
  if (bytes == 0) return InvalidArgumentError("Tensor::empty: shape " + shape.to_string() + " is empty");
  MCKE_ASSIGN_OR_RETURN(std::shared_ptr<Storage> s, Storage::create(alloc, bytes, stream));
  return Tensor(std::move(s), 0, shape, dtype);
}

StatusOr<Tensor> Tensor::reshape(Shape new_shape) const {
  if (new_shape.numel() != shape_.numel())
    return InvalidArgumentError("Tensor::reshape: " + shape_.to_string() + " -> " +
                                new_shape.to_string() + " changes the element count");
  return Tensor(storage_, byte_offset_, new_shape, dtype_);
}

StatusOr<Tensor> Tensor::slice(dim_t elem_offset, Shape shape) const {
  if (elem_offset < 0 || elem_offset + shape.numel() > shape_.numel())
    return InvalidArgumentError("Tensor::slice: out of range");
  return Tensor(storage_, byte_offset_ + static_cast<std::size_t>(elem_offset) * dtype_size(dtype_),
                shape, dtype_);
}

StatusOr<Tensor> Tensor::from_storage(std::shared_ptr<Storage> s, std::size_t byte_offset,
                                      Shape shape, DType dtype) {
  if (!s) return InvalidArgumentError("Tensor::from_storage: null storage");
  if (byte_offset + shape.bytes(dtype) > s->bytes())
    return InvalidArgumentError("Tensor::from_storage: view [" + std::to_string(byte_offset) + ", " +
                                std::to_string(byte_offset + shape.bytes(dtype)) +
                                ") exceeds the storage's " + std::to_string(s->bytes()) + " bytes");
  return Tensor(std::move(s), byte_offset, shape, dtype);
}

std::string Tensor::to_string() const {
  std::ostringstream os;
  os << "Tensor" << shape_.to_string() << " " << dtype_name(dtype_) << " @" << data_ptr();
  return os.str();
}

Status Tensor::copy_from_host(const void* src, std::size_t bytes, rt::StreamHandle stream) {
  if (!defined()) return FailedPreconditionError("copy_from_host: undefined tensor");
  if (bytes > nbytes()) return InvalidArgumentError("copy_from_host: more bytes than the tensor holds");
  const int rc = mcke_rt_memcpy_async(data_ptr(), src, bytes, 0, stream);
  if (rc != MCKE_STATUS_OK) return Status(static_cast<StatusCode>(rc), mcke_last_error());
  // The source is pageable host memory the caller may release on return.
  const int rc2 = mcke_rt_stream_synchronize(stream);
  if (rc2 != MCKE_STATUS_OK) return Status(static_cast<StatusCode>(rc2), mcke_last_error());
  note_use(stream);
  return OkStatus();
}

Status Tensor::copy_to_host(void* dst, std::size_t bytes, rt::StreamHandle stream) const {
  if (!defined()) return FailedPreconditionError("copy_to_host: undefined tensor");
  if (bytes > nbytes()) return InvalidArgumentError("copy_to_host: more bytes than the tensor holds");
  const int rc = mcke_rt_memcpy_async(dst, data_ptr(), bytes, 1, stream);
  if (rc != MCKE_STATUS_OK) return Status(static_cast<StatusCode>(rc), mcke_last_error());
  note_use(stream);
  return OkStatus();
}

}  // namespace mcke
