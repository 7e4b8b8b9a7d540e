// mcke/core/dtype.hpp -- element types (reference include/mcke/core/dtype.hpp:33-95;
// same enumerator values).  Only kF32 reaches a kernel in this build.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string_view>

#include "mcke/core/config.hpp"

namespace mcke {

enum class DType : std::uint8_t { kF32 = 0, kF16, kBF16, kI32, kU8, kCount };

[[nodiscard]] MCKE_HOST_DEVICE constexpr std::size_t dtype_size(DType t) noexcept {
  switch (t) {
    case DType::kF32: return 4;
    case DType::kF16: return 2;
    case DType::kBF16: return 2;
    case DType::kI32: return 4;
    case DType::kU8: return 1;
    default: return 0;
  }
}

[[nodiscard]] constexpr std::string_view dtype_name(DType t) noexcept {
  switch (t) {
    case DType::kF32: return "f32";
    case DType::kF16: return "f16";
    case DType::kBF16: return "bf16";
    case DType::kI32: return "i32";
    case DType::kU8: return "u8";
    default: return "invalid";
  }
}

template <typename T> struct DTypeOf {};
template <> struct DTypeOf<float> { static constexpr DType value = DType::kF32; };
template <> struct DTypeOf<std::int32_t> { static constexpr DType value = DType::kI32; };
template <> struct DTypeOf<std::uint8_t> { static constexpr DType value = DType::kU8; };
template <typename T> inline constexpr DType kDTypeOf = DTypeOf<T>::value;

}  // namespace mcke
