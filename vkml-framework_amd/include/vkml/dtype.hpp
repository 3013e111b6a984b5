#pragma once

#include <cstddef>
#include <cstdint>
#include <string_view>

namespace vkml {

// Element types a tensor can hold (reference: include/vkml/dtype.hpp:12).
// F16 and BF16 host data are passed as raw bytes; kernels compute in f32.
enum class DType : std::uint8_t { F32, F16, BF16, I32 };

constexpr std::size_t element_size(DType dtype) noexcept {
    switch (dtype) {
        case DType::F16:
        case DType::BF16: return 2;
        case DType::F32:
        case DType::I32: break;
    }
    return 4;
}

std::string_view to_string(DType dtype) noexcept;

}  // namespace vkml
