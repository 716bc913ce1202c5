#pragma once

// Element types (reference src/tensor/dtype.h:17, same enumerators in the same order; the numeric values are the
// C-ABI's xs_dtype for the first eight). The HIP backend handles the dense ones; the weight formats after Bool are
// named so that a graph holding them is refused by name.

#include <cstddef>
#include <cstdint>
#include <string_view>

namespace xs {

enum class DType : uint8_t { F32, F16, BF16, I64, I32, I8, U8, Bool, Q8, Q4, F8, Block, F4 };

size_t dtype_size(DType t);
std::string_view dtype_name(DType t);
bool is_float(DType t);  // f32, f16, bf16

}  // namespace xs
