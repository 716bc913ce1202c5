// The TurboQuant KV formats' launchers (kv_turbo.hip), for the C-ABI entry points of kv_quant.hip.
#pragma once

#include "common.h"

namespace xs_hip {

// Rows [rows, width] (width a multiple of 128) as codes [rows * width / 128, 16 * bits] bytes and f16 norms
// [rows * width / 128]; bits 4, 3 or 2.
int turbo_quantize(hipStream_t s, int bits, xs_dtype x_dtype, const void* x, void* codes, void* norms, int64_t rows,
                   int64_t width);
// The rotated values such codes and norms store, in out_dtype.
int turbo_dequantize(hipStream_t s, int bits, const void* codes, const void* norms, xs_dtype out_dtype, void* out,
                     int64_t rows, int64_t width);

}  // namespace xs_hip
