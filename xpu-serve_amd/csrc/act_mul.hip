// The unary family (sycl_be::unary, src/backend/sycl/sycl_kernels.h:21-25; cpu-ref semantics ops.cpp:209-258) and the
// activation-times-gate entry points for gfx950: act_mul, unary_bias, and the biased gated-MLP activation over
// row-strided operands (the SwiGLU of a gated MLP: reference src/models/common/blocks.cpp:23-27, fused by the SYCL
// planner as unary_bias + act_mul, src/backend/sycl/sycl_backend.cpp:1004-1047). All run the 2-D kernel of ew.h.
#include "ew.h"

namespace xs_hip {
namespace {

using ew::Ew2D;

std::string i2s(int64_t v) { return std::to_string(v); }

bool act_ok(xs_unary_op act) {
    return act == XS_UNARY_SILU || act == XS_UNARY_SIGMOID || act == XS_UNARY_GELU_TANH || act == XS_UNARY_GELU;
}

}  // namespace
}  // namespace xs_hip

using namespace xs_hip;

extern "C" {

int xs_hip_unary(void* stream, xs_unary_op op, xs_dtype x_dtype, const void* x, xs_dtype y_dtype, void* y, int64_t n,
                 float a, float b) {
    if (static_cast<int>(op) < XS_UNARY_SCALE || static_cast<int>(op) > XS_UNARY_GELU)
        return fail(XS_HIP_EINVAL, "xs_hip_unary: unknown op " + i2s(op));
    if (n < 0) return fail(XS_HIP_EINVAL, "xs_hip_unary: n " + i2s(n));
    if (n == 0) return XS_HIP_OK;
    if (x == nullptr || y == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_unary: null buffer");
    if (op == XS_UNARY_SOFTCAP && !(a != 0.0f))
        return fail(XS_HIP_EINVAL, "xs_hip_unary: softcap " + std::to_string(a) + " must be nonzero");
    Ew2D e{x, nullptr, nullptr, y, n, 0, 0, n, 1, n, ew::kUnary, op};
    e.pa = a;
    e.pb = b;
    return ew::dispatch_unary(as_stream(stream), e, x_dtype, y_dtype, "xs_hip_unary");
}

int xs_hip_act_mul(void* stream, xs_unary_op act, xs_dtype x_dtype, const void* x, const void* b, xs_dtype y_dtype,
                   void* y, int64_t n) {
    if (!act_ok(act))
        return fail(XS_HIP_EINVAL, "xs_hip_act_mul: act must be silu, sigmoid, gelu_tanh or gelu, got " + i2s(act));
    if (n < 0) return fail(XS_HIP_EINVAL, "xs_hip_act_mul: n " + i2s(n));
    if (n == 0) return XS_HIP_OK;
    if (x == nullptr || b == nullptr || y == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_act_mul: null buffer");
    const Ew2D e{x, b, nullptr, y, n, n, 0, n, 1, n, ew::kActMul, act};
    return ew::dispatch_act<ew::kActMul>(as_stream(stream), e, x_dtype, y_dtype, "xs_hip_act_mul");
}

int xs_hip_unary_bias(void* stream, xs_unary_op act, const float* x, const float* bias, xs_dtype y_dtype, void* y,
                      int64_t n, int64_t period) {
    if (!act_ok(act))
        return fail(XS_HIP_EINVAL, "xs_hip_unary_bias: act must be silu, sigmoid, gelu_tanh or gelu, got " + i2s(act));
    if (n < 0 || period <= 0 || n % period != 0)
        return fail(XS_HIP_EINVAL, "xs_hip_unary_bias: n " + i2s(n) + " is not a multiple of period " + i2s(period));
    if (n == 0) return XS_HIP_OK;
    if (x == nullptr || bias == nullptr || y == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_unary_bias: null buffer");
    const Ew2D e{x, nullptr, bias, y, period, 0, 0, period, n / period, period, ew::kActBias, act};
    return ew::dispatch_act<ew::kActBias>(as_stream(stream), e, XS_F32, y_dtype, "xs_hip_unary_bias");
}

int xs_hip_act_bias_mul_2d(void* stream, xs_unary_op act, xs_dtype x_dtype, const void* x, int64_t x_row_stride,
                           const void* b, int64_t b_row_stride, const void* bias, xs_dtype y_dtype, void* y,
                           int64_t y_row_stride, int64_t rows, int64_t cols) {
    if (!act_ok(act))
        return fail(XS_HIP_EINVAL,
                    "xs_hip_act_bias_mul_2d: act must be silu, sigmoid, gelu_tanh or gelu, got " + i2s(act));
    if (rows < 0 || cols < 0)
        return fail(XS_HIP_EINVAL, "xs_hip_act_bias_mul_2d: shape [" + i2s(rows) + ", " + i2s(cols) + "]");
    if (rows == 0 || cols == 0) return XS_HIP_OK;
    if (x == nullptr || b == nullptr || y == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_act_bias_mul_2d: null buffer");
    if ((rows > 1 && (x_row_stride < cols || b_row_stride < cols || y_row_stride < cols)) || x_row_stride < 0 ||
        b_row_stride < 0 || y_row_stride < 0)
        return fail(XS_HIP_EINVAL, "xs_hip_act_bias_mul_2d: row strides " + i2s(x_row_stride) + ", " +
                                       i2s(b_row_stride) + ", " + i2s(y_row_stride) + " are shorter than a row of " +
                                       i2s(cols));
    const Ew2D e{x, b, bias, y, x_row_stride, b_row_stride, 0, y_row_stride, rows, cols,
                 bias != nullptr ? ew::kActBiasMul : ew::kActMul, act};
    if (bias != nullptr)
        return ew::dispatch_act<ew::kActBiasMul>(as_stream(stream), e, x_dtype, y_dtype, "xs_hip_act_bias_mul_2d");
    return ew::dispatch_act<ew::kActMul>(as_stream(stream), e, x_dtype, y_dtype, "xs_hip_act_bias_mul_2d");
}

}  // extern "C"
