// Elementwise and broadcast entry points for gfx950: numpy-broadcast binary ops, the same-shape and row-vector fast
// paths, the fused residual forms and dtype conversion. The row-structured ones run the 2-D kernel of ew.h.
//
// The general broadcast kernel does numpy broadcasting over up to 6 dims with arbitrary strides (sycl_be::binary,
// sycl_kernels.cpp:88-102; cpu_ref::map_binary, src/backend/cpu_ref/ops.cpp:68-93), after the host has dropped
// size-1 dims and merged dims that are contiguous for all three operands; a unit of work is 8 consecutive elements of
// the innermost dim (128-bit accesses) when the strides allow, one element otherwise.
#include <algorithm>
#include <cmath>

#include "ew.h"

namespace xs_hip {
namespace {

using ew::Ew2D;
using ew::load8;
using ew::store8;

// ---------------------------------------------------------------------------------------------------------------
// General broadcast.

struct Bcast {
    int rank;
    int64_t out[XS_MAX_RANK];
    int64_t sa[XS_MAX_RANK], sb[XS_MAX_RANK], sy[XS_MAX_RANK];
};

// One unit is 8 (VEC) or 1 consecutive elements of the innermost dim; its multi-index is decoded dim by dim.
__device__ __forceinline__ float binary_apply(int op, float a, float b) {
    return op == ew::kAdd ? a + b : op == ew::kMul ? a * b : a / b;
}

template <typename TA, typename TB, typename TY, bool VEC>
__global__ __launch_bounds__(kBlock) void bcast_kernel(const void* __restrict__ pa, const void* __restrict__ pb,
                                                       void* __restrict__ py, Bcast d, int op, int64_t units) {
    using SA = typename TA::storage;
    using SB = typename TB::storage;
    using SY = typename TY::storage;
    const SA* a = static_cast<const SA*>(pa);
    const SB* b = static_cast<const SB*>(pb);
    SY* y = static_cast<SY*>(py);
    constexpr int E = VEC ? 8 : 1;
    const int last = d.rank - 1;
    const int64_t inner_units = d.out[last] / E;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t u = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; u < units; u += stride) {
        int64_t rest = u / inner_units;
        const int64_t i_last = (u - rest * inner_units) * E;
        int64_t oa = i_last * d.sa[last], ob = i_last * d.sb[last], oy = i_last * d.sy[last];
        for (int k = last - 1; k >= 0; --k) {
            const int64_t q = rest / d.out[k];
            const int64_t i = rest - q * d.out[k];
            rest = q;
            oa += i * d.sa[k];
            ob += i * d.sb[k];
            oy += i * d.sy[k];
        }
        if constexpr (VEC) {
            float fa[8], fb[8], out[8];
            if (d.sa[last] == 1) load8<TA>(a + oa, fa);
            else {
                const float v = TA::load(a[oa]);
#pragma unroll
                for (int i = 0; i < 8; ++i) fa[i] = v;
            }
            if (d.sb[last] == 1) load8<TB>(b + ob, fb);
            else {
                const float v = TB::load(b[ob]);
#pragma unroll
                for (int i = 0; i < 8; ++i) fb[i] = v;
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) out[i] = binary_apply(op, fa[i], fb[i]);
            store8<TY>(y + oy, out);
        } else {
            y[oy] = TY::store(binary_apply(op, TA::load(a[oa]), TB::load(b[ob])));
        }
    }
}

// Drops size-1 dims and merges a dim into the next inner one when all three operands are contiguous across them.
Bcast collapse(const xs_broadcast& in) {
    Bcast d{};
    d.rank = 0;
    for (int i = 0; i < in.rank; ++i) {
        if (in.out[i] == 1) continue;
        d.out[d.rank] = in.out[i];
        d.sa[d.rank] = in.stride_a[i];
        d.sb[d.rank] = in.stride_b[i];
        d.sy[d.rank] = in.stride_y[i];
        ++d.rank;
    }
    if (d.rank == 0) {
        d.rank = 1;
        d.out[0] = 1;
        d.sa[0] = d.sb[0] = d.sy[0] = 1;
        return d;
    }
    Bcast m{};
    m.rank = 1;
    m.out[0] = d.out[0];
    m.sa[0] = d.sa[0];
    m.sb[0] = d.sb[0];
    m.sy[0] = d.sy[0];
    for (int i = 1; i < d.rank; ++i) {
        const int j = m.rank - 1;  // outer dim j merges with inner dim i when stride_j == stride_i * out_i for all
        if (m.sa[j] == d.sa[i] * d.out[i] && m.sb[j] == d.sb[i] * d.out[i] && m.sy[j] == d.sy[i] * d.out[i]) {
            m.out[j] *= d.out[i];
            m.sa[j] = d.sa[i];
            m.sb[j] = d.sb[i];
            m.sy[j] = d.sy[i];
        } else {
            m.out[m.rank] = d.out[i];
            m.sa[m.rank] = d.sa[i];
            m.sb[m.rank] = d.sb[i];
            m.sy[m.rank] = d.sy[i];
            ++m.rank;
        }
    }
    return m;
}

template <typename TA, typename TB, typename TY>
int launch_bcast(hipStream_t s, const void* a, const void* b, void* y, const Bcast& d, int op, int64_t n) {
    const int last = d.rank - 1;
    bool vec = d.out[last] % 8 == 0 && d.sy[last] == 1 && (d.sa[last] == 0 || d.sa[last] == 1) &&
               (d.sb[last] == 0 || d.sb[last] == 1) && aligned16(y);
    if (vec && d.sa[last] == 1) vec = aligned16(a);
    if (vec && d.sb[last] == 1) vec = aligned16(b);
    for (int k = 0; vec && k < last; ++k)
        vec = (d.sa[k] % 8 == 0 || d.sa[last] == 0) && (d.sb[k] % 8 == 0 || d.sb[last] == 0) && d.sy[k] % 8 == 0;
    // A broadcast inner dim read as a scalar needs no alignment, but its outer strides still must keep 8 | index.
    if (vec) {
        const int64_t units = n / 8;
        bcast_kernel<TA, TB, TY, true><<<grid_for(units, kBlock * 4), kBlock, 0, s>>>(a, b, y, d, op, units);
    } else {
        bcast_kernel<TA, TB, TY, false><<<grid_for(n, kBlock * 4), kBlock, 0, s>>>(a, b, y, d, op, n);
    }
    return check_launch("xs_hip_binary");
}

template <typename TA, typename TB>
int bcast_y(hipStream_t s, const void* a, const void* b, void* y, const Bcast& d, int op, int64_t n, xs_dtype yt) {
    switch (yt) {
        case XS_F32: return launch_bcast<TA, TB, F32>(s, a, b, y, d, op, n);
        case XS_F16: return launch_bcast<TA, TB, F16>(s, a, b, y, d, op, n);
        case XS_BF16: return launch_bcast<TA, TB, BF16>(s, a, b, y, d, op, n);
        default: return fail(XS_HIP_EINVAL, std::string("xs_hip_binary: y must be f32, f16 or bf16, got ") + dtype_name(yt));
    }
}
template <typename TA>
int bcast_b(hipStream_t s, const void* a, const void* b, void* y, const Bcast& d, int op, int64_t n, xs_dtype bt,
            xs_dtype yt) {
    switch (bt) {
        case XS_F32: return bcast_y<TA, F32>(s, a, b, y, d, op, n, yt);
        case XS_F16: return bcast_y<TA, F16>(s, a, b, y, d, op, n, yt);
        case XS_BF16: return bcast_y<TA, BF16>(s, a, b, y, d, op, n, yt);
        default: return fail(XS_HIP_EINVAL, std::string("xs_hip_binary: b must be f32, f16 or bf16, got ") + dtype_name(bt));
    }
}

int binary_op_code(xs_binary_op op) {
    switch (op) {
        case XS_BINARY_ADD: return ew::kAdd;
        case XS_BINARY_MUL: return ew::kMul;
        case XS_BINARY_DIV: return ew::kDiv;
    }
    return -1;
}

// The 2-D kernel for a binary op code.
int dispatch_binary(hipStream_t s, const Ew2D& e, xs_dtype x_dtype, xs_dtype y_dtype, const char* what) {
    switch (e.op) {
        case ew::kAdd: return ew::dispatch<ew::kAdd, 0>(s, e, x_dtype, y_dtype, what);
        case ew::kMul: return ew::dispatch<ew::kMul, 0>(s, e, x_dtype, y_dtype, what);
        default: return ew::dispatch<ew::kDiv, 0>(s, e, x_dtype, y_dtype, what);
    }
}

std::string i2s(int64_t v) { return std::to_string(v); }

}  // namespace
}  // namespace xs_hip

using namespace xs_hip;

extern "C" {

int xs_hip_binary(void* stream, xs_binary_op op, xs_dtype a_dtype, const void* a, xs_dtype b_dtype, const void* b,
                  xs_dtype y_dtype, void* y, const xs_broadcast* bc) {
    const int code = binary_op_code(op);
    if (code < 0) return fail(XS_HIP_EINVAL, "xs_hip_binary: unknown op " + i2s(op));
    if (bc == nullptr || bc->rank < 0 || bc->rank > XS_MAX_RANK)
        return fail(XS_HIP_EINVAL, "xs_hip_binary: missing or bad broadcast descriptor");
    int64_t n = 1;
    for (int i = 0; i < bc->rank; ++i) {
        if (bc->out[i] < 0) return fail(XS_HIP_EINVAL, "xs_hip_binary: negative dim " + i2s(bc->out[i]));
        n *= bc->out[i];
    }
    if (n == 0) return XS_HIP_OK;
    if (a == nullptr || b == nullptr || y == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_binary: null buffer");
    const Bcast d = collapse(*bc);
    const hipStream_t s = as_stream(stream);
    // Contiguous same-shape and row-vector operands take the 2-D kernel.
    if (a_dtype == b_dtype && d.rank <= 2) {
        const int last = d.rank - 1;
        const bool inner_ok = d.sa[last] == 1 && d.sy[last] == 1 && (d.sb[last] == 1);
        if (inner_ok) {
            Ew2D e{a, b, nullptr, y, 0, 0, 0, 0, 1, d.out[last], code, 0};
            if (d.rank == 2) {
                e.rows = d.out[0];
                e.sa = d.sa[0];
                e.sb = d.sb[0];
                e.sy = d.sy[0];
            } else {
                e.sa = e.sb = e.sy = d.out[0];
            }
            return dispatch_binary(s, e, a_dtype, y_dtype, "xs_hip_binary");
        }
    }
    switch (a_dtype) {
        case XS_F32: return bcast_b<F32>(s, a, b, y, d, code, n, b_dtype, y_dtype);
        case XS_F16: return bcast_b<F16>(s, a, b, y, d, code, n, b_dtype, y_dtype);
        case XS_BF16: return bcast_b<BF16>(s, a, b, y, d, code, n, b_dtype, y_dtype);
        default: return fail(XS_HIP_EINVAL, std::string("xs_hip_binary: a must be f32, f16 or bf16, got ") + dtype_name(a_dtype));
    }
}

int xs_hip_binary_same(void* stream, xs_binary_op op, xs_dtype dtype, const void* a, const void* b, xs_dtype y_dtype,
                       void* y, int64_t n) {
    const int code = binary_op_code(op);
    if (code < 0) return fail(XS_HIP_EINVAL, "xs_hip_binary_same: unknown op " + i2s(op));
    if (n < 0) return fail(XS_HIP_EINVAL, "xs_hip_binary_same: n " + i2s(n));
    if (n == 0) return XS_HIP_OK;
    if (a == nullptr || b == nullptr || y == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_binary_same: null buffer");
    Ew2D e{a, b, nullptr, y, n, n, 0, n, 1, n, code, 0};
    return dispatch_binary(as_stream(stream), e, dtype, y_dtype, "xs_hip_binary_same");
}

int xs_hip_binary_period(void* stream, xs_binary_op op, xs_dtype dtype, const void* a, const void* b,
                         xs_dtype y_dtype, void* y, int64_t n, int64_t period) {
    const int code = binary_op_code(op);
    if (code < 0) return fail(XS_HIP_EINVAL, "xs_hip_binary_period: unknown op " + i2s(op));
    if (n < 0 || period <= 0 || n % period != 0)
        return fail(XS_HIP_EINVAL, "xs_hip_binary_period: n " + i2s(n) + " is not a multiple of period " + i2s(period));
    if (n == 0) return XS_HIP_OK;
    if (a == nullptr || b == nullptr || y == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_binary_period: null buffer");
    Ew2D e{a, b, nullptr, y, period, 0, 0, period, n / period, period, code, 0};
    return dispatch_binary(as_stream(stream), e, dtype, y_dtype, "xs_hip_binary_period");
}

int xs_hip_add_mul(void* stream, const float* a, const float* b, const float* c, xs_dtype y_dtype, void* y, int64_t n,
                   int64_t period) {
    if (n < 0 || period <= 0 || n % period != 0)
        return fail(XS_HIP_EINVAL, "xs_hip_add_mul: n " + i2s(n) + " is not a multiple of period " + i2s(period));
    if (n == 0) return XS_HIP_OK;
    if (a == nullptr || b == nullptr || c == nullptr || y == nullptr)
        return fail(XS_HIP_EINVAL, "xs_hip_add_mul: null buffer");
    Ew2D e{a, b, c, y, period, period, 0, period, n / period, period, ew::kAddMul, 0};
    return ew::dispatch<ew::kAddMul, 0>(as_stream(stream), e, XS_F32, y_dtype, "xs_hip_add_mul");
}

int xs_hip_add3(void* stream, const float* a, const float* b, const float* c, xs_dtype y_dtype, void* y, int64_t n,
                int64_t period) {
    if (n < 0 || period <= 0 || n % period != 0)
        return fail(XS_HIP_EINVAL, "xs_hip_add3: n " + i2s(n) + " is not a multiple of period " + i2s(period));
    if (n == 0) return XS_HIP_OK;
    if (a == nullptr || b == nullptr || c == nullptr || y == nullptr)
        return fail(XS_HIP_EINVAL, "xs_hip_add3: null buffer");
    Ew2D e{a, b, c, y, period, period, 0, period, n / period, period, ew::kAdd3, 0};
    return ew::dispatch<ew::kAdd3, 0>(as_stream(stream), e, XS_F32, y_dtype, "xs_hip_add3");
}

int xs_hip_convert(void* stream, xs_dtype x_dtype, const void* x, xs_dtype y_dtype, void* y, int64_t n) {
    if (n < 0) return fail(XS_HIP_EINVAL, "xs_hip_convert: n " + i2s(n));
    if (n == 0) return XS_HIP_OK;
    if (x == nullptr || y == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_convert: null buffer");
    Ew2D e{x, nullptr, nullptr, y, n, 0, 0, n, 1, n, ew::kCopy, 0};
    return ew::dispatch<ew::kCopy, 0>(as_stream(stream), e, x_dtype, y_dtype, "xs_hip_convert");
}

}  // extern "C"
