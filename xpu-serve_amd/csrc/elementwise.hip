// Elementwise and broadcast kernels for gfx950.
//
// One 2-D kernel covers every row-structured elementwise op of the reference's device surface
// (src/backend/sycl/sycl_kernels.h:24-55): y[r, c] = f(a[r, c], b[r, c], bias[c]) with a row stride per operand, where
// a row stride of 0 repeats a row vector over the leading dims. That is binary_same (one row), binary_period (b's
// stride 0), act_mul, unary_bias, add_mul, add3, the biased gated-MLP activation on column slices of a fused
// gate|up buffer, and dtype conversion. Each lane handles chunks of 8 consecutive elements of a row (one or two
// 128-bit loads per operand, one or two 128-bit stores), keeps 4 chunks in flight, and the flat chunk index is split
// into (row, column) with a multiply-high division by the chunk count of a row.
//
// A second kernel does numpy broadcasting over up to 6 dims with arbitrary strides (sycl_be::binary,
// sycl_kernels.cpp:88-102; cpu_ref::map_binary, src/backend/cpu_ref/ops.cpp:68-93), after the host has dropped
// size-1 dims and merged dims that are contiguous for all three operands.
//
// Arithmetic: operands widened exactly to f32, each reference op rounded once in f32 in the reference's order; the
// build disables FMA contraction, so a + b * c is two roundings as in cpu-ref. SiLU and sigmoid are evaluated in f32
// (expf of the device math library) in a form that cannot overflow; the GELUs in f64 as cpu-ref does (ops.cpp:216-247).
#include <algorithm>
#include <cmath>

#include "common.h"

namespace xs_hip {
namespace {

enum EwOp : int { kCopy = 0, kAdd, kMul, kDiv, kActMul, kAddMul, kAdd3, kActBias, kActBiasMul };

struct FastDiv32 {
    uint32_t m = 1, s = 0;
    FastDiv32() = default;
    explicit FastDiv32(uint32_t d) {
        s = 0;
        while ((uint64_t{1} << s) < d) ++s;
        m = static_cast<uint32_t>(((uint64_t{1} << 32) * ((uint64_t{1} << s) - d)) / d + 1);
    }
    // floor(n / d) for n < 2^32 (Granlund-Montgomery).
    __device__ __forceinline__ uint32_t div(uint32_t n) const {
        return static_cast<uint32_t>((static_cast<uint64_t>(__umulhi(n, m)) + n) >> s);
    }
};

// Below this input the f32 exponential of the fast forms turns subnormal; those inputs take the reference's f64
// formula instead (a branch no N(0, 1) activation ever takes).
constexpr float kTinyExp = -80.0f;

// x * sigmoid(x) with the exponential of -|x| only, so nothing overflows: sigmoid(x) = 1 / (1 + e) for x >= 0 and
// e / (1 + e) for x < 0, e = exp(-|x|). cpu-ref: d / (1 + exp(-d)) in f64 (ops.cpp:242-247).
__device__ __forceinline__ float silu_f(float x) {
    if (x < kTinyExp) {
        const double d = x;
        return static_cast<float>(d / (1.0 + exp(-d)));
    }
    const float e = expf(-fabsf(x));
    const float s = x >= 0.0f ? 1.0f / (1.0f + e) : e / (1.0f + e);
    return x * s;
}
// cpu-ref: 1 / (1 + exp(-d)) in f64 (ops.cpp:237-239).
__device__ __forceinline__ float sigmoid_f(float x) {
    if (x < kTinyExp) return static_cast<float>(1.0 / (1.0 + exp(-static_cast<double>(x))));
    const float e = expf(-fabsf(x));
    return x >= 0.0f ? 1.0f / (1.0f + e) : e / (1.0f + e);
}
// The two GELUs are evaluated as cpu-ref writes them, in f64 (ops.cpp:220-233): their 1 + tanh / 1 + erf cancel for
// negative x, and cpu-ref's result there is that cancellation's (0 once tanh rounds to -1), which a cancellation-free
// form would not reproduce.
__device__ __forceinline__ float gelu_tanh_f(float x) {
    const double d = x;
    const double inner = sqrt(2.0 / 3.14159265358979323846) * (d + 0.044715 * d * d * d);
    return static_cast<float>(0.5 * d * (1.0 + tanh(inner)));
}
__device__ __forceinline__ float gelu_f(float x) {
    const double d = x;
    return static_cast<float>(0.5 * d * (1.0 + erf(d / 1.41421356237309504880)));
}

__device__ __forceinline__ float act_fn(int act, float x) {
    switch (act) {
        case XS_UNARY_SILU: return silu_f(x);
        case XS_UNARY_SIGMOID: return sigmoid_f(x);
        case XS_UNARY_GELU_TANH: return gelu_tanh_f(x);
        default: return gelu_f(x);
    }
}

__device__ __forceinline__ float ew_apply(int op, int act, float a, float b, float c) {
    switch (op) {
        case kCopy: return a;
        case kAdd: return a + b;
        case kMul: return a * b;
        case kDiv: return a / b;
        case kActMul: return act_fn(act, a) * b;
        case kAddMul: return a + b * c;
        case kAdd3: return a + (b + c);
        case kActBias: return act_fn(act, a + c);
        default: return act_fn(act, a + c) * b;  // kActBiasMul
    }
}

constexpr bool op_reads_b(int op) { return op != kCopy && op != kActBias; }
constexpr bool op_reads_c(int op) { return op == kAddMul || op == kAdd3 || op == kActBias || op == kActBiasMul; }

struct Ew2D {
    const void* a;
    const void* b;
    const void* c;
    void* y;
    int64_t sa, sb, sc, sy;  // row strides in elements (0: the row repeats)
    int64_t rows, cols;
    int op, act;
};

// 8 elements of T from p (two 128-bit loads for f32, one for 16-bit types).
template <typename T>
__device__ __forceinline__ void load8(const typename T::storage* p, float* f) {
    if constexpr (sizeof(typename T::storage) == 4) {
        unpack<T>(ld128(p), f);
        unpack<T>(ld128(p + 4), f + 4);
    } else {
        unpack<T>(ld128(p), f);
    }
}
template <typename T>
__device__ __forceinline__ void store8(typename T::storage* p, const float* f) {
    if constexpr (sizeof(typename T::storage) == 4) {
        st128(p, pack<T>(f));
        st128(p + 4, pack<T>(f + 4));
    } else {
        st128(p, pack<T>(f));
    }
}

// Vector path: cols % 8 == 0, every pointer 16-byte aligned, every nonzero row stride a multiple of 8.
template <typename TX, typename TC, typename TY, int U>
__global__ __launch_bounds__(kBlock) void ew2d_vec(Ew2D e, uint32_t units, FastDiv32 chunks_per_row,
                                                   uint32_t cpr) {
    using SX = typename TX::storage;
    using SC = typename TC::storage;
    using SY = typename TY::storage;
    const SX* a = static_cast<const SX*>(e.a);
    const SX* b = static_cast<const SX*>(e.b);
    const SC* c = static_cast<const SC*>(e.c);
    SY* y = static_cast<SY*>(e.y);
    const bool rb = op_reads_b(e.op), rc = op_reads_c(e.op);
    const uint32_t stride = gridDim.x * kBlock;
    for (uint32_t u0 = blockIdx.x * kBlock + threadIdx.x; u0 < units; u0 += U * stride) {
        float fa[U][8], fb[U][8], fc[U][8];
        int64_t row[U], col[U];
#pragma unroll
        for (int k = 0; k < U; ++k) {
            const uint32_t u = u0 + k * stride;
            if (u < units) {
                const uint32_t r = chunks_per_row.div(u);
                row[k] = r;
                col[k] = static_cast<int64_t>(u - r * cpr) * 8;
                load8<TX>(a + row[k] * e.sa + col[k], fa[k]);
                if (rb) load8<TX>(b + row[k] * e.sb + col[k], fb[k]);
                if (rc) load8<TC>(c + row[k] * e.sc + col[k], fc[k]);
            }
        }
#pragma unroll
        for (int k = 0; k < U; ++k) {
            const uint32_t u = u0 + k * stride;
            if (u < units) {
                float out[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) out[i] = ew_apply(e.op, e.act, fa[k][i], rb ? fb[k][i] : 0.0f, rc ? fc[k][i] : 0.0f);
                store8<TY>(y + row[k] * e.sy + col[k], out);
            }
        }
    }
}

// Scalar path: any shape, alignment and stride.
template <typename TX, typename TC, typename TY>
__global__ __launch_bounds__(kBlock) void ew2d_any(Ew2D e) {
    using SX = typename TX::storage;
    using SC = typename TC::storage;
    using SY = typename TY::storage;
    const SX* a = static_cast<const SX*>(e.a);
    const SX* b = static_cast<const SX*>(e.b);
    const SC* c = static_cast<const SC*>(e.c);
    SY* y = static_cast<SY*>(e.y);
    const bool rb = op_reads_b(e.op), rc = op_reads_c(e.op);
    const int64_t n = e.rows * e.cols;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
        const int64_t r = i / e.cols, col = i - r * e.cols;
        const float fa = TX::load(a[r * e.sa + col]);
        const float fb = rb ? TX::load(b[r * e.sb + col]) : 0.0f;
        const float fc = rc ? TC::load(c[r * e.sc + col]) : 0.0f;
        y[r * e.sy + col] = TY::store(ew_apply(e.op, e.act, fa, fb, fc));
    }
}

template <typename TX, typename TC, typename TY>
int launch_ew2d(hipStream_t s, const Ew2D& e, const char* what) {
    if (e.rows == 0 || e.cols == 0) return XS_HIP_OK;
    const bool rb = op_reads_b(e.op), rc = op_reads_c(e.op);
    bool vec = e.cols % 8 == 0 && aligned16(e.a) && aligned16(e.y) && (!rb || aligned16(e.b)) &&
               (!rc || aligned16(e.c)) && e.sa % 8 == 0 && e.sy % 8 == 0 && (!rb || e.sb % 8 == 0) &&
               (!rc || e.sc % 8 == 0);
    const int64_t cpr = e.cols / 8;
    const int64_t units = e.rows * cpr;
    if (vec && units < (int64_t{1} << 31)) {
        constexpr int U = 4;
        const unsigned grid = grid_for(units, kBlock * U);
        ew2d_vec<TX, TC, TY, U><<<grid, kBlock, 0, s>>>(e, static_cast<uint32_t>(units),
                                                         FastDiv32(static_cast<uint32_t>(cpr)),
                                                         static_cast<uint32_t>(cpr));
    } else {
        ew2d_any<TX, TC, TY><<<grid_for(e.rows * e.cols, kBlock * 4), kBlock, 0, s>>>(e);
    }
    return check_launch(what);
}

template <typename TX, typename TC>
int dispatch_y(hipStream_t s, const Ew2D& e, xs_dtype y_dtype, const char* what) {
    switch (y_dtype) {
        case XS_F32: return launch_ew2d<TX, TC, F32>(s, e, what);
        case XS_F16: return launch_ew2d<TX, TC, F16>(s, e, what);
        case XS_BF16: return launch_ew2d<TX, TC, BF16>(s, e, what);
        default: return fail(XS_HIP_EINVAL, std::string(what) + ": y must be f32, f16 or bf16, got " + dtype_name(y_dtype));
    }
}

// x, b and c share x_dtype.
int dispatch_ew(hipStream_t s, const Ew2D& e, xs_dtype x_dtype, xs_dtype y_dtype, const char* what) {
    switch (x_dtype) {
        case XS_F32: return dispatch_y<F32, F32>(s, e, y_dtype, what);
        case XS_F16: return dispatch_y<F16, F16>(s, e, y_dtype, what);
        case XS_BF16: return dispatch_y<BF16, BF16>(s, e, y_dtype, what);
        default: return fail(XS_HIP_EINVAL, std::string(what) + ": operands must be f32, f16 or bf16, got " + dtype_name(x_dtype));
    }
}

// ---------------------------------------------------------------------------------------------------------------
// General broadcast.

struct Bcast {
    int rank;
    int64_t out[XS_MAX_RANK];
    int64_t sa[XS_MAX_RANK], sb[XS_MAX_RANK], sy[XS_MAX_RANK];
};

// One unit is 8 (VEC) or 1 consecutive elements of the innermost dim; its multi-index is decoded dim by dim.
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
            for (int i = 0; i < 8; ++i) out[i] = ew_apply(op, 0, fa[i], fb[i], 0.0f);
            store8<TY>(y + oy, out);
        } else {
            y[oy] = TY::store(ew_apply(op, 0, TA::load(a[oa]), TB::load(b[ob]), 0.0f));
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
        case XS_BINARY_ADD: return kAdd;
        case XS_BINARY_MUL: return kMul;
        case XS_BINARY_DIV: return kDiv;
    }
    return -1;
}

bool act_ok(xs_unary_op act) {
    return act == XS_UNARY_SILU || act == XS_UNARY_SIGMOID || act == XS_UNARY_GELU_TANH || act == XS_UNARY_GELU;
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
            return dispatch_ew(s, e, a_dtype, y_dtype, "xs_hip_binary");
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
    return dispatch_ew(as_stream(stream), e, dtype, y_dtype, "xs_hip_binary_same");
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
    return dispatch_ew(as_stream(stream), e, dtype, y_dtype, "xs_hip_binary_period");
}

int xs_hip_add_mul(void* stream, const float* a, const float* b, const float* c, xs_dtype y_dtype, void* y, int64_t n,
                   int64_t period) {
    if (n < 0 || period <= 0 || n % period != 0)
        return fail(XS_HIP_EINVAL, "xs_hip_add_mul: n " + i2s(n) + " is not a multiple of period " + i2s(period));
    if (n == 0) return XS_HIP_OK;
    if (a == nullptr || b == nullptr || c == nullptr || y == nullptr)
        return fail(XS_HIP_EINVAL, "xs_hip_add_mul: null buffer");
    Ew2D e{a, b, c, y, period, period, 0, period, n / period, period, kAddMul, 0};
    return dispatch_ew(as_stream(stream), e, XS_F32, y_dtype, "xs_hip_add_mul");
}

int xs_hip_add3(void* stream, const float* a, const float* b, const float* c, xs_dtype y_dtype, void* y, int64_t n,
                int64_t period) {
    if (n < 0 || period <= 0 || n % period != 0)
        return fail(XS_HIP_EINVAL, "xs_hip_add3: n " + i2s(n) + " is not a multiple of period " + i2s(period));
    if (n == 0) return XS_HIP_OK;
    if (a == nullptr || b == nullptr || c == nullptr || y == nullptr)
        return fail(XS_HIP_EINVAL, "xs_hip_add3: null buffer");
    Ew2D e{a, b, c, y, period, period, 0, period, n / period, period, kAdd3, 0};
    return dispatch_ew(as_stream(stream), e, XS_F32, y_dtype, "xs_hip_add3");
}

int xs_hip_act_mul(void* stream, xs_unary_op act, xs_dtype x_dtype, const void* x, const void* b, xs_dtype y_dtype,
                   void* y, int64_t n) {
    if (!act_ok(act)) return fail(XS_HIP_EINVAL, "xs_hip_act_mul: act must be silu, sigmoid, gelu_tanh or gelu, got " + i2s(act));
    if (n < 0) return fail(XS_HIP_EINVAL, "xs_hip_act_mul: n " + i2s(n));
    if (n == 0) return XS_HIP_OK;
    if (x == nullptr || b == nullptr || y == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_act_mul: null buffer");
    Ew2D e{x, b, nullptr, y, n, n, 0, n, 1, n, kActMul, act};
    return dispatch_ew(as_stream(stream), e, x_dtype, y_dtype, "xs_hip_act_mul");
}

int xs_hip_unary_bias(void* stream, xs_unary_op act, const float* x, const float* bias, xs_dtype y_dtype, void* y,
                      int64_t n, int64_t period) {
    if (!act_ok(act)) return fail(XS_HIP_EINVAL, "xs_hip_unary_bias: act must be silu, sigmoid, gelu_tanh or gelu, got " + i2s(act));
    if (n < 0 || period <= 0 || n % period != 0)
        return fail(XS_HIP_EINVAL, "xs_hip_unary_bias: n " + i2s(n) + " is not a multiple of period " + i2s(period));
    if (n == 0) return XS_HIP_OK;
    if (x == nullptr || bias == nullptr || y == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_unary_bias: null buffer");
    Ew2D e{x, nullptr, bias, y, period, 0, 0, period, n / period, period, kActBias, act};
    return dispatch_ew(as_stream(stream), e, XS_F32, y_dtype, "xs_hip_unary_bias");
}

int xs_hip_act_bias_mul_2d(void* stream, xs_unary_op act, xs_dtype x_dtype, const void* x, int64_t x_row_stride,
                           const void* b, int64_t b_row_stride, const void* bias, xs_dtype y_dtype, void* y,
                           int64_t y_row_stride, int64_t rows, int64_t cols) {
    if (!act_ok(act)) return fail(XS_HIP_EINVAL, "xs_hip_act_bias_mul_2d: act must be silu, sigmoid, gelu_tanh or gelu, got " + i2s(act));
    if (rows < 0 || cols < 0) return fail(XS_HIP_EINVAL, "xs_hip_act_bias_mul_2d: shape [" + i2s(rows) + ", " + i2s(cols) + "]");
    if (rows == 0 || cols == 0) return XS_HIP_OK;
    if (x == nullptr || b == nullptr || y == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_act_bias_mul_2d: null buffer");
    if ((rows > 1 && (x_row_stride < cols || b_row_stride < cols || y_row_stride < cols)) ||
        x_row_stride < 0 || b_row_stride < 0 || y_row_stride < 0)
        return fail(XS_HIP_EINVAL, "xs_hip_act_bias_mul_2d: row strides " + i2s(x_row_stride) + ", " + i2s(b_row_stride) +
                                       ", " + i2s(y_row_stride) + " are shorter than a row of " + i2s(cols));
    Ew2D e{x, b, bias, y, x_row_stride, b_row_stride, 0, y_row_stride, rows, cols,
           bias != nullptr ? kActBiasMul : kActMul, act};
    return dispatch_ew(as_stream(stream), e, x_dtype, y_dtype, "xs_hip_act_bias_mul_2d");
}

int xs_hip_convert(void* stream, xs_dtype x_dtype, const void* x, xs_dtype y_dtype, void* y, int64_t n) {
    if (n < 0) return fail(XS_HIP_EINVAL, "xs_hip_convert: n " + i2s(n));
    if (n == 0) return XS_HIP_OK;
    if (x == nullptr || y == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_convert: null buffer");
    Ew2D e{x, nullptr, nullptr, y, n, 0, 0, n, 1, n, kCopy, 0};
    return dispatch_ew(as_stream(stream), e, x_dtype, y_dtype, "xs_hip_convert");
}

}  // extern "C"
