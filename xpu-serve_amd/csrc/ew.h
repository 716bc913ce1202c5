// The row-structured elementwise kernel shared by the binary, residual, activation and conversion entry points.
//
// y[r, c] = f(a[r, c], b[r, c], bias[c]) for r < rows, c < cols, with a row stride per operand (a row stride of 0
// repeats a row vector over the leading dims). f is a compile-time op (and activation), so the per-element code holds
// nothing but the arithmetic. Each lane handles chunks of 8 consecutive elements of a row -- one or two 128-bit loads
// per operand, one or two 128-bit stores -- and keeps U chunks in flight. A workgroup takes one contiguous tile of
// kBlock * U chunks (lane t its chunks t, t + kBlock, ...) and the grid covers the whole tensor, so the workgroups in
// flight at any moment read one contiguous window of memory, which HBM serves faster than the scattered windows of a
// grid-stride loop. The flat chunk index is split into (row, column) with a multiply-high division by the chunk count
// of a row.
//
// Arithmetic: operands widened exactly to f32, each reference op rounded once in f32 in the reference's order; the
// build disables FMA contraction, so a + b * c rounds twice as in cpu-ref. SiLU and sigmoid take a fast f32 form
// (v_exp_f32, v_rcp_f32: a few units in the last f32 place, well inside the parity bar) unless some input of the chunk
// lies below kTinyExp, where the chunk takes cpu-ref's f64 formula; the GELUs always take cpu-ref's f64 formula, whose
// 1 + tanh / 1 + erf cancellation for negative x a cancellation-free form would not reproduce (ops.cpp:216-247).
#pragma once

#include "common.h"

namespace xs_hip {
namespace ew {

enum Op : int { kCopy = 0, kAdd, kMul, kDiv, kActMul, kAddMul, kAdd3, kActBias, kActBiasMul, kUnary };

constexpr bool reads_b(int op) { return op != kCopy && op != kActBias && op != kUnary; }
constexpr bool reads_c(int op) { return op == kAddMul || op == kAdd3 || op == kActBias || op == kActBiasMul; }
constexpr bool has_act(int op) { return op == kActMul || op == kActBias || op == kActBiasMul || op == kUnary; }

// Below this input the fast forms' exponential leaves the normal f32 range; a chunk holding one takes the f64 path.
constexpr float kTinyExp = -80.0f;
constexpr float kLog2e = 1.4426950408889634f;

// cpu-ref's activations in f64, rounded once (ops.cpp:216-247).
template <int ACT>
__device__ __forceinline__ float act_exact(float x) {
    const double d = x;
    if constexpr (ACT == XS_UNARY_SILU) {
        return static_cast<float>(d / (1.0 + exp(-d)));
    } else if constexpr (ACT == XS_UNARY_SIGMOID) {
        return static_cast<float>(1.0 / (1.0 + exp(-d)));
    } else if constexpr (ACT == XS_UNARY_GELU_TANH) {
        const double inner = sqrt(2.0 / 3.14159265358979323846) * (d + 0.044715 * d * d * d);
        return static_cast<float>(0.5 * d * (1.0 + tanh(inner)));
    } else {
        return static_cast<float>(0.5 * d * (1.0 + erf(d / 1.41421356237309504880)));
    }
}

// An empty register barrier: hides the value's origin from the optimizer. Used on unary results before they are
// narrowed, where the compiler would otherwise fold the narrowing of a libm copysign into a bf16 copysign that it
// cannot select on gfx950.
__device__ __forceinline__ float opaque(float v) {
    asm volatile("" : "+v"(v));
    return v;
}

// Every op of the unary family as cpu-ref evaluates it (ops.cpp:209-258), `pa` / `pb` the op's parameters (the scale
// factor, the softcap, the clamp bounds). Scale and Clamp are the reference's f32 arithmetic exactly (Clamp is
// std::min(std::max(v, lo), hi), which keeps a NaN v). Tanh, Softcap and Softplus, which cpu-ref evaluates in f64 and
// rounds once, are evaluated with the device's f32 tanhf / log1pf / expf (a few units in the last f32 place, no
// cancellation: within the parity bar of every output dtype) -- f64 transcendentals would make these memory-bound ops
// VALU-bound. The GELUs keep the f64 formula (their 1 + tanh cancellation needs it).
template <int ACT>
__device__ __forceinline__ float unary_exact(float x, float pa, float pb) {
    if constexpr (ACT == XS_UNARY_SCALE) {
        return x * pa;
    } else if constexpr (ACT == XS_UNARY_TANH) {
        return tanhf(x);
    } else if constexpr (ACT == XS_UNARY_SOFTCAP) {
        return pa * tanhf(x / pa);
    } else if constexpr (ACT == XS_UNARY_SOFTPLUS) {
        return x > 20.0f ? x : log1pf(expf(x));
    } else if constexpr (ACT == XS_UNARY_CLAMP) {
        const float lo = x < pa ? pa : x;
        return pb < lo ? pb : lo;
    } else {
        return act_exact<ACT>(x);
    }
}

// x >= kTinyExp: x / (1 + 2^(-x log2 e)) and 1 / (1 + 2^(-x log2 e)). For an f32 output (`exact_arg`) the rounding
// error of -x log2 e is carried into the exponential (2^(t + dt) = 2^t (1 + dt ln 2)), otherwise |t| <= 116 costs at
// most 7e-6 of relative error, far below half a bf16 / f16 unit.
template <int ACT, bool EXACT_ARG>
__device__ __forceinline__ float act_fast(float x) {
    const float t = -x * kLog2e;
    float e = __builtin_amdgcn_exp2f(t);
    if constexpr (EXACT_ARG) {
        const float dt = fmaf(-x, kLog2e, -t) + (-x) * 1.925963001e-8f;  // log2(e) - kLog2e
        e = fmaf(e, dt * 0.6931471805599453f, e);
    }
    const float r = __builtin_amdgcn_rcpf(1.0f + e);
    if constexpr (ACT == XS_UNARY_SILU) return x * r;
    else return r;
}

constexpr bool act_fast_ok(int act) { return act == XS_UNARY_SILU || act == XS_UNARY_SIGMOID; }

// The pre-activation value of op OP (or the final value for ops without activation).
template <int OP>
__device__ __forceinline__ float pre(float a, float b, float c) {
    if constexpr (OP == kCopy) return a;
    else if constexpr (OP == kAdd) return a + b;
    else if constexpr (OP == kMul) return a * b;
    else if constexpr (OP == kDiv) return a / b;
    else if constexpr (OP == kActMul || OP == kUnary) return a;
    else if constexpr (OP == kAddMul) return a + b * c;
    else if constexpr (OP == kAdd3) return a + (b + c);
    else return a + c;  // kActBias, kActBiasMul
}

// Applies op OP with activation ACT to 8 elements (pre-activation values in v, gate values in b).
template <int OP, int ACT, bool EXACT_ARG>
__device__ __forceinline__ void finish8(float* v, const float* b, float pa, float pb) {
    if constexpr (has_act(OP)) {
        bool slow = !act_fast_ok(ACT);
        if constexpr (act_fast_ok(ACT)) {
            const float m = fminf(fminf(fminf(v[0], v[1]), fminf(v[2], v[3])),
                                  fminf(fminf(v[4], v[5]), fminf(v[6], v[7])));
            slow = !(m >= kTinyExp);  // NaN inputs too: the exact path keeps cpu-ref's NaN
        }
        if (slow) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                v[i] = unary_exact<ACT>(v[i], pa, pb);
                if constexpr (OP == kUnary) v[i] = opaque(v[i]);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = act_fast<ACT, EXACT_ARG>(v[i]);
        }
        if constexpr (OP == kActMul || OP == kActBiasMul) {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = v[i] * b[i];
        }
    }
}

struct Ew2D {
    const void* a;
    const void* b;
    const void* c;
    void* y;
    int64_t sa, sb, sc, sy;  // row strides in elements (0: the row repeats)
    int64_t rows, cols;
    int op, act;
    float pa = 0.0f, pb = 0.0f;  // kUnary's parameters
};

// 8 elements of T at p (two 128-bit loads for f32, one for 16-bit types); NT marks streaming data read once.
template <typename T, bool NT = false>
__device__ __forceinline__ void load8(const typename T::storage* p, float* f) {
    if constexpr (sizeof(typename T::storage) == 4) {
        unpack<T>(NT ? ld128_nt(p) : ld128(p), f);
        unpack<T>(NT ? ld128_nt(p + 4) : ld128(p + 4), f + 4);
    } else {
        unpack<T>(NT ? ld128_nt(p) : ld128(p), f);
    }
}
template <typename T, bool NT = false>
__device__ __forceinline__ void store8(typename T::storage* p, const float* f) {
    if constexpr (sizeof(typename T::storage) == 4) {
        if constexpr (NT) {
            st128_nt(p, pack<T>(f));
            st128_nt(p + 4, pack<T>(f + 4));
        } else {
            st128(p, pack<T>(f));
            st128(p + 4, pack<T>(f + 4));
        }
    } else {
        if constexpr (NT) st128_nt(p, pack<T>(f));
        else st128(p, pack<T>(f));
    }
}

// Threads of a vector-path workgroup.
constexpr int kVecBlock = 64;

// Vector path: cols % 8 == 0, every pointer 16-byte aligned, every nonzero row stride a multiple of 8.
template <typename TX, typename TY, int OP, int ACT, int U>
__global__ __launch_bounds__(kVecBlock) void ew2d_vec(Ew2D e, uint32_t units, FastDiv32 chunks_per_row, uint32_t cpr) {
    using SX = typename TX::storage;
    using SY = typename TY::storage;
    constexpr bool RB = reads_b(OP), RC = reads_c(OP);
    constexpr bool EXACT_ARG = sizeof(SY) == 4;
    const SX* a = static_cast<const SX*>(e.a);
    const SX* b = static_cast<const SX*>(e.b);
    const SX* c = static_cast<const SX*>(e.c);
    SY* y = static_cast<SY*>(e.y);
    constexpr uint32_t stride = kVecBlock;
    {
        const uint32_t u0 = blockIdx.x * (kVecBlock * U) + threadIdx.x;
        float fa[U][8], fb[U][8], fc[U][8];
        int64_t row[U], col[U];
#pragma unroll
        for (int k = 0; k < U; ++k) {
            const uint32_t u = u0 + k * stride;
            if (u < units) {
                const uint32_t r = chunks_per_row.div(u);
                row[k] = r;
                col[k] = static_cast<int64_t>(u - r * cpr) * 8;
                // a and b stream through once (their rows do not repeat in the common case); bias rows repeat.
                load8<TX, true>(a + row[k] * e.sa + col[k], fa[k]);
                if constexpr (RB) load8<TX, true>(b + row[k] * e.sb + col[k], fb[k]);
                if constexpr (RC) load8<TX>(c + row[k] * e.sc + col[k], fc[k]);
            }
        }
#pragma unroll
        for (int k = 0; k < U; ++k) {
            const uint32_t u = u0 + k * stride;
            if (u < units) {
                float v[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = pre<OP>(fa[k][i], RB ? fb[k][i] : 0.0f, RC ? fc[k][i] : 0.0f);
                finish8<OP, ACT, EXACT_ARG>(v, fb[k], e.pa, e.pb);
                store8<TY, true>(y + row[k] * e.sy + col[k], v);
            }
        }
    }
}

// Scalar path: any shape, alignment and stride.
template <typename TX, typename TY, int OP, int ACT>
__global__ __launch_bounds__(kBlock) void ew2d_any(Ew2D e) {
    using SX = typename TX::storage;
    using SY = typename TY::storage;
    constexpr bool RB = reads_b(OP), RC = reads_c(OP);
    const SX* a = static_cast<const SX*>(e.a);
    const SX* b = static_cast<const SX*>(e.b);
    const SX* c = static_cast<const SX*>(e.c);
    SY* y = static_cast<SY*>(e.y);
    const int64_t n = e.rows * e.cols;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
        const int64_t r = i / e.cols, col = i - r * e.cols;
        const float fa = TX::load(a[r * e.sa + col]);
        const float fb = RB ? TX::load(b[r * e.sb + col]) : 0.0f;
        const float fc = RC ? TX::load(c[r * e.sc + col]) : 0.0f;
        float v = pre<OP>(fa, fb, fc);
        if constexpr (has_act(OP)) {
            v = unary_exact<ACT>(v, e.pa, e.pb);
            if constexpr (OP == kUnary) v = opaque(v);
            if constexpr (OP == kActMul || OP == kActBiasMul) v = v * fb;
        }
        y[r * e.sy + col] = TY::store(v);
    }
}

template <typename TX, typename TY, int OP, int ACT>
int launch(hipStream_t s, const Ew2D& e, const char* what) {
    if (e.rows == 0 || e.cols == 0) return XS_HIP_OK;
    constexpr bool RB = reads_b(OP), RC = reads_c(OP);
    const bool vec = e.cols % 8 == 0 && aligned16(e.a) && aligned16(e.y) && (!RB || aligned16(e.b)) &&
                     (!RC || aligned16(e.c)) && e.sa % 8 == 0 && e.sy % 8 == 0 && (!RB || e.sb % 8 == 0) &&
                     (!RC || e.sc % 8 == 0);
    // A single row (a flat tensor) whose length is no multiple of 8: the vector kernel takes all whole chunks and the
    // scalar one the last cols % 8 elements.
    if (!vec && e.rows == 1 && e.cols > 8 && e.cols % 8 != 0) {
        Ew2D head = e;
        head.cols = e.cols / 8 * 8;
        const bool head_vec = aligned16(e.a) && aligned16(e.y) && (!RB || aligned16(e.b)) && (!RC || aligned16(e.c));
        if (head_vec) {
            Ew2D tail = e;
            const int64_t skip = head.cols;
            tail.cols = e.cols - skip;
            tail.a = static_cast<const typename TX::storage*>(e.a) + skip;
            if (RB) tail.b = static_cast<const typename TX::storage*>(e.b) + skip;
            if (RC) tail.c = static_cast<const typename TX::storage*>(e.c) + skip;
            tail.y = static_cast<typename TY::storage*>(e.y) + skip;
            const int rc = launch<TX, TY, OP, ACT>(s, head, what);
            if (rc != XS_HIP_OK) return rc;
            ew2d_any<TX, TY, OP, ACT><<<1, kBlock, 0, s>>>(tail);
            return check_launch(what);
        }
    }
    const int64_t cpr = e.cols / 8;
    const int64_t units = e.rows * cpr;
    if (vec && units < (int64_t{1} << 31)) {
        constexpr int U = 1;
        const unsigned grid = static_cast<unsigned>((units + kVecBlock * U - 1) / (kVecBlock * U));
        ew2d_vec<TX, TY, OP, ACT, U><<<grid, kVecBlock, 0, s>>>(e, static_cast<uint32_t>(units),
                                                            FastDiv32(static_cast<uint32_t>(cpr)),
                                                            static_cast<uint32_t>(cpr));
    } else {
        ew2d_any<TX, TY, OP, ACT><<<grid_for(e.rows * e.cols, kBlock * 4), kBlock, 0, s>>>(e);
    }
    return check_launch(what);
}

template <int OP, int ACT, typename TX>
int dispatch_y(hipStream_t s, const Ew2D& e, xs_dtype y_dtype, const char* what) {
    switch (y_dtype) {
        case XS_F32: return launch<TX, F32, OP, ACT>(s, e, what);
        case XS_F16: return launch<TX, F16, OP, ACT>(s, e, what);
        case XS_BF16: return launch<TX, BF16, OP, ACT>(s, e, what);
        default:
            return fail(XS_HIP_EINVAL, std::string(what) + ": y must be f32, f16 or bf16, got " + dtype_name(y_dtype));
    }
}

// x, b and c share x_dtype.
template <int OP, int ACT>
int dispatch(hipStream_t s, const Ew2D& e, xs_dtype x_dtype, xs_dtype y_dtype, const char* what) {
    switch (x_dtype) {
        case XS_F32: return dispatch_y<OP, ACT, F32>(s, e, y_dtype, what);
        case XS_F16: return dispatch_y<OP, ACT, F16>(s, e, y_dtype, what);
        case XS_BF16: return dispatch_y<OP, ACT, BF16>(s, e, y_dtype, what);
        default:
            return fail(XS_HIP_EINVAL, std::string(what) + ": operands must be f32, f16 or bf16, got " +
                                           dtype_name(x_dtype));
    }
}

// The unary family (kUnary) with a run-time op: one template instance per op.
inline int dispatch_unary(hipStream_t s, const Ew2D& e, xs_dtype x_dtype, xs_dtype y_dtype, const char* what) {
    switch (e.act) {
        case XS_UNARY_SCALE: return dispatch<kUnary, XS_UNARY_SCALE>(s, e, x_dtype, y_dtype, what);
        case XS_UNARY_TANH: return dispatch<kUnary, XS_UNARY_TANH>(s, e, x_dtype, y_dtype, what);
        case XS_UNARY_GELU_TANH: return dispatch<kUnary, XS_UNARY_GELU_TANH>(s, e, x_dtype, y_dtype, what);
        case XS_UNARY_SOFTCAP: return dispatch<kUnary, XS_UNARY_SOFTCAP>(s, e, x_dtype, y_dtype, what);
        case XS_UNARY_SIGMOID: return dispatch<kUnary, XS_UNARY_SIGMOID>(s, e, x_dtype, y_dtype, what);
        case XS_UNARY_SILU: return dispatch<kUnary, XS_UNARY_SILU>(s, e, x_dtype, y_dtype, what);
        case XS_UNARY_SOFTPLUS: return dispatch<kUnary, XS_UNARY_SOFTPLUS>(s, e, x_dtype, y_dtype, what);
        case XS_UNARY_CLAMP: return dispatch<kUnary, XS_UNARY_CLAMP>(s, e, x_dtype, y_dtype, what);
        case XS_UNARY_GELU: return dispatch<kUnary, XS_UNARY_GELU>(s, e, x_dtype, y_dtype, what);
        default: return fail(XS_HIP_EINVAL, std::string(what) + ": unknown unary op " + std::to_string(e.act));
    }
}

// Activation ops with a run-time act: one template instance per activation.
template <int OP>
int dispatch_act(hipStream_t s, const Ew2D& e, xs_dtype x_dtype, xs_dtype y_dtype, const char* what) {
    switch (e.act) {
        case XS_UNARY_SILU: return dispatch<OP, XS_UNARY_SILU>(s, e, x_dtype, y_dtype, what);
        case XS_UNARY_SIGMOID: return dispatch<OP, XS_UNARY_SIGMOID>(s, e, x_dtype, y_dtype, what);
        case XS_UNARY_GELU_TANH: return dispatch<OP, XS_UNARY_GELU_TANH>(s, e, x_dtype, y_dtype, what);
        case XS_UNARY_GELU: return dispatch<OP, XS_UNARY_GELU>(s, e, x_dtype, y_dtype, what);
        default:
            return fail(XS_HIP_EINVAL, std::string(what) + ": act must be silu, sigmoid, gelu_tanh or gelu, got " +
                                           std::to_string(e.act));
    }
}

}  // namespace ew
}  // namespace xs_hip
