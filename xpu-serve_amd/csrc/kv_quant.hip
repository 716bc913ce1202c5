// int8 KV-cache quantize and dequantize for gfx950.
//
// Semantics: quant::quantize_kv_row_i8 and quant::round_trip_kv_i8 (reference src/quant/quant.cpp:259-277), row
// layout quant::kv_row_bytes(I8) = {width codes, one f32 scale} (src/quant/kv_format.cpp:47-48), launchers
// sycl_be::quantize_kv / dequantize_kv (src/backend/sycl/sycl_kv_cache.cpp:33-49, 87-93, 119-150).
//
// Quantize layout: a row of `width` values is spread over LPR lanes (LPR = row bytes / 16, a power of two <= 64), each
// lane holding one 128-bit vector; rows per wave = 64 / LPR. The row's |x| maximum is a DPP reduction inside the LPR
// lanes, so a row never touches LDS. Each lane keeps U rows in flight (U independent 128-bit loads) to cover HBM
// latency. Rounding is the reference's: inv = 127.0f / amax (correctly rounded f32 division), code =
// rint(x * inv) (v_rndne_f32, round half to even) clamped to [-127, 127], scale = amax / 127.0f.
#include "common.h"

namespace xs_hip {
namespace {

// A NaN product has no defined int8 value in the reference (a float-to-int cast of NaN); on the x86-64 host the
// conversion yields INT_MIN whose low byte is 0, so a NaN code is 0 here as there.
__device__ __forceinline__ int quantize_code(float x, float inv) {
    float q = rintf(x * inv);
    if (q != q) return 0;
    q = fminf(fmaxf(q, -127.0f), 127.0f);
    return static_cast<int>(q);
}

template <typename T, int LPR, int U>
__global__ __launch_bounds__(kBlock) void quantize_i8_vec(const typename T::storage* __restrict__ x,
                                                          int8_t* __restrict__ codes, float* __restrict__ scales,
                                                          int64_t rows, int64_t width) {
    constexpr int VEC = vec_elems<T>();
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63;
    const int sub = lane / LPR;
    const int l = lane % LPR;
    const int64_t waves = static_cast<int64_t>(gridDim.x) * (kBlock / 64);
    const int64_t wave_id = static_cast<int64_t>(blockIdx.x) * (kBlock / 64) + (threadIdx.x >> 6);
    const int64_t stride = waves * RPW;
    for (int64_t base = wave_id * RPW + sub; base < rows + 0 * stride; base += U * stride) {
        u32x4 raw[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t r = base + u * stride;
            if (r < rows) raw[u] = ld128_nt(x + r * width + l * VEC);
            else raw[u] = u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t r = base + u * stride;
            float f[VEC];
            unpack<T>(raw[u], f);
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < VEC; ++i) amax = fmaxf(amax, fabsf(f[i]));
            amax = group_reduce<LPR, OpMax>(amax);
            const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
            if (r < rows) {
                if constexpr (VEC == 8) {
                    uint32_t lo = 0, hi = 0;
#pragma unroll
                    for (int i = 0; i < 4; ++i) lo |= (static_cast<uint32_t>(quantize_code(f[i], inv)) & 0xffu) << (8 * i);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        hi |= (static_cast<uint32_t>(quantize_code(f[4 + i], inv)) & 0xffu) << (8 * i);
                    uint2 packed = make_uint2(lo, hi);
                    __builtin_nontemporal_store(packed.x, reinterpret_cast<uint32_t*>(codes + r * width + l * VEC));
                    __builtin_nontemporal_store(packed.y, reinterpret_cast<uint32_t*>(codes + r * width + l * VEC) + 1);
                } else {
                    uint32_t w = 0;
#pragma unroll
                    for (int i = 0; i < 4; ++i) w |= (static_cast<uint32_t>(quantize_code(f[i], inv)) & 0xffu) << (8 * i);
                    __builtin_nontemporal_store(w, reinterpret_cast<uint32_t*>(codes + r * width + l * VEC));
                }
                if (l == 0) scales[r] = amax / 127.0f;
            }
        }
    }
}

// Any width: one wave per row, the row read twice (the second time from cache).
template <typename T>
__global__ __launch_bounds__(kBlock) void quantize_i8_any(const typename T::storage* __restrict__ x,
                                                          int8_t* __restrict__ codes, float* __restrict__ scales,
                                                          int64_t rows, int64_t width) {
    const int lane = threadIdx.x & 63;
    const int64_t waves = static_cast<int64_t>(gridDim.x) * (kBlock / 64);
    for (int64_t r = static_cast<int64_t>(blockIdx.x) * (kBlock / 64) + (threadIdx.x >> 6); r < rows; r += waves) {
        const typename T::storage* xr = x + r * width;
        float amax = 0.0f;
        for (int64_t i = lane; i < width; i += 64) amax = fmaxf(amax, fabsf(T::load(xr[i])));
        amax = group_reduce<64, OpMax>(amax);
        const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
        for (int64_t i = lane; i < width; i += 64)
            codes[r * width + i] = static_cast<int8_t>(quantize_code(T::load(xr[i]), inv));
        if (lane == 0) scales[r] = amax / 127.0f;
    }
}

// Unsigned 32-bit division by a run-time constant: q = (umulhi(n, m) + n) >> s with s = ceil(log2 d),
// m = floor(2^32 (2^s - d) / d) + 1 (Granlund and Montgomery, "Division by invariant integers using
// multiplication", 1994), exact for every n < 2^32.
struct FastDiv {
    uint32_t d = 1, m = 1, s = 0;
    FastDiv() = default;
    explicit FastDiv(uint32_t div) : d(div) {
        s = 0;
        while ((uint64_t{1} << s) < div) ++s;
        m = static_cast<uint32_t>(((uint64_t{1} << 32) * ((uint64_t{1} << s) - div)) / div + 1);
    }
    __device__ __forceinline__ uint32_t div(uint32_t n) const {
        return static_cast<uint32_t>((static_cast<uint64_t>(__umulhi(n, m)) + n) >> s);
    }
};

// out = fl32(code * scale[row]), 16 codes per lane (one 128-bit load), 16 outputs stored as 128-bit vectors.
template <typename Y>
__global__ __launch_bounds__(kBlock) void dequantize_i8_vec(const u32x4* __restrict__ codes,
                                                            const float* __restrict__ scales,
                                                            typename Y::storage* __restrict__ out, uint32_t nvec,
                                                            FastDiv vecs_per_row) {
    constexpr int OV = vec_elems<Y>();  // outputs per 128-bit store
    const uint32_t stride = gridDim.x * kBlock;
    for (uint32_t v = blockIdx.x * kBlock + threadIdx.x; v < nvec; v += stride) {
        const u32x4 raw = ld128_nt(codes + v);
        const float scale = scales[vecs_per_row.div(v)];
        float f[16];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int8_t c = static_cast<int8_t>((raw[w] >> (8 * b)) & 0xffu);
                f[4 * w + b] = static_cast<float>(c) * scale;
            }
        }
        typename Y::storage* o = out + static_cast<int64_t>(v) * 16;
#pragma unroll
        for (int k = 0; k < 16 / OV; ++k) st128_nt(o + k * OV, pack<Y>(f + k * OV));
    }
}

template <typename Y>
__global__ __launch_bounds__(kBlock) void dequantize_i8_any(const int8_t* __restrict__ codes,
                                                            const float* __restrict__ scales,
                                                            typename Y::storage* __restrict__ out, int64_t n,
                                                            int64_t width) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
        out[i] = Y::store(static_cast<float>(codes[i]) * scales[i / width]);
}

template <typename T>
int launch_quantize(hipStream_t s, const void* x, int8_t* codes, float* scales, int64_t rows, int64_t width) {
    using S = typename T::storage;
    const int64_t row_bytes = width * static_cast<int64_t>(sizeof(S));
    const bool vec_ok = row_bytes % 16 == 0 && aligned16(x) && (reinterpret_cast<uintptr_t>(codes) % 8 == 0) &&
                        ((width * 1) % 4 == 0);
    const int64_t lpr = row_bytes / 16;
    const auto* xs = static_cast<const S*>(x);
    constexpr int U = 4;
    auto go = [&](auto kernel, int rpw) {
        const int64_t slots_per_block = (kBlock / 64) * rpw;
        const unsigned grid = grid_for(rows, static_cast<int>(slots_per_block * U));
        kernel<<<grid, kBlock, 0, s>>>(xs, codes, scales, rows, width);
        return check_launch("xs_hip_quantize_kv");
    };
    if (vec_ok) {
        switch (lpr) {
            case 1: return go(quantize_i8_vec<T, 1, U>, 64);
            case 2: return go(quantize_i8_vec<T, 2, U>, 32);
            case 4: return go(quantize_i8_vec<T, 4, U>, 16);
            case 8: return go(quantize_i8_vec<T, 8, U>, 8);
            case 16: return go(quantize_i8_vec<T, 16, U>, 4);
            case 32: return go(quantize_i8_vec<T, 32, U>, 2);
            case 64: return go(quantize_i8_vec<T, 64, U>, 1);
            default: break;
        }
    }
    const unsigned grid = grid_for(rows, kBlock / 64);
    quantize_i8_any<T><<<grid, kBlock, 0, s>>>(xs, codes, scales, rows, width);
    return check_launch("xs_hip_quantize_kv");
}

template <typename Y>
int launch_dequantize(hipStream_t s, const int8_t* codes, const float* scales, void* out, int64_t rows,
                      int64_t width) {
    using S = typename Y::storage;
    const int64_t n = rows * width;
    auto* o = static_cast<S*>(out);
    if (width % 16 == 0 && aligned16(codes) && aligned16(out) && n / 16 < (int64_t{1} << 32)) {
        const uint32_t nvec = static_cast<uint32_t>(n / 16);
        dequantize_i8_vec<Y><<<grid_for(nvec, kBlock * 4), kBlock, 0, s>>>(
            reinterpret_cast<const u32x4*>(codes), scales, o, nvec, FastDiv(static_cast<uint32_t>(width / 16)));
    } else {
        dequantize_i8_any<Y><<<grid_for(n, kBlock * 4), kBlock, 0, s>>>(codes, scales, o, n, width);
    }
    return check_launch("xs_hip_dequantize_kv");
}

int check_kv_format(xs_kv_format format, const char* op) {
    if (format == XS_KV_I8) return XS_HIP_OK;
    if (format == XS_KV_FLOAT)
        return fail(XS_HIP_EINVAL, std::string(op) + ": the float format is stored as it is, not quantized");
    if (format >= XS_KV_TURBO4 && format <= XS_KV_TURBO2)
        return fail(XS_HIP_EUNSUPPORTED, std::string(op) + ": TurboQuant KV formats are not implemented on this device");
    return fail(XS_HIP_EINVAL, std::string(op) + ": unknown KV format " + std::to_string(static_cast<int>(format)));
}

}  // namespace
}  // namespace xs_hip

using namespace xs_hip;

extern "C" {

int xs_hip_quantize_kv(void* stream, xs_kv_format format, xs_dtype x_dtype, const void* x, void* codes, void* scales,
                       int64_t rows, int64_t width) {
    int rc = check_kv_format(format, "xs_hip_quantize_kv");
    if (rc != XS_HIP_OK) return rc;
    if (rows < 0 || width <= 0)
        return fail(XS_HIP_EINVAL, "xs_hip_quantize_kv: rows " + std::to_string(rows) + " of width " +
                                       std::to_string(width));
    if (rows == 0) return XS_HIP_OK;
    if (x == nullptr || codes == nullptr || scales == nullptr)
        return fail(XS_HIP_EINVAL, "xs_hip_quantize_kv: null buffer");
    if (reinterpret_cast<uintptr_t>(scales) % 4 != 0)
        return fail(XS_HIP_EINVAL, "xs_hip_quantize_kv: scales must be 4-byte aligned f32");
    auto* c = static_cast<int8_t*>(codes);
    auto* sc = static_cast<float*>(scales);
    switch (x_dtype) {
        case XS_F32: return launch_quantize<F32>(as_stream(stream), x, c, sc, rows, width);
        case XS_F16: return launch_quantize<F16>(as_stream(stream), x, c, sc, rows, width);
        case XS_BF16: return launch_quantize<BF16>(as_stream(stream), x, c, sc, rows, width);
        default:
            return fail(XS_HIP_EINVAL, std::string("xs_hip_quantize_kv: x must be f32, f16 or bf16, got ") +
                                           dtype_name(x_dtype));
    }
}

int xs_hip_dequantize_kv(void* stream, xs_kv_format format, const void* codes, const void* scales, xs_dtype out_dtype,
                         void* out, int64_t rows, int64_t width) {
    int rc = check_kv_format(format, "xs_hip_dequantize_kv");
    if (rc != XS_HIP_OK) return rc;
    if (rows < 0 || width <= 0)
        return fail(XS_HIP_EINVAL, "xs_hip_dequantize_kv: rows " + std::to_string(rows) + " of width " +
                                       std::to_string(width));
    if (rows == 0) return XS_HIP_OK;
    if (codes == nullptr || scales == nullptr || out == nullptr)
        return fail(XS_HIP_EINVAL, "xs_hip_dequantize_kv: null buffer");
    if (reinterpret_cast<uintptr_t>(scales) % 4 != 0)
        return fail(XS_HIP_EINVAL, "xs_hip_dequantize_kv: scales must be 4-byte aligned f32");
    const auto* c = static_cast<const int8_t*>(codes);
    const auto* sc = static_cast<const float*>(scales);
    switch (out_dtype) {
        case XS_F32: return launch_dequantize<F32>(as_stream(stream), c, sc, out, rows, width);
        case XS_F16: return launch_dequantize<F16>(as_stream(stream), c, sc, out, rows, width);
        case XS_BF16: return launch_dequantize<BF16>(as_stream(stream), c, sc, out, rows, width);
        default:
            return fail(XS_HIP_EINVAL, std::string("xs_hip_dequantize_kv: out must be f32, f16 or bf16, got ") +
                                           dtype_name(out_dtype));
    }
}

}  // extern "C"
