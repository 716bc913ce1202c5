// int8 KV-cache quantize and dequantize for gfx950.
//
// Semantics: quant::quantize_kv_row_i8 and quant::round_trip_kv_i8 (reference src/quant/quant.cpp:259-277), row
// layout quant::kv_row_bytes(I8) = {width codes, one f32 scale} (src/quant/kv_format.cpp:47-48), launchers
// sycl_be::quantize_kv / dequantize_kv (src/backend/sycl/sycl_kv_cache.cpp:33-49, 87-93, 119-150).
//
// Quantize layout: a row of `width` values is spread over L lanes (L = min(16, 128-bit vectors per row)), lane l
// holding the row's vectors l, l + L, ... (VPL of them), so every load instruction reads whole contiguous 256-byte
// runs of a row and every store instruction writes whole contiguous runs of codes -- no partial cache lines, which
// would cost a read of the line before the write. A row's |x| maximum is a DPP reduction inside its L lanes (no LDS).
// Each lane keeps U rows in flight (U * VPL independent 128-bit loads). Rounding is the reference's:
// inv = 127.0f / amax (correctly rounded f32 division), code = rint(x * inv) round half to even,
// scale = amax / 127.0f. rint is taken by adding 1.5 * 2^23 in f32 (the FPU's own round-to-nearest-even) and keeping
// the low byte, which is the code in two's complement since |x * inv| <= 127 (the clamp of the reference can never
// bind); a NaN product (a NaN input, or an infinite row's 0 * inf) leaves a quiet NaN, whose low byte is 0 for every
// f16/bf16 input and for the canonical NaN -- the value x86-64 gives the reference's cast of NaN.
//
// Dequantize layout: a unit is 8 codes (one 64-bit load) and their 8 outputs (one 128-bit store for f16/bf16, two
// for f32); consecutive lanes take consecutive units, so loads and stores are contiguous across the wave, and each
// lane keeps U units (codes and row scales) in flight.
//
// Both kernels give each workgroup one contiguous tile of the tensor and launch as many workgroups as there are
// tiles: the workgroups in flight then read one contiguous window of memory, which HBM serves faster than the
// scattered windows of a grid-stride loop.
#include "common.h"
#include "kv_turbo.h"

namespace xs_hip {
namespace {

// Scalar form of the rounding above (the any-width kernel).
__device__ __forceinline__ int quantize_code(float x, float inv) {
    float q = rintf(x * inv);
    if (q != q) return 0;
    q = fminf(fmaxf(q, -127.0f), 127.0f);
    return static_cast<int>(q);
}

// x * inv + 1.5 * 2^23: the low byte of the sum's bits is rint(x * inv) (|x * inv| <= 127), or 0 for NaN.
__device__ __forceinline__ uint32_t code_bits(float x, float inv) {
    return __float_as_uint(x * inv + 12582912.0f);
}

// code_bits for a row whose 127 / amax overflowed to inf (0 < amax < 127 / FLT_MAX, which only f32 and bf16 inputs
// reach): x * inv is then +-inf for a nonzero x, which the reference's clamp takes to +-127, and NaN for 0 (code 0);
// the scalar form gives exactly that. `huge` is uniform over a row.
template <typename T>
__device__ __forceinline__ uint32_t row_code(float x, float inv, bool huge) {
    if constexpr (T::dtype == XS_F16) return code_bits(x, inv);  // |x| >= 2^-24: 127 / amax is finite
    return huge ? static_cast<uint32_t>(quantize_code(x, inv)) : code_bits(x, inv);
}

// The low bytes of four words, packed in order into one word.
__device__ __forceinline__ uint32_t pack_low_bytes(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const uint32_t ab = __builtin_amdgcn_perm(b, a, 0x0c0c0400u);  // a.b0 | b.b0 << 8
    const uint32_t cd = __builtin_amdgcn_perm(d, c, 0x04000c0cu);  // c.b0 << 16 | d.b0 << 24
    return ab | cd;
}

// Threads of a quantize workgroup.
constexpr int kQBlock = 256;

// Where a quantize writes: rows [0, rows) of codes / scales, or, with `row0` set, rows row0[0] * unit + r of a cache of
// `cap` rows -- the destination read from device memory when the kernel runs (a step replayed from a captured graph
// appends where the cache ends that step). A destination past the cache writes nothing.
struct QuantDest {
    const int64_t* row0 = nullptr;
    int64_t unit = 0, cap = 0;
};

// The first destination row, or -1 when the destination lies outside the cache.
__device__ __forceinline__ int64_t first_row(const QuantDest& d, int64_t rows) {
    if (d.row0 == nullptr) return 0;
    const int64_t off = d.row0[0] * d.unit;
    return off < 0 || off > d.cap - rows ? -1 : off;
}

// A second tensor quantized by the same launch (a step's values beside its keys): workgroups from `first_block` on
// take it, at the same rows of its own cache.
struct QuantSecond {
    const void* x = nullptr;
    int8_t* codes = nullptr;
    float* scales = nullptr;
    unsigned first_block = 0;
};

// MODE 0: one tensor; 1: one tensor at a device-resident destination; 2: two tensors, the destination as in 1 or,
// with no row0, at their buffers' starts.
template <typename T, int L, int VPL, int U, int MODE>
__global__ __launch_bounds__(kQBlock) void quantize_i8_vec(const typename T::storage* __restrict__ x,
                                                          int8_t* __restrict__ codes, float* __restrict__ scales,
                                                          int64_t rows, int64_t width, QuantDest dest,
                                                          QuantSecond second) {
    unsigned block = blockIdx.x;
    if constexpr (MODE == 2) {
        if (block >= second.first_block) {
            x = static_cast<const typename T::storage*>(second.x);
            codes = second.codes;
            scales = second.scales;
            block -= second.first_block;
        }
    }
    if constexpr (MODE != 0) {
        const int64_t off = first_row(dest, rows);
        if (off < 0) return;
        codes += off * width;
        scales += off;
    }
    constexpr int VEC = vec_elems<T>();
    constexpr int RPW = 64 / L;  // rows per wave
    constexpr int WAVES = kQBlock / 64;
    const int lane = threadIdx.x & 63;
    const int sub = lane / L;
    const int l = lane % L;
    // The block's tile: U * WAVES * RPW contiguous rows; wave w takes rows (u * WAVES + w) * RPW + sub.
    constexpr int64_t stride = WAVES * RPW;
    {
        const int64_t base = static_cast<int64_t>(block) * (U * WAVES * RPW) + (threadIdx.x >> 6) * RPW + sub;
        u32x4 raw[U][VPL];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t r = base + u * stride;
#pragma unroll
            for (int k = 0; k < VPL; ++k)
                raw[u][k] = r < rows ? ld128_nt(x + r * width + (l + k * L) * VEC) : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t r = base + u * stride;
            float f[VPL][VEC];
#pragma unroll
            for (int k = 0; k < VPL; ++k) unpack<T>(raw[u][k], f[k]);
            float amax = 0.0f;
#pragma unroll
            for (int k = 0; k < VPL; ++k)
#pragma unroll
                for (int i = 0; i < VEC; ++i) amax = fmaxf(amax, fabsf(f[k][i]));
            amax = group_reduce<L, OpMax>(amax);
            const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
            const bool huge = inv > 3.40282347e38f;
            if (r < rows) {
#pragma unroll
                for (int k = 0; k < VPL; ++k) {
                    int8_t* out = codes + r * width + (l + k * L) * VEC;
                    const uint32_t w0 =
                        pack_low_bytes(row_code<T>(f[k][0], inv, huge), row_code<T>(f[k][1], inv, huge),
                                       row_code<T>(f[k][2], inv, huge), row_code<T>(f[k][3], inv, huge));
                    if constexpr (VEC == 8) {
                        const uint32_t w1 =
                            pack_low_bytes(row_code<T>(f[k][4], inv, huge), row_code<T>(f[k][5], inv, huge),
                                           row_code<T>(f[k][6], inv, huge), row_code<T>(f[k][7], inv, huge));
                        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
                        __builtin_nontemporal_store(u32x2{w0, w1}, reinterpret_cast<u32x2*>(out));
                    } else {
                        __builtin_nontemporal_store(w0, reinterpret_cast<uint32_t*>(out));
                    }
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
                                                          int64_t rows, int64_t width, QuantDest dest) {
    const int64_t off = first_row(dest, rows);
    if (off < 0) return;
    codes += off * width;
    scales += off;
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

// Threads of a dequantize workgroup.
constexpr int kDeqBlock = 64;

// out = fl32(code * scale[row]) for units of 8 codes.
template <typename Y, int U>
__global__ __launch_bounds__(kDeqBlock) void dequantize_i8_vec(const uint64_t* __restrict__ codes,
                                                            const float* __restrict__ scales,
                                                            typename Y::storage* __restrict__ out, uint32_t units,
                                                            FastDiv32 units_per_row) {
    constexpr uint32_t stride = kDeqBlock;
    {
        const uint32_t v0 = blockIdx.x * (kDeqBlock * U) + threadIdx.x;
        uint64_t raw[U];
        float scale[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t v = v0 + u * stride;
            if (v < units) {
                raw[u] = __builtin_nontemporal_load(codes + v);
                scale[u] = scales[units_per_row.div(v)];
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t v = v0 + u * stride;
            if (v < units) {
                float f[8];
#pragma unroll
                for (int b = 0; b < 8; ++b) {
                    const int code = static_cast<int>(static_cast<int8_t>((raw[u] >> (8 * b)) & 0xffu));
                    f[b] = static_cast<float>(code) * scale[u];
                }
                typename Y::storage* o = out + static_cast<int64_t>(v) * 8;
                if constexpr (sizeof(typename Y::storage) == 2) {
                    st128_nt(o, pack<Y>(f));
                } else {
                    st128_nt(o, pack<Y>(f));
                    st128_nt(o + 4, pack<Y>(f + 4));
                }
            }
        }
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
int launch_quantize(hipStream_t s, const void* x, int8_t* codes, float* scales, int64_t rows, int64_t width,
                    const QuantDest& dest, QuantSecond second = QuantSecond{}) {
    using S = typename T::storage;
    const int64_t row_bytes = width * static_cast<int64_t>(sizeof(S));
    const int64_t nvr = row_bytes / 16;  // 128-bit vectors per row
    const bool pair = second.x != nullptr;
    const bool vec_ok = row_bytes % 16 == 0 && aligned16(x) && (reinterpret_cast<uintptr_t>(codes) % 8 == 0) &&
                        (nvr & (nvr - 1)) == 0 && nvr >= 1 && nvr <= 64 &&
                        (!pair || (aligned16(second.x) && reinterpret_cast<uintptr_t>(second.codes) % 8 == 0));
    const auto* xs = static_cast<const S*>(x);
    constexpr int U = 2;
    auto go = [&](auto kernel, auto kernel_dest, auto kernel_pair, int lanes) {
        const int64_t rows_per_tile = (kQBlock / 64) * (64 / lanes) * U;
        const unsigned grid = static_cast<unsigned>((rows + rows_per_tile - 1) / rows_per_tile);
        if (pair) {
            second.first_block = grid;
            kernel_pair<<<2 * grid, kQBlock, 0, s>>>(xs, codes, scales, rows, width, dest, second);
        } else if (dest.row0 != nullptr) {
            kernel_dest<<<grid, kQBlock, 0, s>>>(xs, codes, scales, rows, width, dest, second);
        } else {
            kernel<<<grid, kQBlock, 0, s>>>(xs, codes, scales, rows, width, dest, second);
        }
        return check_launch("xs_hip_quantize_kv");
    };
    if (vec_ok) {
        switch (nvr) {
            case 1:
                return go(quantize_i8_vec<T, 1, 1, U, 0>, quantize_i8_vec<T, 1, 1, U, 1>,
                          quantize_i8_vec<T, 1, 1, U, 2>, 1);
            case 2:
                return go(quantize_i8_vec<T, 2, 1, U, 0>, quantize_i8_vec<T, 2, 1, U, 1>,
                          quantize_i8_vec<T, 2, 1, U, 2>, 2);
            case 4:
                return go(quantize_i8_vec<T, 4, 1, U, 0>, quantize_i8_vec<T, 4, 1, U, 1>,
                          quantize_i8_vec<T, 4, 1, U, 2>, 4);
            case 8:
                return go(quantize_i8_vec<T, 8, 1, U, 0>, quantize_i8_vec<T, 8, 1, U, 1>,
                          quantize_i8_vec<T, 8, 1, U, 2>, 8);
            case 16:
                return go(quantize_i8_vec<T, 16, 1, U, 0>, quantize_i8_vec<T, 16, 1, U, 1>,
                          quantize_i8_vec<T, 16, 1, U, 2>, 16);
            case 32:
                return go(quantize_i8_vec<T, 16, 2, U, 0>, quantize_i8_vec<T, 16, 2, U, 1>,
                          quantize_i8_vec<T, 16, 2, U, 2>, 16);
            case 64:
                return go(quantize_i8_vec<T, 16, 4, U, 0>, quantize_i8_vec<T, 16, 4, U, 1>,
                          quantize_i8_vec<T, 16, 4, U, 2>, 16);
            default: break;
        }
    }
    const unsigned grid = grid_for(rows, kBlock / 64);
    quantize_i8_any<T><<<grid, kBlock, 0, s>>>(xs, codes, scales, rows, width, dest);
    if (pair)  // the second tensor by a second launch on this path
        quantize_i8_any<T><<<grid, kBlock, 0, s>>>(static_cast<const S*>(second.x), second.codes, second.scales, rows,
                                                   width, dest);
    return check_launch("xs_hip_quantize_kv");
}

template <typename Y>
int launch_dequantize(hipStream_t s, const int8_t* codes, const float* scales, void* out, int64_t rows,
                      int64_t width) {
    using S = typename Y::storage;
    const int64_t n = rows * width;
    auto* o = static_cast<S*>(out);
    if (width % 8 == 0 && reinterpret_cast<uintptr_t>(codes) % 8 == 0 && aligned16(out) && n / 8 < (int64_t{1} << 31)) {
        // (below 2^31 units no lane index wraps in 32 bits)
        const uint32_t units = static_cast<uint32_t>(n / 8);
        constexpr int U = 1;
        dequantize_i8_vec<Y, U><<<(units + kDeqBlock * U - 1) / (kDeqBlock * U), kDeqBlock, 0, s>>>(
            reinterpret_cast<const uint64_t*>(codes), scales, o, units, FastDiv32(static_cast<uint32_t>(width / 8)));
    } else {
        dequantize_i8_any<Y><<<grid_for(n, kBlock * 4), kBlock, 0, s>>>(codes, scales, o, n, width);
    }
    return check_launch("xs_hip_dequantize_kv");
}

// Bits a code of a TurboQuant format (quant::turbo_bits, src/quant/kv_format.cpp).
int turbo_bits(xs_kv_format f) { return f == XS_KV_TURBO4 ? 4 : f == XS_KV_TURBO3 ? 3 : 2; }

int check_kv_format(xs_kv_format format, const char* op) {
    if (format == XS_KV_I8) return XS_HIP_OK;
    if (format == XS_KV_FLOAT)
        return fail(XS_HIP_EINVAL, std::string(op) + ": the float format is stored as it is, not quantized");
    if (format >= XS_KV_TURBO4 && format <= XS_KV_TURBO2) return XS_HIP_OK;
    return fail(XS_HIP_EINVAL, std::string(op) + ": unknown KV format " + std::to_string(static_cast<int>(format)));
}

int quantize_i8(void* stream, xs_dtype x_dtype, const void* x, void* codes, void* scales, int64_t rows, int64_t width,
                const QuantDest& dest, const char* what, const QuantSecond& second = QuantSecond{}) {
    auto* c = static_cast<int8_t*>(codes);
    auto* sc = static_cast<float*>(scales);
    switch (x_dtype) {
        case XS_F32: return launch_quantize<F32>(as_stream(stream), x, c, sc, rows, width, dest, second);
        case XS_F16: return launch_quantize<F16>(as_stream(stream), x, c, sc, rows, width, dest, second);
        case XS_BF16: return launch_quantize<BF16>(as_stream(stream), x, c, sc, rows, width, dest, second);
        default:
            return fail(XS_HIP_EINVAL, std::string(what) + ": x must be f32, f16 or bf16, got " + dtype_name(x_dtype));
    }
}

// ---- The float KV format: a step's keys and values appended as rows of the cache's float type -------------------
//
// The Float format stores each appended row as the precision's float (quant::round_trip_kv leaves it as is:
// src/quant/kv_format.cpp:57-61): f16 rows at f16 precision (the SYCL session's to_half, sycl_backend.cpp:2224-2228,
// RNE), f32 rows at f32. One launch writes keys and values: unit u of 8 elements (or one element, off the vector path)
// of row r goes to row `first` + r of its cache, `first` = row0[0] * unit rows when the destination is read from
// device memory (a step replayed from a captured graph), rows past the cache written nowhere.
template <typename XT, typename YT, bool VEC>
__global__ __launch_bounds__(256) void kv_store_rows(const void* k, const void* v, void* ky, void* vy, int64_t rows,
                                                     int64_t width, QuantDest dest) {
    int64_t first = 0, limit = rows;
    if (dest.row0 != nullptr) {
        first = dest.row0[0] * dest.unit;
        limit = first < 0 ? 0 : (dest.cap - first < rows ? dest.cap - first : rows);
    }
    const int64_t per = VEC ? 8 : 1;
    const int64_t units = limit > 0 ? limit * (width / per) : 0;
    const int64_t total = v != nullptr ? 2 * units : units;  // no values: keys only
    for (int64_t u = blockIdx.x * 256 + threadIdx.x; u < total; u += static_cast<int64_t>(gridDim.x) * 256) {
        const bool is_v = u >= units;
        const int64_t e = (is_v ? u - units : u) * per;  // element of the step's [rows, width]
        const auto* x = static_cast<const typename XT::storage*>(is_v ? v : k) + e;
        auto* y = static_cast<typename YT::storage*>(is_v ? vy : ky) + first * width + e;
        if constexpr (VEC) {
            float f[8];
            if constexpr (sizeof(typename XT::storage) == 4) {
                unpack<XT>(ld128(x), f);
                unpack<XT>(ld128(x + 4), f + 4);
            } else {
                unpack<XT>(ld128(x), f);
            }
            if constexpr (sizeof(typename YT::storage) == 4) {
                st128(y, pack<YT>(f));
                st128(y + 4, pack<YT>(f + 4));
            } else {
                st128(y, pack<YT>(f));
            }
        } else {
            *y = YT::store(XT::load(*x));
        }
    }
}

template <typename XT, typename YT>
int launch_kv_store(hipStream_t s, const void* k, const void* v, void* ky, void* vy, int64_t rows, int64_t width,
                    const QuantDest& dest, const char* what) {
    const bool vec = width % 8 == 0 && aligned16(k) && aligned16(v) && aligned16(ky) && aligned16(vy);  // null: aligned
    const int64_t units = 2 * rows * (vec ? width / 8 : width);
    const unsigned grid = grid_for(units, 256);
    if (vec) kv_store_rows<XT, YT, true><<<grid, 256, 0, s>>>(k, v, ky, vy, rows, width, dest);
    else kv_store_rows<XT, YT, false><<<grid, 256, 0, s>>>(k, v, ky, vy, rows, width, dest);
    return check_launch(what);
}

template <typename XT>
int kv_store_from(hipStream_t s, xs_dtype row_dtype, const void* k, const void* v, void* ky, void* vy, int64_t rows,
                  int64_t width, const QuantDest& dest, const char* what) {
    if (row_dtype == XS_F16) return launch_kv_store<XT, F16>(s, k, v, ky, vy, rows, width, dest, what);
    return launch_kv_store<XT, F32>(s, k, v, ky, vy, rows, width, dest, what);
}

}  // namespace
}  // namespace xs_hip

using namespace xs_hip;

extern "C" {

int xs_hip_quantize_kv(void* stream, xs_kv_format format, xs_dtype x_dtype, const void* x, void* codes, void* scales,
                       int64_t rows, int64_t width) {
    int rc = check_kv_format(format, "xs_hip_quantize_kv");
    if (rc != XS_HIP_OK) return rc;
    if (format != XS_KV_I8)
        return turbo_quantize(as_stream(stream), turbo_bits(format), x_dtype, x, codes, scales, rows, width);
    if (rows < 0 || width <= 0)
        return fail(XS_HIP_EINVAL, "xs_hip_quantize_kv: rows " + std::to_string(rows) + " of width " +
                                       std::to_string(width));
    if (rows == 0) return XS_HIP_OK;
    if (x == nullptr || codes == nullptr || scales == nullptr)
        return fail(XS_HIP_EINVAL, "xs_hip_quantize_kv: null buffer");
    if (reinterpret_cast<uintptr_t>(scales) % 4 != 0)
        return fail(XS_HIP_EINVAL, "xs_hip_quantize_kv: scales must be 4-byte aligned f32");
    return quantize_i8(stream, x_dtype, x, codes, scales, rows, width, QuantDest{}, "xs_hip_quantize_kv");
}

int xs_hip_quantize_kv_pair(void* stream, xs_dtype x_dtype, const void* k, const void* v, void* k_codes, void* k_scales,
                            void* v_codes, void* v_scales, int64_t rows, int64_t width, const int64_t* row0,
                            int64_t rows_per_unit, int64_t capacity_rows) {
    const char* what = "xs_hip_quantize_kv_pair";
    if (rows < 0 || width <= 0 || (row0 != nullptr && (rows_per_unit < 0 || capacity_rows < 0)))
        return fail(XS_HIP_EINVAL, std::string(what) + ": rows " + std::to_string(rows) + " of width " +
                                       std::to_string(width) + ", " + std::to_string(rows_per_unit) +
                                       " rows a unit, capacity " + std::to_string(capacity_rows));
    if (rows == 0) return XS_HIP_OK;
    if (k == nullptr || v == nullptr || k_codes == nullptr || k_scales == nullptr || v_codes == nullptr ||
        v_scales == nullptr)
        return fail(XS_HIP_EINVAL, std::string(what) + ": null buffer");
    if (reinterpret_cast<uintptr_t>(k_scales) % 4 != 0 || reinterpret_cast<uintptr_t>(v_scales) % 4 != 0 ||
        reinterpret_cast<uintptr_t>(row0) % 8 != 0)
        return fail(XS_HIP_EINVAL, std::string(what) + ": scales must be 4-byte and row0 8-byte aligned");
    const QuantDest dest = row0 != nullptr ? QuantDest{row0, rows_per_unit, capacity_rows} : QuantDest{};
    return quantize_i8(stream, x_dtype, k, k_codes, k_scales, rows, width, dest, what,
                       QuantSecond{v, static_cast<int8_t*>(v_codes), static_cast<float*>(v_scales), 0});
}

int xs_hip_quantize_kv_at(void* stream, xs_dtype x_dtype, const void* x, void* codes, void* scales, int64_t rows,
                          int64_t width, const int64_t* row0, int64_t rows_per_unit, int64_t capacity_rows) {
    const char* what = "xs_hip_quantize_kv_at";
    if (rows < 0 || width <= 0 || rows_per_unit < 0 || capacity_rows < 0)
        return fail(XS_HIP_EINVAL, std::string(what) + ": rows " + std::to_string(rows) + " of width " +
                                       std::to_string(width) + ", " + std::to_string(rows_per_unit) +
                                       " rows a unit, capacity " + std::to_string(capacity_rows));
    if (rows == 0) return XS_HIP_OK;
    if (x == nullptr || codes == nullptr || scales == nullptr || row0 == nullptr)
        return fail(XS_HIP_EINVAL, std::string(what) + ": null buffer");
    if (reinterpret_cast<uintptr_t>(scales) % 4 != 0 || reinterpret_cast<uintptr_t>(row0) % 8 != 0)
        return fail(XS_HIP_EINVAL, std::string(what) + ": scales must be 4-byte and row0 8-byte aligned");
    return quantize_i8(stream, x_dtype, x, codes, scales, rows, width, QuantDest{row0, rows_per_unit, capacity_rows},
                       what);
}

int xs_hip_quantize_kv_turbo_at(void* stream, xs_kv_format format, xs_dtype x_dtype, const void* x, void* codes,
                                void* norms, int64_t rows, int64_t width, const int64_t* row0, int64_t rows_per_unit,
                                int64_t capacity_rows) {
    const char* what = "xs_hip_quantize_kv_turbo_at";
    if (format < XS_KV_TURBO4 || format > XS_KV_TURBO2)
        return fail(XS_HIP_EINVAL, std::string(what) + ": format " + std::to_string(static_cast<int>(format)) +
                                       " is not a TurboQuant format");
    if (rows < 0 || rows_per_unit < 0 || capacity_rows < 0)
        return fail(XS_HIP_EINVAL, std::string(what) + ": rows " + std::to_string(rows) + ", " +
                                       std::to_string(rows_per_unit) + " rows a unit, capacity " +
                                       std::to_string(capacity_rows));
    if (row0 == nullptr) return fail(XS_HIP_EINVAL, std::string(what) + ": null row0");
    return turbo_quantize(as_stream(stream), turbo_bits(format), x_dtype, x, codes, norms, rows, width, row0,
                          rows_per_unit, capacity_rows);
}

int xs_hip_dequantize_kv(void* stream, xs_kv_format format, const void* codes, const void* scales, xs_dtype out_dtype,
                         void* out, int64_t rows, int64_t width) {
    int rc = check_kv_format(format, "xs_hip_dequantize_kv");
    if (rc != XS_HIP_OK) return rc;
    if (format != XS_KV_I8)
        return turbo_dequantize(as_stream(stream), turbo_bits(format), codes, scales, out_dtype, out, rows, width);
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

int xs_hip_kv_store_pair(void* stream, xs_dtype x_dtype, const void* k, const void* v, xs_dtype row_dtype,
                         void* k_rows, void* v_rows, int64_t rows, int64_t width, const int64_t* row0,
                         int64_t rows_per_unit, int64_t capacity_rows) {
    const char* what = "xs_hip_kv_store_pair";
    if (rows < 0 || width <= 0 || (row0 != nullptr && (rows_per_unit < 0 || capacity_rows < 0)))
        return fail(XS_HIP_EINVAL, std::string(what) + ": rows " + std::to_string(rows) + " of width " +
                                       std::to_string(width) + ", " + std::to_string(rows_per_unit) +
                                       " rows a unit, capacity " + std::to_string(capacity_rows));
    if (!is_float_dtype(x_dtype) || (row_dtype != XS_F16 && row_dtype != XS_F32))
        return fail(XS_HIP_EUNSUPPORTED, std::string(what) + ": " + dtype_name(x_dtype) + " rows into a cache of " +
                                             dtype_name(row_dtype) + " (inputs f32, f16 or bf16; cache f16 or f32)");
    if (rows == 0) return XS_HIP_OK;
    if (k == nullptr || k_rows == nullptr || (v == nullptr) != (v_rows == nullptr))
        return fail(XS_HIP_EINVAL, std::string(what) + ": null buffer");
    if (reinterpret_cast<uintptr_t>(row0) % 8 != 0)
        return fail(XS_HIP_EINVAL, std::string(what) + ": row0 must be 8-byte aligned");
    const QuantDest dest = row0 != nullptr ? QuantDest{row0, rows_per_unit, capacity_rows} : QuantDest{};
    const hipStream_t s = as_stream(stream);
    switch (x_dtype) {
        case XS_F32: return kv_store_from<F32>(s, row_dtype, k, v, k_rows, v_rows, rows, width, dest, what);
        case XS_F16: return kv_store_from<F16>(s, row_dtype, k, v, k_rows, v_rows, rows, width, dest, what);
        default: return kv_store_from<BF16>(s, row_dtype, k, v, k_rows, v_rows, rows, width, dest, what);
    }
}

}  // extern "C"
