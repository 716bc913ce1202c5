// Rotate-half (NeoX) RoPE for gfx950.
//
// Semantics: cpu_ref::rope (reference src/backend/cpu_ref/ops.cpp:343-399), spec graph.h Rope (src/graph/graph.h:
// 119-127): for a pair (c1, c2 = c1 + W/2) of a section of width W, angle = double(pos) * double(inv_freq[i]),
// c, s = cos, sin(angle) in f64, y1 = fl32(x1 * c - x2 * s), y2 = fl32(x2 * c + x1 * s) with the products and sums in
// f64; channels past `rotary` pass through. Axial positions [T, S] rotate section s by positions[:, s]; with pair_axes
// one section whose pair i reads positions[:, pair_axes[i]]. Launcher replaced: sycl_be::rope
// (src/backend/sycl/sycl_kernels.h:114-116, sycl_kernels.cpp:1678-1717), which uses an f32 angle; this kernel keeps the
// reference CPU path's f64 angle, so its outputs round from the same f64 values cpu-ref computes.
//
// Layout: a block takes a tile of TT tokens. Its threads first fill an LDS table of (cos, sin) in f64 for the tile's
// TT x pairs entries -- one sincos per (token, pair), shared by every head of the token -- then each unit of work
// (token, head, VEC consecutive pairs) loads VEC values of x1 and of x2 with 128-bit loads, rotates them in f64, and
// stores the two 128-bit (or narrower, by output dtype) vectors.
#include <cmath>

#include "common.h"

namespace xs_hip {
namespace {

struct RopeArgs {
    const void* x;
    const void* pos;
    const float* inv_freq;
    void* y;
    const int32_t* pair_axes;
    int64_t tokens, heads, dim, rotary, sections;
    int tile_tokens;
};

template <typename I>
__device__ __forceinline__ int64_t pos_at(const void* p, int64_t i) {
    return static_cast<int64_t>(static_cast<const I*>(p)[i]);
}

// Stores N consecutive outputs (N = 1, 4 or 8) of type T.
template <typename T, int N>
__device__ __forceinline__ void store_n(typename T::storage* p, const float* f) {
    if constexpr (N == 1) {
        p[0] = T::store(f[0]);
    } else if constexpr (N * sizeof(typename T::storage) == 16) {
        st128(p, pack<T>(f));
    } else if constexpr (N * sizeof(typename T::storage) == 32) {
        st128(p, pack<T>(f));
        st128(p + 16 / sizeof(typename T::storage), pack<T>(f + 16 / sizeof(typename T::storage)));
    } else {  // 4 x 16-bit = 8 bytes
        uint2 v;
        v.x = static_cast<uint32_t>(T::store(f[0])) | (static_cast<uint32_t>(T::store(f[1])) << 16);
        v.y = static_cast<uint32_t>(T::store(f[2])) | (static_cast<uint32_t>(T::store(f[3])) << 16);
        *reinterpret_cast<uint2*>(p) = v;
    }
}

template <typename T, int N>
__device__ __forceinline__ void load_n(const typename T::storage* p, float* f) {
    if constexpr (N == 1) {
        f[0] = T::load(p[0]);
    } else {
        static_assert(N * sizeof(typename T::storage) == 16, "one 128-bit vector");
        unpack<T>(ld128_nt(p), f);
    }
}

constexpr int kMaxTableEntries = 2048;  // (cos, sin) f64 pairs: 32 KiB of LDS

template <typename TX, typename TY, typename I, int VEC>
__global__ __launch_bounds__(kBlock) void rope_kernel(RopeArgs a) {
    using SX = typename TX::storage;
    using SY = typename TY::storage;
    __shared__ double2 table[kMaxTableEntries];

    const int64_t pairs = a.rotary / 2;
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * a.tile_tokens;
    const int tt_n = static_cast<int>(a.tokens - t0 < a.tile_tokens ? a.tokens - t0 : a.tile_tokens);
    const bool axes = a.pair_axes != nullptr;
    const int64_t width = axes ? a.rotary : a.rotary / a.sections;  // section width
    const int64_t half = width / 2;

    // (cos, sin) of every (token, pair) of the tile.
    const int entries = tt_n * static_cast<int>(pairs);
    for (int e = threadIdx.x; e < entries; e += kBlock) {
        const int tt = e / static_cast<int>(pairs);
        const int64_t p = e - static_cast<int64_t>(tt) * pairs;
        const int64_t t = t0 + tt;
        int64_t sec, i;
        if (axes) {
            // Axes outside [0, sections) are a caller error the host cannot see in device memory; clamp so the read
            // stays in bounds.
            sec = a.pair_axes[p];
            sec = sec < 0 ? 0 : (sec >= a.sections ? a.sections - 1 : sec);
            i = p;
        } else {
            sec = p / half;
            i = p - sec * half;
        }
        const double pos = static_cast<double>(pos_at<I>(a.pos, t * a.sections + sec));
        const double angle = pos * static_cast<double>(a.inv_freq[i]);
        double s, c;
        sincos(angle, &s, &c);
        table[e] = make_double2(c, s);
    }
    __syncthreads();

    const SX* x = static_cast<const SX*>(a.x);
    SY* y = static_cast<SY*>(a.y);
    const int pv_per_head = static_cast<int>(pairs / VEC);
    const int rot_units = tt_n * static_cast<int>(a.heads) * pv_per_head;
    for (int u = threadIdx.x; u < rot_units; u += kBlock) {
        const int tt = u / (static_cast<int>(a.heads) * pv_per_head);
        const int rem = u - tt * static_cast<int>(a.heads) * pv_per_head;
        const int h = rem / pv_per_head;
        const int p0 = (rem - h * pv_per_head) * VEC;
        int64_t c1;
        if (axes) {
            c1 = p0;
        } else {
            const int64_t sec = p0 / half;
            c1 = sec * width + (p0 - sec * half);
        }
        const int64_t base = ((t0 + tt) * a.heads + h) * a.dim;
        float x1[VEC], x2[VEC], y1[VEC], y2[VEC];
        load_n<TX, VEC>(x + base + c1, x1);
        load_n<TX, VEC>(x + base + c1 + half, x2);
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
            const double2 cs = table[tt * pairs + p0 + k];
            const double d1 = x1[k], d2 = x2[k];
            y1[k] = static_cast<float>(d1 * cs.x - d2 * cs.y);
            y2[k] = static_cast<float>(d2 * cs.x + d1 * cs.y);
        }
        store_n<TY, VEC>(y + base + c1, y1);
        store_n<TY, VEC>(y + base + c1 + half, y2);
    }

    // Channels past the rotary dims pass through (unless y is x).
    if (a.rotary < a.dim && static_cast<const void*>(a.x) != a.y) {
        const int64_t rest = a.dim - a.rotary;
        const int64_t units = static_cast<int64_t>(tt_n) * a.heads * rest;
        for (int64_t u = threadIdx.x; u < units; u += kBlock) {
            const int64_t row = u / rest;
            const int64_t c = a.rotary + (u - row * rest);
            const int64_t at = (t0 * a.heads + row) * a.dim + c;
            y[at] = TY::store(TX::load(x[at]));
        }
    }
}

template <typename TX, typename TY, typename I>
int launch_rope(hipStream_t s, RopeArgs a) {
    constexpr int VEC = vec_elems<TX>();
    const int64_t pairs = a.rotary / 2;
    const bool axes = a.pair_axes != nullptr;
    const int64_t half = axes ? pairs : (a.rotary / a.sections) / 2;
    const bool vec = half % VEC == 0 && a.dim % VEC == 0 && aligned16(a.x) && aligned16(a.y) &&
                     (sizeof(typename TY::storage) * VEC >= 16 || reinterpret_cast<uintptr_t>(a.y) % 8 == 0);
    // Tokens per block: enough rotation units for two per thread, within the LDS table.
    const int64_t units_per_token = a.heads * (pairs / (vec ? VEC : 1));
    int64_t tt = units_per_token > 0 ? (2 * kBlock + units_per_token - 1) / units_per_token : 1;
    if (tt < 1) tt = 1;
    const int64_t max_tt = pairs > 0 ? kMaxTableEntries / pairs : 64;
    if (tt > max_tt) tt = max_tt;
    if (tt > 64) tt = 64;
    a.tile_tokens = static_cast<int>(tt);
    const unsigned grid = static_cast<unsigned>((a.tokens + tt - 1) / tt);
    if (vec) rope_kernel<TX, TY, I, VEC><<<grid, kBlock, 0, s>>>(a);
    else rope_kernel<TX, TY, I, 1><<<grid, kBlock, 0, s>>>(a);
    return check_launch("xs_hip_rope");
}

template <typename TX, typename TY>
int rope_pos(hipStream_t s, const RopeArgs& a, xs_dtype pos_dtype) {
    switch (pos_dtype) {
        case XS_I32: return launch_rope<TX, TY, int32_t>(s, a);
        case XS_I64: return launch_rope<TX, TY, int64_t>(s, a);
        default: return fail(XS_HIP_EINVAL, std::string("xs_hip_rope: positions must be i32 or i64, got ") + dtype_name(pos_dtype));
    }
}

template <typename TX>
int rope_y(hipStream_t s, const RopeArgs& a, xs_dtype pos_dtype, xs_dtype y_dtype) {
    switch (y_dtype) {
        case XS_F32: return rope_pos<TX, F32>(s, a, pos_dtype);
        case XS_F16: return rope_pos<TX, F16>(s, a, pos_dtype);
        case XS_BF16: return rope_pos<TX, BF16>(s, a, pos_dtype);
        default: return fail(XS_HIP_EINVAL, std::string("xs_hip_rope: y must be f32, f16 or bf16, got ") + dtype_name(y_dtype));
    }
}

std::string i2s(int64_t v) { return std::to_string(v); }

}  // namespace
}  // namespace xs_hip

using namespace xs_hip;

extern "C" {

int xs_hip_rope(void* stream, xs_dtype x_dtype, const void* x, xs_dtype pos_dtype, const void* positions,
                const float* inv_freq, xs_dtype y_dtype, void* y, int64_t tokens, int64_t heads, int64_t dim,
                int64_t rotary, int64_t sections, const int32_t* pair_axes) {
    if (rotary == 0) rotary = dim;
    if (tokens < 0 || heads <= 0 || dim <= 0 || rotary < 0 || rotary > dim || sections <= 0)
        return fail(XS_HIP_EINVAL, "xs_hip_rope: x [" + i2s(tokens) + ", " + i2s(heads) + ", " + i2s(dim) + "], rotary " +
                                       i2s(rotary) + ", sections " + i2s(sections));
    if (pair_axes == nullptr && (rotary % (2 * sections) != 0))
        return fail(XS_HIP_EINVAL, "xs_hip_rope: rotary dims " + i2s(rotary) + " do not split into " + i2s(sections) +
                                       " sections of pairs");
    if (pair_axes != nullptr && rotary % 2 != 0)
        return fail(XS_HIP_EINVAL, "xs_hip_rope: rotary dims " + i2s(rotary) + " are odd");
    if (tokens == 0) return XS_HIP_OK;
    if (x == nullptr || positions == nullptr || inv_freq == nullptr || y == nullptr)
        return fail(XS_HIP_EINVAL, "xs_hip_rope: null buffer");
    if (rotary / 2 > kMaxTableEntries)
        return fail(XS_HIP_EUNSUPPORTED, "xs_hip_rope: " + i2s(rotary / 2) + " pairs per head exceed " + i2s(kMaxTableEntries));
    if (tokens > 0x7fffffffLL || heads * (rotary / 2) > (int64_t{1} << 24))
        return fail(XS_HIP_EUNSUPPORTED, "xs_hip_rope: shape too large");
    if (x != y) {
        // y may be x, but may not overlap it otherwise.
        const int esx = float_size(x_dtype), esy = float_size(y_dtype);
        const char* xb = static_cast<const char*>(x);
        const char* yb = static_cast<const char*>(y);
        const int64_t n = tokens * heads * dim;
        if (esx > 0 && esy > 0 && xb < yb + n * esy && yb < xb + n * esx)
            return fail(XS_HIP_EINVAL, "xs_hip_rope: y overlaps x without being x");
    }
    const RopeArgs a{x, positions, inv_freq, y, pair_axes, tokens, heads, dim, rotary, sections, 1};
    const hipStream_t s = as_stream(stream);
    switch (x_dtype) {
        case XS_F32: return rope_y<F32>(s, a, pos_dtype, y_dtype);
        case XS_F16: return rope_y<F16>(s, a, pos_dtype, y_dtype);
        case XS_BF16: return rope_y<BF16>(s, a, pos_dtype, y_dtype);
        default: return fail(XS_HIP_EINVAL, std::string("xs_hip_rope: x must be f32, f16 or bf16, got ") + dtype_name(x_dtype));
    }
}

}  // extern "C"
