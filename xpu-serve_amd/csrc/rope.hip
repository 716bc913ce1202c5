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
// Layout: a block of 256 threads takes a tile of TT tokens (about four units of work per thread). It first fills an LDS
// table of (cos, sin) in f64 for the tile's TT x pairs entries -- one sincos per (token, pair), shared by every head of
// the token; one f64 pair of padding every 8 entries spreads the 8 entries a wave reads at once over distinct LDS
// banks. Then thread t walks the tile's units t, t + 256, ... -- a unit is (token, head, VEC consecutive pairs): one
// 128-bit load of x1 and one of x2, the rotation, two stores -- so a wave's units are 64 consecutive ones and its loads
// cover whole half-rows of consecutive heads. The rotation is an f64 FMA of the exactly widened inputs, rounded to f32
// and then to y's dtype, as cpu-ref's f64 expression is. (Measured on MI355X: 256-thread blocks beat 320- and
// 640-thread ones that give each thread one fixed unit, and beat splitting a head row across lanes.)
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
    // An optional second tensor of the same tokens (K beside Q): x2 / y2 [tokens, heads2, dim]; heads2 = 0 for none.
    const void* x2;
    void* y2;
    int64_t heads2;
};

// The element offset of (token t, head h) and the tensor it lies in: heads [0, heads) are x / y, heads
// [heads, heads + heads2) the second tensor.
template <typename SX, typename SY>
__device__ __forceinline__ int64_t head_at(const RopeArgs& a, int64_t t, int h, const SX*& x, SY*& y) {
    if (h < a.heads) {
        x = static_cast<const SX*>(a.x);
        y = static_cast<SY*>(a.y);
        return (t * a.heads + h) * a.dim;
    }
    x = static_cast<const SX*>(a.x2);
    y = static_cast<SY*>(a.y2);
    return (t * a.heads2 + (h - a.heads)) * a.dim;
}

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
        v.x = pack2<T>(f[0], f[1]);
        v.y = pack2<T>(f[2], f[3]);
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

constexpr int kMaxTableEntries = 1024;  // (cos, sin) f64 pairs per block, before padding: 18 KiB of LDS
constexpr int kTableSlots = kMaxTableEntries + kMaxTableEntries / 8;

__device__ __forceinline__ int table_slot(int e) { return e + (e >> 3); }

// y1 = x1 c - x2 s, y2 = x2 c + x1 s in f64, each rounded to f32.
template <int VEC>
__device__ __forceinline__ void rotate(const float* x1, const float* x2, const double2* cs, float* y1, float* y2) {
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        const double d1 = x1[k], d2 = x2[k];
        y1[k] = static_cast<float>(fma(d1, cs[k].x, -(d2 * cs[k].y)));
        y2[k] = static_cast<float>(fma(d2, cs[k].x, d1 * cs[k].y));
    }
}

template <typename TX, typename TY, typename I, int VEC>
__global__ __launch_bounds__(kBlock) void rope_kernel(RopeArgs a, FastDiv32 pv_div) {
    using SX = typename TX::storage;
    using SY = typename TY::storage;
    __shared__ double2 table[kTableSlots];

    const int64_t pairs = a.rotary / 2;
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * a.tile_tokens;
    const int tt_n = static_cast<int>(a.tokens - t0 < a.tile_tokens ? a.tokens - t0 : a.tile_tokens);
    const bool axes = a.pair_axes != nullptr;
    const int64_t width = axes ? a.rotary : a.rotary / a.sections;  // section width
    const int64_t half = width / 2;
    const int heads = static_cast<int>(a.heads + a.heads2);
    const int pv_per_head = static_cast<int>(pairs / VEC);
    const int upt = heads * pv_per_head;  // rotation units per token

    // The thread's first unit is loaded before the table is built, so its HBM latency overlaps the sincos work.
    int tt = threadIdx.x / upt;
    int slot = threadIdx.x - tt * upt;
    float x1[VEC], x2[VEC];
    const SX* x = nullptr;
    SY* y = nullptr;
    int64_t base = 0;
    int p0 = 0;
    auto locate = [&]() {
        const int h = static_cast<int>(pv_div.div(static_cast<uint32_t>(slot)));
        p0 = (slot - h * pv_per_head) * VEC;
        int64_t c1 = p0;
        if (!axes) {
            const int64_t sec = p0 / half;
            c1 = sec * width + (p0 - sec * half);
        }
        base = head_at(a, t0 + tt, h, x, y) + c1;
    };
    if (tt < tt_n) {
        locate();
        load_n<TX, VEC>(x + base, x1);
        load_n<TX, VEC>(x + base + half, x2);
    }

    // (cos, sin) of every (token, pair) of the tile.
    const int entries = tt_n * static_cast<int>(pairs);
    for (int e = threadIdx.x; e < entries; e += kBlock) {
        const int te = e / static_cast<int>(pairs);
        const int64_t p = e - static_cast<int64_t>(te) * pairs;
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
        const double pos = static_cast<double>(pos_at<I>(a.pos, (t0 + te) * a.sections + sec));
        const double angle = pos * static_cast<double>(a.inv_freq[i]);
        double sn, cs;
        sincos(angle, &sn, &cs);
        table[table_slot(e)] = make_double2(cs, sn);
    }
    __syncthreads();

    // Thread t takes units t, t + kBlock, ... of the tile; (token, slot) of the next unit follows from the last by
    // adding kBlock to the slot and carrying whole tokens, so no unit needs a division.
    const int carry_t = kBlock / upt, carry_s = kBlock - carry_t * upt;
    bool first = true;
    for (; tt < tt_n;) {
        if (!first) {
            locate();
            load_n<TX, VEC>(x + base, x1);
            load_n<TX, VEC>(x + base + half, x2);
        }
        first = false;
        float y1[VEC], y2[VEC];
        double2 cs[VEC];
#pragma unroll
        for (int k = 0; k < VEC; ++k) cs[k] = table[table_slot(tt * static_cast<int>(pairs) + p0 + k)];
        rotate<VEC>(x1, x2, cs, y1, y2);
        store_n<TY, VEC>(y + base, y1);
        store_n<TY, VEC>(y + base + half, y2);
        tt += carry_t;
        slot += carry_s;
        if (slot >= upt) {
            slot -= upt;
            ++tt;
        }
    }

    // Channels past the rotary dims pass through (unless y is x).
    if (a.rotary < a.dim) {
        const int64_t rest = a.dim - a.rotary;
        const int64_t units = static_cast<int64_t>(tt_n) * heads * rest;
        for (int64_t u = threadIdx.x; u < units; u += kBlock) {
            const int64_t th = u / rest;
            const int64_t tu = th / heads;
            const int hu = static_cast<int>(th - tu * heads);
            const SX* xp;
            SY* yp;
            const int64_t at = head_at(a, t0 + tu, hu, xp, yp) + a.rotary + (u - th * rest);
            if (static_cast<const void*>(xp) != static_cast<const void*>(yp)) yp[at] = TY::store(TX::load(xp[at]));
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
                     (a.heads2 == 0 || (aligned16(a.x2) && aligned16(a.y2)));
    const int64_t pv = pairs / (vec ? VEC : 1);
    const int64_t upt = (a.heads + a.heads2) * pv;  // rotation units per token
    // Tile: about four units per thread (measured best on MI355X against two and eight), within the LDS table.
    int64_t tt = (4 * kBlock + upt - 1) / upt;
    const int64_t max_tt = pairs > 0 ? kMaxTableEntries / pairs : 64;
    if (tt > max_tt) tt = max_tt;
    if (tt < 1) tt = 1;
    a.tile_tokens = static_cast<int>(tt);
    const unsigned grid = static_cast<unsigned>((a.tokens + tt - 1) / tt);
    const FastDiv32 pv_div(static_cast<uint32_t>(pv));
    if (vec) rope_kernel<TX, TY, I, VEC><<<grid, kBlock, 0, s>>>(a, pv_div);
    else rope_kernel<TX, TY, I, 1><<<grid, kBlock, 0, s>>>(a, pv_div);
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

namespace xs_hip {
namespace {

int check_overlap(const void* x, const void* y, int64_t n, xs_dtype xt, xs_dtype yt, const char* what) {
    if (x == y) return XS_HIP_OK;
    const int esx = float_size(xt), esy = float_size(yt);
    const char* xb = static_cast<const char*>(x);
    const char* yb = static_cast<const char*>(y);
    if (esx > 0 && esy > 0 && xb < yb + n * esy && yb < xb + n * esx)
        return fail(XS_HIP_EINVAL, std::string(what) + ": y overlaps x without being x");
    return XS_HIP_OK;
}

int rope_common(void* stream, xs_dtype x_dtype, const void* x, xs_dtype pos_dtype, const void* positions,
                const float* inv_freq, xs_dtype y_dtype, void* y, int64_t tokens, int64_t heads, int64_t dim,
                int64_t rotary, int64_t sections, const int32_t* pair_axes, const void* x2, void* y2, int64_t heads2,
                const char* what) {
    if (rotary == 0) rotary = dim;
    if (tokens < 0 || heads <= 0 || heads2 < 0 || dim <= 0 || rotary < 0 || rotary > dim || sections <= 0)
        return fail(XS_HIP_EINVAL, std::string(what) + ": x [" + i2s(tokens) + ", " + i2s(heads) + ", " + i2s(dim) +
                                       "], rotary " + i2s(rotary) + ", sections " + i2s(sections));
    if (pair_axes == nullptr && (rotary % (2 * sections) != 0))
        return fail(XS_HIP_EINVAL, std::string(what) + ": rotary dims " + i2s(rotary) + " do not split into " +
                                       i2s(sections) + " sections of pairs");
    if (pair_axes != nullptr && rotary % 2 != 0)
        return fail(XS_HIP_EINVAL, std::string(what) + ": rotary dims " + i2s(rotary) + " are odd");
    if (tokens == 0) return XS_HIP_OK;
    if (x == nullptr || positions == nullptr || inv_freq == nullptr || y == nullptr ||
        (heads2 > 0 && (x2 == nullptr || y2 == nullptr)))
        return fail(XS_HIP_EINVAL, std::string(what) + ": null buffer");
    if (rotary / 2 > kMaxTableEntries)
        return fail(XS_HIP_EUNSUPPORTED, std::string(what) + ": " + i2s(rotary / 2) + " pairs per head exceed " +
                                             i2s(kMaxTableEntries));
    if (tokens > 0x7fffffffLL || (heads + heads2) * (rotary / 2) > (int64_t{1} << 24))
        return fail(XS_HIP_EUNSUPPORTED, std::string(what) + ": shape too large");
    int rc = check_overlap(x, y, tokens * heads * dim, x_dtype, y_dtype, what);
    if (rc == XS_HIP_OK && heads2 > 0) rc = check_overlap(x2, y2, tokens * heads2 * dim, x_dtype, y_dtype, what);
    if (rc != XS_HIP_OK) return rc;
    const RopeArgs a{x, positions, inv_freq, y, pair_axes, tokens, heads, dim, rotary, sections, 1, x2, y2, heads2};
    const hipStream_t s = as_stream(stream);
    switch (x_dtype) {
        case XS_F32: return rope_y<F32>(s, a, pos_dtype, y_dtype);
        case XS_F16: return rope_y<F16>(s, a, pos_dtype, y_dtype);
        case XS_BF16: return rope_y<BF16>(s, a, pos_dtype, y_dtype);
        default:
            return fail(XS_HIP_EINVAL, std::string(what) + ": x must be f32, f16 or bf16, got " + dtype_name(x_dtype));
    }
}

}  // namespace
}  // namespace xs_hip

extern "C" {

int xs_hip_rope(void* stream, xs_dtype x_dtype, const void* x, xs_dtype pos_dtype, const void* positions,
                const float* inv_freq, xs_dtype y_dtype, void* y, int64_t tokens, int64_t heads, int64_t dim,
                int64_t rotary, int64_t sections, const int32_t* pair_axes) {
    return rope_common(stream, x_dtype, x, pos_dtype, positions, inv_freq, y_dtype, y, tokens, heads, dim, rotary,
                       sections, pair_axes, nullptr, nullptr, 0, "xs_hip_rope");
}

int xs_hip_rope2(void* stream, xs_dtype x_dtype, const void* xa, void* ya, int64_t heads_a, const void* xb, void* yb,
                 int64_t heads_b, xs_dtype pos_dtype, const void* positions, const float* inv_freq, xs_dtype y_dtype,
                 int64_t tokens, int64_t dim, int64_t rotary, int64_t sections, const int32_t* pair_axes) {
    if (heads_b <= 0) return fail(XS_HIP_EINVAL, "xs_hip_rope2: the second tensor has no heads");
    return rope_common(stream, x_dtype, xa, pos_dtype, positions, inv_freq, y_dtype, ya, tokens, heads_a, dim, rotary,
                       sections, pair_axes, xb, yb, heads_b, "xs_hip_rope2");
}

}  // extern "C"
