// TurboQuant KV formats (turbo4, turbo3, turbo2) for gfx950: quantize rows into codes and f16 norms, decode them,
// and the rotation a query takes to be read against them.
//
// Semantics: quant::turbo::quantize_group / decode_group / rotate_group (reference src/quant/kv_turbo.h:14-105,
// src/quant/kv_turbo.cpp:47-129), which every backend repeats in the same f32 arithmetic so that all store the same
// bits. A group of 128 values: n = the sum of squares (each 8-value lane's squares fused-multiply-added in order, the
// 16 lane sums added pairwise 1, 2, 4, 8 lanes apart); w = the values sign-flipped (kSignsBefore), through unnormalized
// Walsh-Hadamard butterflies of spans 1 .. 64, sign-flipped again (kSignsAfter); code = the sign of w and the count of
// edges e_j with w^2 >= fl32(e_j^2 * 128) * n (> when w < 0); norm = f16(sqrt(n / r)), r the chosen magnitudes'
// squares summed like n with plain adds (0 when n is 0). Decoding gives centroid(code) * norm, still rotated. Launchers
// replaced: sycl_be::quantize_kv / dequantize_kv for the Turbo formats and sycl_be::kv_rotate (src/backend/sycl/
// sycl_kernels.h:211-221; sycl_kv_cache.cpp:51-85, 96-106, 149-163).
//
// Layout: a group per 16 lanes, 8 consecutive values per lane (one 16-byte load of f16/bf16, two of f32), four groups
// a wave; a 16-lane set quantizes kQuantRounds groups in turn. The butterflies of spans 1, 2, 4 run inside a lane;
// spans 8, 16, 32, 64 pair lane l with l ^ 1, 2, 4, 8 of the same 16 (DPP quad permutations for 1 and 2, ds_swizzle for
// 4 and 8), one fused multiply-add each. The edge test compares the bit patterns of non-negative floats as integers:
// k = bits(w^2) + (w >= 0), and edge j counts when bits(edge_j) < k -- w^2 >= edge for a non-negative w, w^2 > edge
// for a negative one, in one integer compare -- and a binary search over the ascending edges finds the count. The magnitudes' squares and the centroids
// come from LDS tables. Codes of a group: turbo4 a nibble per value (a lane's 8 codes are one 32-bit word), turbo2 two
// bits per value (a lane's are one 16-bit word), turbo3 the turbo2 layout of the low two bits in bytes 0..31 and the
// third bits as one byte per lane at 32 + lane (kv_turbo.h:84-87).
#include "common.h"
#include "kv_turbo.h"

namespace xs_hip {
namespace {

using namespace turbo;

constexpr int kGroupsPerBlock = kBlock / kLanes;

template <typename X>
__device__ __forceinline__ void load_lane(const typename X::storage* x, float* v) {
    if constexpr (sizeof(typename X::storage) == 4) {
        unpack<X>(ld128_nt(x), v);
        unpack<X>(ld128_nt(x + 4), v + 4);
    } else {
        unpack<X>(ld128_nt(x), v);
    }
}

// Groups a 16-lane set quantizes in turn: its sign masks and tables are made once for all of them.
constexpr int kQuantRounds = 4;

// With `row0` set, the groups go to group row0[0] * unit_groups + g of a cache of cap_groups groups (the destination
// read from device memory when the kernel runs); a destination outside the cache writes nothing.
template <int Bits, typename X>
__global__ __launch_bounds__(kBlock) void turbo_quantize_kernel(const typename X::storage* __restrict__ x,
                                                                uint8_t* __restrict__ codes,
                                                                uint16_t* __restrict__ norms, int64_t groups,
                                                                const int64_t* row0 = nullptr, int64_t unit_groups = 0,
                                                                int64_t cap_groups = 0) {
    if (row0 != nullptr) {
        const int64_t off = row0[0] * unit_groups;
        if (off < 0 || off > cap_groups - groups) return;
        codes += off * (kGroup * Bits / 8);
        norms += off;
    }
    constexpr int NM = kMagnitudes<Bits>;
    __shared__ float mag_sq[NM];
    if (threadIdx.x < NM) mag_sq[threadIdx.x] = Book<Bits>::mags[threadIdx.x] * Book<Bits>::mags[threadIdx.x];
    __syncthreads();
    const int lane = threadIdx.x % kLanes;
    uint32_t before[kLaneValues], after[kLaneValues];
    sign_masks(kSignsBefore, lane, before);
    sign_masks(kSignsAfter, lane, after);
    const uint32_t parity = static_cast<uint32_t>(__builtin_popcount(lane & 15) & 1) << 31;
#pragma unroll
    for (int e = 0; e < kLaneValues; ++e) after[e] ^= parity;  // the sign the cross-lane spans leave (butterflies)

#pragma unroll
    for (int round = 0; round < kQuantRounds; ++round) {
        const int64_t g = (static_cast<int64_t>(blockIdx.x) * kQuantRounds + round) * kGroupsPerBlock +
                          threadIdx.x / kLanes;
        if (g >= groups) return;  // whole 16-lane groups leave together, and the later rounds are later groups

        float v[kLaneValues];
        load_lane<X>(x + g * kGroup + lane * kLaneValues, v);
        float n = 0.0f;
#pragma unroll
        for (int e = 0; e < kLaneValues; ++e) n = fmaf(v[e], v[e], n);
        n = sum_lanes(n);
#pragma unroll
        for (int e = 0; e < kLaneValues; ++e) v[e] = flip(v[e], before[e]);
        butterflies(v, lane);

        // The edges as bit patterns; a NaN in the group makes every edge test fail, as in f32: all-ones edges do
        // that.
        uint32_t edge[NM - 1];
#pragma unroll
        for (int j = 0; j < NM - 1; ++j) edge[j] = n == n ? __float_as_uint(edge_sq<Bits>(j) * n) : 0xffffffffu;
        uint32_t packed = 0, high = 0;
        float r = 0.0f;
#pragma unroll
        for (int e = 0; e < kLaneValues; ++e) {
            const float w = flip(v[e], after[e]);
            const bool negative = w < 0.0f;
            const uint32_t k = __float_as_uint(w * w) + (negative ? 0u : 1u);
            // m = the count of edges below k: a binary search over the ascending edges.
            uint32_t m;
            if constexpr (Bits == 4) {
                const bool c1 = edge[3] < k;
                const bool c2 = (c1 ? edge[5] : edge[1]) < k;
                const uint32_t t3 = c1 ? (c2 ? edge[6] : edge[4]) : (c2 ? edge[2] : edge[0]);
                m = (c1 ? 4u : 0u) + (c2 ? 2u : 0u) + (t3 < k ? 1u : 0u);
            } else if constexpr (Bits == 3) {
                const bool c1 = edge[1] < k;
                m = (c1 ? 2u : 0u) + ((c1 ? edge[2] : edge[0]) < k ? 1u : 0u);
            } else {
                m = edge[0] < k ? 1u : 0u;
            }
            const uint32_t code = negative ? NM - 1 - m : NM + m;
            if constexpr (Bits == 4) {
                packed |= code << (4 * e);
            } else {
                packed |= (code & 3u) << (2 * e);
                if constexpr (Bits == 3) high |= (code >> 2) << e;
            }
            r += mag_sq[m];
        }
        r = sum_lanes(r);
        uint8_t* gc = codes + g * (kGroup * Bits / 8);
        if constexpr (Bits == 4) {
            reinterpret_cast<uint32_t*>(gc)[lane] = packed;
        } else {
            reinterpret_cast<uint16_t*>(gc)[lane] = static_cast<uint16_t>(packed);
            if constexpr (Bits == 3) gc[kGroup / 4 + lane] = static_cast<uint8_t>(high);
        }
        if (lane == 0) norms[g] = f32_to_f16(n > 0.0f ? sqrtf(n / r) : 0.0f);
    }
}

// Threads of a decode workgroup, the groups a 16-lane slice of it takes (kDecU, kDecGroupsPerBlock apart), and the
// groups of a workgroup.
constexpr int kDecBlock = 256;
constexpr int kDecU = 2;
constexpr int kDecGroupsPerBlock = kDecBlock / kLanes;

template <int Bits, typename Y>
__global__ __launch_bounds__(kDecBlock) void turbo_decode_kernel(const uint8_t* __restrict__ codes,
                                                              const uint16_t* __restrict__ norms,
                                                              typename Y::storage* __restrict__ out, int64_t groups) {
    constexpr int NC = 1 << Bits;
    __shared__ float centroid_s[NC];
    const int lane = threadIdx.x % kLanes;
    const int64_t g0 = static_cast<int64_t>(blockIdx.x) * kDecGroupsPerBlock * kDecU + threadIdx.x / kLanes;
    // The groups' codes and norms are requested first, so their latency overlaps the codebook's staging.
    uint32_t packed[kDecU], high[kDecU];
    uint16_t norm_bits[kDecU];
#pragma unroll
    for (int u = 0; u < kDecU; ++u) {
        const int64_t g = g0 + u * kDecGroupsPerBlock;
        packed[u] = high[u] = 0;
        norm_bits[u] = 0;
        if (g < groups) {
            const uint8_t* gc = codes + g * (kGroup * Bits / 8);
            if constexpr (Bits == 4) {
                packed[u] = reinterpret_cast<const uint32_t*>(gc)[lane];
            } else {
                packed[u] = reinterpret_cast<const uint16_t*>(gc)[lane];
                if constexpr (Bits == 3) high[u] = gc[kGroup / 4 + lane];
            }
            norm_bits[u] = norms[g];
        }
    }
    if (threadIdx.x < NC) {
        centroid_s[threadIdx.x] = centroid<Bits>(static_cast<int>(threadIdx.x));
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kDecU; ++u) {
        const int64_t g = g0 + u * kDecGroupsPerBlock;
        if (g >= groups) break;  // later u are later groups
        const float norm = f16_to_f32(norm_bits[u]);
        float v[kLaneValues];
#pragma unroll
        for (int e = 0; e < kLaneValues; ++e) {
            uint32_t code;
            if constexpr (Bits == 4) code = (packed[u] >> (4 * e)) & 15u;
            else code = ((packed[u] >> (2 * e)) & 3u) | (Bits == 3 ? ((high[u] >> e) & 1u) << 2 : 0u);
            v[e] = centroid_s[code] * norm;
        }
        typename Y::storage* o = out + g * kGroup + lane * kLaneValues;
        if constexpr (sizeof(typename Y::storage) == 4) {
            st128_nt(o, pack<Y>(v));
            st128_nt(o + 4, pack<Y>(v + 4));
        } else {
            st128_nt(o, pack<Y>(v));
        }
    }
}

// Each group rotated (signs before, butterflies, 1 / sqrt(128), signs after) or rotated back (the two sign sets
// swapped): quant::turbo::rotate_group (kv_turbo.cpp:118-129).
__global__ __launch_bounds__(kBlock) void turbo_rotate_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                              int64_t groups, bool inverse) {
    const int lane = threadIdx.x % kLanes;
    const int64_t g = static_cast<int64_t>(blockIdx.x) * kGroupsPerBlock + threadIdx.x / kLanes;
    if (g >= groups) return;
    float v[kLaneValues];
    const float* xl = x + g * kGroup + lane * kLaneValues;
    unpack<F32>(ld128(xl), v);
    unpack<F32>(ld128(xl + 4), v + 4);
    rotate8(v, lane, inverse);
    float* yl = y + g * kGroup + lane * kLaneValues;
    st128(yl, pack<F32>(v));
    st128(yl + 4, pack<F32>(v + 4));
}

unsigned blocks_for(int64_t groups, int rounds = 1, int per_block = kGroupsPerBlock) {
    return static_cast<unsigned>((groups + per_block * rounds - 1) / (per_block * rounds));
}

template <int Bits>
int quantize_bits(hipStream_t s, xs_dtype x_dtype, const void* x, uint8_t* codes, uint16_t* norms, int64_t groups,
                  const int64_t* row0, int64_t unit_groups, int64_t cap_groups) {
    const unsigned grid = blocks_for(groups, kQuantRounds);
    switch (x_dtype) {
        case XS_F32:
            turbo_quantize_kernel<Bits, F32><<<grid, kBlock, 0, s>>>(static_cast<const float*>(x), codes, norms, groups,
                                                                     row0, unit_groups, cap_groups);
            break;
        case XS_F16:
            turbo_quantize_kernel<Bits, F16><<<grid, kBlock, 0, s>>>(static_cast<const uint16_t*>(x), codes, norms,
                                                                     groups, row0, unit_groups, cap_groups);
            break;
        case XS_BF16:
            turbo_quantize_kernel<Bits, BF16><<<grid, kBlock, 0, s>>>(static_cast<const uint16_t*>(x), codes, norms,
                                                                      groups, row0, unit_groups, cap_groups);
            break;
        default:
            return fail(XS_HIP_EINVAL, std::string("xs_hip_quantize_kv: x must be f32, f16 or bf16, got ") +
                                           dtype_name(x_dtype));
    }
    return check_launch("xs_hip_quantize_kv");
}

template <int Bits>
int decode_bits(hipStream_t s, const uint8_t* codes, const uint16_t* norms, xs_dtype out_dtype, void* out,
                int64_t groups) {
    switch (out_dtype) {
        case XS_F32:
            turbo_decode_kernel<Bits, F32><<<blocks_for(groups, kDecU, kDecGroupsPerBlock), kDecBlock, 0, s>>>(codes, norms, static_cast<float*>(out),
                                                                                 groups);
            break;
        case XS_F16:
            turbo_decode_kernel<Bits, F16><<<blocks_for(groups, kDecU, kDecGroupsPerBlock), kDecBlock, 0, s>>>(codes, norms,
                                                                                 static_cast<uint16_t*>(out), groups);
            break;
        case XS_BF16:
            turbo_decode_kernel<Bits, BF16><<<blocks_for(groups, kDecU, kDecGroupsPerBlock), kDecBlock, 0, s>>>(codes, norms,
                                                                                  static_cast<uint16_t*>(out), groups);
            break;
        default:
            return fail(XS_HIP_EINVAL, std::string("xs_hip_dequantize_kv: out must be f32, f16 or bf16, got ") +
                                           dtype_name(out_dtype));
    }
    return check_launch("xs_hip_dequantize_kv");
}

int check_turbo(const char* op, int64_t rows, int64_t width, const void* a, const void* b, const void* c) {
    if (rows < 0 || width <= 0 || width % kGroup != 0)
        return fail(XS_HIP_EINVAL, std::string(op) + ": a TurboQuant format needs rows of a multiple of 128 values, got " +
                                       std::to_string(rows) + " rows of " + std::to_string(width));
    if (rows > 0 && (a == nullptr || b == nullptr || c == nullptr))
        return fail(XS_HIP_EINVAL, std::string(op) + ": null buffer");
    if (rows * (width / kGroup) > (int64_t{0xffffffff} - kBlock) / kLanes)  // a lane per 8 values, in 32 bits
        return fail(XS_HIP_EUNSUPPORTED, std::string(op) + ": too many groups");
    return XS_HIP_OK;
}

}  // namespace

int turbo_quantize(hipStream_t s, int bits, xs_dtype x_dtype, const void* x, void* codes, void* norms, int64_t rows,
                   int64_t width, const int64_t* row0, int64_t rows_per_unit, int64_t capacity_rows) {
    int rc = check_turbo("xs_hip_quantize_kv", rows, width, x, codes, norms);
    if (rc != XS_HIP_OK || rows == 0) return rc;
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(codes) % 4 != 0 ||
        reinterpret_cast<uintptr_t>(norms) % 2 != 0)
        return fail(XS_HIP_EINVAL, "xs_hip_quantize_kv: TurboQuant needs x 16-byte, codes 4-byte and norms 2-byte "
                                   "aligned");
    if (row0 != nullptr && reinterpret_cast<uintptr_t>(row0) % 8 != 0)
        return fail(XS_HIP_EINVAL, "xs_hip_quantize_kv: row0 must be 8-byte aligned");
    const int64_t gpr = width / kGroup;  // groups a row
    const int64_t groups = rows * gpr;
    auto* c = static_cast<uint8_t*>(codes);
    auto* nm = static_cast<uint16_t*>(norms);
    const int64_t ug = rows_per_unit * gpr, cg = capacity_rows * gpr;
    if (bits == 4) return quantize_bits<4>(s, x_dtype, x, c, nm, groups, row0, ug, cg);
    if (bits == 3) return quantize_bits<3>(s, x_dtype, x, c, nm, groups, row0, ug, cg);
    return quantize_bits<2>(s, x_dtype, x, c, nm, groups, row0, ug, cg);
}

int turbo_dequantize(hipStream_t s, int bits, const void* codes, const void* norms, xs_dtype out_dtype, void* out,
                     int64_t rows, int64_t width) {
    int rc = check_turbo("xs_hip_dequantize_kv", rows, width, codes, norms, out);
    if (rc != XS_HIP_OK || rows == 0) return rc;
    if (reinterpret_cast<uintptr_t>(out) % 16 != 0 || reinterpret_cast<uintptr_t>(codes) % 4 != 0 ||
        reinterpret_cast<uintptr_t>(norms) % 2 != 0)
        return fail(XS_HIP_EINVAL, "xs_hip_dequantize_kv: TurboQuant needs out 16-byte, codes 4-byte and norms "
                                   "2-byte aligned");
    const int64_t groups = rows * (width / kGroup);
    const auto* c = static_cast<const uint8_t*>(codes);
    const auto* nm = static_cast<const uint16_t*>(norms);
    if (bits == 4) return decode_bits<4>(s, c, nm, out_dtype, out, groups);
    if (bits == 3) return decode_bits<3>(s, c, nm, out_dtype, out, groups);
    return decode_bits<2>(s, c, nm, out_dtype, out, groups);
}

}  // namespace xs_hip

using namespace xs_hip;

extern "C" {

int xs_hip_kv_rotate(void* stream, const float* x, float* y, int64_t rows, int64_t width, int inverse) {
    int rc = check_turbo("xs_hip_kv_rotate", rows, width, x, y, x);
    if (rc != XS_HIP_OK || rows == 0) return rc;
    if (!aligned16(x) || !aligned16(y)) return fail(XS_HIP_EINVAL, "xs_hip_kv_rotate: x and y must be 16-byte aligned");
    const int64_t groups = rows * (width / kGroup);
    turbo_rotate_kernel<<<blocks_for(groups), kBlock, 0, as_stream(stream)>>>(x, y, groups, inverse != 0);
    return check_launch("xs_hip_kv_rotate");
}

}  // extern "C"
