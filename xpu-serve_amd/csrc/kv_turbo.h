// The TurboQuant KV formats (turbo4, turbo3, turbo2): the launchers of kv_turbo.hip for the C-ABI entry points of
// kv_quant.hip, and the device pieces every kernel that reads or writes these formats shares -- the rotation of a
// group of 128 values over 16 lanes of 8 values each, the codebooks, and a lane's codes of a group.
#pragma once

#include "common.h"

namespace xs_hip {

// Rows [rows, width] (width a multiple of 128) as codes [rows * width / 128, 16 * bits] bytes and f16 norms
// [rows * width / 128]; bits 4, 3 or 2.
// With row0 set, the rows go to row row0[0] * rows_per_unit + r of a cache of capacity_rows rows (read from device
// memory when the kernel runs); a destination outside the cache writes nothing.
int turbo_quantize(hipStream_t s, int bits, xs_dtype x_dtype, const void* x, void* codes, void* norms, int64_t rows,
                   int64_t width, const int64_t* row0 = nullptr, int64_t rows_per_unit = 0,
                   int64_t capacity_rows = 0);
// The rotated values such codes and norms store, in out_dtype.
int turbo_dequantize(hipStream_t s, int bits, const void* codes, const void* norms, xs_dtype out_dtype, void* out,
                     int64_t rows, int64_t width);

namespace turbo {

constexpr int kGroup = 128;
constexpr int kLanes = 16;       // lanes a group
constexpr int kLaneValues = 8;   // values a lane

// The rotation's sign flips before and after the transform: bit i % 64 of word i / 64 flips value i
// (kv_turbo.h:27-28; format constants).
constexpr uint64_t kSignsBefore[2] = {0x42f85949e46a0359ull, 0x49f250a9a4c63bbbull};
constexpr uint64_t kSignsAfter[2] = {0x3f628fdc16acee90ull, 0xbea56562b7a5357aull};

// The codebooks: Lloyd-Max magnitudes for a Gaussian of variance 1 / 128 and the borders between neighbours
// (kv_turbo.h:39-56; format constants).
template <int Bits>
struct Book;
template <>
struct Book<2> {
    static constexpr float mags[2] = {0.039994f, 0.133462f};
    static constexpr float edges[1] = {0.086728f};
};
template <>
struct Book<3> {
    static constexpr float mags[4] = {0.021663f, 0.066822f, 0.118786f, 0.190207f};
    static constexpr float edges[3] = {0.044243f, 0.092804f, 0.154496f};
};
template <>
struct Book<4> {
    static constexpr float mags[8] = {0.011349f, 0.034299f, 0.058050f, 0.083292f,
                                      0.111036f, 0.143016f, 0.182877f, 0.241529f};
    static constexpr float edges[7] = {0.022824f, 0.046174f, 0.070671f, 0.097164f, 0.127026f, 0.162947f, 0.212203f};
};

template <int Bits>
constexpr int kMagnitudes = 1 << (Bits - 1);

// fl32(e_j^2 * 128), squared in f64 (kv_turbo.h:57-62).
template <int Bits>
constexpr float edge_sq(int j) {
    const double e = Book<Bits>::edges[j];
    return static_cast<float>(e * e * kGroup);
}

// Sign masks (bit 31) of lane `lane`'s 8 values.
__device__ __forceinline__ void sign_masks(const uint64_t* signs, int lane, uint32_t* mask) {
    const uint32_t bits = static_cast<uint32_t>((lane < 8 ? signs[0] : signs[1]) >> (8 * (lane % 8))) & 0xffu;
#pragma unroll
    for (int e = 0; e < kLaneValues; ++e) mask[e] = ((bits >> e) & 1u) << 31;
}

__device__ __forceinline__ float flip(float v, uint32_t mask) { return __uint_as_float(__float_as_uint(v) ^ mask); }

// The value of lane l ^ M of this lane's 16 (M = 1, 2, 4, 8).
template <int M>
__device__ __forceinline__ float xlane(float v) {
    // The quad permutations as plain DPP moves (no old value to keep), which the compiler folds into their user.
    if constexpr (M == 1) return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), dpp::kQuadXor1, 0xF, 0xF, true));
    else if constexpr (M == 2) return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), dpp::kQuadXor2, 0xF, 0xF, true));
    else return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1f | (M << 10)));  // bit mode, xor M
}

// The 16 lanes' values added pairwise, 1, 2, 4, 8 lanes apart: every lane ends with the same sum.
__device__ __forceinline__ float sum_lanes(float s) {
    s = s + xlane<1>(s);
    s = s + xlane<2>(s);
    s = s + xlane<4>(s);
    return s + xlane<8>(s);
}

// Span 8 M of the butterflies: the lower lane of a pair takes a + b, the upper a - b (a the lower's value, b the
// upper's). Each lane computes own + t * partner with t = +1 (lower) or -1 (upper) in one fused multiply-add, exact
// since t * partner is: the upper lane so holds b - a = -(a - b), its value negated (round to nearest even commutes
// with negation). A lane's values thus come out of the four spans negated when an odd number of its lane bits is set;
// the caller folds that sign into the flips after the transform.
template <int M>
__device__ __forceinline__ void cross_span(float* v, float t) {
#pragma unroll
    for (int e = 0; e < kLaneValues; ++e) v[e] = fmaf(xlane<M>(v[e]), t, v[e]);
}

// The unnormalized Walsh-Hadamard transform of a group, on this lane's 8 values; returns the sign mask (bit 31) the
// cross-lane spans left on them.
__device__ __forceinline__ uint32_t butterflies(float* v, int lane) {
#pragma unroll
    for (int h = 1; h < kLaneValues; h *= 2) {
#pragma unroll
        for (int e = 0; e < kLaneValues; ++e) {
            if (e & h) continue;
            const float a = v[e], b = v[e + h];
            v[e] = a + b;
            v[e + h] = a - b;
        }
    }
    cross_span<1>(v, (lane & 1) ? -1.0f : 1.0f);
    cross_span<2>(v, (lane & 2) ? -1.0f : 1.0f);
    cross_span<4>(v, (lane & 4) ? -1.0f : 1.0f);
    cross_span<8>(v, (lane & 8) ? -1.0f : 1.0f);
    return static_cast<uint32_t>(__builtin_popcount(lane & 15) & 1) << 31;
}

// 1 / sqrt(128), the rotation's normalization.
constexpr float kInvSqrtGroup = 0.08838834764831845f;

// Span 8 M of the butterflies with IEEE results, signed zeros included: the lower lane of a pair takes a + b, the upper
// a - b, each as fma(own, t, partner) with t = +1 or -1 (fma(b, -1, a) is a + (-b), exactly a - b).
template <int M>
__device__ __forceinline__ void cross_span_exact(float* v, float t) {
#pragma unroll
    for (int e = 0; e < kLaneValues; ++e) v[e] = fmaf(v[e], t, xlane<M>(v[e]));
}

// This lane's 8 values of a group rotated in place (signs before, butterflies, 1 / sqrt(128), signs after), or rotated
// back (`inverse`: the two sign sets swapped): quant::turbo::rotate_group (reference src/quant/kv_turbo.cpp:118-129),
// bit for bit. All 16 lanes of the group take part.
__device__ __forceinline__ void rotate8(float* v, int lane, bool inverse) {
    uint32_t mask[kLaneValues];
    sign_masks(inverse ? kSignsAfter : kSignsBefore, lane, mask);
#pragma unroll
    for (int e = 0; e < kLaneValues; ++e) v[e] = flip(v[e], mask[e]);
#pragma unroll
    for (int h = 1; h < kLaneValues; h *= 2) {
#pragma unroll
        for (int e = 0; e < kLaneValues; ++e) {
            if (e & h) continue;
            const float a = v[e], b = v[e + h];
            v[e] = a + b;
            v[e + h] = a - b;
        }
    }
    cross_span_exact<1>(v, (lane & 1) ? -1.0f : 1.0f);
    cross_span_exact<2>(v, (lane & 2) ? -1.0f : 1.0f);
    cross_span_exact<4>(v, (lane & 4) ? -1.0f : 1.0f);
    cross_span_exact<8>(v, (lane & 8) ? -1.0f : 1.0f);
    sign_masks(inverse ? kSignsBefore : kSignsAfter, lane, mask);
#pragma unroll
    for (int e = 0; e < kLaneValues; ++e) v[e] = flip(v[e] * kInvSqrtGroup, mask[e]);
}

// Centroid c of the codebook (c < 2^Bits): the magnitudes mirrored, -mags[NM - 1] .. -mags[0], mags[0] .. mags[NM - 1].
template <int Bits>
__device__ __forceinline__ float centroid(int c) {
    constexpr int NM = kMagnitudes<Bits>;
    return c >= NM ? Book<Bits>::mags[c - NM] : -Book<Bits>::mags[NM - 1 - c];
}

// Bytes of a group's codes.
constexpr int group_bytes(int bits) { return kGroup * bits / 8; }

// Lane `lane`'s 8 codes of the group at `gc` (kv_turbo.h:84-87 of the reference): turbo4 a 32-bit word of nibbles;
// turbo2 a 16-bit word of 2-bit codes; turbo3 that word for the low two bits and byte 32 + lane for the third bits.
template <int Bits>
struct LaneCodes {
    uint32_t low = 0, high = 0;
    __device__ __forceinline__ void load(const uint8_t* gc, int lane) {
        if constexpr (Bits == 4) {
            low = reinterpret_cast<const uint32_t*>(gc)[lane];
        } else {
            low = reinterpret_cast<const uint16_t*>(gc)[lane];
            if constexpr (Bits == 3) high = gc[kGroup / 4 + lane];
        }
    }
    __device__ __forceinline__ uint32_t code(int e) const {
        if constexpr (Bits == 4) return (low >> (4 * e)) & 15u;
        else if constexpr (Bits == 3) return ((low >> (2 * e)) & 3u) | (((high >> e) & 1u) << 2);
        else return (low >> (2 * e)) & 3u;
    }
};

}  // namespace turbo
}  // namespace xs_hip
