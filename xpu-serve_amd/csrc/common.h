// Device and host helpers shared by the gfx950 kernels: dtype widening/narrowing on 128-bit vectors, wave64
// reductions through DPP, launch geometry, and the error state of the C-ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <string>

#include "xs_hip.h"

namespace xs_hip {

// ---------------------------------------------------------------------------------------------------------------
// Error state of the C ABI: a thread-local message per failed call (the text xs::Error carries in the reference).

void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
// Maps a HIP runtime error after a launch or a call to XS_HIP_ERUNTIME with the op's name.
int check_hip(hipError_t e, const char* what);
int check_launch(const char* what);

// Bytes of one element of a float dtype (0 for others).
inline int float_size(xs_dtype t) {
    return t == XS_F32 ? 4 : (t == XS_F16 || t == XS_BF16) ? 2 : 0;
}
inline bool is_float_dtype(xs_dtype t) { return float_size(t) != 0; }
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
const char* dtype_name(xs_dtype t);

// CUs of the current device (256 on MI355X), cached per device.
int device_cus();

// ---------------------------------------------------------------------------------------------------------------
// Scalar conversions, all in hardware: v_cvt_f32_f16 widens exactly; v_cvt_pk_f16_f32 and v_cvt_pk_bf16_f32 (gfx950)
// narrow two values at a time with round-to-nearest-even, overflow to inf and NaN kept a quiet NaN -- the rounding of
// the reference's util/half.h:19-25 and half.cpp:36-56. bf16 widening is a shift.

__device__ __forceinline__ float bf16_to_f32(uint16_t v) { return __uint_as_float(static_cast<uint32_t>(v) << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    const __bf16 h = static_cast<__bf16>(f);
    uint16_t v;
    __builtin_memcpy(&v, &h, 2);
    return v;
}

__device__ __forceinline__ float f16_to_f32(uint16_t v) {
    _Float16 h;
    __builtin_memcpy(&h, &v, 2);
    return static_cast<float>(h);
}

__device__ __forceinline__ uint16_t f32_to_f16(float f) {
    const _Float16 h = static_cast<_Float16>(f);
    uint16_t v;
    __builtin_memcpy(&v, &h, 2);
    return v;
}

// Element type tags used as template parameters: storage type and the widen/narrow pair.
struct F32 {
    using storage = float;
    static constexpr xs_dtype dtype = XS_F32;
    __device__ static float load(float v) { return v; }
    __device__ static float store(float v) { return v; }
};
struct F16 {
    using storage = uint16_t;
    static constexpr xs_dtype dtype = XS_F16;
    __device__ static float load(uint16_t v) { return f16_to_f32(v); }
    __device__ static uint16_t store(float v) { return f32_to_f16(v); }
};
struct BF16 {
    using storage = uint16_t;
    static constexpr xs_dtype dtype = XS_BF16;
    __device__ static float load(uint16_t v) { return bf16_to_f32(v); }
    __device__ static uint16_t store(float v) { return f32_to_bf16(v); }
};

// Elements of T in one 128-bit vector.
template <typename T>
constexpr int vec_elems() {
    return 16 / static_cast<int>(sizeof(typename T::storage));
}

using u32x4 = uint32_t __attribute__((ext_vector_type(4)));

// 128-bit global loads and stores (global_load_dwordx4 / global_store_dwordx4). `nt` marks streaming data that is
// not re-read, so it does not displace other lines in the caches.
__device__ __forceinline__ u32x4 ld128(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ u32x4 ld128_nt(const void* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void st128(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
__device__ __forceinline__ void st128_nt(void* p, u32x4 v) {
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

template <typename T>
__device__ __forceinline__ void unpack(u32x4 raw, float* out) {
    if constexpr (sizeof(typename T::storage) == 4) {
        for (int i = 0; i < 4; ++i) out[i] = __uint_as_float(raw[i]);
    } else {
        for (int i = 0; i < 4; ++i) {
            out[2 * i] = T::load(static_cast<uint16_t>(raw[i] & 0xffffu));
            out[2 * i + 1] = T::load(static_cast<uint16_t>(raw[i] >> 16));
        }
    }
}

// Two values narrowed to T in one 32-bit word (one v_cvt_pk_{f16,bf16}_f32), the first in the low half.
template <typename T>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    if constexpr (T::dtype == XS_F16) {
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        const h2 v = {static_cast<_Float16>(a), static_cast<_Float16>(b)};
        return __builtin_bit_cast(uint32_t, v);
    } else {
        typedef __bf16 b2 __attribute__((ext_vector_type(2)));
        const b2 v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
        return __builtin_bit_cast(uint32_t, v);
    }
}

template <typename T>
__device__ __forceinline__ u32x4 pack(const float* in) {
    u32x4 raw;
    if constexpr (sizeof(typename T::storage) == 4) {
        for (int i = 0; i < 4; ++i) raw[i] = __float_as_uint(in[i]);
    } else {
        for (int i = 0; i < 4; ++i) raw[i] = pack2<T>(in[2 * i], in[2 * i + 1]);
    }
    return raw;
}

// Scalar element access (tails and general-stride paths).
template <typename T>
__device__ __forceinline__ float load_elem(const void* base, int64_t i) {
    return T::load(static_cast<const typename T::storage*>(base)[i]);
}
template <typename T>
__device__ __forceinline__ void store_elem(void* base, int64_t i, float v) {
    static_cast<typename T::storage*>(base)[i] = T::store(v);
}

// ---------------------------------------------------------------------------------------------------------------
// Wave64 reductions. Lanes of a DPP "row" are 16 consecutive lanes; quad_perm, row_half_mirror and row_mirror pair
// every lane with a partner in its 2-, 4-, 8- and 16-lane group, so after those four steps each lane of a 16-lane
// group holds the group's result. Across 16-lane groups the 32- and 64-lane steps use ds_swizzle/bpermute shuffles.

namespace dpp {
constexpr int kQuadXor1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;       // quad_perm [2,3,0,1]
constexpr int kRowHalfMirror = 0x141;  // lane i <-> 7 - i within each 8
constexpr int kRowMirror = 0x140;      // lane i <-> 15 - i within each 16
}  // namespace dpp

template <int Ctrl>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), Ctrl, 0xF, 0xF, false));
}
template <int Ctrl>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(v, v, Ctrl, 0xF, 0xF, false);
}

struct OpMax {
    __device__ static float apply(float a, float b) { return fmaxf(a, b); }
};
struct OpSum {
    __device__ static float apply(float a, float b) { return a + b; }
};

// Reduces over aligned groups of W lanes (W in 2..64, a power of two); every lane of a group gets the result.
// Note: the order of the additions is the same in every lane of the group, so all lanes hold identical bits.
template <int W, typename Op>
__device__ __forceinline__ float group_reduce(float v) {
    static_assert(W >= 1 && W <= 64 && (W & (W - 1)) == 0, "group width");
    if constexpr (W >= 2) v = Op::apply(v, dpp_f<dpp::kQuadXor1>(v));
    if constexpr (W >= 4) v = Op::apply(v, dpp_f<dpp::kQuadXor2>(v));
    if constexpr (W >= 8) v = Op::apply(v, dpp_f<dpp::kRowHalfMirror>(v));
    if constexpr (W >= 16) v = Op::apply(v, dpp_f<dpp::kRowMirror>(v));
    if constexpr (W >= 32) v = Op::apply(v, __shfl_xor(v, 16, 64));
    if constexpr (W >= 64) v = Op::apply(v, __shfl_xor(v, 32, 64));
    return v;
}

template <int Ctrl>
__device__ __forceinline__ double dpp_d(double v) {
    const uint64_t u = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_update_dpp(static_cast<int>(u), static_cast<int>(u), Ctrl, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(static_cast<int>(u >> 32), static_cast<int>(u >> 32), Ctrl, 0xF, 0xF,
                                               false);
    return __longlong_as_double(static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) |
                                                     static_cast<uint32_t>(lo)));
}

// f64 sum over aligned groups of W lanes: the DPP steps of group_reduce on the two halves of each value, then
// shuffles across 16-lane rows. Every lane of a group ends with identical bits.
template <int W>
__device__ __forceinline__ double group_sum_f64(double v) {
    static_assert(W >= 1 && W <= 64 && (W & (W - 1)) == 0, "group width");
    if constexpr (W >= 2) v += dpp_d<dpp::kQuadXor1>(v);
    if constexpr (W >= 4) v += dpp_d<dpp::kQuadXor2>(v);
    if constexpr (W >= 8) v += dpp_d<dpp::kRowHalfMirror>(v);
    if constexpr (W >= 16) v += dpp_d<dpp::kRowMirror>(v);
    if constexpr (W >= 32) v += __shfl_xor(v, 16, 64);
    if constexpr (W >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

// Reductions over the whole wave64 with DPP alone (no LDS-routed shuffle): the four steps within 16-lane rows, then
// row_bcast:15 (row r takes lane 16 r - 1, rows 1 and 3) and row_bcast:31 (rows 2 and 3 take lane 31), after which
// lane 63 holds the wave's result; v_readlane makes it wave-uniform. Lanes a masked DPP step does not write keep the
// operation's identity, so the combination order is fixed and every wave produces the same bits for the same inputs.
namespace dpp {
constexpr int kRowBcast15 = 0x142;
constexpr int kRowBcast31 = 0x143;
}  // namespace dpp

template <int Ctrl, int RowMask>
__device__ __forceinline__ int dpp_masked_i(int v, int identity) {
    return __builtin_amdgcn_update_dpp(identity, v, Ctrl, RowMask, 0xF, false);
}

template <typename Op>
__device__ __forceinline__ float wave_reduce(float v, float identity) {
    v = Op::apply(v, dpp_f<dpp::kQuadXor1>(v));
    v = Op::apply(v, dpp_f<dpp::kQuadXor2>(v));
    v = Op::apply(v, dpp_f<dpp::kRowHalfMirror>(v));
    v = Op::apply(v, dpp_f<dpp::kRowMirror>(v));
    const int id = __float_as_int(identity);
    v = Op::apply(v, __int_as_float(dpp_masked_i<dpp::kRowBcast15, 0xA>(__float_as_int(v), id)));
    v = Op::apply(v, __int_as_float(dpp_masked_i<dpp::kRowBcast31, 0xC>(__float_as_int(v), id)));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

template <int Ctrl, int RowMask>
__device__ __forceinline__ double dpp_masked_d(double v) {  // identity 0.0
    const uint64_t u = __double_as_longlong(v);
    const uint32_t lo = static_cast<uint32_t>(dpp_masked_i<Ctrl, RowMask>(static_cast<int>(u), 0));
    const uint32_t hi = static_cast<uint32_t>(dpp_masked_i<Ctrl, RowMask>(static_cast<int>(u >> 32), 0));
    return __longlong_as_double(static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo));
}

// f64 sum over the wave, as wave_reduce.
__device__ __forceinline__ double wave_sum_f64(double v) {
    v += dpp_d<dpp::kQuadXor1>(v);
    v += dpp_d<dpp::kQuadXor2>(v);
    v += dpp_d<dpp::kRowHalfMirror>(v);
    v += dpp_d<dpp::kRowMirror>(v);
    v += dpp_masked_d<dpp::kRowBcast15, 0xA>(v);
    v += dpp_masked_d<dpp::kRowBcast31, 0xC>(v);
    const uint64_t u = __double_as_longlong(v);
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(u), 63));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(u >> 32), 63));
    return __longlong_as_double(static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo));
}

// A workgroup barrier that orders LDS only. __syncthreads() also waits for every global access the workgroup has in
// flight (its release fence covers global memory), which here would put the latency of an atomic still on its way to
// memory in front of work that does not need it.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ---------------------------------------------------------------------------------------------------------------
// Index arithmetic.

// Granlund-Montgomery division by a run-time constant: floor(n / d) = (umulhi(n, m) + n) >> s for every n < 2^32,
// with s = ceil(log2 d) and m = floor(2^32 (2^s - d) / d) + 1.
struct FastDiv32 {
    uint32_t m = 1, s = 0;
    FastDiv32() = default;
    explicit FastDiv32(uint32_t d) {
        s = 0;
        while ((uint64_t{1} << s) < d) ++s;
        m = static_cast<uint32_t>(((uint64_t{1} << 32) * ((uint64_t{1} << s) - d)) / d + 1);
    }
    __device__ __forceinline__ uint32_t div(uint32_t n) const {
        return static_cast<uint32_t>((static_cast<uint64_t>(__umulhi(n, m)) + n) >> s);
    }
};

// ---------------------------------------------------------------------------------------------------------------
// Launch geometry.

constexpr int kBlock = 256;  // four waves

// Grid size for a grid-stride loop over `items` items of `per_block` each: enough workgroups to fill every CU with
// `waves_per_cu` waves' worth of blocks, never more than the work needs.
inline unsigned grid_for(int64_t items, int per_block, int blocks_per_cu = 8) {
    const int64_t need = (items + per_block - 1) / per_block;
    const int64_t cap = static_cast<int64_t>(device_cus()) * blocks_per_cu;
    const int64_t g = need < cap ? need : cap;
    return static_cast<unsigned>(g < 1 ? 1 : g);
}

inline hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

}  // namespace xs_hip
