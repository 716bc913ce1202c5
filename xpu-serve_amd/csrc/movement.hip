// Data movement on either side of the path for gfx950: Gather (rows of a table by index), Transpose (any permutation
// of up to XS_MAX_RANK axes) and Concat (up to XS_CONCAT_PARTS parts along an axis), the graph ops the SYCL session
// runs through sycl_be::gather / gather_bits, transpose and concat (reference src/backend/sycl/sycl_kernels.h:95-128).
//
// Semantics: cpu_ref::gather, transpose and concat (src/backend/cpu_ref/ops.cpp:157-173, 312-340, 616-637): bytes
// moved as they are, except that Gather widens an f16 or bf16 table's rows to f32 (exactly), as cpu-ref's f32 view of a
// float table gives them (cpu_backend.cpp:370).
//
// Layout: every kernel moves the widest unit (16, 8, 4, 2 or 1 bytes) that divides the row lengths, strides and
// addresses involved, one unit a lane, consecutive lanes on consecutive units of the destination, so stores are whole
// 128-bit vectors wherever the shapes allow. Gather takes 4 elements a lane of each output row; Transpose decomposes
// the destination unit index over the output shape with precomputed divisors (the innermost run contiguous in both
// tensors when the last axis stays put); Concat finds a unit's part among at most 8 by its byte offset in the row.
#include "common.h"

namespace xs_hip {
namespace {

constexpr int kMoveBlock = 256;

// ---- Gather ---------------------------------------------------------------------------------------------------

// out [n, width] = rows ids[r] of table [rows, width]; an id outside [0, rows) gives a row of zeros (cpu-ref refuses
// it by name; on the device a zero row keeps every access inside the table). 4 elements a lane when width % 4 == 0.
// Non-temporal loads and stores: 6.8 against 7.8 us for 2048 rows of a [151936, 2560] bf16 table, on MI355X (in
// 64-thread workgroups 8.0 us). Units from `base` on (a launch covers at most 2^31 units).
template <typename T, typename I, int V>
__global__ __launch_bounds__(kMoveBlock) void gather_kernel(const typename T::storage* __restrict__ table,
                                                            const I* __restrict__ ids, float* __restrict__ out,
                                                            int64_t n, int64_t rows, int64_t width, int64_t base) {
    const int64_t per_row = width / V;
    const int64_t u = base + static_cast<int64_t>(blockIdx.x) * kMoveBlock + threadIdx.x;
    if (u >= n * per_row) return;
    const int64_t r = u / per_row, c = (u - r * per_row) * V;
    const int64_t id = static_cast<int64_t>(ids[r]);
    float v[V];
    if (id >= 0 && id < rows) {
        const typename T::storage* src = table + id * width + c;
        if constexpr (V == 4 && sizeof(typename T::storage) == 4) {
            const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = __uint_as_float(w[e]);
        } else if constexpr (V == 4) {
            const uint64_t w64 = __builtin_nontemporal_load(reinterpret_cast<const uint64_t*>(src));
            const uint2 w = {static_cast<uint32_t>(w64), static_cast<uint32_t>(w64 >> 32)};
            v[0] = T::load(static_cast<uint16_t>(w.x & 0xffffu));
            v[1] = T::load(static_cast<uint16_t>(w.x >> 16));
            v[2] = T::load(static_cast<uint16_t>(w.y & 0xffffu));
            v[3] = T::load(static_cast<uint16_t>(w.y >> 16));
        } else {
#pragma unroll
            for (int e = 0; e < V; ++e) v[e] = T::load(src[e]);
        }
    } else {
#pragma unroll
        for (int e = 0; e < V; ++e) v[e] = 0.0f;
    }
    float* dst = out + r * width + c;
    if constexpr (V == 4) {
        __builtin_nontemporal_store(
            u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])},
            reinterpret_cast<u32x4*>(dst));
    } else {
#pragma unroll
        for (int e = 0; e < V; ++e) dst[e] = v[e];
    }
}

// An i32 table's rows, bits as they are (sycl_be::gather_bits).
struct Bits32 {
    using storage = float;  // the 32-bit words moved as floats: bits unchanged
    __device__ static float load(float v) { return v; }
};

template <typename T, typename I>
void launch_gather(hipStream_t s, const void* table, const void* ids, float* out, int64_t n, int64_t rows,
                   int64_t width, bool vec) {
    const auto* tb = static_cast<const typename T::storage*>(table);
    const auto* id = static_cast<const I*>(ids);
    const int64_t units = n * (vec ? width / 4 : width);
    constexpr int64_t kSlice = int64_t{1} << 31;
    for (int64_t base = 0; base < units; base += kSlice) {
        const int64_t len = units - base < kSlice ? units - base : kSlice;
        const unsigned grid = static_cast<unsigned>((len + kMoveBlock - 1) / kMoveBlock);
        if (vec) gather_kernel<T, I, 4><<<grid, kMoveBlock, 0, s>>>(tb, id, out, n, rows, width, base);
        else gather_kernel<T, I, 1><<<grid, kMoveBlock, 0, s>>>(tb, id, out, n, rows, width, base);
    }
}

template <typename T>
void gather_ids(hipStream_t s, xs_dtype ids_dtype, const void* table, const void* ids, float* out, int64_t n,
                int64_t rows, int64_t width, bool vec) {
    if (ids_dtype == XS_I64) launch_gather<T, int64_t>(s, table, ids, out, n, rows, width, vec);
    else launch_gather<T, int32_t>(s, table, ids, out, n, rows, width, vec);
}

// ---- Transpose --------------------------------------------------------------------------------------------------

// Transpose and concat read and write each unit once: non-temporal loads and stores, one unit a lane in 64-thread
// workgroups. Measured on MI355X (config 3's Q to head-major, config 1's gate|up concat): 23.5 and 27.9 us, against
// 26.1 and 28.3 us in 256-thread workgroups, and 28.5 and 31.1 us with plain loads and stores (a 64 MiB copy: 21.2).
constexpr int kPermBlock = 64;
// Units a launch covers: a grid counts its threads in 32 bits, so larger tensors take several launches at offsets.
constexpr int64_t kPermSlice = int64_t{1} << 31;
template <typename E>
__device__ __forceinline__ E ld_once(const E* p) {
    return __builtin_nontemporal_load(p);
}
template <typename E>
__device__ __forceinline__ void st_once(E* p, E v) {
    __builtin_nontemporal_store(v, p);
}

// out[u] = x[sum_d index_d(u) * stride[d]] over the output shape, in units of E bytes (one element, or, when the
// innermost output axis is x's innermost too, several consecutive elements of it).
struct PermuteArgs {
    int rank;
    int64_t shape[XS_MAX_RANK];   // output shape, the innermost in units
    int64_t stride[XS_MAX_RANK];  // x's unit stride of each output axis
    FastDiv32 div[XS_MAX_RANK];   // shape[d] as 32-bit divisors (the 32-bit kernel)
};

// W32: fewer than 2^32 units -- the index decomposed with 32-bit multiply-high divisions instead of 64-bit ones.
template <typename E, bool W32>
__global__ __launch_bounds__(kPermBlock) void transpose_kernel(const E* __restrict__ x, E* __restrict__ y, int64_t n,
                                                               PermuteArgs p, int64_t base) {
    const int64_t u = base + static_cast<int64_t>(blockIdx.x) * kPermBlock + threadIdx.x;
    if (u >= n) return;
    int64_t off = 0;
    if constexpr (W32) {
        uint32_t rem = static_cast<uint32_t>(u);
        for (int d = p.rank - 1; d >= 0; --d) {
            const uint32_t q = p.div[d].div(rem);
            off += static_cast<int64_t>(rem - q * static_cast<uint32_t>(p.shape[d])) * p.stride[d];
            rem = q;
        }
    } else {
        int64_t rem = u;
        for (int d = p.rank - 1; d >= 0; --d) {
            const int64_t q = rem / p.shape[d];
            off += (rem - q * p.shape[d]) * p.stride[d];
            rem = q;
        }
    }
    st_once(y + u, ld_once(x + off));
}

// ---- Concat -------------------------------------------------------------------------------------------------------

struct ConcatArgs {
    int count;
    const char* src[XS_CONCAT_PARTS];
    int64_t units[XS_CONCAT_PARTS];  // units of a part's row
    int64_t first[XS_CONCAT_PARTS];  // the part's first unit within an output row
    int64_t row;                     // units of an output row
    FastDiv32 row_div;               // row as a 32-bit divisor (the 32-bit kernel)
};

template <typename E, bool W32>
__global__ __launch_bounds__(kPermBlock) void concat_kernel(ConcatArgs a, E* __restrict__ out, int64_t n, int64_t base) {
    const int64_t u = base + static_cast<int64_t>(blockIdx.x) * kPermBlock + threadIdx.x;
    if (u >= n) return;
    const int64_t o = W32 ? static_cast<int64_t>(a.row_div.div(static_cast<uint32_t>(u))) : u / a.row;
    const int64_t c = u - o * a.row;
    int k = 0;
#pragma unroll
    for (int j = 1; j < XS_CONCAT_PARTS; ++j)
        if (j < a.count && c >= a.first[j]) k = j;
    st_once(out + u, ld_once(reinterpret_cast<const E*>(a.src[k]) + o * a.units[k] + (c - a.first[k])));
}

// The widest unit of {16, 8, 4, 2, 1} bytes dividing every value of `bits`.
int64_t unit_of(uint64_t bits) {
    return bits % 16 == 0 ? 16 : bits % 8 == 0 ? 8 : bits % 4 == 0 ? 4 : bits % 2 == 0 ? 2 : 1;
}

template <typename Launch>
int by_unit(int64_t e, Launch&& launch) {
    switch (e) {
        case 16: launch(u32x4{}); break;
        case 8: launch(uint64_t{}); break;
        case 4: launch(uint32_t{}); break;
        case 2: launch(uint16_t{}); break;
        default: launch(uint8_t{}); break;
    }
    return XS_HIP_OK;
}

}  // namespace
}  // namespace xs_hip

using namespace xs_hip;

extern "C" {

int xs_hip_gather(void* stream, xs_dtype table_dtype, const void* table, int64_t rows, int64_t width,
                  xs_dtype ids_dtype, const void* ids, int64_t n, void* out) {
    const char* what = "xs_hip_gather";
    if (rows < 0 || width <= 0 || n < 0)
        return fail(XS_HIP_EINVAL, std::string(what) + ": " + std::to_string(n) + " ids into a table of " +
                                       std::to_string(rows) + " rows of " + std::to_string(width));
    if (table_dtype != XS_F32 && table_dtype != XS_F16 && table_dtype != XS_BF16 && table_dtype != XS_I32)
        return fail(XS_HIP_EUNSUPPORTED, std::string(what) + ": table of " + dtype_name(table_dtype) +
                                             " (supported: f32, f16, bf16, i32)");
    if (ids_dtype != XS_I32 && ids_dtype != XS_I64)
        return fail(XS_HIP_EINVAL, std::string(what) + ": ids of " + dtype_name(ids_dtype) + " (i32 or i64)");
    if (n == 0) return XS_HIP_OK;
    if (table == nullptr || ids == nullptr || out == nullptr || rows == 0)
        return fail(XS_HIP_EINVAL, std::string(what) + ": null buffer or empty table");
    if (n * width > (int64_t{1} << 40)) return fail(XS_HIP_EUNSUPPORTED, std::string(what) + ": too large");
    const int es = table_dtype == XS_F32 || table_dtype == XS_I32 ? 4 : 2;
    const bool vec = width % 4 == 0 && reinterpret_cast<uintptr_t>(table) % (4 * es) == 0 && aligned16(out);
    const hipStream_t s = as_stream(stream);
    auto* o = static_cast<float*>(out);
    switch (table_dtype) {
        case XS_F32: gather_ids<F32>(s, ids_dtype, table, ids, o, n, rows, width, vec); break;
        case XS_F16: gather_ids<F16>(s, ids_dtype, table, ids, o, n, rows, width, vec); break;
        case XS_BF16: gather_ids<BF16>(s, ids_dtype, table, ids, o, n, rows, width, vec); break;
        default: gather_ids<Bits32>(s, ids_dtype, table, ids, o, n, rows, width, vec); break;
    }
    return check_launch(what);
}

int xs_hip_transpose(void* stream, const void* x, void* y, int64_t elem_bytes, int rank, const int64_t* in_shape,
                     const int32_t* perm) {
    const char* what = "xs_hip_transpose";
    if (rank < 1 || rank > XS_MAX_RANK || in_shape == nullptr || perm == nullptr ||
        (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8))
        return fail(XS_HIP_EINVAL, std::string(what) + ": rank " + std::to_string(rank) + ", elements of " +
                                       std::to_string(elem_bytes) + " bytes");
    int64_t in_stride[XS_MAX_RANK], out_shape[XS_MAX_RANK], stride[XS_MAX_RANK];
    bool seen[XS_MAX_RANK] = {};
    int64_t n = 1;
    for (int d = rank - 1; d >= 0; --d) {
        if (in_shape[d] < 0) return fail(XS_HIP_EINVAL, std::string(what) + ": negative dim");
        in_stride[d] = n;
        n *= in_shape[d];
    }
    for (int i = 0; i < rank; ++i) {
        if (perm[i] < 0 || perm[i] >= rank || seen[perm[i]])
            return fail(XS_HIP_EINVAL, std::string(what) + ": perm is not a permutation of " + std::to_string(rank) +
                                           " axes");
        seen[perm[i]] = true;
        out_shape[i] = in_shape[perm[i]];
        stride[i] = in_stride[perm[i]];
    }
    if (n == 0) return XS_HIP_OK;
    if (x == nullptr || y == nullptr) return fail(XS_HIP_EINVAL, std::string(what) + ": null buffer");
    // The innermost output axis moves whole runs when it is x's innermost axis too.
    int64_t e = elem_bytes;
    const int last = rank - 1;
    if (perm[last] == last) {
        e = unit_of(static_cast<uint64_t>(out_shape[last] * elem_bytes) | reinterpret_cast<uintptr_t>(x) |
                    reinterpret_cast<uintptr_t>(y));
        if (e < elem_bytes) e = elem_bytes;
    }
    const int64_t per = e / elem_bytes;  // elements a unit
    // In units: the innermost axis counts units (its stride in x is 1), and every outer axis's stride in x is a
    // multiple of the innermost length, so of a unit.
    PermuteArgs p{};
    p.rank = rank;
    for (int i = 0; i < rank; ++i) {
        p.shape[i] = i == last ? out_shape[i] / per : out_shape[i];
        p.stride[i] = i == last ? stride[i] : stride[i] / per;
    }
    const int64_t units = n / per;
    if (units > (int64_t{1} << 40)) return fail(XS_HIP_EUNSUPPORTED, std::string(what) + ": too large");
    const bool w32 = units < (int64_t{1} << 31);
    if (w32) {
        for (int i = 0; i < rank; ++i) p.div[i] = FastDiv32(static_cast<uint32_t>(p.shape[i]));
    }
    const hipStream_t s = as_stream(stream);
    by_unit(e, [&](auto tag) {
        using E = decltype(tag);
        for (int64_t base = 0; base < units; base += kPermSlice) {
            const int64_t len = units - base < kPermSlice ? units - base : kPermSlice;
            const unsigned grid = static_cast<unsigned>((len + kPermBlock - 1) / kPermBlock);
            if (w32)
                transpose_kernel<E, true><<<grid, kPermBlock, 0, s>>>(static_cast<const E*>(x), static_cast<E*>(y),
                                                                      units, p, base);
            else
                transpose_kernel<E, false><<<grid, kPermBlock, 0, s>>>(static_cast<const E*>(x), static_cast<E*>(y),
                                                                       units, p, base);
        }
    });
    return check_launch(what);
}

int xs_hip_concat(void* stream, int count, const void* const* parts, const int64_t* part_row_bytes, void* out,
                  int64_t outer) {
    const char* what = "xs_hip_concat";
    if (count < 1 || count > XS_CONCAT_PARTS || parts == nullptr || part_row_bytes == nullptr || outer < 0)
        return fail(XS_HIP_EINVAL, std::string(what) + ": " + std::to_string(count) + " parts (1 to " +
                                       std::to_string(XS_CONCAT_PARTS) + ")");
    uint64_t bits = reinterpret_cast<uintptr_t>(out);
    int64_t row = 0;
    for (int k = 0; k < count; ++k) {
        if (part_row_bytes[k] < 0) return fail(XS_HIP_EINVAL, std::string(what) + ": negative part size");
        if (part_row_bytes[k] > 0 && parts[k] == nullptr) return fail(XS_HIP_EINVAL, std::string(what) + ": null part");
        bits |= static_cast<uint64_t>(part_row_bytes[k]) | reinterpret_cast<uintptr_t>(parts[k]);
        row += part_row_bytes[k];
    }
    if (outer == 0 || row == 0) return XS_HIP_OK;
    if (out == nullptr) return fail(XS_HIP_EINVAL, std::string(what) + ": null out");
    const int64_t e = unit_of(bits);
    ConcatArgs a{};
    a.count = count;
    int64_t first = 0;
    for (int k = 0; k < count; ++k) {
        a.src[k] = static_cast<const char*>(parts[k]);
        a.units[k] = part_row_bytes[k] / e;
        a.first[k] = first;
        first += a.units[k];
    }
    // Empty parts keep their (equal) start offset; a later part with the same start wins the lookup, as it should.
    for (int k = count; k < XS_CONCAT_PARTS; ++k) a.first[k] = first;
    a.row = row / e;
    const int64_t units = outer * a.row;
    if (units > (int64_t{1} << 40)) return fail(XS_HIP_EUNSUPPORTED, std::string(what) + ": too large");
    const bool w32 = units < (int64_t{1} << 31);
    if (w32) a.row_div = FastDiv32(static_cast<uint32_t>(a.row));
    const hipStream_t s = as_stream(stream);
    by_unit(e, [&](auto tag) {
        using E = decltype(tag);
        for (int64_t base = 0; base < units; base += kPermSlice) {
            const int64_t len = units - base < kPermSlice ? units - base : kPermSlice;
            const unsigned grid = static_cast<unsigned>((len + kPermBlock - 1) / kPermBlock);
            if (w32) concat_kernel<E, true><<<grid, kPermBlock, 0, s>>>(a, static_cast<E*>(out), units, base);
            else concat_kernel<E, false><<<grid, kPermBlock, 0, s>>>(a, static_cast<E*>(out), units, base);
        }
    });
    return check_launch(what);
}

}  // extern "C"
