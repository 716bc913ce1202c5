// Top-k along the last axis for gfx950, with the vocabulary-wide argmax (k = 1) as the fast path.
//
// Semantics: cpu_ref::topk (reference src/backend/cpu_ref/ops.cpp:663-684): values and i32 indices of the k largest,
// largest first; equal values keep the lower index first (its partial_sort comparator
// in[a] > in[b] || (in[a] == in[b] && a < b); spec src/graph/graph.h:70-71). k = 1 is blocks::argmax_rows
// (src/models/common/blocks.cpp:36-38). Launchers replaced: sycl_be::topk_scratch / topk
// (src/backend/sycl/sycl_kernels.h:61-63; sycl_kernels.cpp:1092-1254).
//
// Order used everywhere here: (v, i) precedes (w, j) when v > w, or v == w and i < j. It is a strict total order on
// non-NaN values (+0 and -0 compare equal, so the lower index wins, and the winner's own bits are reported). NaN is
// never selected; a row with fewer than k non-NaN values reports index 0 and x[0] for the missing places (cpu-ref's
// comparator is not a strict weak order with NaN, so its result there is unspecified).
//
// k = 1: a row is cut into chunks of kChunk values; a block reduces one chunk (one 128-bit load per lane, DPP within
// waves, one LDS stage across waves). A row of one chunk is done there; otherwise each chunk's (value, index) goes to
// scratch and a second launch, one block per row, reduces the row's partials -- no atomics and no waiting between
// workgroups.
// k > 1: one block per row picks the k winners one after another, each pass finding the best element strictly after
// the previous winner in the order above (k passes over the row, the later ones from cache).
#include <cfloat>
#include <climits>

#include "common.h"

namespace xs_hip {
namespace {

constexpr int kChunk = 1024;  // values per block for k = 1: one 128-bit vector per lane
constexpr int64_t kMaxRows = 65535;  // grid.y

// A (value, index) partial as one 64-bit word: the value's bits low, the index high, so it moves with one atomic.
__device__ __forceinline__ uint64_t pack_best(float v, int32_t i) {
    return static_cast<uint64_t>(__float_as_uint(v)) | (static_cast<uint64_t>(static_cast<uint32_t>(i)) << 32);
}

// true when (v, i) precedes (bv, bi).
__device__ __forceinline__ bool better(float v, int32_t i, float bv, int32_t bi) {
    return v > bv || (v == bv && i < bi);
}

template <int Ctrl>
__device__ __forceinline__ void dpp_best(float& v, int32_t& i) {
    const float ov = dpp_f<Ctrl>(v);
    const int32_t oi = dpp_i<Ctrl>(i);
    if (better(ov, oi, v, i)) {
        v = ov;
        i = oi;
    }
}

// Best over the wave; every lane gets it.
__device__ __forceinline__ void wave_best(float& v, int32_t& i) {
    dpp_best<dpp::kQuadXor1>(v, i);
    dpp_best<dpp::kQuadXor2>(v, i);
    dpp_best<dpp::kRowHalfMirror>(v, i);
    dpp_best<dpp::kRowMirror>(v, i);
    for (int off = 16; off < 64; off <<= 1) {
        const float ov = __shfl_xor(v, off, 64);
        const int32_t oi = __shfl_xor(i, off, 64);
        if (better(ov, oi, v, i)) {
            v = ov;
            i = oi;
        }
    }
}

// Best over the block (kBlock threads); every thread gets it.
__device__ __forceinline__ void block_best(float& v, int32_t& i) {
    __shared__ float sv[kBlock / 64];
    __shared__ int32_t si[kBlock / 64];
    wave_best(v, i);
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = v;
        si[threadIdx.x >> 6] = i;
    }
    __syncthreads();
    v = sv[0];
    i = si[0];
    for (int w = 1; w < kBlock / 64; ++w)
        if (better(sv[w], si[w], v, i)) {
            v = sv[w];
            i = si[w];
        }
    __syncthreads();
}

// grid (chunks, rows). A row of one chunk writes its result; otherwise partials [rows][chunks] (packed value, index).
__global__ __launch_bounds__(kBlock) void argmax_chunks(const float* __restrict__ x, float* __restrict__ values,
                                                        int32_t* __restrict__ indices, int64_t width, int chunks,
                                                        uint64_t* __restrict__ partials) {
    const int64_t row = blockIdx.y;
    const int chunk = blockIdx.x;
    const float* xr = x + row * width;
    const int64_t start = static_cast<int64_t>(chunk) * kChunk;
    const int64_t idx = start + threadIdx.x * 4;
    float bv = -INFINITY;
    int32_t bi = INT32_MAX;
    const bool vec_ok = (width % 4 == 0) && (reinterpret_cast<uintptr_t>(x) % 16 == 0);
    if (vec_ok) {
        if (idx < width) {
            float f[4];
            unpack<F32>(ld128_nt(xr + idx), f);
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (better(f[k], static_cast<int32_t>(idx + k), bv, bi)) {
                    bv = f[k];
                    bi = static_cast<int32_t>(idx + k);
                }
        }
    } else {
        for (int k = 0; k < 4; ++k) {
            const int64_t j = idx + k;
            if (j < width) {
                const float v = xr[j];
                if (better(v, static_cast<int32_t>(j), bv, bi)) {
                    bv = v;
                    bi = static_cast<int32_t>(j);
                }
            }
        }
    }
    block_best(bv, bi);
    if (threadIdx.x != 0) return;
    if (chunks == 1) {
        if (bi == INT32_MAX) {  // no non-NaN value
            bi = 0;
            bv = xr[0];
        }
        values[row] = bv;
        indices[row] = bi;
    } else {
        partials[row * chunks + chunk] = pack_best(bv, bi);
    }
}

// grid (rows): the best of a row's partials.
__global__ __launch_bounds__(kBlock) void argmax_final(const float* __restrict__ x, float* __restrict__ values,
                                                       int32_t* __restrict__ indices, int64_t width, int chunks,
                                                       const uint64_t* __restrict__ partials) {
    const int64_t row = blockIdx.x;
    float bv = -INFINITY;
    int32_t bi = INT32_MAX;
    for (int c = threadIdx.x; c < chunks; c += kBlock) {
        const uint64_t b = partials[row * chunks + c];
        const float v = __uint_as_float(static_cast<uint32_t>(b));
        const int32_t i = static_cast<int32_t>(static_cast<uint32_t>(b >> 32));
        if (better(v, i, bv, bi)) {
            bv = v;
            bi = i;
        }
    }
    block_best(bv, bi);
    if (threadIdx.x == 0) {
        if (bi == INT32_MAX) {
            bi = 0;
            bv = x[row * width];
        }
        values[row] = bv;
        indices[row] = bi;
    }
}

// k > 1: one block per row, k selection passes.
__global__ __launch_bounds__(kBlock) void topk_select(const float* __restrict__ x, float* __restrict__ values,
                                                      int32_t* __restrict__ indices, int64_t width, int64_t k) {
    const int64_t row = blockIdx.x;
    const float* xr = x + row * width;
    float pv = INFINITY;  // previous winner; (+inf, -1) precedes every element
    int32_t pi = -1;
    for (int64_t j = 0; j < k; ++j) {
        float bv = -INFINITY;
        int32_t bi = INT32_MAX;
        for (int64_t c = threadIdx.x; c < width; c += kBlock) {
            const float v = xr[c];
            const int32_t ci = static_cast<int32_t>(c);
            if (better(pv, pi, v, ci) && better(v, ci, bv, bi)) {
                bv = v;
                bi = ci;
            }
        }
        block_best(bv, bi);
        if (bi == INT32_MAX) {  // fewer than k non-NaN values
            bi = 0;
            bv = xr[0];
        } else {
            pv = bv;
            pi = bi;
        }
        if (threadIdx.x == 0) {
            values[row * k + j] = bv;
            indices[row * k + j] = bi;
        }
    }
}

int64_t argmax_chunks_of(int64_t width) { return (width + kChunk - 1) / kChunk; }

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

}  // namespace
}  // namespace xs_hip

using namespace xs_hip;

extern "C" {

size_t xs_hip_topk_scratch(int64_t rows, int64_t width, int64_t k) {
    if (rows <= 0 || width <= 0 || k != 1) return 0;
    const int64_t chunks = argmax_chunks_of(width);
    if (chunks <= 1) return 0;
    return align_up(static_cast<size_t>(rows * chunks) * sizeof(uint64_t), 256);
}

int xs_hip_topk(void* stream, const float* x, float* values, int32_t* indices, int64_t rows, int64_t width, int64_t k,
                void* scratch) {
    if (rows < 0 || width <= 0 || k < 1 || k > width)
        return fail(XS_HIP_EINVAL, "xs_hip_topk: topk " + std::to_string(k) + " of " + std::to_string(rows) +
                                       " rows of " + std::to_string(width));
    if (width > INT32_MAX)
        return fail(XS_HIP_EUNSUPPORTED, "xs_hip_topk: rows wider than 2^31 - 1 have no i32 index");
    if (rows == 0) return XS_HIP_OK;
    if (x == nullptr || values == nullptr || indices == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_topk: null buffer");
    const hipStream_t s = as_stream(stream);
    if (k == 1) {
        const int64_t chunks = argmax_chunks_of(width);
        if (rows > kMaxRows || chunks > INT32_MAX)
            return fail(XS_HIP_EUNSUPPORTED, "xs_hip_topk: more than 65535 rows in one call");
        uint64_t* partials = nullptr;
        if (chunks > 1) {
            if (scratch == nullptr)
                return fail(XS_HIP_EINVAL, "xs_hip_topk: argmax over rows of " + std::to_string(width) +
                                               " needs xs_hip_topk_scratch bytes of scratch");
            if (reinterpret_cast<uintptr_t>(scratch) % 8 != 0)
                return fail(XS_HIP_EINVAL, "xs_hip_topk: scratch must be 8-byte aligned");
            partials = static_cast<uint64_t*>(scratch);
        }
        argmax_chunks<<<dim3(static_cast<unsigned>(chunks), static_cast<unsigned>(rows)), kBlock, 0, s>>>(
            x, values, indices, width, static_cast<int>(chunks), partials);
        int rc = check_launch("xs_hip_topk");
        if (rc != XS_HIP_OK || chunks == 1) return rc;
        argmax_final<<<static_cast<unsigned>(rows), kBlock, 0, s>>>(x, values, indices, width, static_cast<int>(chunks),
                                                                     partials);
        return check_launch("xs_hip_topk");
    }
    if (rows > INT32_MAX) return fail(XS_HIP_EUNSUPPORTED, "xs_hip_topk: too many rows");
    topk_select<<<static_cast<unsigned>(rows), kBlock, 0, s>>>(x, values, indices, width, k);
    return check_launch("xs_hip_topk");
}

}  // extern "C"
