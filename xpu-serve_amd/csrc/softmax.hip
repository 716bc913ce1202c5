// Row softmax for gfx950, plain and in the scaled, length-masked form of attention scores.
//
// Semantics: cpu_ref::softmax (reference src/backend/cpu_ref/ops.cpp:644-661): peak = max, sum = sum exp(x - peak),
// y = exp(x - peak) / sum, all in f64, rounded once to f32. The masked form is what cpu-ref evaluates for
// Softmax(Add(Scale(s, scale), mask)) with a 0/-inf key mask: s * scale in f32 (ops.cpp:209-211), -inf on masked keys,
// which come out exactly 0. (Device analog: sycl_be::softmax, src/backend/sycl/sycl_kernels.cpp:1071-1090, and the
// masked attention_softmax, :2047-2104.)
//
// Layout: as the row norms, LPR lanes share a row (16..1024) and hold it in registers (up to NV 128-bit vectors per
// lane), so the row is read from HBM once and written once, and exp is evaluated once per element. Reductions: the max
// in f32 (exact) by DPP within a wave and one LDS stage across waves; x - peak carries its rounding error (TwoSum) into
// exp; the sum is accumulated in f64; y = e * (1 / sum) in f64, rounded once. Masked keys are neither loaded nor
// exponentiated.
//
// Few wide rows (the decode step's [heads, 1, keys] scores) would leave most of the chip idle with one workgroup per
// row, so with caller scratch a row is split over `chunks` workgroups of kChunk keys, in two launches that need no
// atomics or cross-workgroup waits: the first writes each chunk's (max m_j, sum s_j of exp(x - m_j)) to scratch; the
// second reads the row's partials (one lane per chunk: M = max m_j, S = sum s_j exp(m_j - M) in f64), reads its chunk
// again -- from the L2 of the same XCD, since both launches map a chunk to the same workgroup id -- and writes
// exp(x - M) / S.
#include <cmath>

#include "common.h"

namespace xs_hip {
namespace {

struct SoftmaxArgs {
    const float* x;
    float* y;
    int64_t rows, width, row_stride;
    float scale;
    const int64_t* valid_len;  // per row, or null
    int64_t valid_all;
};

// exp(s - peak) with the rounding error of the f32 subtraction folded back in: d + err == s - peak exactly (TwoSum,
// Knuth), and exp(d + err) = exp(d) (1 + err) to first order.
__device__ __forceinline__ float exp_diff(float s, float peak) {
    const float d = s - peak;
    const float bb = d - s;
    const float err = (s - (d - bb)) + (-peak - bb);
    const float e = expf(d);
    return (err != 0.0f && err == err) ? fmaf(e, err, e) : e;
}

template <int LPR, int NV>
__global__ __launch_bounds__(LPR > kBlock ? LPR : kBlock) void softmax_vec(SoftmaxArgs p) {
    constexpr int BLOCK = LPR > kBlock ? LPR : kBlock;
    constexpr int ROWS_PER_BLOCK = BLOCK / LPR;
    constexpr int WAVES_PER_ROW = LPR > 64 ? LPR / 64 : 1;
    constexpr int W = LPR < 64 ? LPR : 64;
    __shared__ float part_max[BLOCK / 64];
    __shared__ double part_sum[BLOCK / 64];

    const int l = threadIdx.x % LPR;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * ROWS_PER_BLOCK + threadIdx.x / LPR;
    const bool live = row < p.rows;
    const int64_t nvec = p.width / 4;
    int64_t valid = p.valid_len != nullptr && live ? p.valid_len[row] : p.valid_all;
    valid = valid < 0 ? 0 : (valid > p.width ? p.width : valid);
    const float* xr = p.x + row * p.row_stride;

    float s[NV][4];
    u32x4 raw[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int64_t v = l + static_cast<int64_t>(k) * LPR;
        if (live && v < nvec && v * 4 < valid) raw[k] = ld128_nt(xr + v * 4);
    }
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int64_t v = l + static_cast<int64_t>(k) * LPR;
        if (live && v < nvec && v * 4 < valid) {
            unpack<F32>(raw[k], s[k]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                s[k][i] = v * 4 + i < valid ? s[k][i] * p.scale : -INFINITY;
                m = fmaxf(m, s[k][i]);
            }
        }
    }
    m = group_reduce<W, OpMax>(m);
    if constexpr (WAVES_PER_ROW > 1) {
        const int wave = threadIdx.x >> 6;
        if ((threadIdx.x & 63) == 0) part_max[wave] = m;
        __syncthreads();
        const int first = (wave / WAVES_PER_ROW) * WAVES_PER_ROW;
        m = part_max[first];
#pragma unroll
        for (int i = 1; i < WAVES_PER_ROW; ++i) m = fmaxf(m, part_max[first + i]);
    }
    // A row whose keys are all masked or -inf has peak -inf and exp(-inf - -inf) = NaN, as in cpu-ref; with nothing
    // loaded the sum stays 0 and 0 * (1 / 0) below is NaN too. A NaN sum makes every output NaN, masked keys included
    // (cpu-ref divides their exp(-inf) = 0 by it).
    double sum = 0.0;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int64_t v = l + static_cast<int64_t>(k) * LPR;
        if (live && v < nvec && v * 4 < valid) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                s[k][i] = v * 4 + i < valid ? exp_diff(s[k][i], m) : 0.0f;
                sum += static_cast<double>(s[k][i]);
            }
        }
    }
    sum = group_sum_f64<W>(sum);
    if constexpr (WAVES_PER_ROW > 1) {
        const int wave = threadIdx.x >> 6;
        if ((threadIdx.x & 63) == 0) part_sum[wave] = sum;
        __syncthreads();
        const int first = (wave / WAVES_PER_ROW) * WAVES_PER_ROW;
        sum = 0.0;
#pragma unroll
        for (int i = 0; i < WAVES_PER_ROW; ++i) sum += part_sum[first + i];
    }
    if (!live) return;
    const double rinv = 1.0 / sum;
    float* yr = p.y + row * p.row_stride;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int64_t v = l + static_cast<int64_t>(k) * LPR;
        if (v < nvec) {
            float o[4];
            const float masked = static_cast<float>(0.0 * rinv);
            if (v * 4 < valid) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    o[i] = v * 4 + i < valid ? static_cast<float>(static_cast<double>(s[k][i]) * rinv) : masked;
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) o[i] = masked;
            }
            st128_nt(yr + v * 4, pack<F32>(o));
        }
    }
}

// Any width or alignment: one block per row, three passes over the row (the later ones from cache).
__global__ __launch_bounds__(kBlock) void softmax_any(SoftmaxArgs p) {
    __shared__ float part_max[kBlock / 64];
    __shared__ double part_sum[kBlock / 64];
    const int64_t row = blockIdx.x;
    int64_t valid = p.valid_len != nullptr ? p.valid_len[row] : p.valid_all;
    valid = valid < 0 ? 0 : (valid > p.width ? p.width : valid);
    const float* xr = p.x + row * p.row_stride;
    float* yr = p.y + row * p.row_stride;
    float m = -INFINITY;
    for (int64_t i = threadIdx.x; i < valid; i += kBlock) m = fmaxf(m, xr[i] * p.scale);
    m = group_reduce<64, OpMax>(m);
    if ((threadIdx.x & 63) == 0) part_max[threadIdx.x >> 6] = m;
    __syncthreads();
    m = part_max[0];
    for (int i = 1; i < kBlock / 64; ++i) m = fmaxf(m, part_max[i]);
    double sum = 0.0;
    for (int64_t i = threadIdx.x; i < valid; i += kBlock) sum += static_cast<double>(exp_diff(xr[i] * p.scale, m));
    sum = group_sum_f64<64>(sum);
    if ((threadIdx.x & 63) == 0) part_sum[threadIdx.x >> 6] = sum;
    __syncthreads();
    sum = 0.0;
    for (int i = 0; i < kBlock / 64; ++i) sum += part_sum[i];
    const double rinv = 1.0 / sum;
    const float masked = static_cast<float>(0.0 * rinv);
    // Read every input of the row before the first write: y may alias x.
    __syncthreads();
    for (int64_t i = threadIdx.x; i < p.width; i += kBlock) {
        yr[i] = i < valid ? static_cast<float>(static_cast<double>(exp_diff(xr[i] * p.scale, m)) * rinv)
                          : masked;
    }
}

constexpr int kChunkVpt = 1;                      // 128-bit vectors per lane in a chunk
constexpr int64_t kChunk = kBlock * kChunkVpt * 4;  // keys per chunk: 1024
constexpr int64_t kMaxRows = 65535;
constexpr int kMaxChunks = 64;                      // the second launch combines a row's partials in one wave

// Max over the block; every thread gets it. `lds` is written once per launch (each reduction has its own array), so
// no barrier follows the reads.
__device__ __forceinline__ float block_max(float v, float* lds) {
    v = group_reduce<64, OpMax>(v);
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
    __syncthreads();
    float m = lds[0];
    for (int i = 1; i < kBlock / 64; ++i) m = fmaxf(m, lds[i]);
    return m;
}

// Sum over the block, as block_max.
__device__ __forceinline__ double block_sum(double v, double* lds) {
    v = group_sum_f64<64>(v);
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
    __syncthreads();
    double s = 0.0;
    for (int i = 0; i < kBlock / 64; ++i) s += lds[i];
    return s;
}

__device__ __forceinline__ int64_t row_valid(const SoftmaxArgs& p, int64_t row) {
    const int64_t v = p.valid_len != nullptr ? p.valid_len[row] : p.valid_all;
    return v < 0 ? 0 : (v > p.width ? p.width : v);
}

// Loads the chunk's valid keys scaled (-inf for masked ones) and returns how many of its vectors are in range.
__device__ __forceinline__ void load_chunk(const SoftmaxArgs& p, int64_t row, int chunk, int64_t valid,
                                           float (&s)[kChunkVpt][4]) {
    const float* xr = p.x + row * p.row_stride;
    const int64_t v0 = chunk * (kChunk / 4);
    const int64_t nvec = p.width / 4;
    u32x4 raw[kChunkVpt];
#pragma unroll
    for (int k = 0; k < kChunkVpt; ++k) {
        const int64_t v = v0 + threadIdx.x + k * kBlock;
        if (v < nvec && v * 4 < valid) raw[k] = ld128(xr + v * 4);
    }
#pragma unroll
    for (int k = 0; k < kChunkVpt; ++k) {
        const int64_t v = v0 + threadIdx.x + k * kBlock;
        if (v < nvec && v * 4 < valid) {
            unpack<F32>(raw[k], s[k]);
#pragma unroll
            for (int i = 0; i < 4; ++i) s[k][i] = v * 4 + i < valid ? s[k][i] * p.scale : -INFINITY;
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) s[k][i] = -INFINITY;
        }
    }
}

// Launch 1, grid (chunks, rows): partial[row][chunk] = (m_j as f32 bits, s_j as f64 bits).
__global__ __launch_bounds__(kBlock) void softmax_partials(SoftmaxArgs p, int chunks, uint64_t* __restrict__ partial) {
    __shared__ float lds_f[kBlock / 64];
    __shared__ double lds_d[kBlock / 64];
    const int64_t row = blockIdx.y;
    const int chunk = blockIdx.x;
    const int64_t valid = row_valid(p, row);
    float s[kChunkVpt][4];
    load_chunk(p, row, chunk, valid, s);
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < kChunkVpt; ++k)
#pragma unroll
        for (int i = 0; i < 4; ++i) m = fmaxf(m, s[k][i]);
    m = block_max(m, lds_f);
    // A chunk whose keys are all masked or -inf adds nothing against any finite M (and its exponentials relative to
    // its own -inf maximum would be NaN), so its sum is 0.
    double sum = 0.0;
    if (m != -INFINITY) {
#pragma unroll
        for (int k = 0; k < kChunkVpt; ++k)
#pragma unroll
            for (int i = 0; i < 4; ++i) sum += static_cast<double>(exp_diff(s[k][i], m));
    }
    sum = block_sum(sum, lds_d);
    if (threadIdx.x == 0) {
        uint64_t* out = partial + (row * chunks + chunk) * 2;
        out[0] = __float_as_uint(m);
        out[1] = static_cast<uint64_t>(__double_as_longlong(sum));
    }
}

// Launch 2, grid (chunks, rows): combines the row's partials and writes the chunk's outputs.
__global__ __launch_bounds__(kBlock) void softmax_finish(SoftmaxArgs p, int chunks,
                                                         const uint64_t* __restrict__ partial) {
    __shared__ float s_M;
    __shared__ double s_S;
    const int64_t row = blockIdx.y;
    const int chunk = blockIdx.x;
    const int64_t valid = row_valid(p, row);
    float s[kChunkVpt][4];
    load_chunk(p, row, chunk, valid, s);
    if (threadIdx.x < 64) {
        const int j = threadIdx.x;
        const uint64_t* pr = partial + row * chunks * 2;
        const float mj = j < chunks ? __uint_as_float(static_cast<uint32_t>(pr[2 * j])) : -INFINITY;
        const double sj = j < chunks ? __longlong_as_double(static_cast<long long>(pr[2 * j + 1])) : 0.0;
        const float M = group_reduce<64, OpMax>(mj);
        // M = -inf: every key masked or -inf; cpu-ref's exp(-inf - (-inf)) makes the row NaN.
        const double t = mj != -INFINITY ? sj * exp(static_cast<double>(mj) - static_cast<double>(M))
                                         : (M == -INFINITY && j < chunks ? static_cast<double>(NAN) : 0.0);
        const double S = group_sum_f64<64>(t);
        if (j == 0) {
            s_M = M;
            s_S = S;
        }
    }
    __syncthreads();
    const float M = s_M;
    const double rinv = 1.0 / s_S;
    float* yr = p.y + row * p.row_stride;
    const int64_t v0 = chunk * (kChunk / 4);
    const int64_t nvec = p.width / 4;
#pragma unroll
    for (int k = 0; k < kChunkVpt; ++k) {
        const int64_t v = v0 + threadIdx.x + k * kBlock;
        if (v < nvec) {
            float o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                // masked keys: exp(-inf - M) = 0 (NaN when the sum is)
                const float e = s[k][i] == -INFINITY ? 0.0f : exp_diff(s[k][i], M);
                o[i] = static_cast<float>(static_cast<double>(e) * rinv);
            }
            st128_nt(yr + v * 4, pack<F32>(o));
        }
    }
}

int64_t split_chunks(int64_t rows, int64_t width) {
    const int64_t chunks = (width + kChunk - 1) / kChunk;
    // Split only rows whose one-workgroup form would leave the chip mostly idle.
    if (chunks < 2 || chunks > kMaxChunks || rows > kMaxRows || rows * 4 >= 1024 || width % 4 != 0) return 0;
    return chunks;
}

size_t split_scratch_bytes(int64_t rows, int64_t chunks) {
    return (static_cast<size_t>(rows * chunks) * 16 + 255) / 256 * 256;
}

template <int LPR>
int go_vec(hipStream_t s, const SoftmaxArgs& p, int nv) {
    constexpr int BLOCK = LPR > kBlock ? LPR : kBlock;
    const unsigned grid = static_cast<unsigned>((p.rows + (BLOCK / LPR) - 1) / (BLOCK / LPR));
    switch (nv) {
        case 1: softmax_vec<LPR, 1><<<grid, BLOCK, 0, s>>>(p); break;
        case 2: softmax_vec<LPR, 2><<<grid, BLOCK, 0, s>>>(p); break;
        case 3: softmax_vec<LPR, 3><<<grid, BLOCK, 0, s>>>(p); break;
        case 4: softmax_vec<LPR, 4><<<grid, BLOCK, 0, s>>>(p); break;
        case 5: softmax_vec<LPR, 5><<<grid, BLOCK, 0, s>>>(p); break;
        case 6: softmax_vec<LPR, 6><<<grid, BLOCK, 0, s>>>(p); break;
        case 7: softmax_vec<LPR, 7><<<grid, BLOCK, 0, s>>>(p); break;
        default: softmax_vec<LPR, 8><<<grid, BLOCK, 0, s>>>(p); break;
    }
    return check_launch("xs_hip_softmax");
}

constexpr int kMaxNv = 8;

int launch_softmax(hipStream_t s, const SoftmaxArgs& p, void* scratch) {
    if (p.rows == 0) return XS_HIP_OK;
    const int64_t chunks = split_chunks(p.rows, p.width);
    if (scratch != nullptr && chunks > 0 && aligned16(p.x) && aligned16(p.y) && p.row_stride % 4 == 0) {
        if (reinterpret_cast<uintptr_t>(scratch) % 16 != 0)
            return fail(XS_HIP_EINVAL, "xs_hip_softmax_masked: scratch must be 16-byte aligned");
        auto* partial = static_cast<uint64_t*>(scratch);
        const dim3 grid(static_cast<unsigned>(chunks), static_cast<unsigned>(p.rows));
        softmax_partials<<<grid, kBlock, 0, s>>>(p, static_cast<int>(chunks), partial);
        int rc = check_launch("xs_hip_softmax_masked");
        if (rc != XS_HIP_OK) return rc;
        softmax_finish<<<grid, kBlock, 0, s>>>(p, static_cast<int>(chunks), partial);
        return check_launch("xs_hip_softmax_masked");
    }
    // The in-register kernel needs whole 128-bit vectors; the three-pass kernel handles y aliasing x by reading the
    // row before writing it, the in-register one trivially (each lane reads its values before writing them).
    const bool vec = p.width % 4 == 0 && p.row_stride % 4 == 0 && aligned16(p.x) && aligned16(p.y);
    const int64_t nvec = p.width / 4;
    if (vec) {
        for (int lpr = 16; lpr <= 1024; lpr *= 2) {
            const int64_t nv = (nvec + lpr - 1) / lpr;
            if (nv > kMaxNv) continue;
            const int n = static_cast<int>(nv);
            switch (lpr) {
                case 16: return go_vec<16>(s, p, n);
                case 32: return go_vec<32>(s, p, n);
                case 64: return go_vec<64>(s, p, n);
                case 128: return go_vec<128>(s, p, n);
                case 256: return go_vec<256>(s, p, n);
                case 512: return go_vec<512>(s, p, n);
                default: return go_vec<1024>(s, p, n);
            }
        }
    }
    softmax_any<<<static_cast<unsigned>(p.rows), kBlock, 0, s>>>(p);
    return check_launch("xs_hip_softmax");
}

}  // namespace
}  // namespace xs_hip

using namespace xs_hip;

extern "C" {

int xs_hip_softmax(void* stream, const float* x, float* y, int64_t rows, int64_t width) {
    if (rows < 0 || width <= 0 || rows > 0x7fffffffLL)
        return fail(XS_HIP_EINVAL, "xs_hip_softmax: " + std::to_string(rows) + " rows of width " + std::to_string(width));
    if (rows == 0) return XS_HIP_OK;
    if (x == nullptr || y == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_softmax: null buffer");
    const SoftmaxArgs p{x, y, rows, width, width, 1.0f, nullptr, width};
    return launch_softmax(as_stream(stream), p, nullptr);
}

size_t xs_hip_softmax_scratch(int64_t rows, int64_t width) {
    if (rows <= 0 || width <= 0) return 0;
    const int64_t chunks = split_chunks(rows, width);
    return chunks > 0 ? split_scratch_bytes(rows, chunks) : 0;
}

int xs_hip_softmax_masked(void* stream, const float* x, float* y, int64_t rows, int64_t width, int64_t row_stride,
                          float scale, const int64_t* valid_len, int64_t valid_len_all, void* scratch) {
    if (rows < 0 || width <= 0 || rows > 0x7fffffffLL || row_stride < width)
        return fail(XS_HIP_EINVAL, "xs_hip_softmax_masked: " + std::to_string(rows) + " rows of width " +
                                       std::to_string(width) + " with row stride " + std::to_string(row_stride));
    if (rows == 0) return XS_HIP_OK;
    if (x == nullptr || y == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_softmax_masked: null buffer");
    const SoftmaxArgs p{x, y, rows, width, row_stride, scale, valid_len, valid_len_all};
    return launch_softmax(as_stream(stream), p, scratch);
}

}  // extern "C"
