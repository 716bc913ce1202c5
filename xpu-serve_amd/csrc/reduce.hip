// Sum over one axis for gfx950: x [outer, dim, inner] -> y [outer, inner], f32.
//
// Semantics: cpu_ref::reduce_sum (reference src/backend/cpu_ref/ops.cpp:686-705): each output is the sum over `dim`
// accumulated in f64 and rounded once to f32. Launcher replaced: sycl_be::reduce_sum (src/backend/sycl/
// sycl_kernels.h:80-81).
//
// Layout: with inner == 1 (a sum along the last axis) each row is one wave: lane l sums the row's 128-bit vectors
// l, l + 64, ... (scalar loads when the row is not 16-byte aligned) in f64, four in flight, and the wave reduces by
// shuffles; four rows share a workgroup. With inner > 1 (a sum across rows) a workgroup takes 64 consecutive columns
// (32 -- one 128-byte line -- when there are fewer such tiles than CUs) of one outer index and splits `dim` in four
// or sixteen slices, one per wave: every load instruction reads whole lines, and the slices' f64 sums are combined
// in LDS. At [512, 2560] over the first axis the 32-column tiles took 4.45 us against 5.4 us for 64 columns (40
// workgroups).
#include "common.h"

namespace xs_hip {
namespace {

// Threads of a row-sum workgroup: one wave, one row (512 rows of 2560: 3.82 us against 3.93 with four rows a
// workgroup).
constexpr int kRowsBlock = 64;

__global__ __launch_bounds__(kRowsBlock) void reduce_rows(const float* x, float* y, int64_t rows, int64_t dim,
                                                          bool vec) {
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (kRowsBlock / 64) + (threadIdx.x >> 6);
    if (row >= rows) return;  // whole waves leave together; no workgroup barrier follows
    const float* xr = x + row * dim;
    double sum = 0.0;
    if (vec) {
        // four vectors in flight per lane
        const int64_t nvec = dim / 4;
        for (int64_t v0 = lane; v0 < nvec; v0 += 4 * 64) {
            u32x4 raw[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int64_t v = v0 + u * 64;
                raw[u] = v < nvec ? ld128_nt(xr + v * 4) : u32x4{0, 0, 0, 0};
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
#pragma unroll
                for (int i = 0; i < 4; ++i) sum += static_cast<double>(__uint_as_float(raw[u][i]));
            }
        }
    } else {
        for (int64_t i = lane; i < dim; i += 64) sum += static_cast<double>(xr[i]);
    }
    sum = group_sum_f64<64>(sum);
    if (lane == 0) y[row] = static_cast<float>(sum);
}

// Columns: a workgroup of SLICES waves takes COLS consecutive columns (64, or 32 -- one 128-byte line -- when column
// tiles are few) of one outer index and splits `dim` in SLICES slices, one a wave; a wave instruction reads 64 / COLS
// rows of the tile, each lane keeping eight loads in flight. The rows a wave read are added by a shuffle, the slices'
// f64 sums in LDS, in a fixed order.
template <int SLICES, int COLS>
__global__ __launch_bounds__(64 * SLICES) void reduce_cols(const float* x, float* y, int64_t dim, int64_t inner,
                                                           uint32_t col_blocks) {
    constexpr int RPW = 64 / COLS;  // rows a wave instruction covers
    __shared__ double part[SLICES][COLS];
    const int c = threadIdx.x % COLS;
    const int sub = (threadIdx.x % 64) / COLS;
    const int slice = threadIdx.x / 64;
    const int64_t o = blockIdx.x / col_blocks;
    const int64_t i = static_cast<int64_t>(blockIdx.x - o * col_blocks) * COLS + c;
    const int64_t per = (dim + SLICES - 1) / SLICES;
    const int64_t d0 = slice * per;
    const int64_t d1 = d0 + per < dim ? d0 + per : dim;
    double sum = 0.0;
    if (i < inner) {
        const float* xp = x + (o * dim) * inner + i;
        int64_t d = d0 + sub;
        for (; d + 7 * RPW < d1; d += 8 * RPW) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = xp[(d + u * RPW) * inner];
#pragma unroll
            for (int u = 0; u < 8; ++u) sum += static_cast<double>(v[u]);
        }
        for (; d < d1; d += RPW) sum += static_cast<double>(xp[d * inner]);
    }
#pragma unroll
    for (int m = COLS; m < 64; m *= 2) sum += __shfl_xor(sum, m, 64);
    if (sub == 0) part[slice][c] = sum;
    __syncthreads();
    if (slice == 0 && sub == 0 && i < inner) {
        double total = part[0][c];
#pragma unroll
        for (int s = 1; s < SLICES; ++s) total += part[s][c];
        y[o * inner + i] = static_cast<float>(total);
    }
}

}  // namespace
}  // namespace xs_hip

using namespace xs_hip;

extern "C" {

int xs_hip_reduce_sum(void* stream, const float* x, float* y, int64_t outer, int64_t dim, int64_t inner) {
    if (outer < 0 || dim < 0 || inner < 0 || outer > 0x7fffffffLL)
        return fail(XS_HIP_EINVAL, "xs_hip_reduce_sum: shape [" + std::to_string(outer) + ", " + std::to_string(dim) +
                                       ", " + std::to_string(inner) + "]");
    if (outer == 0 || inner == 0) return XS_HIP_OK;
    if (x == nullptr && dim > 0) return fail(XS_HIP_EINVAL, "xs_hip_reduce_sum: null buffer");
    if (y == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_reduce_sum: null buffer");
    const hipStream_t s = as_stream(stream);
    if (inner == 1) {
        const bool vec = dim % 4 == 0 && aligned16(x);
        const int64_t blocks = (outer + kRowsBlock / 64 - 1) / (kRowsBlock / 64);
        reduce_rows<<<static_cast<unsigned>(blocks), kRowsBlock, 0, s>>>(x, y, outer, dim, vec);
    } else {
        // Few column tiles get sixteen waves each (more of `dim` in flight) and, below one tile a CU, tiles of one
        // 128-byte line; many get four waves over 64 columns.
        const int64_t cus = static_cast<int64_t>(device_cus());
        const int64_t wide_blocks = (inner + 63) / 64 * outer;
        const int cols = wide_blocks < cus ? 32 : 64;
        const int64_t col_blocks = (inner + cols - 1) / cols;
        if (col_blocks * outer > 0x7fffffffLL)
            return fail(XS_HIP_EUNSUPPORTED, "xs_hip_reduce_sum: " + std::to_string(outer) + " outer indices of " +
                                                 std::to_string(inner) + " columns exceed the launch grid");
        const unsigned grid = static_cast<unsigned>(col_blocks * outer);
        const uint32_t cb = static_cast<uint32_t>(col_blocks);
        if (cols == 32)
            reduce_cols<16, 32><<<grid, 64 * 16, 0, s>>>(x, y, dim, inner, cb);
        else if (col_blocks * outer < 4 * cus)
            reduce_cols<16, 64><<<grid, 64 * 16, 0, s>>>(x, y, dim, inner, cb);
        else
            reduce_cols<4, 64><<<grid, 64 * 4, 0, s>>>(x, y, dim, inner, cb);
    }
    return check_launch("xs_hip_reduce_sum");
}

}  // extern "C"
