// Sum over one axis for gfx950: x [outer, dim, inner] -> y [outer, inner], f32.
//
// Semantics: cpu_ref::reduce_sum (reference src/backend/cpu_ref/ops.cpp:686-705): each output is the sum over `dim`
// accumulated in f64 and rounded once to f32. Launcher replaced: sycl_be::reduce_sum (src/backend/sycl/
// sycl_kernels.h:80-81).
//
// Layout: with inner == 1 (a sum along the last axis) each row is one wave: lane l sums the row's 128-bit vectors
// l, l + 64, ... (scalar loads when the row is not 16-byte aligned) in f64, four in flight, and the wave reduces by
// shuffles; four rows share a workgroup. With inner > 1 (a sum across rows) a workgroup takes 64 consecutive columns
// of one outer index and splits `dim` in four or sixteen slices, one per wave: every load instruction reads 64
// consecutive floats, and the slices' f64 sums are combined in LDS.
#include "common.h"

namespace xs_hip {
namespace {

__global__ __launch_bounds__(kBlock) void reduce_rows(const float* x, float* y, int64_t rows, int64_t dim, bool vec) {
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (kBlock / 64) + (threadIdx.x >> 6);
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

// Columns: a workgroup of SLICES waves takes 64 consecutive columns of one outer index and splits `dim` in SLICES
// slices, one a wave; each lane keeps eight rows' loads in flight. The slices' f64 sums combine in LDS.
constexpr int kCols = 64;

template <int SLICES>
__global__ __launch_bounds__(64 * SLICES) void reduce_cols(const float* x, float* y, int64_t dim, int64_t inner,
                                                           uint32_t col_blocks) {
    __shared__ double part[SLICES][kCols];
    const int c = threadIdx.x % kCols;
    const int slice = threadIdx.x / kCols;
    const int64_t o = blockIdx.x / col_blocks;
    const int64_t i = static_cast<int64_t>(blockIdx.x - o * col_blocks) * kCols + c;
    const int64_t per = (dim + SLICES - 1) / SLICES;
    const int64_t d0 = slice * per;
    const int64_t d1 = d0 + per < dim ? d0 + per : dim;
    double sum = 0.0;
    if (i < inner) {
        const float* xp = x + (o * dim) * inner + i;
        int64_t d = d0;
        for (; d + 8 <= d1; d += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = xp[(d + u) * inner];
#pragma unroll
            for (int u = 0; u < 8; ++u) sum += static_cast<double>(v[u]);
        }
        for (; d < d1; ++d) sum += static_cast<double>(xp[d * inner]);
    }
    part[slice][c] = sum;
    __syncthreads();
    if (slice == 0 && i < inner) {
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
        const int64_t blocks = (outer + kBlock / 64 - 1) / (kBlock / 64);
        reduce_rows<<<static_cast<unsigned>(blocks), kBlock, 0, s>>>(x, y, outer, dim, vec);
    } else {
        const int64_t col_blocks = (inner + kCols - 1) / kCols;
        if (col_blocks * outer > 0x7fffffffLL)
            return fail(XS_HIP_EUNSUPPORTED, "xs_hip_reduce_sum: " + std::to_string(outer) + " outer indices of " +
                                                 std::to_string(inner) + " columns exceed the launch grid");
        // Few column blocks get sixteen waves each (more of `dim` in flight); many get four.
        if (col_blocks * outer < 4 * static_cast<int64_t>(device_cus()))
            reduce_cols<16><<<static_cast<unsigned>(col_blocks * outer), 64 * 16, 0, s>>>(
                x, y, dim, inner, static_cast<uint32_t>(col_blocks));
        else
            reduce_cols<4><<<static_cast<unsigned>(col_blocks * outer), 64 * 4, 0, s>>>(
                x, y, dim, inner, static_cast<uint32_t>(col_blocks));
    }
    return check_launch("xs_hip_reduce_sum");
}

}  // extern "C"
