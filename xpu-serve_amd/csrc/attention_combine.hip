// The split-attention combine and merge over the reference's partial-row layout, for gfx950: the launchers a caller of
// its own split attention (the reference's matmul and flash paths) uses to fold key splits into the output.
//
// Layout (sycl_kernels.h:232-244): part [rows, split, D + 2] -- for each row and split, D unnormalized weighted sums,
// then the split's running max and its sum of exponentials relative to that max; a split that saw no key has max
// -inf. Semantics: sycl_be::attention_combine / attention_merge (src/backend/sycl/sycl_kernels.cpp:1975-2030):
//   combine: out[r, d] = sum_s part[r, s, d] w_s / sum_s part[r, s, D + 1] w_s, w_s = exp(max_s - max), max over the
//            splits, splits with max -inf left out;
//   merge:   acc [rows, D + 2] (a partial row itself) takes in the row's splits, rescaled to the new max; `first` starts
//            acc as their merge alone. attention_combine(acc, split 1) then gives the output.
//
// Layout of the kernels: one wave per row, lanes over the D sums (a row's split maxima and weights are computed by
// every lane alike, from loads of the same few words), so a row's partials are read once, in whole 64-lane spans.
#include <cmath>

#include "common.h"

namespace xs_hip {
namespace {

constexpr int kRowsPerBlock = 4;  // a wave a row, four waves a workgroup

__global__ __launch_bounds__(64 * kRowsPerBlock) void combine_kernel(const float* __restrict__ part,
                                                                     float* __restrict__ out, int64_t rows,
                                                                     int64_t split, int64_t D) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / 64;
    if (r >= rows) return;
    const int lane = threadIdx.x % 64;
    const float* pr = part + r * split * (D + 2);
    float m_all = -INFINITY;
    for (int64_t sp = 0; sp < split; ++sp) m_all = fmaxf(m_all, pr[sp * (D + 2) + D]);
    float denom = 0.0f;
    for (int64_t sp = 0; sp < split; ++sp) {
        const float ms = pr[sp * (D + 2) + D];
        if (ms == -INFINITY) continue;
        denom += pr[sp * (D + 2) + D + 1] * __expf(ms - m_all);
    }
    for (int64_t d = lane; d < D; d += 64) {
        float acc = 0.0f;
        for (int64_t sp = 0; sp < split; ++sp) {
            const float ms = pr[sp * (D + 2) + D];
            if (ms == -INFINITY) continue;
            acc += pr[sp * (D + 2) + d] * __expf(ms - m_all);
        }
        out[r * D + d] = acc / denom;
    }
}

__global__ __launch_bounds__(64 * kRowsPerBlock) void merge_kernel(const float* __restrict__ part, float* acc,
                                                                   int64_t rows, int64_t split, int64_t D, bool first) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / 64;
    if (r >= rows) return;
    const int lane = threadIdx.x % 64;
    const float* pr = part + r * split * (D + 2);
    float* ar = acc + r * (D + 2);
    // Every lane reads the row's running (max, denominator) before lane 0 overwrites them at the end.
    const float m_acc = first ? -INFINITY : ar[D];
    const float l_acc = first ? 0.0f : ar[D + 1];
    float m_all = m_acc;
    for (int64_t sp = 0; sp < split; ++sp) m_all = fmaxf(m_all, pr[sp * (D + 2) + D]);
    if (m_all == -INFINITY) {  // nothing seen yet
        if (first) {
            for (int64_t d = lane; d < D; d += 64) ar[d] = 0.0f;
            if (lane == 0) {
                ar[D] = -INFINITY;
                ar[D + 1] = 0.0f;
            }
        }
        return;
    }
    const float w_acc = m_acc == -INFINITY ? 0.0f : __expf(m_acc - m_all);
    float denom = m_acc == -INFINITY ? 0.0f : l_acc * w_acc;
    for (int64_t sp = 0; sp < split; ++sp) {
        const float ms = pr[sp * (D + 2) + D];
        if (ms == -INFINITY) continue;
        denom += pr[sp * (D + 2) + D + 1] * __expf(ms - m_all);
    }
    for (int64_t d = lane; d < D; d += 64) {
        float v = m_acc == -INFINITY ? 0.0f : ar[d] * w_acc;
        for (int64_t sp = 0; sp < split; ++sp) {
            const float ms = pr[sp * (D + 2) + D];
            if (ms == -INFINITY) continue;
            v += pr[sp * (D + 2) + d] * __expf(ms - m_all);
        }
        ar[d] = v;
    }
    if (lane == 0) {
        ar[D] = m_all;
        ar[D + 1] = denom;
    }
}

int check_args(const char* what, const void* part, const void* out, int64_t rows, int64_t split, int64_t head_dim) {
    if (rows < 0 || split < 1 || head_dim < 1)
        return fail(XS_HIP_EINVAL, std::string(what) + ": " + std::to_string(rows) + " rows, split " +
                                       std::to_string(split) + ", head_dim " + std::to_string(head_dim));
    if (rows > 0 && (part == nullptr || out == nullptr)) return fail(XS_HIP_EINVAL, std::string(what) + ": null buffer");
    if ((rows + kRowsPerBlock - 1) / kRowsPerBlock > 0x7fffffffLL)
        return fail(XS_HIP_EUNSUPPORTED, std::string(what) + ": too many rows");
    return XS_HIP_OK;
}

}  // namespace
}  // namespace xs_hip

using namespace xs_hip;

extern "C" {

int xs_hip_attention_combine(void* stream, const float* part, float* out, int64_t rows, int64_t split,
                             int64_t head_dim) {
    const int rc = check_args("xs_hip_attention_combine", part, out, rows, split, head_dim);
    if (rc != XS_HIP_OK || rows == 0) return rc;
    combine_kernel<<<static_cast<unsigned>((rows + kRowsPerBlock - 1) / kRowsPerBlock), 64 * kRowsPerBlock, 0,
                     as_stream(stream)>>>(part, out, rows, split, head_dim);
    return check_launch("xs_hip_attention_combine");
}

int xs_hip_attention_merge(void* stream, const float* part, float* acc, int64_t rows, int64_t split, int64_t head_dim,
                           int first) {
    const int rc = check_args("xs_hip_attention_merge", part, acc, rows, split, head_dim);
    if (rc != XS_HIP_OK || rows == 0) return rc;
    merge_kernel<<<static_cast<unsigned>((rows + kRowsPerBlock - 1) / kRowsPerBlock), 64 * kRowsPerBlock, 0,
                   as_stream(stream)>>>(part, acc, rows, split, head_dim, first != 0);
    return check_launch("xs_hip_attention_merge");
}

}  // extern "C"
