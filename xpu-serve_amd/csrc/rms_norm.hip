// RMSNorm, with or without the residual add folded in, for gfx950.
//
// Semantics: cpu_ref::rms_norm (reference src/backend/cpu_ref/ops.cpp:260-281): inv_rms = 1 / sqrt(sum(x^2) / width +
// eps) and y = x * inv_rms * w, evaluated in f64 and rounded once to f32; the graph spec says "computed in f32, no +1
// offset" (src/graph/graph.h:57). The residual form is the decoder pattern h = add(h, f(rms_norm(h)))
// (src/models/qwen3/qwen3_decoder.cpp:101-102): cpu-ref evaluates h = fl32(x + r) (ops.cpp:201-203) and then the norm;
// here both happen in one pass that also writes h back (the updated residual).
//
// Layout: LPR lanes share a row (LPR a power of two, 16..1024), each lane holding up to NV 128-bit vectors of the row
// in registers (vector k of lane l is the row's vector l + k * LPR, so every load instruction of a wave is coalesced).
// The sum of squares is summed in f32 per lane, reduced across the LPR lanes with DPP inside a wave and one LDS stage
// across waves; the scale 1 / sqrt(mean + eps) is computed in f64 from that sum; the outputs are formed in f64
// (x * inv_rms * w in the reference's order) and rounded once. The row is read from HBM once.
#include <cmath>

#include "common.h"

namespace xs_hip {
namespace {

struct NormArgs {
    const void* x;      // TX [rows, width]
    const float* r;     // f32 residual or null
    const float* w;     // f32 [width] or null
    const float* bias;  // f32 [width] or null
    float* h_out;       // f32 [rows, width] (residual form) or null
    void* y;            // TY [rows, width]
    int64_t rows, width;
    float eps;
};

template <typename TX, typename TY, int LPR, int NV>
__global__ __launch_bounds__(LPR > kBlock ? LPR : kBlock) void rms_norm_vec(NormArgs p) {
    constexpr int BLOCK = LPR > kBlock ? LPR : kBlock;
    constexpr int VEC = vec_elems<TX>();
    constexpr int ROWS_PER_BLOCK = BLOCK / LPR;
    constexpr int WAVES_PER_ROW = LPR > 64 ? LPR / 64 : 1;
    using SX = typename TX::storage;
    using SY = typename TY::storage;
    __shared__ float partial[BLOCK / 64];

    const int l = threadIdx.x % LPR;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * ROWS_PER_BLOCK + threadIdx.x / LPR;
    const bool live = row < p.rows;
    const int64_t nvec = p.width / VEC;
    const SX* xr = static_cast<const SX*>(p.x) + row * p.width;

    float h[NV][VEC];
    u32x4 raw_x[NV], raw_r[NV * (VEC == 4 ? 1 : 2)];
    // Issue every load of the row first.
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int64_t v = l + static_cast<int64_t>(k) * LPR;
        if (live && v < nvec) {
            raw_x[k] = ld128_nt(xr + v * VEC);
            if (p.r != nullptr) {
                const float* rr = p.r + row * p.width + v * VEC;
                raw_r[k * (VEC == 4 ? 1 : 2)] = ld128_nt(rr);
                if constexpr (VEC == 8) raw_r[2 * k + 1] = ld128_nt(rr + 4);
            }
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int64_t v = l + static_cast<int64_t>(k) * LPR;
        if (live && v < nvec) {
            unpack<TX>(raw_x[k], h[k]);
            if (p.r != nullptr) {
                float fr[VEC];
                unpack<F32>(raw_r[k * (VEC == 4 ? 1 : 2)], fr);
                if constexpr (VEC == 8) unpack<F32>(raw_r[2 * k + 1], fr + 4);
#pragma unroll
                for (int i = 0; i < VEC; ++i) h[k][i] = h[k][i] + fr[i];
                float* ho = p.h_out + row * p.width + v * VEC;
                st128_nt(ho, pack<F32>(h[k]));
                if constexpr (VEC == 8) st128_nt(ho + 4, pack<F32>(h[k] + 4));
            }
#pragma unroll
            for (int i = 0; i < VEC; ++i) ss += h[k][i] * h[k][i];
        }
    }
    ss = group_reduce<(LPR < 64 ? LPR : 64), OpSum>(ss);
    if constexpr (WAVES_PER_ROW > 1) {
        const int wave = threadIdx.x >> 6;
        if ((threadIdx.x & 63) == 0) partial[wave] = ss;
        __syncthreads();
        const int first = (wave / WAVES_PER_ROW) * WAVES_PER_ROW;
        ss = 0.0f;
#pragma unroll
        for (int i = 0; i < WAVES_PER_ROW; ++i) ss += partial[first + i];
    }
    if (!live) return;
    const double inv = 1.0 / sqrt(static_cast<double>(ss) / static_cast<double>(p.width) + static_cast<double>(p.eps));
    SY* yr = static_cast<SY*>(p.y) + row * p.width;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int64_t v = l + static_cast<int64_t>(k) * LPR;
        if (v < nvec) {
            float o[VEC], wv[VEC], bv[VEC];
            if (p.w != nullptr) {
                unpack<F32>(ld128(p.w + v * VEC), wv);
                if constexpr (VEC == 8) unpack<F32>(ld128(p.w + v * VEC + 4), wv + 4);
            }
            if (p.bias != nullptr) {
                unpack<F32>(ld128(p.bias + v * VEC), bv);
                if constexpr (VEC == 8) unpack<F32>(ld128(p.bias + v * VEC + 4), bv + 4);
            }
#pragma unroll
            for (int i = 0; i < VEC; ++i) {
                double t = static_cast<double>(h[k][i]) * inv;
                if (p.w != nullptr) t *= static_cast<double>(wv[i]);
                o[i] = static_cast<float>(t);
                if (p.bias != nullptr) o[i] = o[i] + bv[i];
            }
            if constexpr (sizeof(SY) == 2 && VEC == 4) {
                // four 16-bit outputs: one 64-bit store
                uint2 packed;
                packed.x = pack2<TY>(o[0], o[1]);
                packed.y = pack2<TY>(o[2], o[3]);
                *reinterpret_cast<uint2*>(yr + v * VEC) = packed;
            } else if constexpr (sizeof(SY) == 4 && VEC == 8) {
                st128_nt(yr + v * VEC, pack<TY>(o));
                st128_nt(yr + v * VEC + 4, pack<TY>(o + 4));
            } else {
                st128_nt(yr + v * VEC, pack<TY>(o));
            }
        }
    }
}

// Any width or alignment: one block per row, two passes (the second reads h back from h_out, or x again).
template <typename TX, typename TY>
__global__ __launch_bounds__(kBlock) void rms_norm_any(NormArgs p) {
    using SX = typename TX::storage;
    using SY = typename TY::storage;
    __shared__ float partial[kBlock / 64];
    const int64_t row = blockIdx.x;
    const SX* xr = static_cast<const SX*>(p.x) + row * p.width;
    float ss = 0.0f;
    for (int64_t i = threadIdx.x; i < p.width; i += kBlock) {
        float v = TX::load(xr[i]);
        if (p.r != nullptr) {
            v = v + p.r[row * p.width + i];
            p.h_out[row * p.width + i] = v;
        }
        ss += v * v;
    }
    ss = group_reduce<64, OpSum>(ss);
    if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = 0.0f;
    for (int i = 0; i < kBlock / 64; ++i) ss += partial[i];
    const double inv = 1.0 / sqrt(static_cast<double>(ss) / static_cast<double>(p.width) + static_cast<double>(p.eps));
    SY* yr = static_cast<SY*>(p.y) + row * p.width;
    for (int64_t i = threadIdx.x; i < p.width; i += kBlock) {
        const float v = p.r != nullptr ? p.h_out[row * p.width + i] : TX::load(xr[i]);
        double t = static_cast<double>(v) * inv;
        if (p.w != nullptr) t *= static_cast<double>(p.w[i]);
        float o = static_cast<float>(t);
        if (p.bias != nullptr) o = o + p.bias[i];
        yr[i] = TY::store(o);
    }
}

template <typename TX, typename TY, int LPR>
int go_vec(hipStream_t s, const NormArgs& p, int nv) {
    constexpr int BLOCK = LPR > kBlock ? LPR : kBlock;
    const unsigned grid = static_cast<unsigned>((p.rows + (BLOCK / LPR) - 1) / (BLOCK / LPR));
    switch (nv) {
        case 1: rms_norm_vec<TX, TY, LPR, 1><<<grid, BLOCK, 0, s>>>(p); break;
        case 2: rms_norm_vec<TX, TY, LPR, 2><<<grid, BLOCK, 0, s>>>(p); break;
        case 3: rms_norm_vec<TX, TY, LPR, 3><<<grid, BLOCK, 0, s>>>(p); break;
        case 4: rms_norm_vec<TX, TY, LPR, 4><<<grid, BLOCK, 0, s>>>(p); break;
        case 5: rms_norm_vec<TX, TY, LPR, 5><<<grid, BLOCK, 0, s>>>(p); break;
        case 6: rms_norm_vec<TX, TY, LPR, 6><<<grid, BLOCK, 0, s>>>(p); break;
        case 7: rms_norm_vec<TX, TY, LPR, 7><<<grid, BLOCK, 0, s>>>(p); break;
        default: rms_norm_vec<TX, TY, LPR, 8><<<grid, BLOCK, 0, s>>>(p); break;
    }
    return check_launch("xs_hip_rms_norm");
}

// Lanes per row: the smallest power of two (>= 16) that keeps at most kMaxNv vectors per lane and puts at least
// kTargetWaves waves on the chip (few rows get more lanes each, so the whole chip pulls on HBM), or keeps at most two
// vectors per lane; rows wider than 1024 lanes * kMaxNv vectors take the two-pass kernel.
constexpr int kMaxNv = 8;
constexpr int64_t kTargetWaves = 4096;  // 16 per CU on 256 CUs

template <typename TX, typename TY>
int launch_norm(hipStream_t s, const NormArgs& p) {
    constexpr int VEC = vec_elems<TX>();
    const bool vec = p.width % VEC == 0 && aligned16(p.x) && aligned16(p.y) && (p.r == nullptr || aligned16(p.r)) &&
                     (p.h_out == nullptr || aligned16(p.h_out)) && (p.w == nullptr || aligned16(p.w)) &&
                     (p.bias == nullptr || aligned16(p.bias)) &&
                     (sizeof(typename TY::storage) == 4 || VEC == 8 || reinterpret_cast<uintptr_t>(p.y) % 8 == 0);
    const int64_t nvec = p.width / VEC;
    if (vec) {
        for (int lpr = 16; lpr <= 1024; lpr *= 2) {
            const int64_t nv = (nvec + lpr - 1) / lpr;
            if (nv > kMaxNv) continue;
            if (lpr < 1024 && nv > 2 && p.rows * lpr / 64 < kTargetWaves) continue;
            const int n = static_cast<int>(nv);
            switch (lpr) {
                case 16: return go_vec<TX, TY, 16>(s, p, n);
                case 32: return go_vec<TX, TY, 32>(s, p, n);
                case 64: return go_vec<TX, TY, 64>(s, p, n);
                case 128: return go_vec<TX, TY, 128>(s, p, n);
                case 256: return go_vec<TX, TY, 256>(s, p, n);
                case 512: return go_vec<TX, TY, 512>(s, p, n);
                default: return go_vec<TX, TY, 1024>(s, p, n);
            }
        }
    }
    rms_norm_any<TX, TY><<<static_cast<unsigned>(p.rows), kBlock, 0, s>>>(p);
    return check_launch("xs_hip_rms_norm");
}

template <typename TX>
int dispatch_norm_y(hipStream_t s, const NormArgs& p, xs_dtype y_dtype, const char* what) {
    switch (y_dtype) {
        case XS_F32: return launch_norm<TX, F32>(s, p);
        case XS_F16: return launch_norm<TX, F16>(s, p);
        case XS_BF16: return launch_norm<TX, BF16>(s, p);
        default: return fail(XS_HIP_EINVAL, std::string(what) + ": y must be f32, f16 or bf16, got " + dtype_name(y_dtype));
    }
}

int check_shape(int64_t rows, int64_t width, const char* what) {
    if (rows < 0 || width <= 0 || rows > 0x7fffffffLL)
        return fail(XS_HIP_EINVAL, std::string(what) + ": " + std::to_string(rows) + " rows of width " + std::to_string(width));
    return XS_HIP_OK;
}

}  // namespace
}  // namespace xs_hip

using namespace xs_hip;

extern "C" {

int xs_hip_rms_norm(void* stream, xs_dtype x_dtype, const void* x, const float* w, const float* bias, xs_dtype y_dtype,
                    void* y, int64_t rows, int64_t width, float eps) {
    int rc = check_shape(rows, width, "xs_hip_rms_norm");
    if (rc != XS_HIP_OK || rows == 0) return rc;
    if (x == nullptr || y == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_rms_norm: null buffer");
    const NormArgs p{x, nullptr, w, bias, nullptr, y, rows, width, eps};
    const hipStream_t s = as_stream(stream);
    switch (x_dtype) {
        case XS_F32: return dispatch_norm_y<F32>(s, p, y_dtype, "xs_hip_rms_norm");
        case XS_F16: return dispatch_norm_y<F16>(s, p, y_dtype, "xs_hip_rms_norm");
        case XS_BF16: return dispatch_norm_y<BF16>(s, p, y_dtype, "xs_hip_rms_norm");
        default: return fail(XS_HIP_EINVAL, std::string("xs_hip_rms_norm: x must be f32, f16 or bf16, got ") + dtype_name(x_dtype));
    }
}

int xs_hip_add_rms_norm(void* stream, const float* x, const float* residual, const float* w, const float* bias,
                        float* h_out, xs_dtype y_dtype, void* y, int64_t rows, int64_t width, float eps) {
    int rc = check_shape(rows, width, "xs_hip_add_rms_norm");
    if (rc != XS_HIP_OK || rows == 0) return rc;
    if (x == nullptr || residual == nullptr || h_out == nullptr || y == nullptr)
        return fail(XS_HIP_EINVAL, "xs_hip_add_rms_norm: null buffer");
    const NormArgs p{x, residual, w, bias, h_out, y, rows, width, eps};
    return dispatch_norm_y<F32>(as_stream(stream), p, y_dtype, "xs_hip_add_rms_norm");
}

}  // extern "C"
