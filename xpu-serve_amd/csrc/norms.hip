// Row norms for gfx950: RMSNorm (with or without the residual add folded in), LayerNorm (with an optional shift row
// added first) and the L2 clip.
//
// Semantics: cpu_ref::rms_norm (reference src/backend/cpu_ref/ops.cpp:260-281): inv_rms = 1 / sqrt(sum(x^2) / width +
// eps) and y = x * inv_rms * w, evaluated in f64 and rounded once to f32; the graph spec says "computed in f32, no +1
// offset" (src/graph/graph.h:57). The residual form is the decoder pattern h = add(h, f(rms_norm(h)))
// (src/models/qwen3/qwen3_decoder.cpp:101-102): cpu-ref evaluates h = fl32(x + r) (ops.cpp:201-203) and then the norm;
// here both happen in one pass that also writes h back (the updated residual). LayerNorm is cpu_ref::layer_norm
// (ops.cpp:595-614): mean and the sum of squared deviations in f64, inv = 1 / sqrt(var / width + eps), y =
// fl32((x - mean) * inv * w + b) in f64; the SYCL launcher's shift row (sycl_kernels.h:91-94) is the graph's Add of a
// row before the norm, fl32(x + shift). L2Clip is cpu_ref::l2_clip (ops.cpp:401-412): factor = min(1, threshold /
// (sqrt(sum x^2) + eps)) in f64, y = fl32(x * factor).
//
// Layout: LPR lanes share a row (LPR a power of two, 16..1024), each lane holding up to NV 128-bit vectors of the row
// in registers (vector k of lane l is the row's vector l + k * LPR, so every load instruction of a wave is coalesced).
// Sums (of squares, of values, of squared deviations) are accumulated in f64 as cpu-ref's are -- each f32 square is
// exact in f64 -- per lane, then across the LPR lanes by shuffles inside a wave and one LDS stage across waves; the
// scale is computed in f64 from them and the outputs are formed in f64 in the reference's order and rounded once. The
// row is read from HBM once.
#include <cmath>

#include "common.h"

namespace xs_hip {
namespace {

enum NormMode : int { kRms = 0, kLayer = 1, kL2Clip = 2 };

struct NormArgs {
    const void* x;      // TX [rows, width]
    const float* r;     // f32 residual (RMS) or shift row [width] (LayerNorm), or null
    const float* w;     // f32 [width] or null
    const float* bias;  // f32 [width] or null
    float* h_out;       // f32 [rows, width] (residual form) or null
    void* y;            // TY [rows, width]
    int64_t rows, width;
    float eps;
    float threshold = 0.0f;  // L2 clip
};

// Threads of a workgroup of LPR lanes a row: kBlock when LPR divides it (several rows a workgroup), else one row.
constexpr int norm_block(int lpr) { return lpr < kBlock && kBlock % lpr == 0 ? kBlock : lpr; }

// Sum over the LPR lanes of a row (f64): DPP inside a wave, one LDS stage across the row's waves (an LDS-only barrier:
// the residual stores already issued need not land first). REUSE: `partial` held an earlier sum of this launch, whose
// reads must finish first.
template <int LPR, int BLOCK, bool REUSE = false>
__device__ __forceinline__ double row_sum(double v, double* partial) {
    constexpr int WAVES_PER_ROW = LPR > 64 ? LPR / 64 : 1;
    if constexpr (LPR >= 64) v = wave_sum_f64(v);
    else v = group_sum_f64<LPR>(v);
    if constexpr (WAVES_PER_ROW > 1) {
        const int wave = threadIdx.x >> 6;
        if constexpr (REUSE) lds_barrier();
        if ((threadIdx.x & 63) == 0) partial[wave] = v;
        lds_barrier();
        const int first = (wave / WAVES_PER_ROW) * WAVES_PER_ROW;
        v = 0.0;
#pragma unroll
        for (int i = 0; i < WAVES_PER_ROW; ++i) v += partial[first + i];
    }
    return v;
}

template <typename TX, typename TY, int MODE, int LPR, int NV>
__global__ __launch_bounds__(norm_block(LPR)) void row_norm_vec(NormArgs p) {
    constexpr int BLOCK = norm_block(LPR);
    constexpr int VEC = vec_elems<TX>();
    constexpr int ROWS_PER_BLOCK = BLOCK / LPR;
    using SX = typename TX::storage;
    using SY = typename TY::storage;
    __shared__ double partial[BLOCK / 64];

    const int l = threadIdx.x % LPR;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * ROWS_PER_BLOCK + threadIdx.x / LPR;
    const bool live = row < p.rows;
    const int64_t nvec = p.width / VEC;
    const SX* xr = static_cast<const SX*>(p.x) + row * p.width;

    float h[NV][VEC];
    u32x4 raw_x[NV], raw_r[NV * (VEC == 4 ? 1 : 2)];
    // The weight and bias vectors the outputs need (rows share them: they come from the caches), loaded with the row.
    float wv[NV][VEC], bv[NV][VEC];
    // Issue every load of the row first.
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int64_t v = l + static_cast<int64_t>(k) * LPR;
        if (v < nvec) {
            if (MODE != kL2Clip && p.w != nullptr) {
                unpack<F32>(ld128(p.w + v * VEC), wv[k]);
                if constexpr (VEC == 8) unpack<F32>(ld128(p.w + v * VEC + 4), wv[k] + 4);
            }
            if (MODE != kL2Clip && p.bias != nullptr) {
                unpack<F32>(ld128(p.bias + v * VEC), bv[k]);
                if constexpr (VEC == 8) unpack<F32>(ld128(p.bias + v * VEC + 4), bv[k] + 4);
            }
        }
        if (live && v < nvec) {
            raw_x[k] = ld128_nt(xr + v * VEC);
            if (p.r != nullptr) {
                // the residual row (RMS) or the shift row shared by every row (LayerNorm)
                const float* rr = p.r + (MODE == kRms ? row * p.width : 0) + v * VEC;
                raw_r[k * (VEC == 4 ? 1 : 2)] = ld128_nt(rr);
                if constexpr (VEC == 8) raw_r[2 * k + 1] = ld128_nt(rr + 4);
            }
        }
    }
    double sum = 0.0;
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
                if (MODE == kRms && p.h_out != nullptr) {
                    float* ho = p.h_out + row * p.width + v * VEC;
                    st128_nt(ho, pack<F32>(h[k]));
                    if constexpr (VEC == 8) st128_nt(ho + 4, pack<F32>(h[k] + 4));
                }
            }
#pragma unroll
            for (int i = 0; i < VEC; ++i) {
                const double d = h[k][i];
                sum += MODE == kLayer ? d : d * d;
            }
        }
    }
    sum = row_sum<LPR, BLOCK>(sum, partial);
    const double width = static_cast<double>(p.width);
    double mean = 0.0, scale;
    if constexpr (MODE == kLayer) {
        mean = sum / width;
        double dev = 0.0;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int64_t v = l + static_cast<int64_t>(k) * LPR;
            if (live && v < nvec) {
#pragma unroll
                for (int i = 0; i < VEC; ++i) {
                    const double d = static_cast<double>(h[k][i]) - mean;
                    dev += d * d;
                }
            }
        }
        dev = row_sum<LPR, BLOCK, true>(dev, partial);
        scale = 1.0 / sqrt(dev / width + static_cast<double>(p.eps));
    } else if constexpr (MODE == kL2Clip) {
        const double f = static_cast<double>(p.threshold) / (sqrt(sum) + static_cast<double>(p.eps));
        scale = f < 1.0 ? f : 1.0;
    } else {
        scale = 1.0 / sqrt(sum / width + static_cast<double>(p.eps));
    }
    if (!live) return;
    SY* yr = static_cast<SY*>(p.y) + row * p.width;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int64_t v = l + static_cast<int64_t>(k) * LPR;
        if (v < nvec) {
            float o[VEC];
#pragma unroll
            for (int i = 0; i < VEC; ++i) {
                if constexpr (MODE == kLayer) {
                    double t = (static_cast<double>(h[k][i]) - mean) * scale;
                    if (p.w != nullptr) t *= static_cast<double>(wv[k][i]);
                    if (p.bias != nullptr) t += static_cast<double>(bv[k][i]);
                    o[i] = static_cast<float>(t);
                } else {
                    double t = static_cast<double>(h[k][i]) * scale;
                    if (MODE == kRms && p.w != nullptr) t *= static_cast<double>(wv[k][i]);
                    o[i] = static_cast<float>(t);
                    if (MODE == kRms && p.bias != nullptr) o[i] = o[i] + bv[k][i];
                }
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

// Any width or alignment: one block per row, two or three passes (later passes read h back from h_out, or x again).
template <typename TX, typename TY, int MODE>
__global__ __launch_bounds__(kBlock) void row_norm_any(NormArgs p) {
    using SX = typename TX::storage;
    using SY = typename TY::storage;
    __shared__ double partial[kBlock / 64];
    const int64_t row = blockIdx.x;
    const SX* xr = static_cast<const SX*>(p.x) + row * p.width;
    // the row's value at i after the residual add or the shift
    auto value = [&](int64_t i) {
        float v = TX::load(xr[i]);
        if (p.r != nullptr) v = v + (MODE == kRms ? p.r[row * p.width + i] : p.r[i]);
        return v;
    };
    double sum = 0.0;
    for (int64_t i = threadIdx.x; i < p.width; i += kBlock) {
        const float v = value(i);
        if (MODE == kRms && p.r != nullptr && p.h_out != nullptr) p.h_out[row * p.width + i] = v;
        sum += MODE == kLayer ? static_cast<double>(v) : static_cast<double>(v) * v;
    }
    sum = row_sum<kBlock, kBlock>(sum, partial);
    const double width = static_cast<double>(p.width);
    double mean = 0.0, scale;
    if constexpr (MODE == kLayer) {
        mean = sum / width;
        double dev = 0.0;
        for (int64_t i = threadIdx.x; i < p.width; i += kBlock) {
            const double d = static_cast<double>(value(i)) - mean;
            dev += d * d;
        }
        dev = row_sum<kBlock, kBlock, true>(dev, partial);
        scale = 1.0 / sqrt(dev / width + static_cast<double>(p.eps));
    } else if constexpr (MODE == kL2Clip) {
        const double f = static_cast<double>(p.threshold) / (sqrt(sum) + static_cast<double>(p.eps));
        scale = f < 1.0 ? f : 1.0;
    } else {
        scale = 1.0 / sqrt(sum / width + static_cast<double>(p.eps));
    }
    SY* yr = static_cast<SY*>(p.y) + row * p.width;
    for (int64_t i = threadIdx.x; i < p.width; i += kBlock) {
        const float v = value(i);
        float o;
        if constexpr (MODE == kLayer) {
            double t = (static_cast<double>(v) - mean) * scale;
            if (p.w != nullptr) t *= static_cast<double>(p.w[i]);
            if (p.bias != nullptr) t += static_cast<double>(p.bias[i]);
            o = static_cast<float>(t);
        } else {
            double t = static_cast<double>(v) * scale;
            if (MODE == kRms && p.w != nullptr) t *= static_cast<double>(p.w[i]);
            o = static_cast<float>(t);
            if (MODE == kRms && p.bias != nullptr) o = o + p.bias[i];
        }
        yr[i] = TY::store(o);
    }
}

template <typename TX, typename TY, int MODE, int LPR, int NV>
int go_vec_nv(hipStream_t s, const NormArgs& p, const char* what) {
    constexpr int BLOCK = norm_block(LPR);
    const unsigned grid = static_cast<unsigned>((p.rows + (BLOCK / LPR) - 1) / (BLOCK / LPR));
    row_norm_vec<TX, TY, MODE, LPR, NV><<<grid, BLOCK, 0, s>>>(p);
    return check_launch(what);
}

template <typename TX, typename TY, int MODE, int LPR>
int go_vec(hipStream_t s, const NormArgs& p, int nv, const char* what) {
    constexpr int BLOCK = norm_block(LPR);
    const unsigned grid = static_cast<unsigned>((p.rows + (BLOCK / LPR) - 1) / (BLOCK / LPR));
    switch (nv) {
        case 1: row_norm_vec<TX, TY, MODE, LPR, 1><<<grid, BLOCK, 0, s>>>(p); break;
        case 2: row_norm_vec<TX, TY, MODE, LPR, 2><<<grid, BLOCK, 0, s>>>(p); break;
        case 3: row_norm_vec<TX, TY, MODE, LPR, 3><<<grid, BLOCK, 0, s>>>(p); break;
        case 4: row_norm_vec<TX, TY, MODE, LPR, 4><<<grid, BLOCK, 0, s>>>(p); break;
        case 5: row_norm_vec<TX, TY, MODE, LPR, 5><<<grid, BLOCK, 0, s>>>(p); break;
        case 6: row_norm_vec<TX, TY, MODE, LPR, 6><<<grid, BLOCK, 0, s>>>(p); break;
        case 7: row_norm_vec<TX, TY, MODE, LPR, 7><<<grid, BLOCK, 0, s>>>(p); break;
        default: row_norm_vec<TX, TY, MODE, LPR, 8><<<grid, BLOCK, 0, s>>>(p); break;
    }
    return check_launch(what);
}

// Two vectors per lane in `waves` whole waves per row (a row of exactly 128 * waves vectors, waves not a power of two):
// every lane holds a full share of the row, which the power-of-two layouts leave partly idle (640 vectors: 5 waves
// instead of 8 waves of which 3 hold one vector a lane; measured 4% faster on MI355X at 512 x 2560 f32).
template <typename TX, typename TY, int MODE>
int go_exact(hipStream_t s, const NormArgs& p, int waves, const char* what) {
    switch (waves) {
        case 3: return go_vec_nv<TX, TY, MODE, 192, 2>(s, p, what);
        case 5: return go_vec_nv<TX, TY, MODE, 320, 2>(s, p, what);
        case 6: return go_vec_nv<TX, TY, MODE, 384, 2>(s, p, what);
        case 7: return go_vec_nv<TX, TY, MODE, 448, 2>(s, p, what);
        case 9: return go_vec_nv<TX, TY, MODE, 576, 2>(s, p, what);
        case 10: return go_vec_nv<TX, TY, MODE, 640, 2>(s, p, what);
        case 11: return go_vec_nv<TX, TY, MODE, 704, 2>(s, p, what);
        case 12: return go_vec_nv<TX, TY, MODE, 768, 2>(s, p, what);
        case 13: return go_vec_nv<TX, TY, MODE, 832, 2>(s, p, what);
        case 14: return go_vec_nv<TX, TY, MODE, 896, 2>(s, p, what);
        case 15: return go_vec_nv<TX, TY, MODE, 960, 2>(s, p, what);
        default: return -1;
    }
}

// Lanes per row: the smallest power of two (>= 16) that keeps at most kMaxNv vectors per lane and puts at least
// kTargetWaves waves on the chip (few rows get more lanes each, so the whole chip pulls on HBM), or keeps at most two
// vectors per lane; rows wider than 1024 lanes * kMaxNv vectors take the two-pass kernel.
constexpr int kMaxNv = 8;
constexpr int64_t kTargetWaves = 4096;  // 16 per CU on 256 CUs

template <typename TX, typename TY, int MODE>
int launch_norm(hipStream_t s, const NormArgs& p, const char* what) {
    constexpr int VEC = vec_elems<TX>();
    const bool vec = p.width % VEC == 0 && aligned16(p.x) && aligned16(p.y) && (p.r == nullptr || aligned16(p.r)) &&
                     (p.h_out == nullptr || aligned16(p.h_out)) && (p.w == nullptr || aligned16(p.w)) &&
                     (p.bias == nullptr || aligned16(p.bias)) &&
                     (sizeof(typename TY::storage) == 4 || VEC == 8 || reinterpret_cast<uintptr_t>(p.y) % 8 == 0);
    const int64_t nvec = p.width / VEC;
    if (vec) {
        if (nvec % 128 == 0 && nvec >= 3 * 128 && nvec < 16 * 128) {
            const int rc = go_exact<TX, TY, MODE>(s, p, static_cast<int>(nvec / 128), what);
            if (rc >= 0) return rc;
        }
        for (int lpr = 16; lpr <= 1024; lpr *= 2) {
            const int64_t nv = (nvec + lpr - 1) / lpr;
            if (nv > kMaxNv) continue;
            if (lpr < 1024 && nv > 2 && p.rows * lpr / 64 < kTargetWaves) continue;
            const int n = static_cast<int>(nv);
            switch (lpr) {
                case 16: return go_vec<TX, TY, MODE, 16>(s, p, n, what);
                case 32: return go_vec<TX, TY, MODE, 32>(s, p, n, what);
                case 64: return go_vec<TX, TY, MODE, 64>(s, p, n, what);
                case 128: return go_vec<TX, TY, MODE, 128>(s, p, n, what);
                case 256: return go_vec<TX, TY, MODE, 256>(s, p, n, what);
                case 512: return go_vec<TX, TY, MODE, 512>(s, p, n, what);
                default: return go_vec<TX, TY, MODE, 1024>(s, p, n, what);
            }
        }
    }
    row_norm_any<TX, TY, MODE><<<static_cast<unsigned>(p.rows), kBlock, 0, s>>>(p);
    return check_launch(what);
}

template <typename TX, int MODE>
int dispatch_norm_y(hipStream_t s, const NormArgs& p, xs_dtype y_dtype, const char* what) {
    switch (y_dtype) {
        case XS_F32: return launch_norm<TX, F32, MODE>(s, p, what);
        case XS_F16: return launch_norm<TX, F16, MODE>(s, p, what);
        case XS_BF16: return launch_norm<TX, BF16, MODE>(s, p, what);
        default: return fail(XS_HIP_EINVAL, std::string(what) + ": y must be f32, f16 or bf16, got " + dtype_name(y_dtype));
    }
}

template <int MODE>
int dispatch_norm(hipStream_t s, const NormArgs& p, xs_dtype x_dtype, xs_dtype y_dtype, const char* what) {
    switch (x_dtype) {
        case XS_F32: return dispatch_norm_y<F32, MODE>(s, p, y_dtype, what);
        case XS_F16: return dispatch_norm_y<F16, MODE>(s, p, y_dtype, what);
        case XS_BF16: return dispatch_norm_y<BF16, MODE>(s, p, y_dtype, what);
        default:
            return fail(XS_HIP_EINVAL, std::string(what) + ": x must be f32, f16 or bf16, got " + dtype_name(x_dtype));
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
    return dispatch_norm<kRms>(as_stream(stream), p, x_dtype, y_dtype, "xs_hip_rms_norm");
}

int xs_hip_add_rms_norm(void* stream, const float* x, const float* residual, const float* w, const float* bias,
                        float* h_out, xs_dtype y_dtype, void* y, int64_t rows, int64_t width, float eps) {
    int rc = check_shape(rows, width, "xs_hip_add_rms_norm");
    if (rc != XS_HIP_OK || rows == 0) return rc;
    if (x == nullptr || residual == nullptr || h_out == nullptr || y == nullptr)
        return fail(XS_HIP_EINVAL, "xs_hip_add_rms_norm: null buffer");
    const NormArgs p{x, residual, w, bias, h_out, y, rows, width, eps};
    return dispatch_norm_y<F32, kRms>(as_stream(stream), p, y_dtype, "xs_hip_add_rms_norm");
}

int xs_hip_layer_norm(void* stream, xs_dtype x_dtype, const void* x, const float* shift, const float* w, const float* b,
                      xs_dtype y_dtype, void* y, int64_t rows, int64_t width, float eps) {
    int rc = check_shape(rows, width, "xs_hip_layer_norm");
    if (rc != XS_HIP_OK || rows == 0) return rc;
    if (x == nullptr || y == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_layer_norm: null buffer");
    const NormArgs p{x, shift, w, b, nullptr, y, rows, width, eps};
    return dispatch_norm<kLayer>(as_stream(stream), p, x_dtype, y_dtype, "xs_hip_layer_norm");
}

int xs_hip_l2_clip(void* stream, const float* x, float* y, int64_t rows, int64_t width, float threshold, float eps) {
    int rc = check_shape(rows, width, "xs_hip_l2_clip");
    if (rc != XS_HIP_OK || rows == 0) return rc;
    if (x == nullptr || y == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_l2_clip: null buffer");
    NormArgs p{x, nullptr, nullptr, nullptr, nullptr, y, rows, width, eps};
    p.threshold = threshold;
    return dispatch_norm_y<F32, kL2Clip>(as_stream(stream), p, XS_F32, "xs_hip_l2_clip");
}

}  // extern "C"
