// ORACLE -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.
//
// A CPU restatement of the reference CPU path (cpu-ref) of xpu-serve for the elementwise, broadcast and reduction ops
// that the gfx950 kernels of this repository implement. Only tests/, __graft_entry__.smoke() and bench.py's
// cpu_baseline leg may load it, and only as the checker (or the timed CPU baseline), never as the thing measured on
// the GPU or shipped.
//
// Every function restates one reference function (file:line into the reference tree) on raw f32 arrays: the reference
// normalises float operands to f32 before each op (src/backend/cpu_ref/cpu_backend.cpp:62-70), runs the op in f32 or
// f64 as written there, and returns f32; rounding to an f16/bf16 output is a separate narrowing (src/util/half.{h,cpp}),
// restated here too. Built with g++ and no fast-math or FMA contraction (x86-64 baseline has no FMA), so each
// expression rounds where the reference's does.
//
// How each function is pinned (the test that pins it, in tests/test_oracle.py):
//   ora_f16/bf16 conversions   exhaustive f16 round trip, RNE ties and saturation KATs of tests/unit/test_half.cpp:9-38,
//                              bf16 KAT 39.191836 -> 39.25; goldens from the compiled reference (oracle/_ref)
//   ora_binary                 brute force multi-index broadcast on the reference's shape cases; goldens
//   ora_unary                  closed forms at special points and an f64 evaluation; goldens
//   ora_unary_op               closed forms (tanh/softcap/softplus identities, clamp bounds, NaN), goldens
//   ora_rms_norm               f64 evaluation + invariants (unit rms of the output); goldens
//   ora_layer_norm             invariants (zero mean, unit variance of the unweighted output), goldens
//   ora_l2_clip                invariants (output norm = min(|x|, threshold) to rounding), goldens
//   ora_reduce_sum             exact sums of small integers, numpy f64 sum, goldens
//   ora_attention              one-key and equal-key closed forms, a numpy f64 evaluation, window/causal ranges by
//                              brute force; goldens
//   ora_softmax                f64 evaluation, sum to 1, masked = 0, shift invariance; goldens
//   ora_topk                   the reference's tie KATs (tests/unit/backend/moe_ops_cases.h:76-122); sort brute force
//   ora_rope                   norm preservation per pair, position 0 identity, inv_freq 0 identity, the planted
//                              interleaved-layout control (tests/unit/backend/cpu_ops.cpp:228-251); goldens
//   ora_rope_inv_freq          goldens of blocks::rope_inv_freq; closed form theta^(-2i/d) at exact powers
//   ora_quantize_kv_*          |code| <= 127, round-trip error <= scale / 2, zero rows, goldens (bit-exact)
//   ora_turbo_*                the reference's own fixtures (tests/fixtures/quant/turbo: codes and f16 norm of 43 rows
//                              at 4, 3 and 2 bits, from the format's published implementation), nearest-centroid and
//                              norm-restoring invariants, the rotation's orthogonality and inverse, an f64 WHT by the
//                              Hadamard matrix, the compiled reference (oracle/_ref)
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <numeric>
#include <vector>

namespace {

// ---- src/util/half.cpp:10-56 and src/util/half.h:12-25 ----------------------------------------------------------

float f16_to_f32(uint16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
    const uint32_t exponent = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    uint32_t bits;
    if (exponent == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            // A subnormal: shift the mantissa up until its leading one reaches the implicit bit.
            int shift = 0;
            while ((mant & 0x400u) == 0) {
                mant <<= 1;
                ++shift;
            }
            bits = sign | static_cast<uint32_t>(127 - 15 + 1 - shift) << 23 | (mant & 0x3ffu) << 13;
        }
    } else if (exponent == 0x1f) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | (exponent + (127 - 15)) << 23 | (mant << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

uint16_t f32_to_f16(float f) {
    uint32_t bits;
    std::memcpy(&bits, &f, 4);
    const uint16_t sign = static_cast<uint16_t>((bits >> 16) & 0x8000u);
    const uint32_t mag = bits & 0x7fffffffu;
    if (mag > 0x7f800000u) return static_cast<uint16_t>(sign | 0x7e00u);  // NaN
    if (mag >= 0x477ff000u) return static_cast<uint16_t>(sign | 0x7c00u);  // 65520 and up round to inf
    if (mag < 0x38800000u) {                                              // f16 subnormal or zero
        if (mag < 0x33000000u) return sign;                               // below half the smallest subnormal
        const uint32_t e = mag >> 23;
        const uint32_t m = (mag & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126 - e;  // 14..24
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1);
        const uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (q & 1u))) ++q;
        return static_cast<uint16_t>(sign | q);
    }
    // Normal: rebias the exponent and round the 13 dropped bits to nearest even.
    const uint32_t r = mag + 0xfffu + ((mag >> 13) & 1u);
    return static_cast<uint16_t>(sign | ((r - 0x38000000u) >> 13));
}

float bf16_to_f32(uint16_t v) {
    const uint32_t bits = static_cast<uint32_t>(v) << 16;
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

uint16_t f32_to_bf16(float f) {
    uint32_t bits;
    std::memcpy(&bits, &f, 4);
    if ((bits & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((bits >> 16) | 0x0040u);
    return static_cast<uint16_t>((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);
}

// ---- src/backend/cpu_ref/ops.cpp:42-93 ---------------------------------------------------------------------------

// Right-aligned numpy broadcast; false when the shapes do not broadcast.
bool broadcast_shape(const int64_t* a, int ra, const int64_t* b, int rb, std::vector<int64_t>& out) {
    const int rank = std::max(ra, rb);
    out.assign(static_cast<size_t>(rank), 0);
    for (int i = 0; i < rank; ++i) {
        const int64_t da = i < rank - ra ? 1 : a[i - (rank - ra)];
        const int64_t db = i < rank - rb ? 1 : b[i - (rank - rb)];
        if (!(da == db || da == 1 || db == 1)) return false;
        out[static_cast<size_t>(i)] = da == 1 ? db : da;
    }
    return true;
}

std::vector<int64_t> broadcast_strides(const int64_t* shape, int r, const std::vector<int64_t>& out) {
    std::vector<int64_t> strides(out.size(), 0);
    int64_t stride = 1;
    for (int i = r - 1; i >= 0; --i) {
        const size_t o = static_cast<size_t>(i) + (out.size() - static_cast<size_t>(r));
        strides[o] = shape[i] == 1 ? 0 : stride;
        stride *= shape[i];
    }
    return strides;
}

double act_f64(int act, double d) {
    switch (act) {
        case 2: {  // GeluTanh, ops.cpp:220-226
            const double inner = std::sqrt(2.0 / 3.14159265358979323846) * (d + 0.044715 * d * d * d);
            return 0.5 * d * (1.0 + std::tanh(inner));
        }
        case 4: return 1.0 / (1.0 + std::exp(-d));  // Sigmoid, ops.cpp:237-239
        case 5: return d / (1.0 + std::exp(-d));    // Silu, ops.cpp:242-247
        case 8: return 0.5 * d * (1.0 + std::erf(d / 1.41421356237309504880));  // Gelu, ops.cpp:228-233
        default: return std::numeric_limits<double>::quiet_NaN();
    }
}

int64_t pos_at(const void* p, int is_i64, int64_t i) {
    return is_i64 ? static_cast<const int64_t*>(p)[i] : static_cast<const int32_t*>(p)[i];
}

}  // namespace

extern "C" {

// ---- dtype conversions -----------------------------------------------------------------------------------------

float ora_f16_to_f32(uint16_t h) { return f16_to_f32(h); }
uint16_t ora_f32_to_f16(float f) { return f32_to_f16(f); }
float ora_bf16_to_f32(uint16_t h) { return bf16_to_f32(h); }
uint16_t ora_f32_to_bf16(float f) { return f32_to_bf16(f); }

// dtype: 0 f32, 1 f16, 2 bf16 (the reference's DType values). HostTensor::to_f32 (src/tensor/tensor.cpp:58-84).
void ora_widen(int dtype, const void* src, float* dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        if (dtype == 0) dst[i] = static_cast<const float*>(src)[i];
        else if (dtype == 1) dst[i] = f16_to_f32(static_cast<const uint16_t*>(src)[i]);
        else dst[i] = bf16_to_f32(static_cast<const uint16_t*>(src)[i]);
    }
}

void ora_narrow(int dtype, const float* src, void* dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        if (dtype == 0) static_cast<float*>(dst)[i] = src[i];
        else if (dtype == 1) static_cast<uint16_t*>(dst)[i] = f32_to_f16(src[i]);
        else static_cast<uint16_t*>(dst)[i] = f32_to_bf16(src[i]);
    }
}

// ---- elementwise ---------------------------------------------------------------------------------------------------

// cpu_ref::map_binary (ops.cpp:68-93) with add / mul / div (ops.cpp:201-207, 401-403): op 0 add, 1 mul, 2 div.
// Returns the number of output elements, or -1 when the shapes do not broadcast. `out` holds numel(out) floats.
int64_t ora_binary(int op, const float* a, const int64_t* a_shape, int a_rank, const float* b, const int64_t* b_shape,
                   int b_rank, float* out) {
    std::vector<int64_t> shape;
    if (!broadcast_shape(a_shape, a_rank, b_shape, b_rank, shape)) return -1;
    const std::vector<int64_t> sa = broadcast_strides(a_shape, a_rank, shape);
    const std::vector<int64_t> sb = broadcast_strides(b_shape, b_rank, shape);
    int64_t n = 1;
    for (int64_t d : shape) n *= d;
    std::vector<int64_t> index(shape.size(), 0);
    int64_t oa = 0, ob = 0;
    for (int64_t i = 0; i < n; ++i) {
        const float x = a[oa], y = b[ob];
        out[i] = op == 0 ? x + y : op == 1 ? x * y : x / y;
        for (size_t d = shape.size(); d-- > 0;) {  // odometer step
            oa += sa[d];
            ob += sb[d];
            if (++index[d] < shape[d]) break;
            oa -= sa[d] * shape[d];
            ob -= sb[d] * shape[d];
            index[d] = 0;
        }
    }
    return n;
}

// cpu_ref::scale (ops.cpp:209-211).
void ora_scale(const float* x, float factor, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = x[i] * factor;
}

// cpu_ref::silu / sigmoid / gelu_tanh / gelu (ops.cpp:216-247): f64 evaluation rounded once. act uses the
// UnaryOp values (2 GeluTanh, 4 Sigmoid, 5 Silu, 8 Gelu).
void ora_unary(int act, const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = static_cast<float>(act_f64(act, static_cast<double>(x[i])));
}

// The whole unary family by UnaryOp value (sycl_kernels.h:21) with the op's parameters: cpu_ref::scale, tanh,
// gelu_tanh, softcap, sigmoid, silu, softplus, clamp, gelu (ops.cpp:209-258).
void ora_unary_op(int op, const float* x, float* y, int64_t n, float a, float b) {
    for (int64_t i = 0; i < n; ++i) {
        const float v = x[i];
        switch (op) {
            case 0: y[i] = v * a; break;                                                       // Scale, ops.cpp:209-211
            case 1: y[i] = static_cast<float>(std::tanh(static_cast<double>(v))); break;      // Tanh, :213-215
            case 3:                                                                            // Softcap, :232-236
                y[i] = static_cast<float>(static_cast<double>(a) * std::tanh(static_cast<double>(v) / a));
                break;
            case 6: {                                                                          // Softplus, :249-254
                const double d = v;
                y[i] = static_cast<float>(d > 20.0 ? d : std::log1p(std::exp(d)));
                break;
            }
            case 7: y[i] = std::min(std::max(v, a), b); break;                                // Clamp, :256-258
            default: y[i] = static_cast<float>(act_f64(op, static_cast<double>(v))); break;  // 2, 4, 5, 8
        }
    }
}

// The gated-MLP activation as cpu-ref evaluates Mul(Act(Add(x, bias)), b) node by node on 2-D row-strided f32
// operands (blocks.cpp:23-27; ops.cpp:201-247): g = fl32(x + bias[c]) (no add without bias), a = fl32(act_f64(g)),
// y = fl32(a * b). Strides in elements; y is [rows, cols] contiguous.
void ora_act_bias_mul(int act, const float* x, int64_t x_stride, const float* b, int64_t b_stride, const float* bias,
                      float* y, int64_t rows, int64_t cols) {
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t c = 0; c < cols; ++c) {
            float g = x[r * x_stride + c];
            if (bias != nullptr) g = g + bias[c];
            const float a = static_cast<float>(act_f64(act, static_cast<double>(g)));
            y[r * cols + c] = a * b[r * b_stride + c];
        }
    }
}

// ---- row reductions --------------------------------------------------------------------------------------------

// cpu_ref::rms_norm (ops.cpp:260-281); weight may be null.
void ora_rms_norm(const float* x, const float* weight, float eps, float* y, int64_t rows, int64_t width) {
    for (int64_t row = 0; row < rows; ++row) {
        const float* in = x + row * width;
        float* o = y + row * width;
        double sum_sq = 0;
        for (int64_t i = 0; i < width; ++i) sum_sq += static_cast<double>(in[i]) * in[i];
        const double inv_rms = 1.0 / std::sqrt(sum_sq / static_cast<double>(width) + eps);
        for (int64_t i = 0; i < width; ++i) {
            const double w = weight != nullptr ? weight[i] : 1.0;
            o[i] = static_cast<float>(in[i] * inv_rms * w);
        }
    }
}

// h = x + residual (cpu_ref::add, f32) then y = rms_norm(h, weight) (+ bias, a following f32 Add).
void ora_add_rms_norm(const float* x, const float* residual, const float* weight, const float* bias, float eps,
                      float* h, float* y, int64_t rows, int64_t width) {
    const int64_t n = rows * width;
    for (int64_t i = 0; i < n; ++i) h[i] = x[i] + residual[i];
    ora_rms_norm(h, weight, eps, y, rows, width);
    if (bias != nullptr)
        for (int64_t i = 0; i < n; ++i) y[i] = y[i] + bias[i % width];
}

// cpu_ref::layer_norm (ops.cpp:595-614) of h = x + shift (a cpu_ref::add of a row first, f32; shift may be null);
// weight and bias may be null (1 and 0: the same f64 value as the reference's expression with w = 1, b = 0).
void ora_layer_norm(const float* x, const float* shift, const float* weight, const float* bias, float eps, float* y,
                    int64_t rows, int64_t width) {
    std::vector<float> h(static_cast<size_t>(width));
    for (int64_t r = 0; r < rows; ++r) {
        const float* xr = x + r * width;
        for (int64_t i = 0; i < width; ++i) h[i] = shift != nullptr ? xr[i] + shift[i] : xr[i];
        double mean = 0;
        for (int64_t i = 0; i < width; ++i) mean += h[i];
        mean /= static_cast<double>(width);
        double var = 0;
        for (int64_t i = 0; i < width; ++i) var += (h[i] - mean) * (h[i] - mean);
        const double inv = 1.0 / std::sqrt(var / static_cast<double>(width) + eps);
        for (int64_t i = 0; i < width; ++i) {
            const double w = weight != nullptr ? weight[i] : 1.0;
            const double b = bias != nullptr ? bias[i] : 0.0;
            y[r * width + i] = static_cast<float>((h[i] - mean) * inv * w + b);
        }
    }
}

// cpu_ref::l2_clip (ops.cpp:401-412), with cpu-ref's four-way f64 dot (ops.cpp:96-108).
void ora_l2_clip(const float* x, float* y, int64_t rows, int64_t width, float threshold, float eps) {
    for (int64_t r = 0; r < rows; ++r) {
        const float* in = x + r * width;
        double s0 = 0, s1 = 0, s2 = 0, s3 = 0;
        int64_t i = 0;
        for (; i + 4 <= width; i += 4) {
            s0 += static_cast<double>(in[i]) * in[i];
            s1 += static_cast<double>(in[i + 1]) * in[i + 1];
            s2 += static_cast<double>(in[i + 2]) * in[i + 2];
            s3 += static_cast<double>(in[i + 3]) * in[i + 3];
        }
        for (; i < width; ++i) s0 += static_cast<double>(in[i]) * in[i];
        const double dot = (s0 + s1) + (s2 + s3);
        const double factor = std::min(1.0, threshold / (std::sqrt(dot) + eps));
        for (int64_t k = 0; k < width; ++k) y[r * width + k] = static_cast<float>(in[k] * factor);
    }
}

// cpu_ref::reduce_sum (ops.cpp:686-705): x [outer, dim, inner] -> y [outer, inner], f64 accumulation.
void ora_reduce_sum(const float* x, float* y, int64_t outer, int64_t dim, int64_t inner) {
    for (int64_t o = 0; o < outer; ++o) {
        for (int64_t i = 0; i < inner; ++i) {
            double sum = 0;
            for (int64_t d = 0; d < dim; ++d) sum += x[(o * dim + d) * inner + i];
            y[o * inner + i] = static_cast<float>(sum);
        }
    }
}

// cpu_ref::attention / attend_one (ops.cpp:113-156, 535-594) for causal or full attention with an optional sliding
// window and softcap (no key bias, groups, blocks, relative bias or anchors): q [T, Hq, D], k and v [N, Hkv, D] f32
// (for an int8 cache, the values it stores), out [T, Hq, D]. Scores, softmax and the weighted sum in f64, the dot
// product with cpu-ref's four partial sums (ops.cpp:96-108).
void ora_attention(const float* q, const float* k, const float* v, float* out, int64_t tokens, int64_t q_heads,
                   int64_t kv_heads, int64_t head_dim, int64_t kv_len, float scale, float softcap, int64_t window,
                   int causal) {
    const int64_t per_kv = q_heads / kv_heads;
    std::vector<double> scores(static_cast<size_t>(kv_len)), acc(static_cast<size_t>(head_dim));
    for (int64_t t = 0; t < tokens; ++t) {
        const int64_t pos = kv_len - tokens + t;
        int64_t first = window > 0 ? std::max<int64_t>(0, pos - window + 1) : 0;
        int64_t last = causal ? pos : kv_len - 1;
        if (window > 0) last = std::min(last, pos + window - 1);
        for (int64_t h = 0; h < q_heads; ++h) {
            const float* qh = q + (t * q_heads + h) * head_dim;
            const int64_t kvh = h / per_kv;
            double max_score = -std::numeric_limits<double>::infinity();
            for (int64_t j = first; j <= last; ++j) {
                const float* kj = k + (j * kv_heads + kvh) * head_dim;
                double s0 = 0, s1 = 0, s2 = 0, s3 = 0;
                int64_t i = 0;
                for (; i + 4 <= head_dim; i += 4) {
                    s0 += static_cast<double>(qh[i]) * kj[i];
                    s1 += static_cast<double>(qh[i + 1]) * kj[i + 1];
                    s2 += static_cast<double>(qh[i + 2]) * kj[i + 2];
                    s3 += static_cast<double>(qh[i + 3]) * kj[i + 3];
                }
                for (; i < head_dim; ++i) s0 += static_cast<double>(qh[i]) * kj[i];
                double sc = scale * ((s0 + s1) + (s2 + s3));
                if (softcap > 0.0f) sc = softcap * std::tanh(sc / softcap);
                scores[static_cast<size_t>(j)] = sc;
                max_score = std::max(max_score, sc);
            }
            double denom = 0;
            for (int64_t j = first; j <= last; ++j) {
                scores[static_cast<size_t>(j)] = std::exp(scores[static_cast<size_t>(j)] - max_score);
                denom += scores[static_cast<size_t>(j)];
            }
            std::fill(acc.begin(), acc.end(), 0.0);
            for (int64_t j = first; j <= last; ++j) {
                const double p = scores[static_cast<size_t>(j)] / denom;
                const float* vj = v + (j * kv_heads + kvh) * head_dim;
                for (int64_t d = 0; d < head_dim; ++d) acc[static_cast<size_t>(d)] += p * vj[d];
            }
            float* o = out + (t * q_heads + h) * head_dim;
            for (int64_t d = 0; d < head_dim; ++d) o[d] = static_cast<float>(acc[static_cast<size_t>(d)]);
        }
    }
}

// cpu_ref::softmax (ops.cpp:644-661).
void ora_softmax(const float* x, float* y, int64_t rows, int64_t width) {
    for (int64_t r = 0; r < rows; ++r) {
        const float* in = x + r * width;
        float* o = y + r * width;
        double peak = in[0];
        for (int64_t i = 1; i < width; ++i) peak = std::max(peak, static_cast<double>(in[i]));
        double sum = 0;
        for (int64_t i = 0; i < width; ++i) sum += std::exp(static_cast<double>(in[i]) - peak);
        for (int64_t i = 0; i < width; ++i) o[i] = static_cast<float>(std::exp(static_cast<double>(in[i]) - peak) / sum);
    }
}

// Softmax(Add(Scale(x, scale), mask)) with mask 0 for key < valid_len[row] (or valid_all) and -inf after.
void ora_softmax_masked(const float* x, float* y, int64_t rows, int64_t width, float scale, const int64_t* valid_len,
                        int64_t valid_all) {
    std::vector<float> s(static_cast<size_t>(width));
    for (int64_t r = 0; r < rows; ++r) {
        const int64_t valid = valid_len != nullptr ? valid_len[r] : valid_all;
        for (int64_t i = 0; i < width; ++i) {
            const float v = x[r * width + i] * scale;
            const float mask = i < valid ? 0.0f : -std::numeric_limits<float>::infinity();
            s[static_cast<size_t>(i)] = v + mask;
        }
        ora_softmax(s.data(), y + r * width, 1, width);
    }
}

// cpu_ref::topk (ops.cpp:663-684): ties keep the lower index first.
void ora_topk(const float* x, float* values, int32_t* indices, int64_t rows, int64_t width, int64_t k) {
    std::vector<int32_t> order(static_cast<size_t>(width));
    for (int64_t r = 0; r < rows; ++r) {
        const float* in = x + r * width;
        std::iota(order.begin(), order.end(), 0);
        std::partial_sort(order.begin(), order.begin() + k, order.end(),
                          [&](int32_t a, int32_t b) { return in[a] > in[b] || (in[a] == in[b] && a < b); });
        for (int64_t j = 0; j < k; ++j) {
            indices[r * k + j] = order[static_cast<size_t>(j)];
            values[r * k + j] = in[order[static_cast<size_t>(j)]];
        }
    }
}

// ---- RoPE ---------------------------------------------------------------------------------------------------------

// cpu_ref::rope (ops.cpp:343-399): x [tokens, heads, dim] f32, positions [tokens] or [tokens, sections] (i32 or
// i64), inv_freq f32, rotary 0 = dim, pair_axes (i32 [rotary / 2]) or null.
void ora_rope(const float* x, const void* positions, int pos_is_i64, const float* inv_freq, float* y, int64_t tokens,
              int64_t heads, int64_t dim, int64_t rotary, int64_t sections, const int32_t* pair_axes) {
    const int64_t rotated = rotary == 0 ? dim : rotary;
    std::memcpy(y, x, static_cast<size_t>(tokens * heads * dim) * sizeof(float));  // channels past rotary pass through
    if (pair_axes != nullptr) {
        const int64_t half = rotated / 2;
        for (int64_t t = 0; t < tokens; ++t) {
            for (int64_t i = 0; i < half; ++i) {
                const double pos = static_cast<double>(pos_at(positions, pos_is_i64, t * sections + pair_axes[i]));
                const double angle = pos * inv_freq[i];
                const double c = std::cos(angle), sn = std::sin(angle);
                for (int64_t h = 0; h < heads; ++h) {
                    const int64_t base = (t * heads + h) * dim;
                    const double x1 = x[base + i], x2 = x[base + half + i];
                    y[base + i] = static_cast<float>(x1 * c - x2 * sn);
                    y[base + half + i] = static_cast<float>(x2 * c + x1 * sn);
                }
            }
        }
        return;
    }
    const int64_t width = rotated / sections;
    const int64_t half = width / 2;
    for (int64_t t = 0; t < tokens; ++t) {
        for (int64_t s = 0; s < sections; ++s) {
            const double pos = static_cast<double>(pos_at(positions, pos_is_i64, t * sections + s));
            for (int64_t i = 0; i < half; ++i) {
                const double angle = pos * inv_freq[i];
                const double c = std::cos(angle);
                const double sn = std::sin(angle);
                for (int64_t h = 0; h < heads; ++h) {
                    const int64_t base = (t * heads + h) * dim + s * width;
                    const double x1 = x[base + i], x2 = x[base + half + i];
                    y[base + i] = static_cast<float>(x1 * c - x2 * sn);
                    y[base + half + i] = static_cast<float>(x2 * c + x1 * sn);
                }
            }
        }
    }
}

// blocks::rope_inv_freq (src/models/common/blocks.cpp:131-141).
void ora_rope_inv_freq(double theta, int64_t dim, int64_t pairs, int64_t length, float* out) {
    for (int64_t i = 0; i < length; ++i) {
        out[i] = i < pairs ? static_cast<float>(1.0 / std::pow(theta, static_cast<double>(2 * i) / static_cast<double>(dim)))
                           : 0.0f;
    }
}

// ---- int8 KV ------------------------------------------------------------------------------------------------------

// quant::quantize_kv_row_i8 (src/quant/quant.cpp:259-267). The reference's float-to-int8 cast of a NaN product is
// undefined behaviour in C++; on x86-64 it yields 0 (cvttss2si gives INT_MIN, whose low byte is 0), stated here as 0.
float ora_quantize_kv_row_i8(const float* x, int64_t width, int8_t* codes) {
    float amax = 0.0f;
    for (int64_t i = 0; i < width; ++i) amax = std::max(amax, std::fabs(x[i]));
    const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
    for (int64_t i = 0; i < width; ++i) {
        const float q = std::nearbyint(x[i] * inv);
        codes[i] = q != q ? int8_t{0} : static_cast<int8_t>(std::clamp(q, -127.0f, 127.0f));
    }
    return amax / 127.0f;
}

void ora_quantize_kv(const float* x, int8_t* codes, float* scales, int64_t rows, int64_t width) {
    for (int64_t r = 0; r < rows; ++r) scales[r] = ora_quantize_kv_row_i8(x + r * width, width, codes + r * width);
}

// The dequantize half of quant::round_trip_kv_i8 (quant.cpp:269-277): fl32(code * scale).
void ora_dequantize_kv(const int8_t* codes, const float* scales, float* out, int64_t rows, int64_t width) {
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t i = 0; i < width; ++i) out[r * width + i] = static_cast<float>(codes[r * width + i]) * scales[r];
}

}  // extern "C"

// ---- TurboQuant KV formats: src/quant/kv_turbo.h:14-105, src/quant/kv_turbo.cpp:9-144 ------------------------------
//
// A group of 128 values: n = its sum of squares (8-value lanes fused-multiply-added in order, the 16 lane sums added
// pairwise 1, 2, 4, 8 lanes apart); w = the values sign-flipped, Walsh-Hadamard transformed (unnormalized butterflies
// of spans 1 .. 64), sign-flipped again; code = sign and the count of edges e_j with w^2 >= e_j^2 * 128 * n (> for a
// negative w); norm = f16(sqrt(n / r)), r = the chosen magnitudes' squares summed like n with plain adds (0 when n is
// 0). Decoding gives centroid * norm, still rotated; the rotation is orthogonal with the 1 / sqrt(128) folded in.

namespace {
namespace turbo {

constexpr int kGroup = 128;
constexpr int kLanes = 16;
constexpr int kLaneValues = 8;
constexpr uint64_t kSignsBefore[2] = {0x42f85949e46a0359ull, 0x49f250a9a4c63bbbull};  // kv_turbo.h:27
constexpr uint64_t kSignsAfter[2] = {0x3f628fdc16acee90ull, 0xbea56562b7a5357aull};   // kv_turbo.h:28
// Lloyd-Max magnitudes of a Gaussian of variance 1 / 128 and the borders between them (kv_turbo.h:39-56).
constexpr float kMags2[2] = {0.039994f, 0.133462f};
constexpr float kEdges2[1] = {0.086728f};
constexpr float kMags3[4] = {0.021663f, 0.066822f, 0.118786f, 0.190207f};
constexpr float kEdges3[3] = {0.044243f, 0.092804f, 0.154496f};
constexpr float kMags4[8] = {0.011349f, 0.034299f, 0.058050f, 0.083292f, 0.111036f, 0.143016f, 0.182877f, 0.241529f};
constexpr float kEdges4[7] = {0.022824f, 0.046174f, 0.070671f, 0.097164f, 0.127026f, 0.162947f, 0.212203f};

const float* mags(int bits) { return bits == 4 ? kMags4 : bits == 3 ? kMags3 : kMags2; }
const float* edges(int bits) { return bits == 4 ? kEdges4 : bits == 3 ? kEdges3 : kEdges2; }
int group_bytes(int bits) { return kGroup * bits / 8; }
bool flipped(const uint64_t* signs, int i) { return ((signs[i / 64] >> (i % 64)) & 1u) != 0; }

// Pairwise over lanes 1, 2, 4, 8 apart (every lane ends with the same sum).
float sum_lanes(float* lane) {
    for (int m = 1; m < kLanes; m <<= 1) {
        float next[kLanes];
        for (int l = 0; l < kLanes; ++l) next[l] = lane[l] + lane[l ^ m];
        std::memcpy(lane, next, sizeof(next));
    }
    return lane[0];
}

void butterflies(float* x) {
    for (int h = 1; h < kGroup; h *= 2)
        for (int i = 0; i < kGroup; i += 2 * h)
            for (int j = i; j < i + h; ++j) {
                const float a = x[j], b = x[j + h];
                x[j] = a + b;
                x[j + h] = a - b;
            }
}

// Code c of a magnitude index m: the upper half of the codes positive, ascending (kv_turbo.h:63-66).
uint32_t code_of(int bits, bool negative, uint32_t m) {
    const uint32_t half = 1u << (bits - 1);
    return negative ? half - 1 - m : half + m;
}

float centroid(int bits, uint32_t code) {
    const uint32_t half = 1u << (bits - 1);
    return code >= half ? mags(bits)[code - half] : -mags(bits)[half - 1 - code];
}

// Packing (kv_turbo.h:84-87; kv_turbo.cpp:38-45, 104-109).
void put_code(uint8_t* codes, int bits, int i, uint32_t code) {
    if (bits == 4) {
        codes[i / 2] |= static_cast<uint8_t>(code << (4 * (i % 2)));
        return;
    }
    codes[i / 4] |= static_cast<uint8_t>((code & 3u) << (2 * (i % 4)));
    if (bits == 3) codes[kGroup / 4 + i / 8] |= static_cast<uint8_t>((code >> 2) << (i % 8));
}

uint32_t code_at(const uint8_t* codes, int bits, int i) {
    if (bits == 4) return (codes[i / 2] >> (4 * (i % 2))) & 15u;
    const uint32_t low = (codes[i / 4] >> (2 * (i % 4))) & 3u;
    if (bits == 2) return low;
    return low | (((codes[kGroup / 4 + i / 8] >> (i % 8)) & 1u) << 2);
}

// quant::turbo::quantize_group (kv_turbo.cpp:47-84).
uint16_t quantize_group(const float* x, int bits, uint8_t* codes) {
    float lane[kLanes];
    for (int l = 0; l < kLanes; ++l) {
        float s = 0.0f;
        for (int e = 0; e < kLaneValues; ++e) s = std::fma(x[l * kLaneValues + e], x[l * kLaneValues + e], s);
        lane[l] = s;
    }
    const float n = sum_lanes(lane);
    float w[kGroup];
    for (int i = 0; i < kGroup; ++i) w[i] = flipped(kSignsBefore, i) ? -x[i] : x[i];
    butterflies(w);
    const int nm = 1 << (bits - 1);
    float edge[7];
    for (int j = 0; j < nm - 1; ++j) {
        const double e = edges(bits)[j];
        edge[j] = static_cast<float>(e * e * kGroup) * n;  // edge_sq(j) * n (kv_turbo.h:57-62)
    }
    std::memset(codes, 0, static_cast<size_t>(group_bytes(bits)));
    float chosen[kGroup];
    for (int i = 0; i < kGroup; ++i) {
        const float v = flipped(kSignsAfter, i) ? -w[i] : w[i];
        const bool negative = v < 0.0f;
        const float sq = v * v;
        uint32_t m = 0;
        for (int j = 0; j < nm - 1; ++j) m += (negative ? sq > edge[j] : sq >= edge[j]) ? 1u : 0u;
        put_code(codes, bits, i, code_of(bits, negative, m));
        chosen[i] = mags(bits)[m] * mags(bits)[m];
    }
    for (int l = 0; l < kLanes; ++l) {
        float s = 0.0f;
        for (int e = 0; e < kLaneValues; ++e) s += chosen[l * kLaneValues + e];
        lane[l] = s;
    }
    const float r = sum_lanes(lane);
    return f32_to_f16(n > 0.0f ? std::sqrt(n / r) : 0.0f);
}

// quant::turbo::rotate_group (kv_turbo.cpp:118-129).
void rotate_group(float* x, bool inverse) {
    const uint64_t* first = inverse ? kSignsAfter : kSignsBefore;
    const uint64_t* last = inverse ? kSignsBefore : kSignsAfter;
    for (int i = 0; i < kGroup; ++i) x[i] = flipped(first, i) ? -x[i] : x[i];
    butterflies(x);
    for (int i = 0; i < kGroup; ++i) {
        const float y = x[i] * 0.08838834764831845f;
        x[i] = flipped(last, i) ? -y : y;
    }
}

}  // namespace turbo
}  // namespace

extern "C" {

// Codes [groups, 128 * bits / 8] and f16 norms [groups] of x [groups, 128] (quant::turbo::quantize_group).
void ora_turbo_quantize(const float* x, int64_t groups, int bits, uint8_t* codes, uint16_t* norms) {
    for (int64_t g = 0; g < groups; ++g)
        norms[g] = turbo::quantize_group(x + g * turbo::kGroup, bits, codes + g * turbo::group_bytes(bits));
}

// The rotated values the groups store, centroid * norm (quant::turbo::decode_group, kv_turbo.cpp:86-91).
void ora_turbo_decode(const uint8_t* codes, const uint16_t* norms, int64_t groups, int bits, float* out) {
    for (int64_t g = 0; g < groups; ++g) {
        const float scale = f16_to_f32(norms[g]);
        for (int i = 0; i < turbo::kGroup; ++i)
            out[g * turbo::kGroup + i] =
                turbo::centroid(bits, turbo::code_at(codes + g * turbo::group_bytes(bits), bits, i)) * scale;
    }
}

// Each group of 128 values rotated, or rotated back, in place (quant::turbo::rotate_group).
void ora_turbo_rotate(float* x, int64_t groups, int inverse) {
    for (int64_t g = 0; g < groups; ++g) turbo::rotate_group(x + g * turbo::kGroup, inverse != 0);
}

// The value each code names: 1 << bits entries (kv_turbo.h:68-80, the Tables' centroids).
void ora_turbo_centroids(int bits, float* out) {
    for (uint32_t c = 0; c < (1u << bits); ++c) out[c] = turbo::centroid(bits, c);
}

}  // extern "C"
