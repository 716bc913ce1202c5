// xs_hip_kernels.hpp -- the C++ device-dispatch surface of the MI355X (gfx950) device, `xs::hip_be`, over the C-ABI
// of xs_hip.h.
//
// It keeps the shape of the reference's `xs::sycl_be` launchers (src/backend/sycl/sycl_kernels.h): the same names, the
// same argument order and meaning, element types as template parameters, and the same error behaviour -- a refused
// call throws an exception carrying a diagnosis, where the reference throws xs::Error (src/util/error.h:12-28). Only
// the queue differs: `sycl::queue&` becomes `Stream`, an opaque HIP stream handle (nullptr is the null stream).
// Every launcher enqueues and returns without waiting (sycl_kernels.h:3).
//
// Header-only; links against libxs_hip.so. No HIP, SYCL or torch headers are needed to include it.
//
// The exception type: `xs::hip_be::Error` derives from XS_HIP_ERROR_BASE, which defaults to std::runtime_error. Inside
// the reference tree, include src/util/error.h first and define XS_HIP_ERROR_BASE as ::xs::Error, so that a refused
// launch is the xs::Error every caller of a backend already handles.
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <type_traits>

#include "xs_hip.h"

#ifndef XS_HIP_ERROR_BASE
#define XS_HIP_ERROR_BASE std::runtime_error
#endif

namespace xs::hip_be {

class Error : public XS_HIP_ERROR_BASE {
public:
    explicit Error(const std::string& what) : XS_HIP_ERROR_BASE(what) {}
};

using Stream = void*;

// 16-bit float storage as the kernels read and write it (the bits of IEEE binary16 / bfloat16). The host never does
// arithmetic on these: the reference converts with util/half.h, and so may a caller.
struct half {
    uint16_t bits;
};
struct bf16 {
    uint16_t bits;
};

inline constexpr int kMaxRank = XS_MAX_RANK;  // sycl_kernels.h:19

// sycl_kernels.h:21, in its order (the values are the C-ABI's).
enum class UnaryOp : uint8_t { Scale, Tanh, GeluTanh, Softcap, Sigmoid, Silu, Softplus, Clamp, Gelu };
// sycl_kernels.h:34.
enum class BinaryOp : uint8_t { Add, Mul, Div };
// quant/kv_format.h:11-17.
enum class KvFormat : uint8_t { Float, I8, Turbo4, Turbo3, Turbo2 };

// numpy broadcasting over at most kMaxRank dims: the out shape and the element strides of a and b per out dim (0 where
// the operand is broadcast), sycl_kernels.h:37-42. y is contiguous.
struct Broadcast {
    int rank = 0;
    int64_t out[kMaxRank] = {};
    int64_t stride_a[kMaxRank] = {};
    int64_t stride_b[kMaxRank] = {};
};

// A quantized KV stream (sycl_kernels.h:201-205): codes and scales of rows [N * Hkv].
struct KvStream {
    KvFormat format = KvFormat::I8;
    const uint8_t* codes = nullptr;
    const uint8_t* scales = nullptr;
};

namespace detail {

template <typename T>
constexpr xs_dtype dtype_of() {
    if constexpr (std::is_same_v<T, float>) return XS_F32;
    else if constexpr (std::is_same_v<T, half>) return XS_F16;
    else if constexpr (std::is_same_v<T, bf16>) return XS_BF16;
    else if constexpr (std::is_same_v<T, int32_t>) return XS_I32;
    else if constexpr (std::is_same_v<T, int64_t>) return XS_I64;
    else static_assert(sizeof(T) == 0, "element type without a device dtype");
}

// Turns a C-ABI status into the exception the reference's launchers throw, naming the op.
inline void check(int status, const char* op) {
    if (status == XS_HIP_OK) return;
    throw Error(std::string("hip_be::") + op + ": " + xs_hip_last_error());
}

inline xs_broadcast to_abi(const Broadcast& s) {
    xs_broadcast bc{};
    bc.rank = s.rank;
    int64_t step = 1;
    for (int d = s.rank - 1; d >= 0; --d) {
        bc.out[d] = s.out[d];
        bc.stride_a[d] = s.stride_a[d];
        bc.stride_b[d] = s.stride_b[d];
        bc.stride_y[d] = step;
        step *= s.out[d];
    }
    return bc;
}

}  // namespace detail

// ---- Elementwise and broadcast -------------------------------------------------------------------------------------

// y = op(x); `a` is the scale factor, softcap or lower bound, `b` the upper bound (sycl_kernels.h:21-25). The
// reference's x is f32; here X may also be half or bf16.
template <typename Y, typename X = float>
void unary(Stream q, UnaryOp op, const X* x, Y* y, int64_t n, float a, float b) {
    detail::check(xs_hip_unary(q, static_cast<xs_unary_op>(op), detail::dtype_of<X>(), x, detail::dtype_of<Y>(), y, n,
                               a, b),
                  "unary");
}

// y = act(x) * b, same shapes; act is Silu, GeluTanh, Sigmoid or Gelu (sycl_kernels.h:27-29). X, Y: float, half, bf16.
template <typename X, typename Y>
void act_mul(Stream q, UnaryOp act, const X* x, const X* b, Y* y, int64_t n) {
    detail::check(xs_hip_act_mul(q, static_cast<xs_unary_op>(act), detail::dtype_of<X>(), x, b, detail::dtype_of<Y>(),
                                 y, n),
                  "act_mul");
}

// y = act(x + bias[i % period]) (sycl_kernels.h:30-32).
template <typename Y>
void unary_bias(Stream q, UnaryOp act, const float* x, const float* bias, Y* y, int64_t n, int64_t period) {
    detail::check(xs_hip_unary_bias(q, static_cast<xs_unary_op>(act), x, bias, detail::dtype_of<Y>(), y, n, period),
                  "unary_bias");
}

// The gated activation of 2-D operands with row strides, y = act(x + bias) * b, in one launch: what the reference
// evaluates as unary_bias then act_mul. An extension of this device (no launcher of its own in the reference).
template <typename X, typename Y>
void act_bias_mul_2d(Stream q, UnaryOp act, const X* x, int64_t x_row_stride, const X* b, int64_t b_row_stride,
                     const X* bias, Y* y, int64_t y_row_stride, int64_t rows, int64_t cols) {
    detail::check(xs_hip_act_bias_mul_2d(q, static_cast<xs_unary_op>(act), detail::dtype_of<X>(), x, x_row_stride, b,
                                         b_row_stride, bias, detail::dtype_of<Y>(), y, y_row_stride, rows, cols),
                  "act_bias_mul_2d");
}

// y = a op b under numpy broadcasting (sycl_kernels.h:43-44). `n` is the element count of y.
template <typename Y>
void binary(Stream q, BinaryOp op, const float* a, const float* b, Y* y, int64_t n, const Broadcast& shape) {
    int64_t count = shape.rank > 0 ? 1 : 0;
    for (int d = 0; d < shape.rank; ++d) count *= shape.out[d];
    if (shape.rank > 0 && count != n) {
        throw Error("hip_be::binary: n = " + std::to_string(n) + " but the broadcast shape holds " +
                    std::to_string(count) + " elements");
    }
    const xs_broadcast bc = detail::to_abi(shape);
    detail::check(xs_hip_binary(q, static_cast<xs_binary_op>(op), XS_F32, a, XS_F32, b, detail::dtype_of<Y>(), y, &bc),
                  "binary");
}

// Same shape, and b repeating every `period` elements of a (sycl_kernels.h:45-49).
template <typename Y>
void binary_same(Stream q, BinaryOp op, const float* a, const float* b, Y* y, int64_t n) {
    detail::check(xs_hip_binary_same(q, static_cast<xs_binary_op>(op), XS_F32, a, b, detail::dtype_of<Y>(), y, n),
                  "binary_same");
}
template <typename Y>
void binary_period(Stream q, BinaryOp op, const float* a, const float* b, Y* y, int64_t n, int64_t period) {
    detail::check(
        xs_hip_binary_period(q, static_cast<xs_binary_op>(op), XS_F32, a, b, detail::dtype_of<Y>(), y, n, period),
        "binary_period");
}

// y = a + b * c[i % period] and y = a + (b + c[i % period]) (sycl_kernels.h:50-55).
template <typename Y>
void add_mul(Stream q, const float* a, const float* b, const float* c, Y* y, int64_t n, int64_t period) {
    detail::check(xs_hip_add_mul(q, a, b, c, detail::dtype_of<Y>(), y, n, period), "add_mul");
}
template <typename Y>
void add3(Stream q, const float* a, const float* b, const float* c, Y* y, int64_t n, int64_t period) {
    detail::check(xs_hip_add3(q, a, b, c, detail::dtype_of<Y>(), y, n, period), "add3");
}

// f32 to f16, round to nearest even (sycl_kernels.h:130).
inline void to_half(Stream q, const float* x, half* y, int64_t n) {
    detail::check(xs_hip_convert(q, XS_F32, x, XS_F16, y, n), "to_half");
}
// Any float dtype to any other (the widening and narrowing of tensor.cpp:58-84 and half.cpp:36-56 on the device).
template <typename X, typename Y>
void convert(Stream q, const X* x, Y* y, int64_t n) {
    detail::check(xs_hip_convert(q, detail::dtype_of<X>(), x, detail::dtype_of<Y>(), y, n), "convert");
}

// ---- Row reductions ------------------------------------------------------------------------------------------------

// Rows of `width`: x / rms(x) [* w] [+ bias]; w and bias may be null (sycl_kernels.h:86-90).
template <typename Y>
void rms_norm(Stream q, const float* x, const float* w, const float* bias, Y* y, int64_t rows, int64_t width,
              float eps) {
    detail::check(xs_hip_rms_norm(q, XS_F32, x, w, bias, detail::dtype_of<Y>(), y, rows, width, eps), "rms_norm");
}

// h_out = x + residual, y = rms_norm(h_out) in one pass: the Add then RmsNorm of a decoder's residual stream
// (models/qwen3/qwen3_decoder.cpp:101-102). An extension of this device.
template <typename Y>
void add_rms_norm(Stream q, const float* x, const float* residual, const float* w, const float* bias, float* h_out,
                  Y* y, int64_t rows, int64_t width, float eps) {
    detail::check(xs_hip_add_rms_norm(q, x, residual, w, bias, h_out, detail::dtype_of<Y>(), y, rows, width, eps),
                  "add_rms_norm");
}

// Rows of `width`: (x [+ shift] - mean) / sqrt(var + eps) [* w] [+ b] (sycl_kernels.h:91-94).
template <typename Y>
void layer_norm(Stream q, const float* x, const float* shift, const float* w, const float* b, Y* y, int64_t rows,
                int64_t width, float eps) {
    detail::check(xs_hip_layer_norm(q, XS_F32, x, shift, w, b, detail::dtype_of<Y>(), y, rows, width, eps),
                  "layer_norm");
}

// y = x * min(1, threshold / (|x| + eps)) per row (sycl_kernels.h:141-142).
inline void l2_clip(Stream q, const float* x, float* y, int64_t rows, int64_t width, float threshold, float eps) {
    detail::check(xs_hip_l2_clip(q, x, y, rows, width, threshold, eps), "l2_clip");
}

// y [outer, inner] = the sum over the middle axis of x [outer, dim, inner] (sycl_kernels.h:80-81).
inline void reduce_sum(Stream q, const float* x, float* y, int64_t outer, int64_t dim, int64_t inner) {
    detail::check(xs_hip_reduce_sum(q, x, y, outer, dim, inner), "reduce_sum");
}

// Rows of `width` (sycl_kernels.h:57-58).
inline void softmax(Stream q, const float* x, float* y, int64_t rows, int64_t width) {
    detail::check(xs_hip_softmax(q, x, y, rows, width), "softmax");
}

// Scaled and masked attention-score softmax (keys at or past valid_len come out 0); `scratch` holds
// softmax_masked_scratch bytes or is null. An extension of this device: the reference's attention_softmax
// (sycl_kernels.cpp:2047-2104) is internal to its attention path.
inline size_t softmax_masked_scratch(int64_t rows, int64_t width) { return xs_hip_softmax_scratch(rows, width); }
inline void softmax_masked(Stream q, const float* x, float* y, int64_t rows, int64_t width, int64_t row_stride,
                           float scale, const int64_t* valid_len, int64_t valid_len_all, void* scratch) {
    detail::check(xs_hip_softmax_masked(q, x, y, rows, width, row_stride, scale, valid_len, valid_len_all, scratch),
                  "softmax_masked");
}

// The k largest per row, ties to the lower index (sycl_kernels.h:59-63). The reference's topk_scratch has no k; this
// device's scratch depends on it, so k is an argument here (default 1, argmax).
inline size_t topk_scratch(int64_t rows, int64_t width, int64_t k = 1) { return xs_hip_topk_scratch(rows, width, k); }
inline void topk(Stream q, const float* x, float* values, int32_t* indices, int64_t rows, int64_t width, int64_t k,
                 void* scratch) {
    detail::check(xs_hip_topk(q, x, values, indices, rows, width, k, scratch), "topk");
}

// ---- RoPE ----------------------------------------------------------------------------------------------------------

// x [T, H, D]; positions [T] or [T, sections]; inv_freq [rotary / (2 sections)] (sycl_kernels.h:111-116). The
// reference's x is f32; here X may also be half or bf16 (the f16 Q/K of an f16 step).
template <typename I, typename Y, typename X = float>
void rope(Stream q, const X* x, const I* positions, const float* inv_freq, Y* y, int64_t tokens, int64_t heads,
          int64_t dim, int64_t rotary, int64_t sections, const int32_t* pair_axes = nullptr) {
    detail::check(xs_hip_rope(q, detail::dtype_of<X>(), x, detail::dtype_of<I>(), positions, inv_freq,
                              detail::dtype_of<Y>(), y, tokens, heads, dim, rotary, sections, pair_axes),
                  "rope");
}

// Q and K of a step rotated in one launch (each as rope rotates it). An extension of this device.
template <typename I, typename Y, typename X = float>
void rope_qk(Stream q, const X* xq, Y* yq, int64_t q_heads, const X* xk, Y* yk, int64_t k_heads, const I* positions,
             const float* inv_freq, int64_t tokens, int64_t dim, int64_t rotary, int64_t sections,
             const int32_t* pair_axes = nullptr) {
    detail::check(xs_hip_rope2(q, detail::dtype_of<X>(), xq, yq, q_heads, xk, yk, k_heads, detail::dtype_of<I>(),
                               positions, inv_freq, detail::dtype_of<Y>(), tokens, dim, rotary, sections, pair_axes),
                  "rope_qk");
}

// ---- Quantized KV cache --------------------------------------------------------------------------------------------

// Codes and scales of x [rows, width] (sycl_kernels.h:211-214). The reference's x is f32; X may also be half or bf16.
template <typename X = float>
void quantize_kv(Stream q, KvFormat format, const X* x, uint8_t* codes, uint8_t* scales, int64_t rows, int64_t width) {
    detail::check(xs_hip_quantize_kv(q, static_cast<xs_kv_format>(format), detail::dtype_of<X>(), x, codes, scales,
                                     rows, width),
                  "quantize_kv");
}

// out [rows, width] = the values the rows store (sycl_kernels.h:215-218). CT: float, half or bf16.
template <typename CT>
void dequantize_kv(Stream q, const KvStream& s, CT* out, int64_t rows, int64_t width) {
    detail::check(xs_hip_dequantize_kv(q, static_cast<xs_kv_format>(s.format), s.codes, s.scales,
                                       detail::dtype_of<CT>(), out, rows, width),
                  "dequantize_kv");
}

// y [rows, width] = x with each group of 128 values rotated as the TurboQuant formats rotate a row, or rotated back
// (sycl_kernels.h:219-221).
inline void kv_rotate(Stream q, const float* x, float* y, int64_t rows, int64_t width, bool inverse) {
    detail::check(xs_hip_kv_rotate(q, x, y, rows, width, inverse ? 1 : 0), "kv_rotate");
}

// ---- Attention over the quantized KV cache -------------------------------------------------------------------------

struct KvQuantized {  // sycl_kernels.h:206-208
    KvStream k, v;
};

// The shape fields of sycl_be::AttentionShape (sycl_kernels.h:158-180) this device takes: causal or full attention with
// an optional sliding window and softcap.
struct AttentionShape {
    int64_t tokens = 0;
    int64_t q_heads = 0;
    int64_t kv_heads = 0;
    int64_t head_dim = 0;
    int64_t kv_len = 0;
    float scale = 1.0f;
    float softcap = 0.0f;
    int64_t window = 0;
    bool causal = true;
};

inline int64_t attention_split(const AttentionShape& s) {
    return xs_hip_attention_i8_split(s.tokens, s.kv_heads, s.kv_len);
}
// The split for attention_rows (float caches) and attention_rows_quantized with TurboQuant values.
inline int64_t attention_rows_split(const AttentionShape& s) {
    return xs_hip_attention_rows_split(s.tokens, s.kv_heads, s.kv_len);
}
inline size_t attention_scratch(const AttentionShape& s, int64_t split) {
    return xs_hip_attention_i8_scratch(s.tokens, s.q_heads, s.head_dim, split);
}

// attention_rows_quantized + attention_combine (sycl_kernels.h:238-240): int8 keys and values, both in the same
// TurboQuant format, or int8 keys with TurboQuant values (kv_formats_supported, sycl_kernels.h:209-212); other pairs
// throw. `part` holds attention_scratch(s, split) bytes when split > 1.
inline void attention_rows_quantized(Stream q, const float* qp, const KvQuantized& kv, float* out,
                                     const AttentionShape& s, int64_t split, float* part) {
    detail::check(xs_hip_attention_quantized(q, static_cast<xs_kv_format>(kv.k.format),
                                             static_cast<xs_kv_format>(kv.v.format), qp, kv.k.codes, kv.k.scales,
                                             kv.v.codes, kv.v.scales, out, s.tokens, s.q_heads, s.kv_heads,
                                             s.head_dim, s.kv_len, s.scale, s.softcap, s.window, s.causal ? 1 : 0,
                                             split, part),
                  "attention_rows_quantized");
}

// attention_rows<KV> + attention_combine (sycl_kernels.h, attention_rows / attention_combine) over a float cache, KV =
// half or float: keys and values [kv_len, kv_heads, head_dim]; `part` holds attention_scratch(s, split) bytes when
// split > 1.
template <typename KV>
void attention_rows(Stream q, const float* qp, const KV* k, const KV* v, float* out, const AttentionShape& s,
                    int64_t split, float* part) {
    static_assert(std::is_same_v<KV, half> || std::is_same_v<KV, float>, "float caches hold half or float rows");
    detail::check(xs_hip_attention(q, detail::dtype_of<KV>(), qp, k, v, out, s.tokens, s.q_heads, s.kv_heads,
                                   s.head_dim, s.kv_len, s.scale, s.softcap, s.window, s.causal ? 1 : 0, split, part),
                  "attention_rows");
}

// part [rows, split, D + 2] (D sums, max, denominator per split) merged into out [rows, D] (sycl_kernels.h:240).
inline void attention_combine(Stream q, const float* part, float* out, int64_t rows, int64_t split, int64_t head_dim) {
    detail::check(xs_hip_attention_combine(q, part, out, rows, split, head_dim), "attention_combine");
}
// acc [rows, D + 2] takes in each row's `split` partial rows; `first`: acc starts as their merge (sycl_kernels.h:
// 241-244).
inline void attention_merge(Stream q, const float* part, float* acc, int64_t rows, int64_t split, int64_t head_dim,
                            bool first) {
    detail::check(xs_hip_attention_merge(q, part, acc, rows, split, head_dim, first ? 1 : 0), "attention_merge");
}

// ---- Data movement -------------------------------------------------------------------------------------------------

// out [n, width] = rows ids[r] of table [rows, width] as f32 (sycl_kernels.h:106-107; T float, half or bf16, I int32_t
// or int64_t). The reference's launcher takes no row count; this device needs it to keep an id outside the table from
// reading past it (such an id gives a row of zeros).
template <typename T, typename I>
void gather(Stream q, const T* table, const I* ids, float* out, int64_t n, int64_t width, int64_t rows) {
    detail::check(xs_hip_gather(q, detail::dtype_of<T>(), table, rows, width, detail::dtype_of<I>(), ids, n, out),
                  "gather");
}
// Rows of a table of 32-bit integers, copied as they are (sycl_kernels.h:108-110).
template <typename I>
void gather_bits(Stream q, const uint32_t* table, const I* ids, uint32_t* out, int64_t n, int64_t width,
                 int64_t rows) {
    detail::check(xs_hip_gather(q, XS_I32, table, rows, width, detail::dtype_of<I>(), ids, n, out), "gather_bits");
}

// For each of `outer` blocks: rows [begin, begin + len) of `dim` rows of `inner` elements of `elem` bytes
// (sycl_kernels.h:118-120).
inline void slice(Stream q, const void* x, void* y, size_t elem, int64_t outer, int64_t dim, int64_t begin, int64_t len,
                  int64_t inner) {
    const auto row = static_cast<int64_t>(elem) * inner;
    detail::check(xs_hip_copy_rows(q, static_cast<const char*>(x) + begin * row, dim * row, y, len * row, outer,
                                   len * row),
                  "slice");
}

// y = x with its axes permuted (sycl_kernels.h:121-128): the reference's Permute carries the output shape and x's
// stride of each output axis; this device takes x's shape and the permutation, from which both follow.
inline void transpose(Stream q, const void* x, void* y, size_t elem, int rank, const int64_t* in_shape,
                      const int32_t* perm) {
    detail::check(xs_hip_transpose(q, x, y, static_cast<int64_t>(elem), rank, in_shape, perm), "transpose");
}

// Concat as one copy kernel (sycl_kernels.h:95-104): `outer` rows, each the parts' rows laid end to end.
inline constexpr int kConcatParts = XS_CONCAT_PARTS;
struct ConcatParts {
    int count = 0;
    const void* src[kConcatParts] = {};
    size_t bytes[kConcatParts] = {};  // per outer row
};
inline void concat(Stream q, const ConcatParts& parts, void* out, int64_t outer) {
    int64_t bytes[kConcatParts] = {};
    for (int k = 0; k < parts.count && k < kConcatParts; ++k) bytes[k] = static_cast<int64_t>(parts.bytes[k]);
    detail::check(xs_hip_concat(q, parts.count, parts.src, bytes, out, outer), "concat");
}

// ---- Device memory -------------------------------------------------------------------------------------------------

// Owns `bytes` of device memory, freed on destruction; the counterpart of the SYCL backend's USM DeviceBuffer
// (sycl_backend.cpp:64-107). Move-only.
class DeviceBuffer {
public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t bytes) : bytes_(bytes) {
        if (bytes > 0) detail::check(xs_hip_malloc(&ptr_, bytes), "DeviceBuffer");
    }
    ~DeviceBuffer() { reset(); }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    DeviceBuffer(DeviceBuffer&& o) noexcept : ptr_(o.ptr_), bytes_(o.bytes_) {
        o.ptr_ = nullptr;
        o.bytes_ = 0;
    }
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
        if (this != &o) {
            reset();
            ptr_ = o.ptr_;
            bytes_ = o.bytes_;
            o.ptr_ = nullptr;
            o.bytes_ = 0;
        }
        return *this;
    }
    void reset() {
        if (ptr_ != nullptr) xs_hip_free(ptr_);
        ptr_ = nullptr;
        bytes_ = 0;
    }
    template <typename T = void>
    T* get() const {
        return static_cast<T*>(ptr_);
    }
    size_t bytes() const { return bytes_; }

private:
    void* ptr_ = nullptr;
    size_t bytes_ = 0;
};

}  // namespace xs::hip_be
