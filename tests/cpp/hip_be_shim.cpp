// TEST INFRASTRUCTURE. Exposes the C++ launchers of include/xs_hip_kernels.hpp (xs::hip_be) to the Python parity tests
// through a few extern "C" wrappers, so the C++ surface a reference-side caller would use is the one checked against
// the oracle. Each wrapper catches xs::hip_be::Error and keeps its message for hipbe_last_error().
#include <cstring>
#include <string>
#include <vector>

#include "xs_hip_kernels.hpp"

namespace hb = xs::hip_be;

namespace {
thread_local std::string g_error;

template <typename F>
int guarded(F&& f) {
    try {
        f();
        g_error.clear();
        return 0;
    } catch (const std::runtime_error& e) {  // hip_be::Error is-a std::runtime_error outside the reference tree
        g_error = e.what();
        return 1;
    }
}

// numpy broadcasting of contiguous a and b into a contiguous y, the way a backend fills sycl_be::Broadcast.
hb::Broadcast make_broadcast(const int64_t* as, int ar, const int64_t* bs, int br) {
    hb::Broadcast s;
    s.rank = ar > br ? ar : br;
    int64_t sa = 1, sb = 1;
    for (int d = s.rank - 1; d >= 0; --d) {
        const int ia = d - (s.rank - ar), ib = d - (s.rank - br);
        const int64_t da = ia >= 0 ? as[ia] : 1, db = ib >= 0 ? bs[ib] : 1;
        if (da != db && da != 1 && db != 1) throw hb::Error("shapes do not broadcast");
        s.out[d] = da > db ? da : db;
        if (da == 1 && db == 0) s.out[d] = 0;
        s.stride_a[d] = da == 1 ? 0 : sa;
        s.stride_b[d] = db == 1 ? 0 : sb;
        sa *= da;
        sb *= db;
    }
    return s;
}
}  // namespace

extern "C" {

const char* hipbe_last_error() { return g_error.c_str(); }

int hipbe_swiglu_bf16(void* q, const void* x, int64_t xs, const void* b, int64_t bs, const void* bias, void* y,
                      int64_t ys, int64_t rows, int64_t cols) {
    return guarded([&] {
        hb::act_bias_mul_2d(q, hb::UnaryOp::Silu, static_cast<const hb::bf16*>(x), xs, static_cast<const hb::bf16*>(b),
                            bs, static_cast<const hb::bf16*>(bias), static_cast<hb::bf16*>(y), ys, rows, cols);
    });
}

int hipbe_act_mul_f32(void* q, int act, const float* x, const float* b, float* y, int64_t n) {
    return guarded([&] { hb::act_mul(q, static_cast<hb::UnaryOp>(act), x, b, y, n); });
}

int hipbe_unary_bias_f16(void* q, int act, const float* x, const float* bias, void* y, int64_t n, int64_t period) {
    return guarded(
        [&] { hb::unary_bias(q, static_cast<hb::UnaryOp>(act), x, bias, static_cast<hb::half*>(y), n, period); });
}

int hipbe_binary_f32(void* q, int op, const float* a, const int64_t* as, int ar, const float* b, const int64_t* bs,
                     int br, float* y) {
    return guarded([&] {
        const hb::Broadcast s = make_broadcast(as, ar, bs, br);
        int64_t n = 1;
        for (int d = 0; d < s.rank; ++d) n *= s.out[d];
        hb::binary(q, static_cast<hb::BinaryOp>(op), a, b, y, n, s);
    });
}

int hipbe_binary_n_mismatch() {
    return guarded([&] {
        hb::Broadcast s;
        s.rank = 2;
        s.out[0] = 4;
        s.out[1] = 6;
        hb::binary<float>(nullptr, hb::BinaryOp::Add, nullptr, nullptr, nullptr, 25, s);
    });
}

int hipbe_add_mul_f32(void* q, const float* a, const float* b, const float* c, float* y, int64_t n, int64_t period) {
    return guarded([&] { hb::add_mul(q, a, b, c, y, n, period); });
}

int hipbe_add_rms_norm_f32(void* q, const float* x, const float* r, const float* w, float* h, float* y, int64_t rows,
                           int64_t width, float eps) {
    return guarded([&] { hb::add_rms_norm(q, x, r, w, nullptr, h, y, rows, width, eps); });
}

int hipbe_rms_norm_f16(void* q, const float* x, const float* w, void* y, int64_t rows, int64_t width, float eps) {
    return guarded([&] { hb::rms_norm(q, x, w, nullptr, static_cast<hb::half*>(y), rows, width, eps); });
}

int hipbe_softmax(void* q, const float* x, float* y, int64_t rows, int64_t width) {
    return guarded([&] { hb::softmax(q, x, y, rows, width); });
}

// topk with the scratch the launcher asks for, owned by a DeviceBuffer for the call (synchronised before it is freed).
int hipbe_topk(void* q, const float* x, float* values, int32_t* indices, int64_t rows, int64_t width, int64_t k) {
    return guarded([&] {
        hb::DeviceBuffer scratch(hb::topk_scratch(rows, width, k));
        hb::topk(q, x, values, indices, rows, width, k, scratch.get());
        if (xs_hip_stream_synchronize(q) != XS_HIP_OK) throw hb::Error(xs_hip_last_error());
    });
}

int hipbe_rope_f16(void* q, const void* x, const int32_t* pos, const float* inv_freq, void* y, int64_t tokens,
                   int64_t heads, int64_t dim, int64_t rotary) {
    return guarded([&] {
        hb::rope<int32_t>(q, static_cast<const hb::half*>(x), pos, inv_freq, static_cast<hb::half*>(y), tokens, heads,
                          dim, rotary, 1);
    });
}

int hipbe_quantize_kv_f16(void* q, const void* x, void* codes, void* scales, int64_t rows, int64_t width) {
    return guarded([&] {
        hb::quantize_kv(q, hb::KvFormat::I8, static_cast<const hb::half*>(x), static_cast<uint8_t*>(codes),
                        static_cast<uint8_t*>(scales), rows, width);
    });
}

int hipbe_dequantize_kv_f16(void* q, const void* codes, const void* scales, void* out, int64_t rows, int64_t width) {
    return guarded([&] {
        hb::KvStream s{hb::KvFormat::I8, static_cast<const uint8_t*>(codes), static_cast<const uint8_t*>(scales)};
        hb::dequantize_kv(q, s, static_cast<hb::half*>(out), rows, width);
    });
}

// attention_rows<half> (k_format 0: the Float format at f16) or attention_rows_quantized over keys and values in
// k_format / v_format (KvFormat's values), with the split the launcher suggests and its scratch.
int hipbe_attention(void* q, int k_format, int v_format, const float* qp, const void* k, const void* k_scales, const void* v,
                    const void* v_scales, float* out, int64_t tokens, int64_t q_heads, int64_t kv_heads,
                    int64_t head_dim, int64_t kv_len, float scale) {
    return guarded([&] {
        hb::AttentionShape s;
        s.tokens = tokens;
        s.q_heads = q_heads;
        s.kv_heads = kv_heads;
        s.head_dim = head_dim;
        s.kv_len = kv_len;
        s.scale = scale;
        const int64_t split = k_format == static_cast<int>(hb::KvFormat::I8) && v_format == k_format
                                  ? hb::attention_split(s)
                                  : hb::attention_rows_split(s);
        hb::DeviceBuffer part(hb::attention_scratch(s, split));
        if (k_format == 0) {
            hb::attention_rows(q, qp, static_cast<const hb::half*>(k), static_cast<const hb::half*>(v), out, s, split,
                               static_cast<float*>(part.get()));
        } else {
            hb::KvQuantized kv{{static_cast<hb::KvFormat>(k_format), static_cast<const uint8_t*>(k),
                                static_cast<const uint8_t*>(k_scales)},
                               {static_cast<hb::KvFormat>(v_format), static_cast<const uint8_t*>(v),
                                static_cast<const uint8_t*>(v_scales)}};
            hb::attention_rows_quantized(q, qp, kv, out, s, split, static_cast<float*>(part.get()));
        }
        if (xs_hip_stream_synchronize(q) != XS_HIP_OK) throw hb::Error(xs_hip_last_error());
    });
}

int hipbe_quantize_kv_turbo() {
    return guarded([&] {
        hb::quantize_kv<float>(nullptr, hb::KvFormat::Turbo4, nullptr, nullptr, nullptr, 4, 100);  // not whole groups
    });
}

}  // extern "C"
