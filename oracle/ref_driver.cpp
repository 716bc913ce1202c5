// ORACLE -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.
//
// A C ABI over the reference's own CPU path, compiled from the reference's sources where they lie (see
// oracle/Makefile) into oracle/_ref/libxsref.so. Each function builds a one-op (or few-op) step graph with the
// reference's graph builder (src/graph/graph.h:282-389), compiles it with the reference's cpu-ref backend
// (src/backend/cpu_ref/cpu_backend.h:10) and runs one Session step (src/backend/backend.h:56): the inputs go through
// the backend's own dtype normalisation (cpu_backend.cpp:62-70) and op evaluation (cpu_backend.cpp:351-526), exactly
// as the engine drives it. The int8 KV codes, which no graph output exposes, come from quant::quantize_kv_row_i8
// directly; the KV round trip also runs through the backend's KvCache append (cpu_backend.cpp:529-544).
//
// Used to write the committed golden vectors (tests/golden/gen_golden.py), to cross-check the restatement in
// oracle/oracle.cpp, and as the timed CPU baseline of bench.py when it is present. Return 0 on success, 1 on an
// xs::Error (message via xsref_last_error).
#include <cstring>
#include <limits>
#include <memory>
#include <string>
#include <vector>

#include "backend/backend.h"
#include "backend/cpu_ref/cpu_backend.h"
#include "graph/graph.h"
#include "models/common/blocks.h"
#include "quant/kv_format.h"
#include "quant/kv_turbo.h"
#include "quant/quant.h"
#include "tensor/tensor.h"
#include "util/error.h"
#include "util/half.h"

using namespace xs;
using namespace xs::graph;

namespace {

thread_local std::string g_error;

class NoWeights : public WeightStore {
public:
    const TensorView* find(const std::string&) const override { return nullptr; }
    std::vector<std::string> names() const override { return {}; }
};

DType float_dtype(int d) { return d == 0 ? DType::F32 : d == 1 ? DType::F16 : DType::BF16; }

Dims dims(const int64_t* s, int r) { return Dims(s, s + r); }

HostTensor borrow(DType t, Dims shape, const void* p) { return HostTensor::borrow(t, std::move(shape), const_cast<void*>(p)); }

TensorMap run_graph(const Graph& g, const TensorMap& inputs, const SessionOptions& opt = SessionOptions{}) {
    NoWeights w;
    SessionOptions o = opt;
    o.precision = DType::F32;
    auto backend = make_cpu_ref_backend();
    auto session = backend->compile(g, w, o);
    TensorMap out;
    session->run(inputs, out);
    return out;
}

void copy_f32(const HostTensor& t, float* dst) {
    XS_CHECK(t.dtype() == DType::F32, "expected an f32 output, got ", dtype_name(t.dtype()));
    std::memcpy(dst, t.raw(), static_cast<size_t>(t.numel()) * 4);
}

template <typename F>
int guarded(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        g_error = e.what();
        return 1;
    }
}

Value act_node(Graph& g, int act, Value x) {
    switch (act) {
        case 2: return g.gelu_tanh(x);
        case 4: return g.sigmoid(x);
        case 5: return g.silu(x);
        case 8: return g.gelu(x);
        default: fail("unknown activation ", act);
    }
}

}  // namespace

extern "C" {

const char* xsref_last_error(void) { return g_error.c_str(); }

// ---- data movement: Gather, Transpose, Concat (cpu_backend.cpp:369-370, 413-414, 479-484) ----

void copy_raw(const HostTensor& t, void* dst) {
    std::memcpy(dst, t.raw(), static_cast<size_t>(t.numel()) * dtype_size(t.dtype()));
}

// Rows ids [n] (i32, or i64 with ids_i64) of a table constant [rows, width] of DType table_dtype (F32, F16, BF16 or
// I32); out f32 [n, width], or i32 for an i32 table.
int xsref_gather(int table_dtype, const void* table, int64_t rows, int64_t width, const void* ids, int ids_i64,
                 int64_t n, void* out) {
    return guarded([&] {
        const auto td = static_cast<DType>(table_dtype);
        HostTensor t(td, {rows, width});
        std::memcpy(t.raw(), table, static_cast<size_t>(rows * width) * dtype_size(td));
        Graph g;
        const DType it = ids_i64 ? DType::I64 : DType::I32;
        g.output("out", g.gather(g.constant(t), g.input("ids", it, {n})));
        copy_raw(run_graph(g, {{"ids", borrow(it, {n}, ids)}}).at("out"), out);
    });
}

// x of DType dtype (F32, I32 or I64) and `shape`, its axes permuted by perm.
int xsref_transpose(int dtype, const void* x, const int64_t* shape, int rank, const int32_t* perm, void* out) {
    return guarded([&] {
        const auto dt = static_cast<DType>(dtype);
        Graph g;
        g.output("out", g.transpose(g.input("x", dt, dims(shape, rank)), std::vector<int>(perm, perm + rank)));
        copy_raw(run_graph(g, {{"x", borrow(dt, dims(shape, rank), x)}}).at("out"), out);
    });
}

// `count` parts of DType dtype (F32, I32 or I64), part k of shape shapes[k * rank .. k * rank + rank), joined along
// `axis`.
int xsref_concat(int dtype, int count, const void* const* parts, const int64_t* shapes, int rank, int axis,
                 void* out) {
    return guarded([&] {
        const auto dt = static_cast<DType>(dtype);
        Graph g;
        std::vector<Value> vs;
        TensorMap in;
        for (int k = 0; k < count; ++k) {
            const std::string name = "p" + std::to_string(k);
            vs.push_back(g.input(name, dt, dims(shapes + k * rank, rank)));
            in.emplace(name, borrow(dt, dims(shapes + k * rank, rank), parts[k]));
        }
        g.output("out", g.concat(vs, axis));
        copy_raw(run_graph(g, in).at("out"), out);
    });
}

// ---- util/half ----
void xsref_f32_to_f16(const float* x, uint16_t* y, int64_t n) { convert_f32_to_f16(x, y, static_cast<size_t>(n)); }
void xsref_f16_to_f32(const uint16_t* x, float* y, int64_t n) { convert_f16_to_f32(x, y, static_cast<size_t>(n)); }
void xsref_bf16_to_f32(const uint16_t* x, float* y, int64_t n) { convert_bf16_to_f32(x, y, static_cast<size_t>(n)); }
void xsref_f32_to_bf16(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = f32_to_bf16(x[i]);
}

// out = a op b (op 0 Add, 1 Mul, 2 Div) through the backend; a and b of float dtype a_dtype / b_dtype.
int xsref_binary(int op, int a_dtype, const void* a, const int64_t* a_shape, int a_rank, int b_dtype, const void* b,
                 const int64_t* b_shape, int b_rank, float* out) {
    return guarded([&] {
        Graph g;
        const Value va = g.input("a", float_dtype(a_dtype), dims(a_shape, a_rank));
        const Value vb = g.input("b", float_dtype(b_dtype), dims(b_shape, b_rank));
        g.output("out", op == 0 ? g.add(va, vb) : op == 1 ? g.mul(va, vb) : g.div(va, vb));
        const TensorMap res = run_graph(g, {{"a", borrow(float_dtype(a_dtype), dims(a_shape, a_rank), a)},
                                            {"b", borrow(float_dtype(b_dtype), dims(b_shape, b_rank), b)}});
        copy_f32(res.at("out"), out);
    });
}

// out [rows, cols] = act(x + bias) * up (no Add when bias is null), x/up/bias of float dtype `dtype`, contiguous.
int xsref_act_bias_mul(int act, int dtype, const void* x, const void* up, const void* bias, int64_t rows, int64_t cols,
                       float* out) {
    return guarded([&] {
        const DType t = float_dtype(dtype);
        Graph g;
        Value gate = g.input("gate", t, {rows, cols});
        TensorMap in{{"gate", borrow(t, {rows, cols}, x)}, {"up", borrow(t, {rows, cols}, up)}};
        if (bias != nullptr) {
            gate = g.add(gate, g.input("bias", t, {cols}));
            in.emplace("bias", borrow(t, {cols}, bias));
        }
        g.output("out", g.mul(act_node(g, act, gate), g.input("up", t, {rows, cols})));
        copy_f32(run_graph(g, in).at("out"), out);
    });
}

// Softmax(Add(Scale(x, scale), mask)), mask 0 before valid_len[row] (or valid_all) and -inf from there.
int xsref_softmax_masked(const float* x, int64_t rows, int64_t width, float scale, const int64_t* valid_len,
                         int64_t valid_all, int apply_scale_and_mask, float* out) {
    return guarded([&] {
        Graph g;
        Value s = g.input("x", DType::F32, {rows, width});
        TensorMap in{{"x", borrow(DType::F32, {rows, width}, x)}};
        HostTensor mask(DType::F32, {rows, width});
        if (apply_scale_and_mask) {
            for (int64_t r = 0; r < rows; ++r) {
                const int64_t valid = valid_len != nullptr ? valid_len[r] : valid_all;
                for (int64_t i = 0; i < width; ++i)
                    mask.data<float>()[r * width + i] = i < valid ? 0.0f : -std::numeric_limits<float>::infinity();
            }
            s = g.add(g.scale(s, scale), g.input("mask", DType::F32, {rows, width}));
            in.emplace("mask", mask);
        }
        g.output("out", g.softmax(s));
        copy_f32(run_graph(g, in).at("out"), out);
    });
}

// out = rms_norm(x, w) (w may be null), x of float dtype x_dtype.
int xsref_rms_norm(int x_dtype, const void* x, const float* w, float eps, int64_t rows, int64_t width, float* out) {
    return guarded([&] {
        Graph g;
        const Value vx = g.input("x", float_dtype(x_dtype), {rows, width});
        Value y;
        if (w != nullptr) {
            HostTensor wt(DType::F32, {width});
            std::memcpy(wt.raw(), w, static_cast<size_t>(width) * 4);
            y = g.rms_norm(vx, g.constant(wt), eps);
        } else {
            y = g.rms_norm(vx, eps);
        }
        g.output("out", y);
        copy_f32(run_graph(g, {{"x", borrow(float_dtype(x_dtype), {rows, width}, x)}}).at("out"), out);
    });
}

// h = Add(x, residual); out = RmsNorm(h, w): both outputs.
int xsref_add_rms_norm(const float* x, const float* residual, const float* w, float eps, int64_t rows, int64_t width,
                       float* h_out, float* out) {
    return guarded([&] {
        Graph g;
        const Value h = g.add(g.input("x", DType::F32, {rows, width}), g.input("r", DType::F32, {rows, width}));
        HostTensor wt(DType::F32, {width});
        std::memcpy(wt.raw(), w, static_cast<size_t>(width) * 4);
        g.output("h", h);
        g.output("out", g.rms_norm(h, g.constant(wt), eps));
        const TensorMap res = run_graph(
            g, {{"x", borrow(DType::F32, {rows, width}, x)}, {"r", borrow(DType::F32, {rows, width}, residual)}});
        copy_f32(res.at("h"), h_out);
        copy_f32(res.at("out"), out);
    });
}

int xsref_topk(const float* x, int64_t rows, int64_t width, int64_t k, float* values, int32_t* indices) {
    return guarded([&] {
        Graph g;
        const auto [v, i] = g.topk(g.input("x", DType::F32, {rows, width}), k);
        g.output("values", v);
        g.output("indices", i);
        const TensorMap res = run_graph(g, {{"x", borrow(DType::F32, {rows, width}, x)}});
        copy_f32(res.at("values"), values);
        const HostTensor& it = res.at("indices");
        XS_CHECK(it.dtype() == DType::I32, "topk indices are not i32");
        std::memcpy(indices, it.raw(), static_cast<size_t>(it.numel()) * 4);
    });
}

// Rope of x [tokens, heads, dim] (float dtype x_dtype); positions [tokens] (sections 1, no pair_axes) or
// [tokens, sections], i32 or i64; pair_axes i32 [rotary / 2] or null.
int xsref_rope(int x_dtype, const void* x, int64_t tokens, int64_t heads, int64_t dim, const void* positions,
               int pos_is_i64, int64_t sections, const float* inv_freq, int64_t n_freq, int64_t rotary,
               const int32_t* pair_axes, float* out) {
    return guarded([&] {
        Graph g;
        const DType pt = pos_is_i64 ? DType::I64 : DType::I32;
        const Dims pshape = (sections == 1 && pair_axes == nullptr) ? Dims{tokens} : Dims{tokens, sections};
        const Value vx = g.input("x", float_dtype(x_dtype), {tokens, heads, dim});
        const Value vp = g.input("pos", pt, pshape);
        HostTensor ft(DType::F32, {n_freq});
        std::memcpy(ft.raw(), inv_freq, static_cast<size_t>(n_freq) * 4);
        Value axes;
        if (pair_axes != nullptr) {
            HostTensor at(DType::I32, {(rotary == 0 ? dim : rotary) / 2});
            std::memcpy(at.raw(), pair_axes, static_cast<size_t>(at.numel()) * 4);
            axes = g.constant(at);
        }
        g.output("out", g.rope(vx, vp, g.constant(ft), rotary, axes));
        const TensorMap res =
            run_graph(g, {{"x", borrow(float_dtype(x_dtype), {tokens, heads, dim}, x)}, {"pos", borrow(pt, pshape, positions)}});
        copy_f32(res.at("out"), out);
    });
}

// y = op(x) for the unary family by UnaryOp value (0 Scale, 1 Tanh, 2 GeluTanh, 3 Softcap, 4 Sigmoid, 5 Silu,
// 6 Softplus, 7 Clamp, 8 Gelu), a / b the op's parameters; f32 [n].
int xsref_unary(int op, const float* x, int64_t n, float a, float b, float* out) {
    return guarded([&] {
        Graph g;
        const Value v = g.input("x", DType::F32, {n});
        Value y;
        switch (op) {
            case 0: y = g.scale(v, a); break;
            case 1: y = g.tanh(v); break;
            case 2: y = g.gelu_tanh(v); break;
            case 3: y = g.softcap(v, a); break;
            case 4: y = g.sigmoid(v); break;
            case 5: y = g.silu(v); break;
            case 6: y = g.softplus(v); break;
            case 7: y = g.clamp(v, a, b); break;
            case 8: y = g.gelu(v); break;
            default: fail("unknown unary op ", op);
        }
        g.output("out", y);
        copy_f32(run_graph(g, {{"x", borrow(DType::F32, {n}, x)}}).at("out"), out);
    });
}

// LayerNorm(Add(x, shift) or x, w, b) over rows of `width`, f32; shift may be null, w and b may not.
int xsref_layer_norm(const float* x, const float* shift, const float* w, const float* b, float eps, int64_t rows,
                     int64_t width, float* out) {
    return guarded([&] {
        Graph g;
        Value h = g.input("x", DType::F32, {rows, width});
        auto row = [&](const float* p) {
            HostTensor t(DType::F32, {width});
            std::memcpy(t.raw(), p, static_cast<size_t>(width) * 4);
            return g.constant(t);
        };
        if (shift != nullptr) h = g.add(h, row(shift));
        g.output("out", g.layer_norm(h, row(w), row(b), eps));
        copy_f32(run_graph(g, {{"x", borrow(DType::F32, {rows, width}, x)}}).at("out"), out);
    });
}

int xsref_l2_clip(const float* x, int64_t rows, int64_t width, float threshold, float eps, float* out) {
    return guarded([&] {
        Graph g;
        g.output("out", g.l2_clip(g.input("x", DType::F32, {rows, width}), threshold, eps));
        copy_f32(run_graph(g, {{"x", borrow(DType::F32, {rows, width}, x)}}).at("out"), out);
    });
}

// ReduceSum over axis 1 of x [outer, dim, inner].
int xsref_reduce_sum(const float* x, int64_t outer, int64_t dim, int64_t inner, float* out) {
    return guarded([&] {
        Graph g;
        g.output("out", g.reduce_sum(g.input("x", DType::F32, {outer, dim, inner}), 1));
        copy_f32(run_graph(g, {{"x", borrow(DType::F32, {outer, dim, inner}, x)}}).at("out"), out);
    });
}

// Attention with AttentionAttrs {scale, sliding_window, softcap, causal}. Causal or windowed attention is driven as the
// engine drives it: one prefill step of `kv_len` tokens whose keys and values go through a KvCache slot (kv_i8: the
// session's int8 cache, so the backend itself stores the round-tripped values) and whose queries q [kv_len, Hq, D] all
// attend; the caller keeps the rows it wants. Otherwise q [tokens, Hq, D] attends to k, v [kv_len, Hkv, D] directly.
int xsref_attention(const float* q, const float* k, const float* v, int64_t tokens, int64_t q_heads, int64_t kv_heads,
                    int64_t head_dim, int64_t kv_len, float scale, float softcap, int64_t window, int causal, int kv_i8,
                    float* out) {
    return guarded([&] {
        Graph g;
        AttentionAttrs attrs;
        attrs.scale = scale;
        attrs.softcap = softcap;
        attrs.sliding_window = window;
        attrs.causal = causal != 0;
        SessionOptions o;
        TensorMap in;
        const Dims kd{kv_len, kv_heads, head_dim};
        if (causal || window > 0 || kv_i8) {
            XS_CHECK(tokens == kv_len, "a cached attention step takes as many queries as keys");
            const int slot = g.add_kv_slot(kv_heads, head_dim, 0, "kv");
            const auto [ka, va] = g.kv_cache(slot, g.input("k", DType::F32, {kT, kv_heads, head_dim}),
                                             g.input("v", DType::F32, {kT, kv_heads, head_dim}));
            g.output("out", g.attention(g.input("q", DType::F32, {kT, q_heads, head_dim}), ka, va, attrs));
            o.max_context = kv_len;
            if (kv_i8) o.kv = quant::KvFormats{quant::KvFormat::I8, quant::KvFormat::I8};
        } else {
            g.output("out", g.attention(g.input("q", DType::F32, {tokens, q_heads, head_dim}),
                                        g.input("k", DType::F32, kd), g.input("v", DType::F32, kd), attrs));
        }
        in.emplace("q", borrow(DType::F32, {tokens, q_heads, head_dim}, q));
        in.emplace("k", borrow(DType::F32, kd, k));
        in.emplace("v", borrow(DType::F32, kd, v));
        copy_f32(run_graph(g, in, o).at("out"), out);
    });
}

int xsref_rope_inv_freq(double theta, int64_t dim, int64_t pairs, int64_t length, float* out) {
    return guarded([&] { copy_f32(blocks::rope_inv_freq(theta, dim, pairs, length), out); });
}

float xsref_quantize_kv_row_i8(const float* x, int64_t width, int8_t* codes) {
    return quant::quantize_kv_row_i8(x, width, codes);
}

void xsref_round_trip_kv_i8(float* x, int64_t rows, int64_t width) { quant::round_trip_kv_i8(x, rows, width); }

// quantize_kv_row_i8 over `rows` rows in one call (codes [rows, width], scales [rows]): the reference's quantize loop
// without a Python call per row, for timing.
void xsref_quantize_kv_rows(const float* x, int64_t rows, int64_t width, int8_t* codes, float* scales) {
    for (int64_t r = 0; r < rows; ++r) scales[r] = quant::quantize_kv_row_i8(x + r * width, width, codes + r * width);
}

// The KV rows a session's int8 cache holds after appending k, v [tokens, kv_heads, head_dim] (float dtype `dtype`):
// KvCache through the backend with kv = i8 for keys and values.
int xsref_kv_cache_i8(int dtype, const void* k, const void* v, int64_t tokens, int64_t kv_heads, int64_t head_dim,
                      float* k_out, float* v_out) {
    return guarded([&] {
        Graph g;
        const int slot = g.add_kv_slot(kv_heads, head_dim, 0, "kv");
        const auto [ka, va] = g.kv_cache(slot, g.input("k", float_dtype(dtype), {kT, kv_heads, head_dim}),
                                         g.input("v", float_dtype(dtype), {kT, kv_heads, head_dim}));
        g.output("k_all", ka);
        g.output("v_all", va);
        SessionOptions o;
        o.kv = quant::KvFormats{quant::KvFormat::I8, quant::KvFormat::I8};
        o.max_context = tokens;
        const TensorMap res = run_graph(g, {{"k", borrow(float_dtype(dtype), {tokens, kv_heads, head_dim}, k)},
                                            {"v", borrow(float_dtype(dtype), {tokens, kv_heads, head_dim}, v)}},
                                        o);
        copy_f32(res.at("k_all"), k_out);
        copy_f32(res.at("v_all"), v_out);
    });
}

// TurboQuant groups through the reference's own functions (src/quant/kv_turbo.cpp): codes, f16 norms, decoded
// (rotated) values, the rotation.
void xsref_turbo_quantize(const float* x, int64_t groups, int bits, uint8_t* codes, uint16_t* norms) {
    for (int64_t g = 0; g < groups; ++g)
        norms[g] = quant::turbo::quantize_group(x + g * quant::turbo::kGroup, bits,
                                                codes + g * quant::turbo::group_bytes(bits));
}

void xsref_turbo_decode(const uint8_t* codes, const uint16_t* norms, int64_t groups, int bits, float* out) {
    for (int64_t g = 0; g < groups; ++g)
        quant::turbo::decode_group(codes + g * quant::turbo::group_bytes(bits), norms[g], bits,
                                   out + g * quant::turbo::kGroup);
}

void xsref_turbo_rotate(float* x, int64_t groups, int inverse) {
    for (int64_t g = 0; g < groups; ++g) quant::turbo::rotate_group(x + g * quant::turbo::kGroup, inverse != 0);
}

}  // extern "C"
