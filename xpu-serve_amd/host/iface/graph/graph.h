#pragma once

// The step graph the backend compiles (reference src/graph/graph.h:25-391), restated for the HIP backend's
// standalone build: the same op kinds in the same order, the same attribute structs and node layout, and the builder
// methods of the ops this backend runs (plus matmul and transpose, which it refuses by name). Symbolic dims kT (tokens
// of the step) and kL (tokens in the KV cache after the step); computed values are f32. In the reference tree the
// backend includes the reference's own header instead.

#include <cstdint>
#include <string>
#include <string_view>
#include <utility>
#include <variant>
#include <vector>

#include "io/safetensors.h"
#include "tensor/tensor.h"

namespace xs::graph {

inline constexpr int64_t kT = -1;
inline constexpr int64_t kL = -2;
inline constexpr int64_t kSliceEnd = INT64_MAX;

std::string dim_to_string(int64_t d);
std::string shape_to_string(const Dims& dims);

struct Value {
    int32_t node = -1;
    int32_t index = 0;
    bool valid() const { return node >= 0; }
    friend bool operator==(const Value&, const Value&) = default;
};

// Reference graph.h:41-92, in its order.
enum class OpKind : uint8_t {
    Input, Weight, Constant, Gather, MatMul, Add, Mul, Scale, Tanh, GeluTanh, Softcap, Sigmoid, Silu, Softplus, Clamp,
    RmsNorm, LayerNorm, Reshape, Slice, Transpose, Rope, KvCache, Attention, CausalConv, GatedDelta, Div, Softmax,
    TopK, ReduceSum, ExpertMatMul, SignMatMul, PrevRow, Concat, KvRead, Gelu, MhcRoute, StreamMix, Conv2d, L2Clip,
    DynamicConv,
};

std::string_view op_name(OpKind kind);

struct InputAttrs { std::string name; };
struct WeightAttrs { std::string name; };
struct ConstantAttrs { HostTensor value; };
struct ScaleAttrs { float factor = 1.0f; };
struct SoftcapAttrs { float cap = 0.0f; };
struct NormAttrs { float eps = 1e-6f; };
struct ReshapeAttrs { Dims shape; };
struct SliceAttrs {
    int axis = 0;
    int64_t begin = 0;
    int64_t end = kSliceEnd;
};
struct ClampAttrs {
    float lo = 0.0f;
    float hi = 0.0f;
};
struct TransposeAttrs { std::vector<int> perm; };
struct KvCacheAttrs { int slot = -1; };
struct RopeAttrs { int64_t rotary_dim = 0; };
struct TopKAttrs { int64_t k = 1; };
struct AxisAttrs { int axis = 0; };
struct L2ClipAttrs {
    float threshold = 0.0f;
    float eps = 1e-6f;
};
// Reference graph.h:200-209; the visibility rules are its comment's (graph.h:176-199).
struct AttentionAttrs {
    float scale = 1.0f;
    int64_t sliding_window = 0;
    float softcap = 0.0f;
    bool causal = true;
    int64_t block = 0;
    bool grouped = false;
    int64_t rel_extent = 0;
    bool anchored = false;
};

using Attrs = std::variant<std::monostate, InputAttrs, WeightAttrs, ConstantAttrs, ScaleAttrs, SoftcapAttrs,
                           ClampAttrs, NormAttrs, ReshapeAttrs, SliceAttrs, TransposeAttrs, KvCacheAttrs, RopeAttrs,
                           AttentionAttrs, TopKAttrs, AxisAttrs, L2ClipAttrs>;

struct TensorType {
    DType dtype = DType::F32;
    Dims shape;
};

struct Node {
    OpKind kind = OpKind::Input;
    std::vector<Value> inputs;
    Attrs attrs;
    std::vector<TensorType> outputs;
    std::string label;
};

struct KvSlot {
    int64_t num_kv_heads = 0;
    int64_t head_dim = 0;
    int64_t sliding_window = 0;
    std::string label;
};

struct GraphOutput {
    std::string name;
    Value value;
};

class Graph {
public:
    Value input(const std::string& name, DType dtype, Dims shape);
    Value weight(const WeightStore& store, const std::string& name);
    Value constant(HostTensor value);

    Value matmul(Value x, Value w);
    Value add(Value a, Value b);
    Value mul(Value a, Value b);
    Value div(Value a, Value b);
    Value scale(Value x, float factor);
    Value tanh(Value x);
    Value gelu_tanh(Value x);
    Value gelu(Value x);
    Value softcap(Value x, float cap);
    Value sigmoid(Value x);
    Value silu(Value x);
    Value softplus(Value x);
    Value clamp(Value x, float lo, float hi);
    Value rms_norm(Value x, float eps);
    Value rms_norm(Value x, Value weight, float eps);
    Value l2_clip(Value x, float threshold, float eps = 1e-6f);
    Value layer_norm(Value x, Value weight, Value bias, float eps);
    Value reshape(Value x, Dims shape);
    Value slice(Value x, int axis, int64_t begin, int64_t end = kSliceEnd);
    Value transpose(Value x, std::vector<int> perm);
    Value gather(Value table, Value ids);
    Value concat(const std::vector<Value>& parts, int axis);
    Value rope(Value x, Value positions, Value inv_freq, int64_t rotary_dim = 0, Value pair_axes = {});
    int add_kv_slot(int64_t num_kv_heads, int64_t head_dim, int64_t sliding_window, std::string label);
    std::pair<Value, Value> kv_cache(int slot, Value k, Value v);
    std::pair<Value, Value> kv_read(int slot);
    Value attention(Value q, Value k_all, Value v_all, const AttentionAttrs& attrs);
    Value softmax(Value x);
    std::pair<Value, Value> topk(Value x, int64_t k);
    Value reduce_sum(Value x, int axis);

    void output(const std::string& name, Value v);

    class Scope {
    public:
        Scope(Graph& g, std::string_view name);
        ~Scope();
        Scope(const Scope&) = delete;
        Scope& operator=(const Scope&) = delete;

    private:
        Graph& g_;
        size_t prev_size_;
    };

    const std::vector<Node>& nodes() const { return nodes_; }
    const Node& node(Value v) const;
    const TensorType& type(Value v) const;
    const std::vector<GraphOutput>& outputs() const { return outputs_; }
    const std::vector<KvSlot>& kv_slots() const { return kv_slots_; }
    bool stateful() const { return !kv_slots_.empty(); }
    bool has_fixed_state() const { return false; }
    std::vector<Value> inputs() const;

    void validate() const;
    std::string dump() const;

private:
    Value add_node(OpKind kind, std::vector<Value> inputs, Attrs attrs, std::vector<TensorType> outputs,
                   std::string_view what = {});
    Value binary(OpKind kind, Value a, Value b);
    Value unary(OpKind kind, Value x, Attrs attrs);
    std::string where(Value v) const;

    std::vector<Node> nodes_;
    std::vector<GraphOutput> outputs_;
    std::vector<KvSlot> kv_slots_;
    std::string scope_;
};

}  // namespace xs::graph
