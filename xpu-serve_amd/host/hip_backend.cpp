// The HIP backend: xs::Backend and xs::Session (reference src/backend/backend.h:46-92) on an MI355X (gfx950), running
// step graphs through the kernels of libxs_hip.so (include/xs_hip.h).
//
// It is written against the reference's interface headers -- graph/graph.h, backend/backend.h, tensor/tensor.h,
// io/safetensors.h, quant/kv_format.h, util/error.h -- and compiles unchanged against the restatement of them beside
// it (host/iface) or against the reference's own (src/), where it is the backend registry.cpp adds under XS_HAVE_HIP.
//
// What a session does, per program (cf. the SYCL session, src/backend/sycl/sycl_backend.cpp):
//  - compile: validates the graph, refuses by name every op it has no kernel for, plans fusions (below), uploads
//    weights and constants once (in their stored dtype, plus an f32 copy where a kernel reads f32), and sizes the
//    KV slots, shared by label between the programs, for SessionOptions::max_context tokens;
//  - run: resolves T from the inputs (and L from the slots), plans the step's activations into one device arena by
//    liveness (cached per T and `only` set), uploads the inputs, launches the steps in graph order on the session's
//    stream, and copies the requested outputs back as f32 (integer outputs in their dtype). Slots advance only after
//    every launch went in, so a refused step leaves the state as it was. Host copies go through page-locked staging,
//    asynchronously, and the step waits once. A step that repeats (same plan, same power-of-two bucket of L) is
//    captured into a HIP graph and replayed (the "graphs" backend option, on by default): where the KV append writes
//    and how many keys the attention reads come from a device-resident step record, so one capture serves every L of
//    its bucket (Program::launch_all).
//
// Fusions (static, per program), each one launch for what the graph spells as several nodes; a node is folded into
// its consumer only when that consumer is its sole reader and it is not a graph output:
//  - Mul(act(x), b) and Mul(act(Add(x, bias)), b), act in {Silu, GeluTanh, Sigmoid, Gelu}, bias a row vector: one
//    act-bias-mul over row-strided operands, so x and b may be column slices of one buffer (a fused gate|up
//    projection), read in place (sycl_backend.cpp:1004-1047 fuses the first two forms);
//  - act(Add(x, b)), b a row vector: one unary-bias launch (sycl_backend.cpp:1031-1047);
//  - Add(a, Add(b, c)) and Add(a, Mul(b, c)), c a row vector or full: add3 / add_mul (sycl_backend.cpp:1048-1098);
//  - Add(RmsNorm(x [, w]), c), c a row vector: the norm with a bias (sycl_backend.cpp:1062-1068);
//  - LayerNorm(Add(x, c)), c a row vector: the norm with a shift (sycl_backend.cpp:1100-1118);
//  - RmsNorm(Add(x, r) [, w]): one pass that writes the sum (the updated residual stream, still read by later nodes)
//    and the norm (no reference counterpart: the reference launches the add and the norm);
//  - two Ropes of the same positions and frequencies (a step's Q and K): one launch (no reference counterpart);
//  - a KvCache's keys and values, of one dtype: one quantize launch (no reference counterpart).
// Reshape is a view; Slice is a view when it keeps whole leading rows or only an act-bias-mul reads it, else a copy.
//
// KV formats (SessionOptions::kv): every pair the reference's device takes -- the Float format (rows of the
// precision's float: f16 at f16 precision, the reference's default; f32 at f32), as the SYCL session stores them; i8
// keys and values (int8 codes and f32 scales); a TurboQuant format for both (codes and f16 norms per 128 values); or i8
// keys with TurboQuant values. SessionOptions::precision is f16 or f32, as for cpu-ref (cpu_backend.cpp:75-76), and as there
// the activations are computed and kept in f32 either way (cpu_backend.cpp:611); the precision picks the Float
// format's row type.
//
// What it refuses: MatMul and the other ops with no kernel here (the GEMM path is outside this library), a precision
// other than f16 or f32, the KV format pairs the reference's device refuses too, a TurboQuant format over a head_dim
// that is not a multiple of 128, KV outputs read by anything but Attention, and attention with a key bias, groups,
// blocks, relative bias or an anchored window.
#include <algorithm>
#include <cstring>
#include <limits>
#include <map>
#include <memory>
#include <set>
#include <string>
#include <utility>
#include <variant>
#include <vector>

#include "backend/backend.h"
#include "util/error.h"
#include "xs_hip.h"

namespace xs {
namespace {

using graph::Graph;
using graph::kL;
using graph::kT;
using graph::Node;
using graph::OpKind;
using graph::Value;

void check(int rc, std::string_view what) {
    if (rc != XS_HIP_OK) fail("hip: ", what, ": ", xs_hip_last_error());
}

xs_dtype abi(DType t) {
    switch (t) {
        case DType::F32: return XS_F32;
        case DType::F16: return XS_F16;
        case DType::BF16: return XS_BF16;
        case DType::I64: return XS_I64;
        case DType::I32: return XS_I32;
        case DType::I8: return XS_I8;
        case DType::U8: return XS_U8;
        case DType::Bool: return XS_BOOL;
        default: fail("hip: dtype ", dtype_name(t), " is not a dense element type");
    }
}

size_t align_up(size_t n) { return (n + 255) & ~size_t{255}; }
// A node whose launch uses the session's zero-filled sync scratch rather than an arena block.
constexpr int32_t kSyncScratch = -2;

// Device memory owned by the session.
class DeviceMemory {
public:
    DeviceMemory() = default;
    explicit DeviceMemory(size_t bytes) { grow(bytes); }
    DeviceMemory(const DeviceMemory&) = delete;
    DeviceMemory& operator=(const DeviceMemory&) = delete;
    DeviceMemory(DeviceMemory&& o) noexcept : p_(std::exchange(o.p_, nullptr)), n_(std::exchange(o.n_, 0)) {}
    DeviceMemory& operator=(DeviceMemory&& o) noexcept {
        std::swap(p_, o.p_);
        std::swap(n_, o.n_);
        return *this;
    }
    ~DeviceMemory() {
        if (p_ != nullptr) xs_hip_free(p_);
    }
    // At least `bytes`; the contents are not kept when it grows. True when the memory moved.
    bool grow(size_t bytes) {
        if (bytes <= n_) return false;
        if (p_ != nullptr) check(xs_hip_free(p_), "free");
        p_ = nullptr;
        n_ = 0;
        check(xs_hip_malloc(&p_, std::max<size_t>(bytes, 256)), "malloc");
        n_ = std::max<size_t>(bytes, 256);
        return true;
    }
    char* get() const { return static_cast<char*>(p_); }
    size_t size() const { return n_; }

private:
    void* p_ = nullptr;
    size_t n_ = 0;
};

// Page-locked host memory owned by the session: the staging of a step's host copies, which then run asynchronously.
class PinnedMemory {
public:
    PinnedMemory() = default;
    PinnedMemory(const PinnedMemory&) = delete;
    PinnedMemory& operator=(const PinnedMemory&) = delete;
    ~PinnedMemory() {
        if (p_ != nullptr) xs_hip_host_free(p_);
    }
    // At least `bytes`; the contents are not kept when it grows (only between steps, when no copy is pending).
    void grow(size_t bytes) {
        if (bytes <= n_) return;
        if (p_ != nullptr) check(xs_hip_host_free(p_), "free");
        p_ = nullptr;
        n_ = 0;
        check(xs_hip_host_alloc(&p_, bytes), "host alloc");
        n_ = bytes;
    }
    char* get() const { return static_cast<char*>(p_); }

private:
    void* p_ = nullptr;
    size_t n_ = 0;
};

// f32 from IEEE binary16 / bfloat16 bits, exactly (the widening of the reference's util/half.h).
float widen(DType t, uint16_t h) {
    uint32_t bits;
    if (t == DType::BF16) {
        bits = static_cast<uint32_t>(h) << 16;
    } else {
        const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
        const uint32_t exp = (h >> 10) & 0x1fu;
        uint32_t man = h & 0x3ffu;
        if (exp == 0x1f) {
            bits = sign | 0x7f800000u | (man << 13);
        } else if (exp != 0) {
            bits = sign | ((exp + 112) << 23) | (man << 13);
        } else if (man == 0) {
            bits = sign;
        } else {  // subnormal: normalize
            int e = -1;
            do {
                man <<= 1;
                ++e;
            } while ((man & 0x400u) == 0);
            bits = sign | (static_cast<uint32_t>(112 - e) << 23) | ((man & 0x3ffu) << 13);
        }
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// ---------------------------------------------------------------------------------------------------------------
// The static plan of a program.

enum class Op : uint8_t {
    None,        // no launch: a leaf, an input, a view, a KV read, or computed in another node's launch
    Binary,      // Add / Mul / Div with broadcasting
    Unary,       // Scale ... Gelu
    ActMul,      // act(x [+ bias]) * b over row-strided operands; reads {x, b [, bias]}
    UnaryBias,   // act(x + bias); reads {x, bias}
    Add3,        // a + (b + c); reads {a, b, c}
    AddMul,      // a + b * c; reads {a, b, c}
    RmsNorm,     // reads {x [, w] [, bias]}
    AddRmsNorm,  // h = x + r (into the Add node's memory), y = rms_norm(h) [* w]; reads {x, r [, w]}
    LayerNorm,   // reads {x, w, b [, shift]}
    L2Clip,
    Softmax,
    TopK,
    ReduceSum,
    Rope,        // reads {x, positions, inv_freq [, pair_axes]}; with a partner, both ropes in one launch
    KvAppend,    // quantizes the step's k, v into the slot
    Attention,   // reads {q, k_all, v_all}
    SliceCopy,   // a Slice that must be contiguous
    Gather,      // rows of a table by ids; reads {table, ids}
    Transpose,   // reads {x}
    Concat,      // reads the parts
};

struct NodePlan {
    Op op = Op::None;
    std::vector<Value> reads;
    int act = -1;              // xs_unary_op of Unary / ActMul / UnaryBias
    bool has_w = false;        // RmsNorm / AddRmsNorm: a weight among the reads
    bool has_bias = false;     // ActMul, RmsNorm: a bias last among the reads; LayerNorm: a shift
    int32_t partner = -1;      // Rope: the other rope of the launch; AddRmsNorm: the Add it writes
    int32_t run_at = -1;       // a node computed inside another node's launch: that node
    bool folded = false;       // its value exists only inside that launch (no memory of its own)
    bool strided_view = false; // Slice read in place by act-bias-muls
};

// A value's storage in a run.
enum class Where : uint8_t { None, Arena, Leaf, LeafF32, Slot };
struct Loc {
    Where where = Where::None;
    int32_t id = -1;      // arena block, leaf node, or slot
    int which = 0;        // slot: 0 keys, 1 values
    int64_t offset = 0;   // bytes from the block's / leaf's start
    int64_t row_stride = 0;  // strided views: bytes between rows (0: contiguous)
};

// Bytes of one row (a token's head of `dim` values) of a quantized format: its codes, and the scales beside them
// (quant::kv_row_bytes, reference src/quant/kv_format.cpp:45-55).
int64_t kv_code_bytes(quant::KvFormat f, int64_t dim) {
    const int bits = quant::turbo_bits(f);
    return bits == 0 ? dim : dim / 128 * 16 * bits;
}
int64_t kv_scale_bytes(quant::KvFormat f, int64_t dim) { return quant::turbo_bits(f) == 0 ? 4 : dim / 128 * 2; }
xs_kv_format kv_abi(quant::KvFormat f) { return static_cast<xs_kv_format>(static_cast<int>(f)); }

struct KvState {
    int64_t heads = 0, dim = 0, cap = 0;
    int64_t len = 0;
    // What the slot stores (SessionOptions::kv), for the keys (kc, ks) and the values (vc, vs): I8 -- codes int8
    // [cap, heads, dim] and scales f32 [cap, heads]; a TurboQuant format -- codes [cap * heads * dim / 128, 16 bits]
    // bytes and f16 norms [cap * heads * dim / 128]; or, both streams alike, the Float format's rows [cap, heads,
    // dim] of F16 (f16 precision) or F32 in kc / vc. `rows` is the Float format's row type, I8 for the others.
    DType rows = DType::I8;
    quant::KvFormat kf = quant::KvFormat::I8, vf = quant::KvFormat::I8;
    bool both_i8() const { return kf == quant::KvFormat::I8 && vf == quant::KvFormat::I8; }
    DeviceMemory kc, ks, vc, vs;
    std::string label;
};

struct Leaf {
    DeviceMemory data;  // stored dtype
    DeviceMemory f32;   // an f32 copy, for float leaves some kernel reads as f32
    DType dtype = DType::F32;
};

class HipSession;

// One compiled program.
class Program {
public:
    Program(const Graph& g, HipSession& s, size_t index);  // plans; touches no device
    ~Program();
    Program(const Program&) = delete;
    Program& operator=(const Program&) = delete;
    void upload();                                          // weights and constants to the device

    void run(const TensorMap& inputs, TensorMap& outputs, std::span<const std::string> only);
    int64_t cached() const;
    void truncate(int64_t n);

private:
    struct RunPlan {
        std::vector<std::vector<Dims>> shapes;  // resolved per value
        std::vector<std::vector<Loc>> locs;
        std::vector<char> live;                 // nodes whose launch runs
        std::vector<int32_t> conv;              // per (node, output 0): arena block of its f32 conversion, or -1
        std::vector<std::vector<Value>> convert_before;  // per node: values converted to f32 before its launch
        std::vector<size_t> block_offset;       // arena offset of each block
        std::vector<int32_t> scratch;           // per node: its scratch block, -1, or kSyncScratch
        std::vector<size_t> scratch_bytes;
        size_t arena_bytes = 0;
        size_t sync_bytes = 0;                  // the session's zero-filled scratch the step's launches need
        // Captured steps by key-count bucket (see Program::run): the executable graph, the arena generation its
        // addresses belong to, and how often the bucket has run.
        struct Captured {
            void* exec = nullptr;
            uint64_t arena_gen = 0;
            int runs = 0;
        };
        std::map<int, Captured> graphs;
    };

    const std::vector<char>& live_for(std::span<const std::string> only);
    RunPlan& plan_for(int64_t T, std::span<const std::string> only);
    Dims resolve(const Dims& d, int64_t T, int64_t L) const;
    bool needs_f32(size_t node, size_t operand) const;
    // replay_cap > 0: the launch goes into a captured graph, the KV append and attention read the step record
    // (first row, key count) from device memory, and the attention's split is the one of replay_cap keys.
    void launch(size_t i, const RunPlan& p, int64_t T, int64_t L, int64_t replay_cap = 0);
    void launch_all(RunPlan& p, int64_t T, int64_t L);
    char* ptr(const RunPlan& p, Value v) const;
    const char* ptr_f32(const RunPlan& p, Value v) const;
    DType dtype(Value v) const { return dt_[static_cast<size_t>(v.node)][static_cast<size_t>(v.index)]; }
    size_t base_node(Value v) const;
    std::string leaf_key(size_t node) const;

    Graph g_;
    HipSession& s_;
    size_t index_;
    std::vector<NodePlan> plan_;
    std::vector<std::vector<DType>> dt_;  // device dtype of every value
    std::vector<int> slot_of_;            // graph KV slot -> session slot
    bool appends_ = false, reads_kv_ = false;
    std::map<std::string, std::vector<char>> live_;
    std::map<std::pair<int64_t, std::string>, RunPlan> plans_;
};

class HipSession final : public Session {
public:
    HipSession(std::span<const Graph* const> programs, const WeightStore& weights, const SessionOptions& options);
    ~HipSession() override {
        if (stream_ != nullptr) xs_hip_stream_destroy(stream_);
    }

    void run(size_t program, const TensorMap& inputs, TensorMap& outputs, std::span<const std::string> only) override {
        XS_CHECK(program < programs_.size(), "hip: no program ", program, " (", programs_.size(), " compiled)");
        programs_[program]->run(inputs, outputs, only);
    }
    int64_t num_cached(size_t program) const override {
        XS_CHECK(program < programs_.size(), "hip: no program ", program);
        return programs_[program]->cached();
    }
    void reset() override {
        for (KvState& k : kv_) k.len = 0;
    }
    void truncate(size_t program, int64_t n) override {
        XS_CHECK(program < programs_.size(), "hip: no program ", program);
        programs_[program]->truncate(n);
    }

    void* stream() const { return stream_; }
    const WeightStore& weights() const { return weights_; }
    const SessionOptions& options() const { return options_; }
    std::vector<KvState>& kv() { return kv_; }
    // Device copies of leaves: weights by name ("w:<name>", shared by the programs), constants by program and node.
    std::map<std::string, Leaf>& leaves() { return leaves_; }
    DeviceMemory& arena() { return arena_; }
    // Grows the arena; when it moves, every captured step (which holds its addresses) is stale.
    void grow_arena(size_t bytes) {
        if (arena_.grow(bytes)) ++arena_gen_;
    }
    uint64_t arena_gen() const { return arena_gen_; }
    // Scratch of the launches whose workgroups combine partials within one launch (the split softmax): zero-filled
    // when allocated, and every such launch leaves it ready for the next, so the session's launches (one stream, in
    // order) share it. Growing it moves it, as the arena.
    char* sync() const { return sync_.get(); }
    void grow_sync(size_t bytes) {
        if (bytes == 0 || !sync_.grow(bytes)) return;
        check(xs_hip_memset(sync_.get(), 0, sync_.size(), stream_), "sync scratch");
        ++arena_gen_;
    }
    // HIP-graph replay of repeated steps: the "graphs" backend option ("1", the default, or "0").
    bool graphs() const { return graphs_; }
    // The step record a replayed step reads from device memory: [first token the step appends, keys held]. Its host
    // copy is the first 16 bytes of the staging.
    const int64_t* step_record() const { return reinterpret_cast<const int64_t*>(step_.get()); }
    void set_step(int64_t first, int64_t keys) {
        auto* h = reinterpret_cast<int64_t*>(staging_.get());
        h[0] = first;
        h[1] = keys;
        check(xs_hip_memcpy_h2d_async(step_.get(), h, 2 * sizeof(int64_t), stream_), "step record");
    }
    // The step's host staging: the step record, then the inputs and outputs (256-byte aligned pieces).
    char* staging(size_t bytes) {
        staging_.grow(std::max<size_t>(bytes, 256));
        return staging_.get();
    }

    int slot_for(const graph::KvSlot& s) {
        for (size_t i = 0; i < kv_.size(); ++i) {
            if (kv_[i].label == s.label) {
                XS_CHECK(kv_[i].heads == s.num_kv_heads && kv_[i].dim == s.head_dim, "hip: kv slot '", s.label,
                         "' declared with different shapes by two programs");
                return static_cast<int>(i);
            }
        }
        KvState k;  // its memory comes with the device, after every program is planned
        k.heads = s.num_kv_heads;
        k.dim = s.head_dim;
        k.cap = options_.max_context;
        k.label = s.label;
        k.kf = options_.kv.k;
        k.vf = options_.kv.v;
        k.rows = options_.kv.k == quant::KvFormat::Float ? options_.precision : DType::I8;
        XS_CHECK((quant::turbo_bits(k.kf) == 0 && quant::turbo_bits(k.vf) == 0) || k.dim % 128 == 0,
                 "hip: kv slot '", s.label, "': a TurboQuant KV format needs a head_dim that is a multiple of 128, got ",
                 k.dim);
        kv_.push_back(std::move(k));
        return static_cast<int>(kv_.size() - 1);
    }

private:
    const WeightStore& weights_;
    SessionOptions options_;
    void* stream_ = nullptr;
    std::vector<KvState> kv_;
    std::map<std::string, Leaf> leaves_;
    DeviceMemory arena_;
    DeviceMemory sync_;
    uint64_t arena_gen_ = 0;
    bool graphs_ = true;
    DeviceMemory step_;
    PinnedMemory staging_;
    std::vector<std::unique_ptr<Program>> programs_;
};

// ---------------------------------------------------------------------------------------------------------------
// Compile.

int act_of(OpKind k) {
    switch (k) {
        case OpKind::Silu: return XS_UNARY_SILU;
        case OpKind::GeluTanh: return XS_UNARY_GELU_TANH;
        case OpKind::Sigmoid: return XS_UNARY_SIGMOID;
        case OpKind::Gelu: return XS_UNARY_GELU;
        default: return -1;
    }
}

int unary_of(OpKind k) {
    switch (k) {
        case OpKind::Scale: return XS_UNARY_SCALE;
        case OpKind::Tanh: return XS_UNARY_TANH;
        case OpKind::GeluTanh: return XS_UNARY_GELU_TANH;
        case OpKind::Softcap: return XS_UNARY_SOFTCAP;
        case OpKind::Sigmoid: return XS_UNARY_SIGMOID;
        case OpKind::Silu: return XS_UNARY_SILU;
        case OpKind::Softplus: return XS_UNARY_SOFTPLUS;
        case OpKind::Clamp: return XS_UNARY_CLAMP;
        case OpKind::Gelu: return XS_UNARY_GELU;
        default: return -1;
    }
}

Program::Program(const Graph& g, HipSession& s, size_t index) : g_(g), s_(s), index_(index) {
    g_.validate();
    const auto& nodes = g_.nodes();
    const size_t n = nodes.size();
    const auto where = [&](size_t i) {
        return str_cat("node ", i, " (", nodes[i].label.empty() ? "-" : nodes[i].label, ": ",
                       graph::op_name(nodes[i].kind), ")");
    };

    // Device dtypes: inputs and leaves as given, computed values f32 (TopK indices i32), views as their source.
    dt_.resize(n);
    for (size_t i = 0; i < n; ++i) {
        const Node& nd = nodes[i];
        dt_[i].resize(nd.outputs.size(), DType::F32);
        switch (nd.kind) {
            case OpKind::Input:
            case OpKind::Weight:
            case OpKind::Constant:
                dt_[i][0] = nd.outputs[0].dtype;
                XS_CHECK(is_float(dt_[i][0]) || dt_[i][0] == DType::I32 || dt_[i][0] == DType::I64, "hip: ", where(i),
                         " holds ", dtype_name(dt_[i][0]), "; this backend takes f32, f16, bf16, i32 and i64 tensors");
                break;
            case OpKind::Reshape:
            case OpKind::Slice: dt_[i][0] = dtype(nd.inputs[0]); break;
            case OpKind::TopK: dt_[i][1] = DType::I32; break;
            // Data movement keeps integers as they are; floats come out f32, as every computed value here.
            case OpKind::Gather: dt_[i][0] = dtype(nd.inputs[0]) == DType::I32 ? DType::I32 : DType::F32; break;
            case OpKind::Transpose:
            case OpKind::Concat: dt_[i][0] = is_float(dtype(nd.inputs[0])) ? DType::F32 : dtype(nd.inputs[0]); break;
            default: break;
        }
    }

    // Ops this backend runs, and the readers of every value.
    std::vector<int> readers(n, 0);
    std::vector<std::vector<size_t>> reader_nodes(n);
    for (size_t i = 0; i < n; ++i) {
        for (const Value& in : nodes[i].inputs) {
            ++readers[static_cast<size_t>(in.node)];
            reader_nodes[static_cast<size_t>(in.node)].push_back(i);
        }
    }
    for (const auto& o : g_.outputs()) readers[static_cast<size_t>(o.value.node)] += 2;  // never fused away
    plan_.resize(n);
    for (size_t i = 0; i < n; ++i) {
        const Node& nd = nodes[i];
        NodePlan& p = plan_[i];
        p.reads = nd.inputs;
        switch (nd.kind) {
            case OpKind::Input:
            case OpKind::Weight:
            case OpKind::Constant:
            case OpKind::Reshape:
            case OpKind::KvRead: break;
            case OpKind::Slice: p.op = Op::SliceCopy; break;
            case OpKind::Gather: p.op = Op::Gather; break;
            case OpKind::Transpose:
                p.op = Op::Transpose;
                XS_CHECK(nd.outputs[0].shape.size() <= XS_MAX_RANK, "hip: ", where(i), ": a transpose of rank ",
                         nd.outputs[0].shape.size(), " (at most ", XS_MAX_RANK, ")");
                break;
            case OpKind::Concat:
                p.op = Op::Concat;
                XS_CHECK(nd.inputs.size() <= XS_CONCAT_PARTS, "hip: ", where(i), ": a concat of ", nd.inputs.size(),
                         " parts (at most ", XS_CONCAT_PARTS, " in one launch)");
                break;
            case OpKind::Add:
            case OpKind::Mul:
            case OpKind::Div: p.op = Op::Binary; break;
            case OpKind::Scale:
            case OpKind::Tanh:
            case OpKind::GeluTanh:
            case OpKind::Softcap:
            case OpKind::Sigmoid:
            case OpKind::Silu:
            case OpKind::Softplus:
            case OpKind::Clamp:
            case OpKind::Gelu:
                p.op = Op::Unary;
                p.act = unary_of(nd.kind);
                break;
            case OpKind::RmsNorm:
                p.op = Op::RmsNorm;
                p.has_w = nd.inputs.size() == 2;
                break;
            case OpKind::LayerNorm: p.op = Op::LayerNorm; break;
            case OpKind::L2Clip: p.op = Op::L2Clip; break;
            case OpKind::Softmax: p.op = Op::Softmax; break;
            case OpKind::TopK: p.op = Op::TopK; break;
            case OpKind::ReduceSum: p.op = Op::ReduceSum; break;
            case OpKind::Rope:
                p.op = Op::Rope;
                XS_CHECK(nodes[i].outputs[0].shape.size() == 3, "hip: ", where(i), ": rope of rows of several a token");
                break;
            case OpKind::KvCache: p.op = Op::KvAppend; break;
            case OpKind::Attention: {
                p.op = Op::Attention;
                const auto& a = std::get<graph::AttentionAttrs>(nd.attrs);
                XS_CHECK(nd.inputs.size() == 3 && a.block == 0 && !a.grouped && a.rel_extent == 0 && !a.anchored,
                         "hip: ", where(i), ": attention with a key bias, groups, blocks, a relative bias or an "
                         "anchored window is not supported");
                const Value k = nd.inputs[1], v = nd.inputs[2];
                const OpKind kk = nodes[static_cast<size_t>(k.node)].kind;
                XS_CHECK((kk == OpKind::KvCache || kk == OpKind::KvRead) && k.node == v.node && k.index == 0 &&
                             v.index == 1,
                         "hip: ", where(i), ": attention reads the keys and values of one KV slot (KvCache or KvRead "
                         "outputs); this backend has no attention over computed keys");
                break;
            }
            default:
                fail("hip: ", where(i), " is not supported by the HIP backend (it runs the elementwise, norm, "
                     "softmax, top-k, reduce, RoPE, gather, transpose, concat, KV cache and attention ops)");
        }
    }
    // KV outputs feed attention only: the slots hold the cache's own format (int8 codes, or f16 / f32 rows).
    for (size_t i = 0; i < n; ++i) {
        if (nodes[i].kind != OpKind::KvCache && nodes[i].kind != OpKind::KvRead) continue;
        for (size_t r : reader_nodes[i]) {
            XS_CHECK(nodes[r].kind == OpKind::Attention, "hip: ", where(i), " is read by ", where(r),
                     "; the KV cache is read only by attention on this backend");
        }
        for (const auto& o : g_.outputs())
            XS_CHECK(static_cast<size_t>(o.value.node) != i, "hip: graph output '", o.name, "' is a KV cache");
    }
    if (!g_.kv_slots().empty()) {
        const auto& kv = s_.options().kv;
        // The pairs the reference's device reads (sycl_kernels.h:209-212): one format for both, or int8 keys with
        // TurboQuant values.
        XS_CHECK(kv.k == kv.v || (kv.k == quant::KvFormat::I8 && quant::turbo_bits(kv.v) != 0),
                 "hip: a KV cache with keys in ", quant::kv_format_name(kv.k), " and values in ",
                 quant::kv_format_name(kv.v),
                 " is not supported: both take one format, or the keys i8 and the values a turbo format");
        for (const auto& slot : g_.kv_slots()) slot_of_.push_back(s_.slot_for(slot));
    }
    for (const Node& nd : nodes) {
        appends_ |= nd.kind == OpKind::KvCache;
        reads_kv_ |= nd.kind == OpKind::KvRead;
    }

    // ---- Fusions.
    const auto shape = [&](Value v) -> const Dims& { return g_.type(v).shape; };
    const auto row_vector = [&](Value v, const Dims& out) {
        const Dims& sh = shape(v);
        return sh.size() == 1 && !out.empty() && sh[0] == out.back();
    };
    const auto foldable = [&](size_t u) { return readers[u] == 1 && plan_[u].run_at < 0 && plan_[u].op != Op::None; };
    const auto fold = [&](size_t u, size_t into) {
        plan_[u].run_at = static_cast<int32_t>(into);
        plan_[u].folded = true;
        plan_[u].op = Op::None;
        plan_[u].reads.clear();
    };
    // A last-axis slice (read in place through its row stride) or a contiguous value of the shape.
    const auto strided_ok = [&](Value v, const Dims& out) {
        if (shape(v) != out) return false;
        const Node& nd = nodes[static_cast<size_t>(v.node)];
        if (nd.kind != OpKind::Slice) return true;
        return std::get<graph::SliceAttrs>(nd.attrs).axis == static_cast<int>(out.size()) - 1;
    };
    // act-bias-mul: Mul(act(x), b) / Mul(act(Add(x, bias)), b).
    for (size_t i = 0; i < n; ++i) {
        if (nodes[i].kind != OpKind::Mul || plan_[i].op != Op::Binary) continue;
        const Dims& out = nodes[i].outputs[0].shape;
        if (out.empty()) continue;
        for (size_t k = 0; k < 2; ++k) {
            const Value a = nodes[i].inputs[k], b = nodes[i].inputs[1 - k];
            const auto u = static_cast<size_t>(a.node);
            const int act = act_of(nodes[u].kind);
            if (act < 0 || !foldable(u) || !strided_ok(b, out)) continue;
            Value x = nodes[u].inputs[0];
            Value bias{};
            const auto ax = static_cast<size_t>(x.node);
            if (nodes[ax].kind == OpKind::Add && foldable(ax)) {
                for (size_t j = 0; j < 2; ++j) {
                    const Value xa = nodes[ax].inputs[j], c = nodes[ax].inputs[1 - j];
                    if (strided_ok(xa, out) && row_vector(c, out) && dtype(c) == dtype(xa)) {
                        x = xa;
                        bias = c;
                        break;
                    }
                }
            }
            if (!strided_ok(x, out) || dtype(x) != dtype(b)) continue;
            if (bias.valid()) fold(ax, i);
            fold(u, i);
            NodePlan& p = plan_[i];
            p.op = Op::ActMul;
            p.act = act;
            p.reads = {x, b};
            if (bias.valid()) {
                p.reads.push_back(bias);
                p.has_bias = true;
            }
            break;
        }
    }
    // unary-bias: act(Add(x, b)), b a row vector.
    for (size_t i = 0; i < n; ++i) {
        if (plan_[i].op != Op::Unary || act_of(nodes[i].kind) < 0) continue;
        const auto u = static_cast<size_t>(nodes[i].inputs[0].node);
        if (nodes[u].kind != OpKind::Add || !foldable(u)) continue;
        const Dims& out = nodes[i].outputs[0].shape;
        for (size_t k = 0; k < 2; ++k) {
            const Value x = nodes[u].inputs[k], c = nodes[u].inputs[1 - k];
            if (shape(x) != out || !row_vector(c, out)) continue;
            fold(u, i);
            plan_[i].op = Op::UnaryBias;
            plan_[i].act = act_of(nodes[i].kind);
            plan_[i].reads = {x, c};
            break;
        }
    }
    // Add(RmsNorm(..), c) / Add(a, Add(b, c)) / Add(a, Mul(b, c)).
    for (size_t i = 0; i < n; ++i) {
        if (nodes[i].kind != OpKind::Add || plan_[i].op != Op::Binary) continue;
        const Dims& out = nodes[i].outputs[0].shape;
        for (size_t k = 0; k < 2; ++k) {
            const Value x = nodes[i].inputs[k], other = nodes[i].inputs[1 - k];
            const auto u = static_cast<size_t>(x.node);
            if (!foldable(u) || shape(x) != out) continue;
            if (plan_[u].op == Op::RmsNorm && !plan_[u].has_bias && row_vector(other, out)) {
                const std::vector<Value> r = plan_[u].reads;
                const bool has_w = plan_[u].has_w;
                fold(u, i);
                plan_[i].op = Op::RmsNorm;
                plan_[i].reads = r;
                plan_[i].reads.push_back(other);
                plan_[i].has_w = has_w;
                plan_[i].has_bias = true;
                break;
            }
            if (shape(other) != out) continue;
            if (plan_[u].op == Op::Binary && nodes[u].kind == OpKind::Add) {
                const Value b = nodes[u].inputs[0], c = nodes[u].inputs[1];
                const bool c_row = shape(b) == out && (row_vector(c, out) || shape(c) == out);
                const bool b_row = shape(c) == out && row_vector(b, out);
                if (!c_row && !b_row) continue;
                fold(u, i);
                plan_[i].op = Op::Add3;
                plan_[i].reads = c_row ? std::vector<Value>{other, b, c} : std::vector<Value>{other, c, b};
                break;
            }
            if (plan_[u].op == Op::Binary && nodes[u].kind == OpKind::Mul) {
                const Value b = nodes[u].inputs[0], c = nodes[u].inputs[1];
                const bool b_full = shape(b) == out, c_full = shape(c) == out;
                if (!(b_full && (c_full || row_vector(c, out))) && !(c_full && row_vector(b, out))) continue;
                fold(u, i);
                plan_[i].op = Op::AddMul;
                plan_[i].reads = b_full ? std::vector<Value>{other, b, c} : std::vector<Value>{other, c, b};
                break;
            }
        }
    }
    // LayerNorm(Add(x, c)), c a row vector.
    for (size_t i = 0; i < n; ++i) {
        if (plan_[i].op != Op::LayerNorm) continue;
        const auto u = static_cast<size_t>(nodes[i].inputs[0].node);
        if (nodes[u].kind != OpKind::Add || plan_[u].op != Op::Binary || !foldable(u)) continue;
        const Dims& out = nodes[i].outputs[0].shape;
        for (size_t k = 0; k < 2; ++k) {
            const Value x = nodes[u].inputs[k], c = nodes[u].inputs[1 - k];
            if (shape(x) != out || !row_vector(c, out)) continue;
            fold(u, i);
            plan_[i].reads = {x, nodes[i].inputs[1], nodes[i].inputs[2], c};
            plan_[i].has_bias = true;
            break;
        }
    }
    // RmsNorm(Add(x, r)): the norm's launch writes the sum too, when every other reader of the sum comes later.
    for (size_t i = 0; i < n; ++i) {
        if (plan_[i].op != Op::RmsNorm || plan_[i].has_bias || nodes[i].kind != OpKind::RmsNorm) continue;
        const auto u = static_cast<size_t>(nodes[i].inputs[0].node);
        if (nodes[u].kind != OpKind::Add || plan_[u].op != Op::Binary || plan_[u].run_at >= 0) continue;
        const Value x = nodes[u].inputs[0], r = nodes[u].inputs[1];
        const Dims& out = nodes[i].outputs[0].shape;
        if (shape(x) != out || shape(r) != out) continue;
        const auto& rn = reader_nodes[u];
        if (std::any_of(rn.begin(), rn.end(), [&](size_t r2) { return r2 < i; })) continue;
        plan_[u].op = Op::None;
        plan_[u].reads.clear();
        plan_[u].run_at = static_cast<int32_t>(i);
        NodePlan& p = plan_[i];
        p.op = Op::AddRmsNorm;
        p.partner = static_cast<int32_t>(u);
        p.reads = {x, r};
        if (p.has_w) p.reads.push_back(nodes[i].inputs[1]);
    }
    // Two ropes of one positions / frequency pair: the later one's launch does both, when nothing reads the earlier
    // one's result before it.
    for (size_t j = 0; j < n; ++j) {
        if (plan_[j].op != Op::Rope || plan_[j].partner >= 0 || nodes[j].inputs.size() != 3) continue;
        for (size_t i = 0; i < j; ++i) {
            if (plan_[i].op != Op::Rope || plan_[i].partner >= 0 || nodes[i].inputs.size() != 3) continue;
            const Node &a = nodes[i], &b = nodes[j];
            if (!(a.inputs[1] == b.inputs[1]) || !(a.inputs[2] == b.inputs[2])) continue;
            if (std::get<graph::RopeAttrs>(a.attrs).rotary_dim != std::get<graph::RopeAttrs>(b.attrs).rotary_dim) continue;
            if (dtype(a.inputs[0]) != dtype(b.inputs[0]) || shape(a.inputs[0])[0] != shape(b.inputs[0])[0] ||
                shape(a.inputs[0])[2] != shape(b.inputs[0])[2])
                continue;
            const auto& rn = reader_nodes[i];
            if (std::any_of(rn.begin(), rn.end(), [&](size_t r) { return r <= j; })) continue;
            plan_[i].op = Op::None;
            plan_[i].run_at = static_cast<int32_t>(j);
            plan_[j].partner = static_cast<int32_t>(i);
            break;
        }
    }
    // Slices: a view when whole leading rows are kept or every reader is an act-bias-mul taking it strided.
    for (size_t i = 0; i < n; ++i) {
        if (nodes[i].kind != OpKind::Slice) continue;
        const auto& a = std::get<graph::SliceAttrs>(nodes[i].attrs);
        const Dims& in = shape(nodes[i].inputs[0]);
        bool leading = true;
        for (int d = 0; d < a.axis; ++d) leading &= in[static_cast<size_t>(d)] == 1;
        bool all_strided = a.axis == static_cast<int>(in.size()) - 1 && !reader_nodes[i].empty();
        for (size_t r : reader_nodes[i]) {
            const size_t at = plan_[r].run_at >= 0 ? static_cast<size_t>(plan_[r].run_at) : r;
            all_strided &= plan_[at].op == Op::ActMul;
        }
        for (const auto& o : g_.outputs()) all_strided &= static_cast<size_t>(o.value.node) != i;
        if (leading) plan_[i].op = Op::None;
        else if (all_strided) {
            plan_[i].op = Op::None;
            plan_[i].strided_view = true;
        }
    }
    // An act-bias-mul whose operand is read through a slice of a slice, or a contiguous-only view of a strided one,
    // cannot use one row stride: such slices are copied (never the case for a gate|up split).
    for (size_t i = 0; i < n; ++i) {
        if (!plan_[i].strided_view) continue;
        const Value src = nodes[i].inputs[0];
        const Node& sn = nodes[static_cast<size_t>(src.node)];
        if ((sn.kind == OpKind::Slice && plan_[static_cast<size_t>(src.node)].op == Op::None) || sn.kind == OpKind::Reshape) {
            plan_[i].strided_view = false;
            plan_[i].op = Op::SliceCopy;
        }
    }

}

// Weights and constants, uploaded once in their stored dtype; float ones that are not f32 also as f32, for the
// kernels that read f32 operands. A weight is one device copy for every program of the session.
void Program::upload() {
    const auto& nodes = g_.nodes();
    for (size_t i = 0; i < nodes.size(); ++i) {
        const Node& nd = nodes[i];
        if (nd.kind != OpKind::Weight && nd.kind != OpKind::Constant) continue;
        const std::string key = leaf_key(i);
        if (s_.leaves().count(key) != 0) continue;
        TensorView view;
        if (nd.kind == OpKind::Weight) view = s_.weights().get(std::get<graph::WeightAttrs>(nd.attrs).name);
        else view = std::get<graph::ConstantAttrs>(nd.attrs).value.view();
        const void* data = view.data;
        XS_CHECK(data != nullptr || view.numel() == 0, "hip: ", nd.label, " has no data");
        Leaf leaf;
        leaf.dtype = view.dtype;
        const size_t bytes = view.nbytes();
        leaf.data.grow(bytes);
        if (bytes > 0) check(xs_hip_memcpy_h2d(leaf.data.get(), data, bytes, s_.stream()), "upload");
        if (view.dtype != DType::F32 && is_float(view.dtype)) {
            std::vector<float> f(static_cast<size_t>(view.numel()));
            const auto* h = static_cast<const uint16_t*>(data);
            for (size_t e = 0; e < f.size(); ++e) f[e] = widen(view.dtype, h[e]);
            leaf.f32.grow(f.size() * 4);
            if (!f.empty()) check(xs_hip_memcpy_h2d(leaf.f32.get(), f.data(), f.size() * 4, s_.stream()), "upload");
        }
        s_.leaves()[key] = std::move(leaf);
    }
}

std::string Program::leaf_key(size_t node) const {
    const Node& nd = g_.nodes()[node];
    if (nd.kind == OpKind::Weight) return "w:" + std::get<graph::WeightAttrs>(nd.attrs).name;
    return "c:" + std::to_string(index_) + ":" + std::to_string(node);
}

// ---------------------------------------------------------------------------------------------------------------
// Run plans.

size_t Program::base_node(Value v) const {
    size_t i = static_cast<size_t>(v.node);
    const auto& nodes = g_.nodes();
    while (true) {
        const Node& nd = nodes[i];
        if (nd.kind == OpKind::Reshape || (nd.kind == OpKind::Slice && plan_[i].op == Op::None)) {
            i = static_cast<size_t>(nd.inputs[0].node);
            continue;
        }
        return i;
    }
}

Dims Program::resolve(const Dims& d, int64_t T, int64_t L) const {
    Dims out = d;
    for (int64_t& x : out) x = x == kT ? T : x == kL ? L : x;
    return out;
}

// Whether the launch of node `node` reads its operand `operand` as f32.
bool Program::needs_f32(size_t node, size_t operand) const {
    const NodePlan& p = plan_[node];
    switch (p.op) {
        case Op::Binary:
        case Op::Unary:
        case Op::SliceCopy:
        case Op::KvAppend:
        case Op::Gather: return false;  // the gather widens a 16-bit table's rows itself
        case Op::ActMul: return false;  // x, b and bias share one dtype (checked when fused)
        case Op::RmsNorm:
        case Op::LayerNorm: return operand > 0;
        case Op::Rope: return operand == 2;
        case Op::Attention: return operand == 0;
        default: return true;
    }
}

const std::vector<char>& Program::live_for(std::span<const std::string> only) {
    std::string key;
    for (const std::string& name : only) key += name + '\n';
    const auto it = live_.find(key);
    if (it != live_.end()) return it->second;
    const auto& nodes = g_.nodes();
    std::vector<char> live(nodes.size(), 0);
    std::vector<size_t> stack;
    const auto need = [&](size_t i) {
        if (live[i] == 0) {
            live[i] = 1;
            stack.push_back(i);
        }
    };
    if (only.empty()) {
        for (const auto& o : g_.outputs()) need(static_cast<size_t>(o.value.node));
    }
    for (const std::string& name : only) {
        const auto out = std::find_if(g_.outputs().begin(), g_.outputs().end(),
                                      [&](const auto& o) { return o.name == name; });
        XS_CHECK(out != g_.outputs().end(), "hip: the program has no output '", name, "'");
        need(static_cast<size_t>(out->value.node));
    }
    for (size_t i = 0; i < nodes.size(); ++i) {
        if (nodes[i].kind == OpKind::KvCache) need(i);  // the state advances whatever is asked
    }
    while (!stack.empty()) {
        const size_t i = stack.back();
        stack.pop_back();
        for (const Value& in : nodes[i].inputs) need(static_cast<size_t>(in.node));
        if (plan_[i].run_at >= 0) need(static_cast<size_t>(plan_[i].run_at));
        for (const Value& in : plan_[i].reads) need(static_cast<size_t>(in.node));
        if (plan_[i].partner >= 0) need(static_cast<size_t>(plan_[i].partner));
    }
    return live_.emplace(std::move(key), std::move(live)).first->second;
}

Program::RunPlan& Program::plan_for(int64_t T, std::span<const std::string> only) {
    std::string key;
    for (const std::string& name : only) key += name + '\n';
    const auto it = plans_.find({T, key});
    if (it != plans_.end()) return it->second;

    const auto& nodes = g_.nodes();
    const size_t n = nodes.size();
    RunPlan p;
    p.live = live_for(only);
    p.shapes.resize(n);
    p.locs.resize(n);
    p.conv.assign(n, -1);
    p.convert_before.resize(n);
    p.scratch.assign(n, -1);
    p.scratch_bytes.assign(n, 0);
    for (size_t i = 0; i < n; ++i) {
        p.shapes[i].resize(nodes[i].outputs.size());
        p.locs[i].resize(nodes[i].outputs.size());
        for (size_t j = 0; j < nodes[i].outputs.size(); ++j) p.shapes[i][j] = resolve(nodes[i].outputs[j].shape, T, 0);
    }
    // The step at which each node's value is written: its own launch, the launch it was folded into, or before the
    // first launch (inputs).
    std::vector<int64_t> def(n, -1);
    for (size_t i = 0; i < n; ++i) def[i] = plan_[i].run_at >= 0 ? plan_[i].run_at : static_cast<int64_t>(i);
    // Blocks: (bytes, first step, last step).
    struct Block {
        size_t bytes;
        int64_t first, last;
    };
    std::vector<Block> blocks;
    std::vector<std::vector<int32_t>> block_of(n);
    const int64_t end = static_cast<int64_t>(n) + 1;
    for (size_t i = 0; i < n; ++i) {
        block_of[i].assign(nodes[i].outputs.size(), -1);
        if (!p.live[i]) continue;
        const Node& nd = nodes[i];
        switch (nd.kind) {
            case OpKind::Weight:
            case OpKind::Constant: p.locs[i][0] = Loc{Where::Leaf, static_cast<int32_t>(i)}; continue;
            case OpKind::KvCache:
            case OpKind::KvRead: {
                const int slot = slot_of_[static_cast<size_t>(std::get<graph::KvCacheAttrs>(nd.attrs).slot)];
                p.locs[i][0] = Loc{Where::Slot, slot, 0};
                p.locs[i][1] = Loc{Where::Slot, slot, 1};
                continue;
            }
            case OpKind::Reshape: continue;  // located below, as a view
            default:
                if (plan_[i].folded) continue;
                break;
        }
        switch (nd.kind) {
            case OpKind::Slice:
                if (plan_[i].op == Op::None) continue;
                break;
            default: break;
        }
        for (size_t j = 0; j < nd.outputs.size(); ++j) {
            const size_t bytes = static_cast<size_t>(numel(p.shapes[i][j])) * dtype_size(dt_[i][j]);
            block_of[i][j] = static_cast<int32_t>(blocks.size());
            blocks.push_back({align_up(std::max<size_t>(bytes, 1)), nd.kind == OpKind::Input ? -1 : def[i], def[i]});
        }
    }
    // Views take their source's block.
    for (size_t i = 0; i < n; ++i) {
        if (!p.live[i]) continue;
        const Node& nd = nodes[i];
        if (nd.kind == OpKind::Reshape || (nd.kind == OpKind::Slice && plan_[i].op == Op::None)) {
            const size_t b = base_node(Value{static_cast<int32_t>(i), 0});
            block_of[i][0] = block_of[b][0];
        }
    }
    // Last uses: every launch's reads (through views), conversions, and the graph outputs (copied out at the end).
    const auto use = [&](Value v, int64_t step) {
        const int32_t b = block_of[static_cast<size_t>(v.node)][static_cast<size_t>(v.index)];
        if (b >= 0) blocks[static_cast<size_t>(b)].last = std::max(blocks[static_cast<size_t>(b)].last, step);
    };
    std::map<std::pair<int32_t, int32_t>, std::pair<int64_t, int64_t>> conv_span;  // value -> (first, last) step
    for (size_t i = 0; i < n; ++i) {
        if (!p.live[i] || plan_[i].op == Op::None) continue;
        for (size_t k = 0; k < plan_[i].reads.size(); ++k) {
            const Value v = plan_[i].reads[k];
            use(v, static_cast<int64_t>(i));
            if (needs_f32(i, k) && dtype(v) != DType::F32 && is_float(dtype(v)) &&
                nodes[base_node(v)].kind != OpKind::Weight && nodes[base_node(v)].kind != OpKind::Constant) {
                auto [cit, fresh] = conv_span.try_emplace({v.node, v.index}, std::make_pair(static_cast<int64_t>(i),
                                                                                            static_cast<int64_t>(i)));
                if (!fresh) cit->second.second = static_cast<int64_t>(i);
            }
        }
        if (plan_[i].partner >= 0 && plan_[i].op == Op::Rope) {
            for (const Value& v : nodes[static_cast<size_t>(plan_[i].partner)].inputs) use(v, static_cast<int64_t>(i));
        }
    }
    for (const auto& o : g_.outputs()) {
        if (!p.live[static_cast<size_t>(o.value.node)]) continue;
        use(o.value, end);
        if (is_float(dtype(o.value)) && dtype(o.value) != DType::F32) {
            auto [cit, fresh] = conv_span.try_emplace({o.value.node, o.value.index}, std::make_pair(end, end));
            if (!fresh) cit->second.second = end;
        }
    }
    for (const auto& [v, span] : conv_span) {
        if (span.first < static_cast<int64_t>(n)) p.convert_before[static_cast<size_t>(span.first)].push_back(Value{v.first, v.second});
        const size_t bytes = static_cast<size_t>(numel(p.shapes[static_cast<size_t>(v.first)][static_cast<size_t>(v.second)])) * 4;
        if (v.second == 0) p.conv[static_cast<size_t>(v.first)] = static_cast<int32_t>(blocks.size());
        blocks.push_back({align_up(std::max<size_t>(bytes, 1)), span.first, span.second});
    }
    // Scratch of the launches that split rows over workgroups.
    const int64_t max_len = s_.options().max_context;
    for (size_t i = 0; i < n; ++i) {
        if (!p.live[i]) continue;
        size_t bytes = 0;
        const Node& nd = nodes[i];
        if (plan_[i].op == Op::TopK) {
            const Dims& x = p.shapes[static_cast<size_t>(nd.inputs[0].node)][static_cast<size_t>(nd.inputs[0].index)];
            const int64_t width = x.back();
            bytes = xs_hip_topk_scratch(numel(x) / std::max<int64_t>(width, 1), width,
                                        std::get<graph::TopKAttrs>(nd.attrs).k);
        } else if (plan_[i].op == Op::Softmax) {
            // Not in the arena: a split softmax needs its scratch zero-filled at entry (and leaves it so).
            const Dims& x = p.shapes[i][0];
            const size_t sync = xs_hip_softmax_scratch(numel(x) / std::max<int64_t>(x.back(), 1), x.back());
            if (sync > 0) {
                p.scratch[i] = kSyncScratch;
                p.sync_bytes = std::max(p.sync_bytes, sync);
            }
            continue;
        } else if (plan_[i].op == Op::Attention) {
            const Dims& q = p.shapes[i][0];
            const Dims& k = g_.type(nd.inputs[1]).shape;
            // The split grows with the keys: sized for max_context, enough for every L of the session, whichever
            // reader (int8 or float rows) runs.
            const int64_t split = std::max({xs_hip_attention_i8_split(q[0], k[1], max_len),
                                            xs_hip_attention_rows_split(q[0], k[1], max_len),
                                            xs_hip_attention_rows_split_kv(XS_KV_FLOAT, XS_F16, q[0], q[1], k[1],
                                                                           max_len, q[2])});
            bytes = xs_hip_attention_i8_scratch(q[0], q[1], q[2], split);
        }
        if (bytes == 0) continue;
        p.scratch[i] = static_cast<int32_t>(blocks.size());
        p.scratch_bytes[i] = bytes;
        blocks.push_back({align_up(bytes), static_cast<int64_t>(i), static_cast<int64_t>(i)});
    }
    // Offsets: blocks in order of first use, each at the lowest offset free over its whole span.
    std::vector<size_t> order(blocks.size());
    for (size_t b = 0; b < blocks.size(); ++b) order[b] = b;
    std::stable_sort(order.begin(), order.end(), [&](size_t a, size_t b) { return blocks[a].first < blocks[b].first; });
    p.block_offset.assign(blocks.size(), 0);
    std::vector<size_t> placed;
    for (size_t b : order) {
        std::vector<std::pair<size_t, size_t>> busy;
        for (size_t o : placed) {
            if (blocks[o].last >= blocks[b].first && blocks[o].first <= blocks[b].last)
                busy.emplace_back(p.block_offset[o], p.block_offset[o] + blocks[o].bytes);
        }
        std::sort(busy.begin(), busy.end());
        size_t at = 0;
        for (const auto& [lo, hi] : busy) {
            if (at + blocks[b].bytes <= lo) break;
            at = std::max(at, hi);
        }
        p.block_offset[b] = at;
        p.arena_bytes = std::max(p.arena_bytes, at + blocks[b].bytes);
        placed.push_back(b);
    }
    // Locations.
    for (size_t i = 0; i < n; ++i) {
        if (!p.live[i]) continue;
        for (size_t j = 0; j < nodes[i].outputs.size(); ++j) {
            if (p.locs[i][j].where != Where::None || block_of[i][j] < 0) continue;
            p.locs[i][j] = Loc{Where::Arena, block_of[i][j], 0, 0, 0};
        }
    }
    for (size_t i = 0; i < n; ++i) {  // views, in graph order (a view's source is located first)
        if (!p.live[i]) continue;
        const Node& nd = nodes[i];
        if (nd.kind == OpKind::Reshape) {
            p.locs[i][0] = p.locs[static_cast<size_t>(nd.inputs[0].node)][static_cast<size_t>(nd.inputs[0].index)];
        } else if (nd.kind == OpKind::Slice && plan_[i].op == Op::None) {
            const auto& a = std::get<graph::SliceAttrs>(nd.attrs);
            const Dims& in = p.shapes[static_cast<size_t>(nd.inputs[0].node)][static_cast<size_t>(nd.inputs[0].index)];
            const int64_t dim = in[static_cast<size_t>(a.axis)];
            const int64_t begin = a.begin < 0 ? a.begin + dim : a.begin;
            int64_t inner = 1;
            for (size_t d = static_cast<size_t>(a.axis) + 1; d < in.size(); ++d) inner *= in[d];
            const auto es = static_cast<int64_t>(dtype_size(dt_[i][0]));
            Loc l = p.locs[static_cast<size_t>(nd.inputs[0].node)][static_cast<size_t>(nd.inputs[0].index)];
            l.offset += begin * inner * es;
            if (plan_[i].strided_view) l.row_stride = dim * es;
            p.locs[i][0] = l;
        }
    }
    return plans_.emplace(std::make_pair(T, key), std::move(p)).first->second;
}

char* Program::ptr(const RunPlan& p, Value v) const {
    const Loc& l = p.locs[static_cast<size_t>(v.node)][static_cast<size_t>(v.index)];
    switch (l.where) {
        case Where::Arena:
            return s_.arena().get() + p.block_offset[static_cast<size_t>(l.id)] + static_cast<size_t>(l.offset);
        case Where::Leaf: return s_.leaves().at(leaf_key(static_cast<size_t>(l.id))).data.get() + l.offset;
        default: fail("hip: value of node ", v.node, " has no memory in this run");
    }
}

const char* Program::ptr_f32(const RunPlan& p, Value v) const {
    if (dtype(v) == DType::F32 || !is_float(dtype(v))) return ptr(p, v);
    const size_t b = base_node(v);
    const Node& bn = g_.nodes()[b];
    if (bn.kind == OpKind::Weight || bn.kind == OpKind::Constant) {
        const Loc& l = p.locs[static_cast<size_t>(v.node)][static_cast<size_t>(v.index)];
        return s_.leaves().at(leaf_key(b)).f32.get() + l.offset / static_cast<int64_t>(dtype_size(dtype(v))) * 4;
    }
    const int32_t c = p.conv[static_cast<size_t>(v.node)];
    XS_CHECK(c >= 0 && v.index == 0, "hip: no f32 copy of node ", v.node, " was planned");
    return s_.arena().get() + p.block_offset[static_cast<size_t>(c)];
}

// ---------------------------------------------------------------------------------------------------------------
// Launches.

void Program::launch(size_t i, const RunPlan& p, int64_t T, int64_t L, int64_t replay_cap) {
    const Node& nd = g_.nodes()[i];
    const NodePlan& np = plan_[i];
    void* const st = s_.stream();
    const Dims& out = p.shapes[i][0];
    const int64_t count = numel(out);
    const auto in_shape = [&](Value v) -> const Dims& {
        return p.shapes[static_cast<size_t>(v.node)][static_cast<size_t>(v.index)];
    };
    const auto f32 = [&](size_t k) { return reinterpret_cast<const float*>(ptr_f32(p, np.reads[k])); };
    const auto rows_of = [](const Dims& d) { return d.empty() ? int64_t{1} : numel(d) / std::max<int64_t>(d.back(), 1); };
    // f32 copies of 16-bit activations read as f32, made before their first such reader (the copy's block lives
    // until the last).
    for (const Value& v : p.convert_before[i]) {
        const int32_t c = p.conv[static_cast<size_t>(v.node)];
        check(xs_hip_convert(st, abi(dtype(v)), ptr(p, v), XS_F32, s_.arena().get() + p.block_offset[static_cast<size_t>(c)],
                             numel(in_shape(v))),
              graph::op_name(nd.kind));
    }
    const std::string what(graph::op_name(nd.kind));
    switch (np.op) {
        case Op::None: return;
        case Op::Binary: {
            const Value a = np.reads[0], b = np.reads[1];
            const xs_binary_op op = nd.kind == OpKind::Add ? XS_BINARY_ADD : nd.kind == OpKind::Mul ? XS_BINARY_MUL
                                                                                                    : XS_BINARY_DIV;
            const Dims& as = in_shape(a);
            const Dims& bs = in_shape(b);
            if (as == out && bs == out && dtype(a) == dtype(b)) {
                check(xs_hip_binary_same(st, op, abi(dtype(a)), ptr(p, a), ptr(p, b), XS_F32, ptr(p, Value{static_cast<int32_t>(i), 0}), count), what);
            } else if (as == out && bs.size() == 1 && !out.empty() && bs[0] == out.back() && dtype(a) == dtype(b) && count > 0) {
                check(xs_hip_binary_period(st, op, abi(dtype(a)), ptr(p, a), ptr(p, b), XS_F32,
                                           ptr(p, Value{static_cast<int32_t>(i), 0}), count, bs[0]),
                      what);
            } else {
                xs_broadcast bc;
                check(xs_hip_broadcast_fill(&bc, as.data(), static_cast<int32_t>(as.size()), bs.data(),
                                            static_cast<int32_t>(bs.size())),
                      what);
                check(xs_hip_binary(st, op, abi(dtype(a)), ptr(p, a), abi(dtype(b)), ptr(p, b), XS_F32,
                                    ptr(p, Value{static_cast<int32_t>(i), 0}), &bc),
                      what);
            }
            return;
        }
        case Op::Unary: {
            float a = 0.0f, b = 0.0f;
            if (nd.kind == OpKind::Scale) a = std::get<graph::ScaleAttrs>(nd.attrs).factor;
            if (nd.kind == OpKind::Softcap) a = std::get<graph::SoftcapAttrs>(nd.attrs).cap;
            if (nd.kind == OpKind::Clamp) {
                a = std::get<graph::ClampAttrs>(nd.attrs).lo;
                b = std::get<graph::ClampAttrs>(nd.attrs).hi;
            }
            const Value x = np.reads[0];
            check(xs_hip_unary(st, static_cast<xs_unary_op>(np.act), abi(dtype(x)), ptr(p, x), XS_F32,
                               ptr(p, Value{static_cast<int32_t>(i), 0}), count, a, b),
                  what);
            return;
        }
        case Op::ActMul: {
            const Value x = np.reads[0], b = np.reads[1];
            const int64_t cols = out.back();
            const int64_t rows = rows_of(out);
            const auto stride = [&](Value v) {
                const Loc& l = p.locs[static_cast<size_t>(v.node)][static_cast<size_t>(v.index)];
                return l.row_stride > 0 ? l.row_stride / static_cast<int64_t>(dtype_size(dtype(v))) : cols;
            };
            check(xs_hip_act_bias_mul_2d(st, static_cast<xs_unary_op>(np.act), abi(dtype(x)), ptr(p, x), stride(x),
                                         ptr(p, b), stride(b), np.has_bias ? ptr(p, np.reads[2]) : nullptr, XS_F32,
                                         ptr(p, Value{static_cast<int32_t>(i), 0}), cols, rows, cols),
                  "act-bias-mul (" + what + ")");
            return;
        }
        case Op::UnaryBias:
            check(xs_hip_unary_bias(st, static_cast<xs_unary_op>(np.act), f32(0), f32(1), XS_F32,
                                    ptr(p, Value{static_cast<int32_t>(i), 0}), count, out.back()),
                  "unary-bias (" + what + ")");
            return;
        case Op::Add3:
        case Op::AddMul: {
            const Dims& cs = in_shape(np.reads[2]);
            const int64_t period = cs == out ? std::max<int64_t>(count, 1) : cs[0];
            const auto fn = np.op == Op::Add3 ? xs_hip_add3 : xs_hip_add_mul;
            check(fn(st, f32(0), f32(1), f32(2), XS_F32, ptr(p, Value{static_cast<int32_t>(i), 0}), count, period),
                  np.op == Op::Add3 ? "add3" : "add_mul");
            return;
        }
        case Op::RmsNorm: {
            const Value x = np.reads[0];
            // The norm node: this one, or (Add(RmsNorm(..), c)) the norm folded into it.
            size_t norm = i;
            if (nd.kind == OpKind::Add) {
                for (const Value& in : nd.inputs) {
                    const auto u = static_cast<size_t>(in.node);
                    if (plan_[u].run_at == static_cast<int32_t>(i) && g_.nodes()[u].kind == OpKind::RmsNorm) norm = u;
                }
            }
            const float e = std::get<graph::NormAttrs>(g_.nodes()[norm].attrs).eps;
            const float* w = np.has_w ? f32(1) : nullptr;
            const float* bias = np.has_bias ? f32(np.reads.size() - 1) : nullptr;
            check(xs_hip_rms_norm(st, abi(dtype(x)), ptr(p, x), w, bias, XS_F32,
                                  ptr(p, Value{static_cast<int32_t>(i), 0}), rows_of(out), out.back(), e),
                  "RmsNorm");
            return;
        }
        case Op::AddRmsNorm: {
            const float e = std::get<graph::NormAttrs>(nd.attrs).eps;
            check(xs_hip_add_rms_norm(st, f32(0), f32(1), np.has_w ? f32(2) : nullptr, nullptr,
                                      reinterpret_cast<float*>(ptr(p, Value{np.partner, 0})), XS_F32,
                                      ptr(p, Value{static_cast<int32_t>(i), 0}), rows_of(out), out.back(), e),
                  "Add+RmsNorm");
            return;
        }
        case Op::LayerNorm: {
            const Value x = np.reads[0];
            const float e = std::get<graph::NormAttrs>(nd.attrs).eps;
            check(xs_hip_layer_norm(st, abi(dtype(x)), ptr(p, x), np.has_bias ? f32(3) : nullptr, f32(1), f32(2),
                                    XS_F32, ptr(p, Value{static_cast<int32_t>(i), 0}), rows_of(out), out.back(), e),
                  what);
            return;
        }
        case Op::L2Clip: {
            const auto& a = std::get<graph::L2ClipAttrs>(nd.attrs);
            check(xs_hip_l2_clip(st, f32(0), reinterpret_cast<float*>(ptr(p, Value{static_cast<int32_t>(i), 0})),
                                 rows_of(out), out.back(), a.threshold, a.eps),
                  what);
            return;
        }
        case Op::Softmax: {
            float* y = reinterpret_cast<float*>(ptr(p, Value{static_cast<int32_t>(i), 0}));
            const int64_t rows = rows_of(out), width = out.back();
            if (p.scratch[i] == kSyncScratch) {
                check(xs_hip_softmax_masked(st, f32(0), y, rows, width, width, 1.0f, nullptr, width, s_.sync()), what);
            } else {
                check(xs_hip_softmax(st, f32(0), y, rows, width), what);
            }
            return;
        }
        case Op::TopK: {
            const Dims& x = in_shape(np.reads[0]);
            const int64_t k = std::get<graph::TopKAttrs>(nd.attrs).k;
            check(xs_hip_topk(st, f32(0), reinterpret_cast<float*>(ptr(p, Value{static_cast<int32_t>(i), 0})),
                              reinterpret_cast<int32_t*>(ptr(p, Value{static_cast<int32_t>(i), 1})), rows_of(x),
                              x.back(), k,
                              p.scratch[i] >= 0 ? s_.arena().get() + p.block_offset[static_cast<size_t>(p.scratch[i])]
                                                : nullptr),
                  what);
            return;
        }
        case Op::ReduceSum: {
            const Dims& x = in_shape(np.reads[0]);
            const auto axis = static_cast<size_t>(std::get<graph::AxisAttrs>(nd.attrs).axis);
            int64_t outer = 1, inner = 1;
            for (size_t d = 0; d < axis; ++d) outer *= x[d];
            for (size_t d = axis + 1; d < x.size(); ++d) inner *= x[d];
            check(xs_hip_reduce_sum(st, f32(0), reinterpret_cast<float*>(ptr(p, Value{static_cast<int32_t>(i), 0})),
                                    outer, x[axis], inner),
                  what);
            return;
        }
        case Op::Rope: {
            const Value x = np.reads[0], pos = np.reads[1];
            const Dims& xs = in_shape(x);
            const Dims& ps = in_shape(pos);
            const int64_t sections = ps.size() == 2 ? ps[1] : 1;
            const int64_t rotary = std::get<graph::RopeAttrs>(nd.attrs).rotary_dim;
            const int32_t* pair_axes = nullptr;
            if (np.reads.size() == 4) {
                XS_CHECK(dtype(np.reads[3]) == DType::I32, "hip: rope pair_axes must be i32");
                pair_axes = reinterpret_cast<const int32_t*>(ptr(p, np.reads[3]));
            }
            XS_CHECK(dtype(pos) == DType::I32 || dtype(pos) == DType::I64, "hip: rope positions must be i32 or i64");
            if (np.partner >= 0) {
                const Node& other = g_.nodes()[static_cast<size_t>(np.partner)];
                const Value xa = other.inputs[0];
                check(xs_hip_rope2(st, abi(dtype(x)), ptr(p, xa), ptr(p, Value{np.partner, 0}), in_shape(xa)[1],
                                   ptr(p, x), ptr(p, Value{static_cast<int32_t>(i), 0}), xs[1], abi(dtype(pos)),
                                   ptr(p, pos), f32(2), XS_F32, xs[0], xs[2], rotary, sections, pair_axes),
                      "Rope (Q and K)");
            } else {
                check(xs_hip_rope(st, abi(dtype(x)), ptr(p, x), abi(dtype(pos)), ptr(p, pos), f32(2), XS_F32,
                                  ptr(p, Value{static_cast<int32_t>(i), 0}), xs[0], xs[1], xs[2], rotary, sections,
                                  pair_axes),
                      what);
            }
            return;
        }
        case Op::KvAppend: {
            const int slot = slot_of_[static_cast<size_t>(std::get<graph::KvCacheAttrs>(nd.attrs).slot)];
            KvState& kv = s_.kv()[static_cast<size_t>(slot)];
            const int64_t first = L - T;  // rows [L - T, L) of the slot
            const Value k = np.reads[0], v = np.reads[1];
            if (kv.rows != DType::I8) {  // the Float format: rows of the precision's float
                const bool at = replay_cap > 0;  // the first token read from the step record at replay
                const size_t skip = at ? 0 : static_cast<size_t>(first * kv.heads * kv.dim) * dtype_size(kv.rows);
                const int64_t* row0 = at ? s_.step_record() : nullptr;
                const xs_dtype rd = abi(kv.rows);
                if (dtype(k) == dtype(v)) {
                    check(xs_hip_kv_store_pair(st, abi(dtype(k)), ptr(p, k), ptr(p, v), rd, kv.kc.get() + skip,
                                               kv.vc.get() + skip, T * kv.heads, kv.dim, row0, kv.heads,
                                               kv.cap * kv.heads),
                          "KvCache");
                } else {
                    check(xs_hip_kv_store_pair(st, abi(dtype(k)), ptr(p, k), nullptr, rd, kv.kc.get() + skip, nullptr,
                                               T * kv.heads, kv.dim, row0, kv.heads, kv.cap * kv.heads),
                          "KvCache");
                    check(xs_hip_kv_store_pair(st, abi(dtype(v)), ptr(p, v), nullptr, rd, kv.vc.get() + skip, nullptr,
                                               T * kv.heads, kv.dim, row0, kv.heads, kv.cap * kv.heads),
                          "KvCache");
                }
                return;
            }
            if (!kv.both_i8()) {  // a TurboQuant stream: keys and values by a launch each
                for (int which = 0; which < 2; ++which) {
                    const quant::KvFormat f = which == 0 ? kv.kf : kv.vf;
                    const Value x = np.reads[static_cast<size_t>(which)];
                    char* codes = (which == 0 ? kv.kc : kv.vc).get();
                    char* scales = (which == 0 ? kv.ks : kv.vs).get();
                    if (replay_cap > 0) {  // the first token read from the step record at replay
                        if (f == quant::KvFormat::I8)
                            check(xs_hip_quantize_kv_at(st, abi(dtype(x)), ptr(p, x), codes, scales, T * kv.heads,
                                                        kv.dim, s_.step_record(), kv.heads, kv.cap * kv.heads),
                                  "KvCache");
                        else
                            check(xs_hip_quantize_kv_turbo_at(st, kv_abi(f), abi(dtype(x)), ptr(p, x), codes, scales,
                                                              T * kv.heads, kv.dim, s_.step_record(), kv.heads,
                                                              kv.cap * kv.heads),
                                  "KvCache");
                    } else {
                        const int64_t cb = kv_code_bytes(f, kv.dim), sb = kv_scale_bytes(f, kv.dim);
                        check(xs_hip_quantize_kv(st, kv_abi(f), abi(dtype(x)), ptr(p, x),
                                                 codes + first * kv.heads * cb, scales + first * kv.heads * sb,
                                                 T * kv.heads, kv.dim),
                              "KvCache");
                    }
                }
                return;
            }
            if (dtype(k) == dtype(v)) {  // keys and values in one launch
                const bool at = replay_cap > 0;  // the first token read from the step record at replay
                const int64_t skip = at ? 0 : first * kv.heads;
                check(xs_hip_quantize_kv_pair(st, abi(dtype(k)), ptr(p, k), ptr(p, v), kv.kc.get() + skip * kv.dim,
                                              kv.ks.get() + skip * 4, kv.vc.get() + skip * kv.dim,
                                              kv.vs.get() + skip * 4, T * kv.heads, kv.dim,
                                              at ? s_.step_record() : nullptr, kv.heads, kv.cap * kv.heads),
                      "KvCache");
                return;
            }
            for (int which = 0; which < 2; ++which) {
                const Value x = np.reads[static_cast<size_t>(which)];
                char* codes = (which == 0 ? kv.kc : kv.vc).get();
                char* scales = (which == 0 ? kv.ks : kv.vs).get();
                if (replay_cap > 0) {  // the first token read from the step record at replay
                    check(xs_hip_quantize_kv_at(st, abi(dtype(x)), ptr(p, x), codes, scales, T * kv.heads, kv.dim,
                                                s_.step_record(), kv.heads, kv.cap * kv.heads),
                          "KvCache");
                } else {
                    check(xs_hip_quantize_kv(st, XS_KV_I8, abi(dtype(x)), ptr(p, x), codes + first * kv.heads * kv.dim,
                                             scales + first * kv.heads * 4, T * kv.heads, kv.dim),
                          "KvCache");
                }
            }
            return;
        }
        case Op::Attention: {
            const auto& a = std::get<graph::AttentionAttrs>(nd.attrs);
            const Value q = np.reads[0];
            const Loc& kl = p.locs[static_cast<size_t>(np.reads[1].node)][0];
            KvState& kv = s_.kv()[static_cast<size_t>(kl.id)];
            const Dims& qs = in_shape(q);
            const int64_t keys = replay_cap > 0 ? replay_cap : L;
            const int64_t split = kv.both_i8() ? xs_hip_attention_i8_split(qs[0], kv.heads, keys)
                                               : xs_hip_attention_rows_split_kv(kv_abi(kv.kf), abi(kv.rows), qs[0],
                                                                                qs[1], kv.heads, keys, kv.dim);
            auto* out_p = reinterpret_cast<float*>(ptr(p, Value{static_cast<int32_t>(i), 0}));
            char* scratch = split > 1 ? s_.arena().get() + p.block_offset[static_cast<size_t>(p.scratch[i])] : nullptr;
            if (kv.rows != DType::I8) {  // the Float format's rows
                if (replay_cap > 0) {
                    check(xs_hip_attention_at(st, abi(kv.rows), f32(0), kv.kc.get(), kv.vc.get(), out_p, qs[0], qs[1],
                                              kv.heads, qs[2], kv.cap, s_.step_record() + 1, a.scale, a.softcap,
                                              a.sliding_window, a.causal ? 1 : 0, split, scratch),
                          what);
                } else {
                    check(xs_hip_attention(st, abi(kv.rows), f32(0), kv.kc.get(), kv.vc.get(), out_p, qs[0], qs[1],
                                           kv.heads, qs[2], L, a.scale, a.softcap, a.sliding_window, a.causal ? 1 : 0,
                                           split, scratch),
                          what);
                }
                return;
            }
            if (!kv.both_i8()) {  // TurboQuant values, with keys in the same format or in int8
                if (replay_cap > 0) {  // the key count read from the step record at replay
                    check(xs_hip_attention_quantized_at(st, kv_abi(kv.kf), kv_abi(kv.vf), f32(0), kv.kc.get(),
                                                        kv.ks.get(), kv.vc.get(), kv.vs.get(), out_p, qs[0], qs[1],
                                                        kv.heads, qs[2], kv.cap, s_.step_record() + 1, a.scale,
                                                        a.softcap, a.sliding_window, a.causal ? 1 : 0, split, scratch),
                          what);
                } else {
                    check(xs_hip_attention_quantized(st, kv_abi(kv.kf), kv_abi(kv.vf), f32(0), kv.kc.get(),
                                                     kv.ks.get(), kv.vc.get(), kv.vs.get(), out_p, qs[0], qs[1],
                                                     kv.heads, qs[2], L, a.scale, a.softcap, a.sliding_window,
                                                     a.causal ? 1 : 0, split, scratch),
                          what);
                }
                return;
            }
            if (replay_cap > 0) {  // the key count read from the step record at replay
                check(xs_hip_attention_i8_at(st, f32(0), kv.kc.get(), kv.ks.get(), kv.vc.get(), kv.vs.get(), out_p,
                                             qs[0], qs[1], kv.heads, qs[2], kv.cap, s_.step_record() + 1, a.scale,
                                             a.softcap, a.sliding_window, a.causal ? 1 : 0, split, scratch),
                      what);
            } else {
                check(xs_hip_attention_i8(st, f32(0), kv.kc.get(), kv.ks.get(), kv.vc.get(), kv.vs.get(), out_p, qs[0],
                                          qs[1], kv.heads, qs[2], L, a.scale, a.softcap, a.sliding_window,
                                          a.causal ? 1 : 0, split, scratch),
                      what);
            }
            return;
        }
        case Op::Gather: {
            const Value table = np.reads[0], ids = np.reads[1];
            const Dims& ts = in_shape(table);
            check(xs_hip_gather(st, abi(dtype(table)), ptr(p, table), ts[0], ts[1], abi(dtype(ids)), ptr(p, ids),
                                numel(in_shape(ids)), ptr(p, Value{static_cast<int32_t>(i), 0})),
                  what);
            return;
        }
        case Op::Transpose: {
            const Value x = np.reads[0];
            const Dims& xs = in_shape(x);
            const auto& perm = std::get<graph::TransposeAttrs>(nd.attrs).perm;
            const std::vector<int32_t> pm(perm.begin(), perm.end());
            const void* src = is_float(dtype(x)) ? static_cast<const void*>(f32(0)) : ptr(p, x);
            check(xs_hip_transpose(st, src, ptr(p, Value{static_cast<int32_t>(i), 0}),
                                   static_cast<int64_t>(dtype_size(dtype(Value{static_cast<int32_t>(i), 0}))),
                                   static_cast<int>(xs.size()), xs.data(), pm.data()),
                  what);
            return;
        }
        case Op::Concat: {
            const int axis = std::get<graph::AxisAttrs>(nd.attrs).axis;
            int64_t outer = 1;
            for (int d = 0; d < axis; ++d) outer *= out[static_cast<size_t>(d)];
            const auto es = static_cast<int64_t>(dtype_size(dtype(Value{static_cast<int32_t>(i), 0})));
            const void* src[XS_CONCAT_PARTS] = {};
            int64_t bytes[XS_CONCAT_PARTS] = {};
            for (size_t k = 0; k < np.reads.size(); ++k) {
                const Value v = np.reads[k];
                src[k] = is_float(dtype(v)) ? static_cast<const void*>(f32(k)) : ptr(p, v);
                bytes[k] = outer > 0 ? numel(in_shape(v)) / outer * es : 0;
            }
            check(xs_hip_concat(st, static_cast<int>(np.reads.size()), src, bytes,
                                ptr(p, Value{static_cast<int32_t>(i), 0}), outer),
                  what);
            return;
        }
        case Op::SliceCopy: {
            const auto& a = std::get<graph::SliceAttrs>(nd.attrs);
            const Value x = np.reads[0];
            const Dims& in = in_shape(x);
            const int64_t dim = in[static_cast<size_t>(a.axis)];
            const int64_t begin = a.begin < 0 ? a.begin + dim : a.begin;
            int64_t outer = 1, inner = 1;
            for (size_t d = 0; d < static_cast<size_t>(a.axis); ++d) outer *= in[d];
            for (size_t d = static_cast<size_t>(a.axis) + 1; d < in.size(); ++d) inner *= in[d];
            const auto es = static_cast<int64_t>(dtype_size(dtype(x)));
            const int64_t len = out[static_cast<size_t>(a.axis)];
            check(xs_hip_copy_rows(st, ptr(p, x) + begin * inner * es, dim * inner * es,
                                   ptr(p, Value{static_cast<int32_t>(i), 0}), len * inner * es, outer, len * inner * es),
                  what);
            return;
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// Run.

void Program::run(const TensorMap& inputs, TensorMap& outputs, std::span<const std::string> only) {
    const auto& nodes = g_.nodes();
    // T from the inputs.
    int64_t T = -1;
    for (const Value& v : g_.inputs()) {
        const Node& nd = nodes[static_cast<size_t>(v.node)];
        const std::string& name = std::get<graph::InputAttrs>(nd.attrs).name;
        const auto it = inputs.find(name);
        XS_CHECK(it != inputs.end(), "hip: graph input '", name, "' was not given");
        const HostTensor& t = it->second;
        const Dims& want = nd.outputs[0].shape;
        XS_CHECK(t.dtype() == nd.outputs[0].dtype && t.rank() == want.size(), "hip: input '", name, "' is ",
                 dtype_name(t.dtype()), dims_to_string(t.shape()), ", the graph takes ",
                 dtype_name(nd.outputs[0].dtype), graph::shape_to_string(want));
        for (size_t d = 0; d < want.size(); ++d) {
            if (want[d] == kT) {
                XS_CHECK(T < 0 || T == t.dim(d), "hip: input '", name, "' has ", t.dim(d), " tokens, another ", T);
                T = t.dim(d);
            } else {
                XS_CHECK(want[d] == t.dim(d), "hip: input '", name, "' is ", dims_to_string(t.shape()),
                         ", the graph takes ", graph::shape_to_string(want));
            }
        }
    }
    if (T < 0) T = 1;
    XS_CHECK(T >= 1 || !appends_, "hip: a step appending to the KV cache needs at least one token");
    // L, and room in the slots, before anything runs.
    int64_t L = 0;
    if (!slot_of_.empty()) {
        const KvState& kv0 = s_.kv()[static_cast<size_t>(slot_of_[0])];
        L = appends_ ? kv0.len + T : kv0.len;
        for (const int slot : slot_of_) {
            const KvState& kv = s_.kv()[static_cast<size_t>(slot)];
            XS_CHECK(L <= kv.cap, "hip: ", L, " tokens exceed SessionOptions::max_context ", kv.cap, " (slot '",
                     kv.label, "')");
            XS_CHECK(!reads_kv_ || kv.len > 0 || T == 0, "hip: slot '", kv.label, "' holds no tokens to read");
        }
    }
    RunPlan& p = plan_for(T, only);
    s_.grow_arena(p.arena_bytes);
    s_.grow_sync(p.sync_bytes);
    // The host side goes through page-locked staging, so every copy is asynchronous and the step waits once: the step
    // record, then the inputs, then the outputs.
    size_t stage_bytes = 256;
    for (const Value& v : g_.inputs()) {
        const auto i = static_cast<size_t>(v.node);
        if (p.live[i]) stage_bytes += align_up(inputs.at(std::get<graph::InputAttrs>(nodes[i].attrs).name).nbytes());
    }
    for (const auto& o : g_.outputs()) {
        if (!only.empty() && std::find(only.begin(), only.end(), o.name) == only.end()) continue;
        const DType d = dtype(o.value);
        const Dims& shape = p.shapes[static_cast<size_t>(o.value.node)][static_cast<size_t>(o.value.index)];
        stage_bytes += align_up(static_cast<size_t>(numel(shape)) * dtype_size(is_float(d) ? DType::F32 : d));
    }
    char* const stage = s_.staging(stage_bytes);
    size_t at = 256;
    // Inputs.
    for (const Value& v : g_.inputs()) {
        const auto i = static_cast<size_t>(v.node);
        if (!p.live[i]) continue;
        const HostTensor& t = inputs.at(std::get<graph::InputAttrs>(nodes[i].attrs).name);
        if (t.nbytes() > 0) {
            std::memcpy(stage + at, t.raw(), t.nbytes());
            check(xs_hip_memcpy_h2d_async(ptr(p, v), stage + at, t.nbytes(), s_.stream()), "input upload");
            at += align_up(t.nbytes());
        }
    }
    launch_all(p, T, L);
    // Outputs: f32 for floats (16-bit values widened on the device), integers as they are.
    TensorMap result;
    std::vector<std::pair<std::string, size_t>> staged;  // output, its place in the staging
    for (const auto& o : g_.outputs()) {
        if (!only.empty() && std::find(only.begin(), only.end(), o.name) == only.end()) continue;
        const DType d = dtype(o.value);
        const Dims& shape = p.shapes[static_cast<size_t>(o.value.node)][static_cast<size_t>(o.value.index)];
        HostTensor t(is_float(d) ? DType::F32 : d, shape);
        const char* src = ptr(p, o.value);
        if (is_float(d) && d != DType::F32) {
            const int32_t c = p.conv[static_cast<size_t>(o.value.node)];
            XS_CHECK(c >= 0, "hip: no f32 copy of output '", o.name, "'");
            char* dst = s_.arena().get() + p.block_offset[static_cast<size_t>(c)];
            check(xs_hip_convert(s_.stream(), abi(d), src, XS_F32, dst, numel(shape)), "output");
            src = dst;
        }
        if (t.nbytes() > 0) {
            check(xs_hip_memcpy_d2h_async(stage + at, src, t.nbytes(), s_.stream()), "output download");
            staged.emplace_back(o.name, at);
            at += align_up(t.nbytes());
        }
        result[o.name] = std::move(t);
    }
    check(xs_hip_stream_synchronize(s_.stream()), "step");
    for (const auto& [name, off] : staged) {
        HostTensor& t = result.at(name);
        std::memcpy(t.raw(), stage + off, t.nbytes());
    }
    if (appends_) {
        for (const int slot : slot_of_) s_.kv()[static_cast<size_t>(slot)].len = L;
    }
    for (auto& [name, t] : result) outputs[name] = std::move(t);
}

// The step's launches. With graphs on, a (plan, key-count bucket) that runs a second time is captured into a HIP
// graph, and later runs replay it: the bucket is the smallest power of two >= L (capped at the slots' capacity), the
// attention takes that bucket's split, and the KV append and attention read where to append and how many keys there
// are from the step record uploaded before the replay. A one-off step (a prefill of a new length) runs eagerly.
void Program::launch_all(RunPlan& p, int64_t T, int64_t L) {
    const auto each = [&](int64_t replay_cap) {
        for (size_t i = 0; i < g_.nodes().size(); ++i) {
            if (p.live[i] && plan_[i].op != Op::None) launch(i, p, T, L, replay_cap);
        }
    };
    // Graphs off, or a reading step with fewer keys than queries (whose refusal comes from the launch): eagerly.
    if (!s_.graphs() || (!appends_ && L < T)) return each(0);
    int64_t cap = 0;  // the bucket's key count (0 without KV slots)
    if (!slot_of_.empty()) {
        cap = 1;
        while (cap < L) cap *= 2;
        for (const int slot : slot_of_) cap = std::min(cap, s_.kv()[static_cast<size_t>(slot)].cap);
        cap = std::max<int64_t>(cap, 1);
    }
    RunPlan::Captured& g = p.graphs[static_cast<int>(cap)];
    if (g.exec != nullptr && g.arena_gen != s_.arena_gen()) {  // the arena moved under it
        check(xs_hip_graph_destroy(g.exec), "graph");
        g = RunPlan::Captured{};
    }
    s_.set_step(L - T, L);
    if (g.exec == nullptr && ++g.runs >= 2) {
        check(xs_hip_stream_begin_capture(s_.stream()), "capture");
        try {
            each(std::max<int64_t>(cap, 1));
        } catch (...) {
            void* discard = nullptr;
            xs_hip_stream_end_capture(s_.stream(), &discard);
            if (discard != nullptr) xs_hip_graph_destroy(discard);
            throw;
        }
        check(xs_hip_stream_end_capture(s_.stream(), &g.exec), "capture");
        g.arena_gen = s_.arena_gen();
    }
    if (g.exec != nullptr) {
        check(xs_hip_graph_launch(g.exec, s_.stream()), "graph replay");
    } else {
        each(0);
    }
}

Program::~Program() {
    for (auto& [key, plan] : plans_) {
        for (auto& [cap, g] : plan.graphs) {
            if (g.exec != nullptr) xs_hip_graph_destroy(g.exec);
        }
    }
}

int64_t Program::cached() const {
    if (slot_of_.empty() || !appends_) return 0;
    return s_.kv()[static_cast<size_t>(slot_of_[0])].len;
}

void Program::truncate(int64_t n) {
    const int64_t have = cached();
    XS_CHECK(n >= 0 && n <= have, "hip: cannot truncate to ", n, " tokens; ", have, " are cached");
    if (!appends_) return;
    for (const int slot : slot_of_) s_.kv()[static_cast<size_t>(slot)].len = n;
}

HipSession::HipSession(std::span<const Graph* const> programs, const WeightStore& weights,
                       const SessionOptions& options)
    : weights_(weights), options_(options) {
    XS_CHECK(!programs.empty(), "hip: nothing to compile");
    XS_CHECK(options_.max_context > 0, "hip: max_context ", options_.max_context);
    XS_CHECK(options_.rewind_tokens >= 0, "hip: rewind_tokens ", options_.rewind_tokens);
    // As cpu-ref (cpu_backend.cpp:75-76, 611): f16 or f32, and activations computed in f32 either way; the precision
    // picks the Float KV format's row type (f16 rows at f16 precision, f32 rows at f32).
    XS_CHECK(options_.precision == DType::F16 || options_.precision == DType::F32,
             "hip: session precision must be f16 or f32, got ", dtype_name(options_.precision));
    for (const auto& [key, value] : options_.extra) {
        XS_CHECK(key == "graphs", "hip: unknown backend option '", key, "' (known: graphs)");
        XS_CHECK(value == "0" || value == "1", "hip: backend option graphs=", value, " (expected 0 or 1)");
        graphs_ = value == "1";
    }
    // Plan every program first: what this backend cannot run is refused before any device work.
    for (size_t i = 0; i < programs.size(); ++i) programs_.push_back(std::make_unique<Program>(*programs[i], *this, i));
    int count = 0;
    check(xs_hip_device_count(&count), "device count");
    XS_CHECK(count > 0, "hip: no HIP device");
    int device = 0;
    if (!options_.device.empty()) {
        const std::string& d = options_.device;
        const std::string n = d.rfind("GPU.", 0) == 0 ? d.substr(4) : std::string();
        XS_CHECK(!n.empty() && n.size() < 6 && n.find_first_not_of("0123456789") == std::string::npos, "hip: device '",
                 d, "' (expected GPU.<n>)");
        device = std::stoi(n);
        XS_CHECK(device >= 0 && device < count, "hip: device '", d, "' (", count, " present)");
    }
    check(xs_hip_set_device(device), "set device");
    check(xs_hip_stream_create(&stream_), "stream");
    try {
        for (KvState& k : kv_) {
            const auto rows = static_cast<size_t>(k.cap * k.heads);
            if (k.kf == quant::KvFormat::Float) {
                const size_t width = static_cast<size_t>(k.dim) * dtype_size(k.rows);
                k.kc.grow(rows * width);
                k.vc.grow(rows * width);
            } else {
                k.kc.grow(rows * static_cast<size_t>(kv_code_bytes(k.kf, k.dim)));
                k.ks.grow(rows * static_cast<size_t>(kv_scale_bytes(k.kf, k.dim)));
                k.vc.grow(rows * static_cast<size_t>(kv_code_bytes(k.vf, k.dim)));
                k.vs.grow(rows * static_cast<size_t>(kv_scale_bytes(k.vf, k.dim)));
            }
        }
        step_.grow(2 * sizeof(int64_t));
        staging(256);
        for (auto& p : programs_) p->upload();
        check(xs_hip_stream_synchronize(stream_), "weight upload");
    } catch (...) {
        // The destructor does not run for a constructor that throws: wait for what was queued, then let the stream go.
        xs_hip_stream_synchronize(stream_);
        xs_hip_stream_destroy(stream_);
        stream_ = nullptr;
        throw;
    }
}

class HipBackend final : public Backend {
public:
    std::string_view name() const override { return "hip"; }
    std::vector<DeviceInfo> devices() const override {
        int count = 0;
        if (xs_hip_device_count(&count) != XS_HIP_OK) return {};
        std::vector<DeviceInfo> out;
        for (int d = 0; d < count; ++d) {
            char name[256] = {0};
            uint64_t bytes = 0;
            int cus = 0;
            if (xs_hip_device_info(d, name, sizeof(name), &bytes, &cus) != XS_HIP_OK) continue;
            out.push_back(DeviceInfo{"GPU." + std::to_string(d), name, bytes, false});
        }
        return out;
    }
    std::unique_ptr<Session> compile(std::span<const Graph* const> programs, const WeightStore& weights,
                                     const SessionOptions& options) override {
        return std::make_unique<HipSession>(programs, weights, options);
    }
};

}  // namespace

std::unique_ptr<Backend> make_hip_backend() { return std::make_unique<HipBackend>(); }

}  // namespace xs
