// TEST INFRASTRUCTURE: extern "C" access to the HIP backend (libxs_session.so) for the Python tests -- graph
// building through xs::graph::Graph's builders, named weights, Backend::compile and Session::run / num_cached / reset
// / truncate. Values cross as node * 8 + output index; errors as a nonzero status (or null / -1) with the message in
// xst_error(). Every call catches the backend's xs::Error, so a refusal reads as its diagnosis.
#include <cstring>
#include <map>
#include <memory>
#include <algorithm>
#include <chrono>
#include <string>
#include <vector>

#include "backend/backend.h"
#include "util/error.h"

using namespace xs;
using graph::Graph;
using graph::Value;

namespace {

thread_local std::string g_error;

int64_t enc(Value v) { return static_cast<int64_t>(v.node) * 8 + v.index; }
Value dec(int64_t e) { return e < 0 ? Value{} : Value{static_cast<int32_t>(e / 8), static_cast<int32_t>(e % 8)}; }
Dims dims(int rank, const int64_t* d) { return Dims(d, d + rank); }

template <typename F>
int64_t guard(F&& f) {
    try {
        return f();
    } catch (const std::exception& e) {
        g_error = e.what();
        return -1;
    }
}

// Weights owning their bytes.
struct Store {
    MapWeights views;
    std::vector<HostTensor> owned;
};

struct SessionBox {
    std::unique_ptr<Backend> backend;
    std::unique_ptr<Session> session;
    TensorMap outputs;
};

}  // namespace

extern "C" {

const char* xst_error() { return g_error.c_str(); }

const char* xst_backends() {
    static std::string s;
    s.clear();
    for (const std::string& b : available_backends()) s += (s.empty() ? "" : ",") + b;
    return s.c_str();
}

void* xsg_new() { return new Graph(); }
void xsg_free(void* g) { delete static_cast<Graph*>(g); }

int64_t xsg_input(void* g, const char* name, int dtype, int rank, const int64_t* d) {
    return guard([&] { return enc(static_cast<Graph*>(g)->input(name, static_cast<DType>(dtype), dims(rank, d))); });
}

int64_t xsg_weight(void* g, void* store, const char* name) {
    return guard([&] { return enc(static_cast<Graph*>(g)->weight(static_cast<Store*>(store)->views, name)); });
}

int64_t xsg_constant(void* g, int dtype, int rank, const int64_t* d, const void* data) {
    return guard([&] {
        HostTensor t(static_cast<DType>(dtype), dims(rank, d));
        if (t.nbytes() > 0) std::memcpy(t.raw(), data, t.nbytes());
        return enc(static_cast<Graph*>(g)->constant(std::move(t)));
    });
}

int64_t xsg_matmul(void* g, int64_t x, int64_t w) {
    return guard([&] { return enc(static_cast<Graph*>(g)->matmul(dec(x), dec(w))); });
}

// kind: 0 add, 1 mul, 2 div
int64_t xsg_binary(void* g, int kind, int64_t a, int64_t b) {
    return guard([&] {
        Graph& gr = *static_cast<Graph*>(g);
        return enc(kind == 0 ? gr.add(dec(a), dec(b)) : kind == 1 ? gr.mul(dec(a), dec(b)) : gr.div(dec(a), dec(b)));
    });
}

// kind: the OpKind value of Scale, Tanh, GeluTanh, Softcap, Sigmoid, Silu, Softplus, Clamp, Gelu
int64_t xsg_unary(void* g, int kind, int64_t x, float p0, float p1) {
    return guard([&] {
        Graph& gr = *static_cast<Graph*>(g);
        const Value v = dec(x);
        switch (static_cast<graph::OpKind>(kind)) {
            case graph::OpKind::Scale: return enc(gr.scale(v, p0));
            case graph::OpKind::Tanh: return enc(gr.tanh(v));
            case graph::OpKind::GeluTanh: return enc(gr.gelu_tanh(v));
            case graph::OpKind::Softcap: return enc(gr.softcap(v, p0));
            case graph::OpKind::Sigmoid: return enc(gr.sigmoid(v));
            case graph::OpKind::Silu: return enc(gr.silu(v));
            case graph::OpKind::Softplus: return enc(gr.softplus(v));
            case graph::OpKind::Clamp: return enc(gr.clamp(v, p0, p1));
            case graph::OpKind::Gelu: return enc(gr.gelu(v));
            default: fail("not a unary op kind: ", kind);
        }
    });
}

int64_t xsg_rms_norm(void* g, int64_t x, int64_t w, float eps) {
    return guard([&] {
        Graph& gr = *static_cast<Graph*>(g);
        return enc(w < 0 ? gr.rms_norm(dec(x), eps) : gr.rms_norm(dec(x), dec(w), eps));
    });
}

int64_t xsg_layer_norm(void* g, int64_t x, int64_t w, int64_t b, float eps) {
    return guard([&] { return enc(static_cast<Graph*>(g)->layer_norm(dec(x), dec(w), dec(b), eps)); });
}

int64_t xsg_l2_clip(void* g, int64_t x, float threshold, float eps) {
    return guard([&] { return enc(static_cast<Graph*>(g)->l2_clip(dec(x), threshold, eps)); });
}

int64_t xsg_reshape(void* g, int64_t x, int rank, const int64_t* d) {
    return guard([&] { return enc(static_cast<Graph*>(g)->reshape(dec(x), dims(rank, d))); });
}

int64_t xsg_slice(void* g, int64_t x, int axis, int64_t begin, int64_t end) {
    return guard([&] { return enc(static_cast<Graph*>(g)->slice(dec(x), axis, begin, end)); });
}

int64_t xsg_transpose(void* g, int64_t x, int rank, const int32_t* perm) {
    return guard([&] { return enc(static_cast<Graph*>(g)->transpose(dec(x), std::vector<int>(perm, perm + rank))); });
}

int64_t xsg_gather(void* g, int64_t table, int64_t ids) {
    return guard([&] { return enc(static_cast<Graph*>(g)->gather(dec(table), dec(ids))); });
}

int64_t xsg_concat(void* g, int count, const int64_t* parts, int axis) {
    return guard([&] {
        std::vector<Value> vs;
        for (int k = 0; k < count; ++k) vs.push_back(dec(parts[k]));
        return enc(static_cast<Graph*>(g)->concat(vs, axis));
    });
}

int64_t xsg_rope(void* g, int64_t x, int64_t positions, int64_t inv_freq, int64_t rotary, int64_t pair_axes) {
    return guard([&] {
        return enc(static_cast<Graph*>(g)->rope(dec(x), dec(positions), dec(inv_freq), rotary, dec(pair_axes)));
    });
}

int64_t xsg_kv_slot(void* g, int64_t heads, int64_t dim, int64_t window, const char* label) {
    return guard([&] { return static_cast<int64_t>(static_cast<Graph*>(g)->add_kv_slot(heads, dim, window, label)); });
}

int64_t xsg_kv_cache(void* g, int slot, int64_t k, int64_t v) {
    return guard([&] { return enc(static_cast<Graph*>(g)->kv_cache(slot, dec(k), dec(v)).first); });
}

int64_t xsg_kv_read(void* g, int slot) {
    return guard([&] { return enc(static_cast<Graph*>(g)->kv_read(slot).first); });
}

int64_t xsg_attention(void* g, int64_t q, int64_t k, int64_t v, float scale, int64_t window, float softcap,
                      int causal) {
    return guard([&] {
        graph::AttentionAttrs a;
        a.scale = scale;
        a.sliding_window = window;
        a.softcap = softcap;
        a.causal = causal != 0;
        return enc(static_cast<Graph*>(g)->attention(dec(q), dec(k), dec(v), a));
    });
}

int64_t xsg_softmax(void* g, int64_t x) {
    return guard([&] { return enc(static_cast<Graph*>(g)->softmax(dec(x))); });
}

int64_t xsg_topk(void* g, int64_t x, int64_t k) {
    return guard([&] { return enc(static_cast<Graph*>(g)->topk(dec(x), k).first); });
}

int64_t xsg_reduce_sum(void* g, int64_t x, int axis) {
    return guard([&] { return enc(static_cast<Graph*>(g)->reduce_sum(dec(x), axis)); });
}

int xsg_output(void* g, const char* name, int64_t v) {
    return static_cast<int>(guard([&] {
        static_cast<Graph*>(g)->output(name, dec(v));
        return int64_t{0};
    }));
}

// The graph's output names, one a line (the same buffer protocol as xsg_dump).
int64_t xsg_outputs(void* g, char* buf, int64_t len) {
    return guard([&] {
        std::string s;
        for (const auto& o : static_cast<Graph*>(g)->outputs()) s += o.name + "\n";
        if (buf != nullptr && len > 0) {
            const size_t n = std::min<size_t>(s.size(), static_cast<size_t>(len - 1));
            std::memcpy(buf, s.data(), n);
            buf[n] = 0;
        }
        return static_cast<int64_t>(s.size());
    });
}

int64_t xsg_dump(void* g, char* buf, int64_t len) {
    return guard([&] {
        const std::string s = static_cast<Graph*>(g)->dump();
        if (buf != nullptr && len > 0) {
            const size_t n = std::min<size_t>(s.size(), static_cast<size_t>(len - 1));
            std::memcpy(buf, s.data(), n);
            buf[n] = 0;
        }
        return static_cast<int64_t>(s.size());
    });
}

void* xsw_new() { return new Store(); }
void xsw_free(void* s) { delete static_cast<Store*>(s); }

int xsw_add(void* store, const char* name, int dtype, int rank, const int64_t* d, const void* data) {
    return static_cast<int>(guard([&] {
        Store& s = *static_cast<Store*>(store);
        HostTensor t(static_cast<DType>(dtype), dims(rank, d));
        if (t.nbytes() > 0) std::memcpy(t.raw(), data, t.nbytes());
        s.views.add(name, t.view());
        s.owned.push_back(std::move(t));
        return int64_t{0};
    }));
}

// kv_k / kv_v: KvFormat values (0 float, 1 i8, ...); precision: a DType value.
void* xss_compile(int nprog, void* const* graphs, void* store, int precision, int64_t max_context, int kv_k, int kv_v,
                  const char* device) {
    try {
        auto box = std::make_unique<SessionBox>();
        box->backend = make_backend("hip");
        SessionOptions o;
        o.precision = static_cast<DType>(precision);
        o.max_context = max_context;
        o.kv.k = static_cast<quant::KvFormat>(kv_k);
        o.kv.v = static_cast<quant::KvFormat>(kv_v);
        o.device = device != nullptr ? device : "";
        std::vector<const Graph*> progs;
        for (int i = 0; i < nprog; ++i) progs.push_back(static_cast<const Graph*>(graphs[i]));
        box->session = box->backend->compile(progs, static_cast<Store*>(store)->views, o);
        return box.release();
    } catch (const std::exception& e) {
        g_error = e.what();
        return nullptr;
    }
}

// xss_compile with backend options: "key=value" pairs separated by ';' (SessionOptions::extra).
void* xss_compile_opts(int nprog, void* const* graphs, void* store, int precision, int64_t max_context, int kv_k,
                       int kv_v, const char* device, const char* extra) {
    try {
        auto box = std::make_unique<SessionBox>();
        box->backend = make_backend("hip");
        SessionOptions o;
        o.precision = static_cast<DType>(precision);
        o.max_context = max_context;
        o.kv.k = static_cast<quant::KvFormat>(kv_k);
        o.kv.v = static_cast<quant::KvFormat>(kv_v);
        o.device = device != nullptr ? device : "";
        std::string rest = extra != nullptr ? extra : "";
        while (!rest.empty()) {
            const size_t end = rest.find(';');
            const std::string kv = rest.substr(0, end);
            rest = end == std::string::npos ? "" : rest.substr(end + 1);
            const size_t eq = kv.find('=');
            if (!kv.empty()) o.extra[kv.substr(0, eq)] = eq == std::string::npos ? "" : kv.substr(eq + 1);
        }
        std::vector<const Graph*> progs;
        for (int i = 0; i < nprog; ++i) progs.push_back(static_cast<const Graph*>(graphs[i]));
        box->session = box->backend->compile(progs, static_cast<Store*>(store)->views, o);
        return box.release();
    } catch (const std::exception& e) {
        g_error = e.what();
        return nullptr;
    }
}

void xss_free(void* s) { delete static_cast<SessionBox*>(s); }

int xss_run(void* s, int64_t program, int n_in, const char* const* names, const int* dtypes, const int* ranks,
            const int64_t* all_dims, const void* const* datas, int n_only, const char* const* only) {
    return static_cast<int>(guard([&] {
        SessionBox& b = *static_cast<SessionBox*>(s);
        TensorMap in;
        const int64_t* d = all_dims;
        for (int i = 0; i < n_in; ++i) {
            in[names[i]] = HostTensor::borrow(static_cast<DType>(dtypes[i]), dims(ranks[i], d), const_cast<void*>(datas[i]));
            d += ranks[i];
        }
        std::vector<std::string> o(only, only + n_only);
        b.outputs.clear();
        b.session->run(static_cast<size_t>(program), in, b.outputs, o);
        return int64_t{0};
    }));
}

// Runs `program` `iters` times on the same inputs and stores the mean wall time of one Session::run in *us_per_run:
// the backend's step cost (inputs up, launches or a graph replay, outputs down, the wait) timed from C++.
int xss_time_runs(void* s, int64_t program, int n_in, const char* const* names, const int* dtypes, const int* ranks,
                  const int64_t* all_dims, const void* const* datas, int iters, double* us_per_run) {
    return static_cast<int>(guard([&] {
        SessionBox& b = *static_cast<SessionBox*>(s);
        TensorMap in;
        const int64_t* d = all_dims;
        for (int i = 0; i < n_in; ++i) {
            in[names[i]] = HostTensor::borrow(static_cast<DType>(dtypes[i]), dims(ranks[i], d), const_cast<void*>(datas[i]));
            d += ranks[i];
        }
        const auto t0 = std::chrono::steady_clock::now();
        for (int k = 0; k < iters; ++k) {
            b.outputs.clear();
            b.session->run(static_cast<size_t>(program), in, b.outputs, {});
        }
        const std::chrono::duration<double, std::micro> dt = std::chrono::steady_clock::now() - t0;
        *us_per_run = dt.count() / std::max(iters, 1);
        return int64_t{0};
    }));
}

// The output `name` of the last run: dtype, rank, dims (up to 8) and a pointer valid until the next run.
int xss_output(void* s, const char* name, int* dtype, int* rank, int64_t* d, const void** data) {
    return static_cast<int>(guard([&] {
        SessionBox& b = *static_cast<SessionBox*>(s);
        const auto it = b.outputs.find(name);
        if (it == b.outputs.end()) fail("no output '", name, "' in the last run");
        const HostTensor& t = it->second;
        *dtype = static_cast<int>(t.dtype());
        *rank = static_cast<int>(t.rank());
        for (size_t i = 0; i < t.rank() && i < 8; ++i) d[i] = t.dim(i);
        *data = t.raw();
        return int64_t{0};
    }));
}

int64_t xss_num_cached(void* s, int64_t program) {
    return guard([&] { return static_cast<SessionBox*>(s)->session->num_cached(static_cast<size_t>(program)); });
}

int xss_reset(void* s) {
    return static_cast<int>(guard([&] {
        static_cast<SessionBox*>(s)->session->reset();
        return int64_t{0};
    }));
}

int xss_truncate(void* s, int64_t program, int64_t n) {
    return static_cast<int>(guard([&] {
        static_cast<SessionBox*>(s)->session->truncate(static_cast<size_t>(program), n);
        return int64_t{0};
    }));
}

}  // extern "C"
