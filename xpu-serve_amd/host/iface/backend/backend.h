#pragma once

// The backend interface (reference src/backend/backend.h:20-92): a Backend compiles step graphs into a Session that
// runs them over one sequence and owns its KV state. Same classes, members and contracts; restated for the HIP
// backend's standalone build.

#include <cstdint>
#include <map>
#include <memory>
#include <span>
#include <string>
#include <string_view>
#include <vector>

#include "graph/graph.h"
#include "io/safetensors.h"
#include "quant/kv_format.h"
#include "tensor/tensor.h"

namespace xs {

struct DeviceInfo {
    std::string id;
    std::string name;
    uint64_t memory_bytes = 0;
    bool integrated = false;
};

struct SessionOptions {
    std::string device;
    DType precision = DType::F16;
    int64_t max_context = 8192;
    quant::KvFormats kv;
    int64_t rewind_tokens = 0;
    std::map<std::string, std::string> extra;
};

class Session {
public:
    virtual ~Session() = default;
    virtual void run(size_t program, const TensorMap& inputs, TensorMap& outputs, std::span<const std::string> only) = 0;
    void run(size_t program, const TensorMap& inputs, TensorMap& outputs) { run(program, inputs, outputs, {}); }
    void run(const TensorMap& inputs, TensorMap& outputs) { run(0, inputs, outputs, {}); }
    virtual int64_t num_cached(size_t program) const = 0;
    int64_t num_cached() const { return num_cached(0); }
    virtual void reset() = 0;
    virtual void truncate(size_t program, int64_t n) = 0;
    void truncate(int64_t n) { truncate(0, n); }
};

class Backend {
public:
    virtual ~Backend() = default;
    virtual std::string_view name() const = 0;
    virtual std::vector<DeviceInfo> devices() const = 0;
    virtual std::unique_ptr<Session> compile(std::span<const graph::Graph* const> programs, const WeightStore& weights,
                                             const SessionOptions& options) = 0;
    std::unique_ptr<Session> compile(const graph::Graph& graph, const WeightStore& weights,
                                     const SessionOptions& options) {
        const graph::Graph* programs[] = {&graph};
        return compile(programs, weights, options);
    }
};

std::vector<std::string> available_backends();
std::unique_ptr<Backend> make_backend(std::string_view name);

// The HIP backend (hip_backend.cpp): what the reference's registry adds under XS_HAVE_HIP.
std::unique_ptr<Backend> make_hip_backend();

}  // namespace xs
