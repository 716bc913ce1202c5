// The standalone build's implementation of the interface surface the HIP backend compiles against: dtypes, host
// tensors, weight views, KV format names and the backend registry (reference src/tensor/dtype.cpp,
// src/tensor/tensor.cpp, src/io/safetensors.cpp's WeightStore::get, src/quant/kv_format.cpp,
// src/backend/registry.cpp:11-30). In the reference tree the reference's own files provide these.
#include <cstring>
#include <sstream>

#include "backend/backend.h"
#include "util/error.h"

namespace xs {

size_t dtype_size(DType t) {
    switch (t) {
        case DType::F32: case DType::I32: return 4;
        case DType::F16: case DType::BF16: return 2;
        case DType::I64: return 8;
        case DType::I8: case DType::U8: case DType::Bool: return 1;
        default: fail("dtype ", dtype_name(t), " has no element size");
    }
}

std::string_view dtype_name(DType t) {
    static constexpr std::string_view names[] = {"f32", "f16", "bf16", "i64", "i32", "i8", "u8", "bool",
                                                 "q8",  "q4",  "f8",   "block", "f4"};
    const auto i = static_cast<size_t>(t);
    return i < std::size(names) ? names[i] : "?";
}

bool is_float(DType t) { return t == DType::F32 || t == DType::F16 || t == DType::BF16; }

int64_t numel(const Dims& dims) {
    int64_t n = 1;
    for (const int64_t d : dims) n *= d;
    return n;
}

std::string dims_to_string(const Dims& dims) {
    std::ostringstream os;
    os << '[';
    for (size_t i = 0; i < dims.size(); ++i) os << (i ? ", " : "") << dims[i];
    os << ']';
    return os.str();
}

HostTensor::HostTensor(DType dtype, Dims shape) : dtype_(dtype), shape_(std::move(shape)) {
    for (const int64_t d : shape_) XS_CHECK(d >= 0, "host tensor dim ", d, " in ", dims_to_string(shape_));
    const size_t bytes = std::max<size_t>(nbytes(), 1);
    storage_ = std::shared_ptr<void>(::operator new(bytes), [](void* p) { ::operator delete(p); });
    std::memset(storage_.get(), 0, bytes);
    data_ = storage_.get();
}

HostTensor HostTensor::borrow(DType dtype, Dims shape, void* data) {
    HostTensor t;
    t.dtype_ = dtype;
    t.shape_ = std::move(shape);
    t.data_ = data;
    return t;
}

HostTensor HostTensor::clone() const {
    HostTensor t(dtype_, shape_);
    if (nbytes() > 0) std::memcpy(t.data_, data_, nbytes());
    return t;
}

HostTensor HostTensor::reshaped(Dims shape) const {
    XS_CHECK(xs::numel(shape) == numel(), "reshape ", dims_to_string(shape_), " -> ", dims_to_string(shape));
    HostTensor t = *this;
    t.shape_ = std::move(shape);
    return t;
}

const TensorView& WeightStore::get(const std::string& name) const {
    const TensorView* v = find(name);
    if (v == nullptr) fail("weight '", name, "' not found");
    return *v;
}

const TensorView* MapWeights::find(const std::string& name) const {
    const auto it = views_.find(name);
    return it == views_.end() ? nullptr : &it->second;
}

std::vector<std::string> MapWeights::names() const {
    std::vector<std::string> out;
    for (const auto& [name, view] : views_) out.push_back(name);
    return out;
}

namespace quant {
std::string_view kv_format_name(KvFormat f) {
    switch (f) {
        case KvFormat::Float: return "auto";
        case KvFormat::I8: return "i8";
        case KvFormat::Turbo4: return "turbo4";
        case KvFormat::Turbo3: return "turbo3";
        case KvFormat::Turbo2: return "turbo2";
    }
    return "?";
}
}  // namespace quant

std::vector<std::string> available_backends() { return {"hip"}; }

std::unique_ptr<Backend> make_backend(std::string_view name) {
    if (name == "hip") return make_hip_backend();
    fail("unknown backend '", name, "'; available: hip");
}

}  // namespace xs
