#pragma once

// Host tensors as the backend interface passes them (reference src/tensor/tensor.h:74-116): a dense row-major
// HostTensor with shared storage, a non-owning TensorView, and TensorMap. Only what the HIP backend and its tests use.

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "tensor/dtype.h"

namespace xs {

using Dims = std::vector<int64_t>;

int64_t numel(const Dims& dims);
std::string dims_to_string(const Dims& dims);

struct TensorView {
    DType dtype = DType::F32;
    Dims shape;
    const void* data = nullptr;

    int64_t numel() const { return xs::numel(shape); }
    size_t nbytes() const { return static_cast<size_t>(numel()) * dtype_size(dtype); }
};

class HostTensor {
public:
    HostTensor() = default;
    HostTensor(DType dtype, Dims shape);  // zero-filled storage
    static HostTensor borrow(DType dtype, Dims shape, void* data);

    DType dtype() const { return dtype_; }
    const Dims& shape() const { return shape_; }
    int64_t dim(size_t i) const { return shape_.at(i); }
    size_t rank() const { return shape_.size(); }
    int64_t numel() const { return xs::numel(shape_); }
    size_t nbytes() const { return static_cast<size_t>(numel()) * dtype_size(dtype_); }
    bool empty() const { return data_ == nullptr; }

    void* raw() { return data_; }
    const void* raw() const { return data_; }
    template <typename T>
    T* data() { return static_cast<T*>(data_); }
    template <typename T>
    const T* data() const { return static_cast<const T*>(data_); }

    TensorView view() const { return {dtype_, shape_, data_}; }
    HostTensor clone() const;
    HostTensor reshaped(Dims shape) const;

private:
    DType dtype_ = DType::F32;
    Dims shape_;
    std::shared_ptr<void> storage_;
    void* data_ = nullptr;
};

using TensorMap = std::map<std::string, HostTensor>;

}  // namespace xs
