#pragma once

// Named weights as a backend receives them (reference src/io/safetensors.h:15-25): find / names / get. Files are out of
// scope here; MapWeights holds views of caller-owned memory, which is how the tests and the bench feed weights.

#include <map>
#include <string>
#include <vector>

#include "tensor/tensor.h"

namespace xs {

class WeightStore {
public:
    virtual ~WeightStore() = default;
    virtual const TensorView* find(const std::string& name) const = 0;  // nullptr when absent
    virtual std::vector<std::string> names() const = 0;

    const TensorView& get(const std::string& name) const;  // throws naming the weight when absent
    bool contains(const std::string& name) const { return find(name) != nullptr; }
};

class MapWeights final : public WeightStore {
public:
    void add(const std::string& name, TensorView view) { views_[name] = std::move(view); }
    const TensorView* find(const std::string& name) const override;
    std::vector<std::string> names() const override;

private:
    std::map<std::string, TensorView> views_;
};

}  // namespace xs
