// tensor_table.h -- name -> tensor map with the reference's ownership
// convention (include/onnx/tensor_table.h:22-145): intermediates, weights
// and packed weights are owned (unique_ptr); external inputs and outputs are
// borrowed (reference_wrapper).  Operators only ever receive references.
#pragma once

#include <memory>
#include <string>
#include <unordered_map>
#include <variant>

#include "onnx/tensor.h"

namespace lcml::onnx {

class TensorTable {
    using Entry = std::variant<std::reference_wrapper<ITensor>, std::unique_ptr<ITensor>>;
    std::unordered_map<std::string, Entry> map_;

public:
    void bind(std::string name, ITensor &t) { map_.insert_or_assign(std::move(name), Entry{std::ref(t)}); }
    void own(std::string name, std::unique_ptr<ITensor> t) { map_.insert_or_assign(std::move(name), Entry{std::move(t)}); }
    bool contains(std::string_view name) const { return map_.find(std::string(name)) != map_.end(); }
    bool is_owned(std::string_view name) const {
        auto it = map_.find(std::string(name));
        return it != map_.end() && it->second.index() == 1;
    }
    ITensor &at(std::string_view name) {
        auto it = map_.find(std::string(name));
        LCML_ASSERT(it != map_.end(), "TensorTable: key not found: %.*s", (int)name.size(), name.data());
        if (it->second.index() == 0) return std::get<0>(it->second).get();
        return *std::get<1>(it->second);
    }
    void erase(std::string_view name) { map_.erase(std::string(name)); }
    void clear() { map_.clear(); }
    size_t size() const { return map_.size(); }
};

}  // namespace lcml::onnx
