// operator.h -- operator base class of the host layer.
//
// Same interface as the reference's Operator (include/onnx/operator.h:16-54):
// forward() over spans of tensor references, the is_output_view /
// can_operate_inplace / need_outline / set_environment / set_warp_size hooks,
// and a name.  Here forward() runs eagerly: it launches HIP work on the
// network's stream instead of emitting kernel AST.
#pragma once

#include <functional>
#include <span>
#include <string>

#include "onnx/tensor.h"

namespace lcml::onnx {

class Node;
class NetworkInstance;
class TensorTable;

class Operator {
    std::string name_;

public:
    Operator() = delete;
    virtual ~Operator() = default;
    Operator(const Operator &) = default;
    Operator(Operator &&) noexcept = default;
    Operator &operator=(const Operator &) = default;
    Operator &operator=(Operator &&) noexcept = default;

    explicit Operator(std::string name) : name_(std::move(name)) {}
    const std::string &get_name() const { return name_; }

    virtual void forward(std::span<std::reference_wrapper<ITensor>> inputs,
                         std::span<std::reference_wrapper<ITensor>> outputs) = 0;

    virtual bool is_output_view([[maybe_unused]] size_t output_index, [[maybe_unused]] const Node &node) const {
        return false;
    }
    // Gemm / MatMul / Conv never run in place (operator.h:40-47 of the reference).
    virtual bool can_operate_inplace() const { return false; }
    virtual bool need_outline() const { return true; }
    // called once per forward, before forward(), with the executing network
    virtual void set_environment(NetworkInstance &, TensorTable &) {}
    virtual void set_warp_size(uint32_t) {}
};

}  // namespace lcml::onnx
