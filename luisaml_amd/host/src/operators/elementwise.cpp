// Add / Sub / Mul / Div on FLOAT, FLOAT8E4M3FN and FLOAT8E5M2 tensors with
// numpy broadcasting, as the reference's Binary operators
// (src/onnx/operators/binary.cpp:335-345; broadcasting 59-182; the quantised
// path 184-285: decode both operands, the op in half, encode).  All three
// tensors share one element type (binary.cpp:301-303).
#include "common.h"

namespace lcml::onnx {
namespace {

using namespace ops;

class BinaryOp : public StreamOperator {
    int op_;

public:
    BinaryOp(const char *name, int op) : StreamOperator(name), op_(op) {}
    bool can_operate_inplace() const override { return true; }
    void forward(std::span<std::reference_wrapper<ITensor>> inputs,
                 std::span<std::reference_wrapper<ITensor>> outputs) override {
        LCML_ASSERT(inputs.size() == 2 && outputs.size() == 1, "Binary operator requires 2 inputs and 1 output.");
        ITensor &a = inputs[0], &b = inputs[1], &y = outputs[0];
        LCML_ASSERT(a.element_type_index() == b.element_type_index() &&
                        a.element_type_index() == y.element_type_index(),
                    "Binary op: all tensors must have the same element type.");
        const int dt = fp8_path_dtype(a);
        LCML_ASSERT(dt != 0, "Binary op: FLOAT, FLOAT8E4M3FN or FLOAT8E5M2 tensors only");
        std::vector<int64_t> sa, sb, sy;
        for (size_t i = 0; i < a.ndim(); ++i) sa.push_back(a.shape(i));
        for (size_t i = 0; i < b.ndim(); ++i) sb.push_back(b.shape(i));
        for (size_t i = 0; i < y.ndim(); ++i) sy.push_back(y.shape(i));
        // the C ABI checks that y's shape is the broadcast of a's and b's
        check(lcml_fp8_binary(op_, dt, a.device_data(), sa.data(), (int)sa.size(), b.device_data(), sb.data(),
                              (int)sb.size(), y.device_data(), sy.data(), (int)sy.size(), stream_),
              get_name().c_str());
    }
};

}  // namespace

REGISTER_TO_DEFAULT_OPSET(Add) { return std::make_unique<BinaryOp>("Add", LCML_BINARY_ADD); };
REGISTER_TO_DEFAULT_OPSET(Sub) { return std::make_unique<BinaryOp>("Sub", LCML_BINARY_SUB); };
REGISTER_TO_DEFAULT_OPSET(Mul) { return std::make_unique<BinaryOp>("Mul", LCML_BINARY_MUL); };
REGISTER_TO_DEFAULT_OPSET(Div) { return std::make_unique<BinaryOp>("Div", LCML_BINARY_DIV); };

}  // namespace lcml::onnx
