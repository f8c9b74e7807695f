// common.h -- helpers shared by the operator implementations.
#pragma once

#include <hip/hip_runtime.h>

#include "lcml_fp8.h"
#include "onnx/network_instance.h"
#include "onnx/onnx.h"

namespace lcml::onnx::ops {

inline void check(int rc, const char *op) { LCML_ASSERT(rc == 0, "%s: %s", op, lcml_fp8_last_error()); }

template <typename T>
inline bool is_type(const ITensor &t) {
    return t.element_type_index() == refl::type_index_of<T>();
}

// Base for operators that launch on the executing network's stream.
class StreamOperator : public Operator {
protected:
    hipStream_t stream_ = nullptr;

public:
    using Operator::Operator;
    void set_environment(NetworkInstance &env, TensorTable &) override { stream_ = env.stream(); }
};

// [outer, axis_len, inner] view of a tensor for a per-axis scale of
// `nscale` entries (nscale == 1: per tensor).
struct AxisView {
    int64_t outer, axis_len, inner;
};
inline AxisView axis_view(const ITensor &t, int axis, size_t nscale) {
    int64_t n = t.size();
    if (nscale == 1) return {1, 1, n};
    int nd = (int)t.ndim();
    if (axis < 0) axis += nd;
    LCML_ASSERT(axis >= 0 && axis < nd, "axis %d out of range for rank %d", axis, nd);
    LCML_ASSERT(t.shape(axis) == nscale, "per-axis scale has %zu entries, dimension %d has %u", nscale, axis,
                t.shape(axis));
    int64_t outer = 1, inner = 1;
    for (int i = 0; i < axis; ++i) outer *= t.shape(i);
    for (int i = axis + 1; i < nd; ++i) inner *= t.shape(i);
    return {outer, (int64_t)t.shape(axis), inner};
}

// The optional zero-point input of Q/DQ: ONNX requires 0 for float8 types.
// A constant zero point is verified; a runtime one (DynamicQuantizeLinear's
// output) is zero by that operator's definition.
// The zero point's type is the quantised type (ONNX): it must match `q`.
inline void check_zero_point(std::span<std::reference_wrapper<ITensor>> inputs, size_t idx, const ITensor &q,
                             const char *op) {
    if (inputs.size() <= idx) return;
    ITensor &zp = inputs[idx];
    LCML_ASSERT(zp.element_type_index() == q.element_type_index(), "%s: the zero point type must be the fp8 type",
                op);
    const std::vector<uint8_t> *bytes = nullptr;
    if (auto *c = dynamic_cast<ConstTensor<FP8E4M3FN> *>(&zp)) bytes = &c->const_data();
    if (auto *c = dynamic_cast<ConstTensor<FP8E5M2> *>(&zp)) bytes = &c->const_data();
    if (bytes)
        for (uint8_t b : *bytes) LCML_ASSERT(b == 0, "%s: float8 zero point must be 0", op);
}

// ONNX element type of a float / fp8 tensor for the C ABI (0 if neither)
inline int fp8_path_dtype(const ITensor &t) {
    if (is_type<float>(t)) return LCML_DTYPE_FLOAT;
    if (is_type<FP8E4M3FN>(t)) return LCML_DTYPE_FLOAT8E4M3FN;
    if (is_type<FP8E5M2>(t)) return LCML_DTYPE_FLOAT8E5M2;
    return 0;
}

inline int out_dtype_code(const ITensor &y, const char *op) {
    if (is_type<float>(y)) return LCML_DTYPE_FLOAT;
    if (is_type<BFloat16>(y)) return LCML_DTYPE_BFLOAT16;
    LCML_ASSERT(false, "%s: output element type %.*s (float or bfloat16 supported)", op,
                (int)y.element_type_name().size(), y.element_type_name().data());
    return 0;
}

// Gemm C broadcast description for the C ABI.
struct CArgs {
    const float *ptr = nullptr;
    int ndim = 0;
    int64_t d0 = 0, d1 = 0;
};
inline CArgs c_args(ITensor *c) {
    CArgs a;
    if (!c) return a;
    LCML_ASSERT(is_type<float>(*c), "Gemm: C must be float");
    a.ptr = static_cast<const float *>(c->device_data());
    a.ndim = (int)c->ndim();
    a.d0 = c->ndim() >= 1 ? c->shape(0) : 0;
    a.d1 = c->ndim() >= 2 ? c->shape(1) : 0;
    return a;
}

}  // namespace lcml::onnx::ops
