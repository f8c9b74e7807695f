// QuantizeLinear / DequantizeLinear / DynamicQuantizeLinear / Cast for
// FLOAT <-> FLOAT8E4M3FN.  The reference registers none of the first three
// (its loader rejects them, src/onnx/onnx.cpp:228-229); its only fp8
// conversion is Cast (src/onnx/operators/cast.cpp:39-77, attrs 149-162),
// whose fp32->fp8 branch goes through half precision.  Here every
// float->E4M3 conversion is the exact FP8E4M3FN::from_float
// (include/onnx/fp_quantized.h:149-223) and every E4M3->float the exact
// to_float (226-249), on the GPU, bit for bit.
#include "common.h"

namespace lcml::onnx {
namespace {

using namespace ops;

class QuantizeLinear : public StreamOperator {
    int axis_;

public:
    QuantizeLinear(int axis, int saturate) : StreamOperator("QuantizeLinear"), axis_(axis) {
        LCML_ASSERT(saturate == 1, "QuantizeLinear: saturate=0 is not supported for FLOAT8E4M3FN");
    }
    void forward(std::span<std::reference_wrapper<ITensor>> inputs,
                 std::span<std::reference_wrapper<ITensor>> outputs) override {
        LCML_ASSERT(inputs.size() >= 2 && outputs.size() == 1, "QuantizeLinear requires 2-3 inputs and 1 output.");
        ITensor &x = inputs[0], &s = inputs[1], &y = outputs[0];
        LCML_ASSERT(is_type<float>(x) && is_type<float>(s), "QuantizeLinear: x and y_scale must be float");
        LCML_ASSERT(is_type<FP8E4M3FN>(y), "QuantizeLinear: only FLOAT8E4M3FN outputs are supported");
        LCML_ASSERT(x.size() == y.size(), "QuantizeLinear: x and y sizes differ");
        check_zero_point(inputs, 2, "QuantizeLinear");
        AxisView v = axis_view(x, axis_, s.size());
        check(lcml_fp8_quantize(static_cast<const float *>(x.device_data()), static_cast<uint8_t *>(y.device_data()),
                                v.outer, v.axis_len, v.inner, static_cast<const float *>(s.device_data()), stream_),
              "QuantizeLinear");
    }
};

class DequantizeLinear : public StreamOperator {
    int axis_;

public:
    explicit DequantizeLinear(int axis) : StreamOperator("DequantizeLinear"), axis_(axis) {}
    void forward(std::span<std::reference_wrapper<ITensor>> inputs,
                 std::span<std::reference_wrapper<ITensor>> outputs) override {
        LCML_ASSERT(inputs.size() >= 2 && outputs.size() == 1, "DequantizeLinear requires 2-3 inputs and 1 output.");
        ITensor &x = inputs[0], &s = inputs[1], &y = outputs[0];
        LCML_ASSERT(is_type<FP8E4M3FN>(x), "DequantizeLinear: only FLOAT8E4M3FN inputs are supported");
        LCML_ASSERT(is_type<float>(s) && is_type<float>(y), "DequantizeLinear: x_scale and y must be float");
        LCML_ASSERT(x.size() == y.size(), "DequantizeLinear: x and y sizes differ");
        check_zero_point(inputs, 2, "DequantizeLinear");
        AxisView v = axis_view(x, axis_, s.size());
        check(lcml_fp8_dequantize(static_cast<const uint8_t *>(x.device_data()), static_cast<float *>(y.device_data()),
                                  v.outer, v.axis_len, v.inner, static_cast<const float *>(s.device_data()), stream_),
              "DequantizeLinear");
    }
};

// DynamicQuantizeLinear with a FLOAT8E4M3FN output: y_scale = amax/448
// (1 when that is not a positive finite number), y_zero_point = 0.
class DynamicQuantizeLinear : public StreamOperator {
    std::unique_ptr<DeviceBuffer> ws_;

public:
    DynamicQuantizeLinear() : StreamOperator("DynamicQuantizeLinear") {}
    void forward(std::span<std::reference_wrapper<ITensor>> inputs,
                 std::span<std::reference_wrapper<ITensor>> outputs) override {
        LCML_ASSERT(inputs.size() == 1 && outputs.size() >= 2, "DynamicQuantizeLinear requires 1 input, 2-3 outputs.");
        ITensor &x = inputs[0], &y = outputs[0], &s = outputs[1];
        LCML_ASSERT(is_type<float>(x) && is_type<float>(s), "DynamicQuantizeLinear: x and y_scale must be float");
        LCML_ASSERT(is_type<FP8E4M3FN>(y), "DynamicQuantizeLinear: only FLOAT8E4M3FN outputs are supported");
        if (!ws_) ws_ = std::make_unique<DeviceBuffer>(LCML_FP8_DYNAMIC_WORKSPACE_BYTES);
        check(lcml_fp8_quantize_dynamic(static_cast<const float *>(x.device_data()),
                                        static_cast<uint8_t *>(y.device_data()), x.size(),
                                        static_cast<float *>(s.device_data()), ws_->data(), stream_),
              "DynamicQuantizeLinear");
        if (outputs.size() > 2) {
            ITensor &zp = outputs[2];
            LCML_ASSERT(hipMemsetAsync(zp.device_data(), 0, zp.size(), stream_) == hipSuccess,
                        "DynamicQuantizeLinear: zero point");
        }
    }
};

// Cast between FLOAT and FLOAT8E4M3FN: an exact encode / decode with scale 1.
class Cast : public StreamOperator {
    std::unique_ptr<DeviceBuffer> one_;

public:
    Cast(DataType to, int saturate) : StreamOperator("Cast") {
        LCML_ASSERT(to == DataType::FLOAT || to == DataType::FLOAT8E4M3FN,
                    "Cast: only FLOAT <-> FLOAT8E4M3FN is on the FP8 path");
        LCML_ASSERT(saturate == 1 || to != DataType::FLOAT8E4M3FN, "Cast: saturate=0 is not supported");
    }
    void forward(std::span<std::reference_wrapper<ITensor>> inputs,
                 std::span<std::reference_wrapper<ITensor>> outputs) override {
        ITensor &x = inputs[0], &y = outputs[0];
        LCML_ASSERT(x.size() == y.size(), "Cast: sizes differ");
        if (!one_) {
            one_ = std::make_unique<DeviceBuffer>(sizeof(float));
            const float v = 1.0f;
            LCML_ASSERT(hipMemcpy(one_->data(), &v, sizeof v, hipMemcpyHostToDevice) == hipSuccess, "Cast");
        }
        const float *one = static_cast<const float *>(one_->data());
        if (is_type<float>(x) && is_type<FP8E4M3FN>(y))
            check(lcml_fp8_quantize(static_cast<const float *>(x.device_data()), static_cast<uint8_t *>(y.device_data()),
                                    1, 1, x.size(), one, stream_), "Cast");
        else if (is_type<FP8E4M3FN>(x) && is_type<float>(y))
            check(lcml_fp8_dequantize(static_cast<const uint8_t *>(x.device_data()), static_cast<float *>(y.device_data()),
                                      1, 1, x.size(), one, stream_), "Cast");
        else
            LCML_ASSERT(false, "Cast: unsupported element types");
    }
};

}  // namespace

REGISTER_TO_DEFAULT_OPSET(QuantizeLinear) {
    return std::make_unique<QuantizeLinear>(attr_int(node, "axis", 1), attr_int(node, "saturate", 1));
};
REGISTER_TO_DEFAULT_OPSET(DequantizeLinear) { return std::make_unique<DequantizeLinear>(attr_int(node, "axis", 1)); };
REGISTER_TO_DEFAULT_OPSET(DynamicQuantizeLinear) { return std::make_unique<DynamicQuantizeLinear>(); };
REGISTER_TO_DEFAULT_OPSET(Cast) {
    return std::make_unique<Cast>((DataType)attr_int(node, "to", 1), attr_int(node, "saturate", 1));
};

}  // namespace lcml::onnx
