// QuantizeLinear / DequantizeLinear / DynamicQuantizeLinear / Cast for
// FLOAT <-> FLOAT8E4M3FN / FLOAT8E5M2.  The reference registers none of the
// first three (its loader rejects them, src/onnx/onnx.cpp:228-229); its only
// fp8 conversion is Cast (src/onnx/operators/cast.cpp:39-77, attrs 149-162),
// whose fp32->fp8 branch goes through half precision.  Here every
// float->fp8 conversion is the exact FP8E4M3FN / FP8E5M2 from_float
// (include/onnx/fp_quantized.h:149-223, 272-346) and every fp8->float the
// exact to_float (226-249, 350-377), on the GPU, bit for bit.
#include "common.h"

namespace lcml::onnx {
namespace {

using namespace ops;

class QuantizeLinear : public StreamOperator {
    int axis_, saturate_;

public:
    QuantizeLinear(int axis, int saturate) : StreamOperator("QuantizeLinear"), axis_(axis), saturate_(saturate) {
        LCML_ASSERT(saturate == 0 || saturate == 1, "QuantizeLinear: saturate must be 0 or 1");
    }
    void forward(std::span<std::reference_wrapper<ITensor>> inputs,
                 std::span<std::reference_wrapper<ITensor>> outputs) override {
        LCML_ASSERT(inputs.size() >= 2 && outputs.size() == 1, "QuantizeLinear requires 2-3 inputs and 1 output.");
        ITensor &x = inputs[0], &s = inputs[1], &y = outputs[0];
        LCML_ASSERT(is_type<float>(x) && is_type<float>(s), "QuantizeLinear: x and y_scale must be float");
        LCML_ASSERT(x.size() == y.size(), "QuantizeLinear: x and y sizes differ");
        check_zero_point(inputs, 2, y, "QuantizeLinear");
        AxisView v = axis_view(x, axis_, s.size());
        const float *xp = static_cast<const float *>(x.device_data()), *sp = static_cast<const float *>(s.device_data());
        uint8_t *yp = static_cast<uint8_t *>(y.device_data());
        if (is_type<FP8E4M3FN>(y)) {
            // FP8E4M3FN::from_float saturates to +-448 by itself; ONNX's
            // saturate=0 (overflow to NaN) has no counterpart in that encoder
            LCML_ASSERT(saturate_ == 1, "QuantizeLinear: saturate=0 is not supported for FLOAT8E4M3FN");
            check(lcml_fp8_quantize(xp, yp, v.outer, v.axis_len, v.inner, sp, stream_), "QuantizeLinear");
        } else {
            LCML_ASSERT(is_type<FP8E5M2>(y), "QuantizeLinear: FLOAT8E4M3FN or FLOAT8E5M2 outputs only");
            check(lcml_fp8_quantize_e5m2(xp, yp, v.outer, v.axis_len, v.inner, sp, saturate_, stream_),
                  "QuantizeLinear");
        }
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
        LCML_ASSERT(is_type<float>(s) && is_type<float>(y), "DequantizeLinear: x_scale and y must be float");
        LCML_ASSERT(x.size() == y.size(), "DequantizeLinear: x and y sizes differ");
        check_zero_point(inputs, 2, x, "DequantizeLinear");
        AxisView v = axis_view(x, axis_, s.size());
        const uint8_t *xp = static_cast<const uint8_t *>(x.device_data());
        const float *sp = static_cast<const float *>(s.device_data());
        float *yp = static_cast<float *>(y.device_data());
        if (is_type<FP8E4M3FN>(x)) {
            check(lcml_fp8_dequantize(xp, yp, v.outer, v.axis_len, v.inner, sp, stream_), "DequantizeLinear");
        } else {
            LCML_ASSERT(is_type<FP8E5M2>(x), "DequantizeLinear: FLOAT8E4M3FN or FLOAT8E5M2 inputs only");
            check(lcml_fp8_dequantize_e5m2(xp, yp, v.outer, v.axis_len, v.inner, sp, stream_), "DequantizeLinear");
        }
    }
};

// DynamicQuantizeLinear with a FLOAT8E4M3FN output: y_scale = amax/448
// (1 when that is not a positive finite number), y_zero_point = 0.
class DynamicQuantizeLinear : public StreamOperator {
    std::unique_ptr<DeviceBuffer> ws_, zero_;

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
            // y_zero_point = 0, written by a kernel (Cast of fp32 zeros) so
            // that steady-state forwards launch kernels only
            ITensor &zp = outputs[2];
            LCML_ASSERT(is_type<FP8E4M3FN>(zp), "DynamicQuantizeLinear: zero point must be FLOAT8E4M3FN");
            if (!zero_ || zero_->bytes() < zp.size() * sizeof(float)) {
                zero_ = std::make_unique<DeviceBuffer>(zp.size() * sizeof(float));
                const hipError_t e = hipMemset(zero_->data(), 0, zero_->bytes());
                LCML_ASSERT(e == hipSuccess, "DynamicQuantizeLinear: hipMemset: %s", hipGetErrorString(e));
            }
            check(lcml_fp8_cast(zero_->data(), LCML_DTYPE_FLOAT, zp.device_data(), LCML_DTYPE_FLOAT8E4M3FN,
                                zp.size(), stream_),
                  "DynamicQuantizeLinear");
        }
    }
};

// Cast between FLOAT, FLOAT8E4M3FN and FLOAT8E5M2 with the CPU codecs; as in
// the reference, `saturate` only concerns float -> int casts (cast.cpp:86-98)
// and is not consulted for fp8.
class Cast : public StreamOperator {
public:
    Cast(DataType to, int) : StreamOperator("Cast") {
        LCML_ASSERT(to == DataType::FLOAT || to == DataType::FLOAT8E4M3FN || to == DataType::FLOAT8E5M2,
                    "Cast: only FLOAT, FLOAT8E4M3FN and FLOAT8E5M2 are on the FP8 path");
    }
    void forward(std::span<std::reference_wrapper<ITensor>> inputs,
                 std::span<std::reference_wrapper<ITensor>> outputs) override {
        ITensor &x = inputs[0], &y = outputs[0];
        LCML_ASSERT(x.size() == y.size(), "Cast: sizes differ");
        const int xt = fp8_path_dtype(x), yt = fp8_path_dtype(y);
        LCML_ASSERT(xt && yt, "Cast: unsupported element types");
        if (x.device_data() == y.device_data() && xt == yt) return;  // same storage, same type
        check(lcml_fp8_cast(x.device_data(), xt, y.device_data(), yt, x.size(), stream_), "Cast");
    }
};

}  // namespace

// opset 21's blocked quantisation (block_size > 0) is outside this path:
// per-tensor and per-axis scales only
REGISTER_TO_DEFAULT_OPSET(QuantizeLinear) {
    LCML_ASSERT(attr_int(node, "block_size", 0) == 0, "QuantizeLinear: blocked quantisation is not supported");
    return std::make_unique<QuantizeLinear>(attr_int(node, "axis", 1), attr_int(node, "saturate", 1));
};
REGISTER_TO_DEFAULT_OPSET(DequantizeLinear) {
    LCML_ASSERT(attr_int(node, "block_size", 0) == 0, "DequantizeLinear: blocked quantisation is not supported");
    return std::make_unique<DequantizeLinear>(attr_int(node, "axis", 1));
};
REGISTER_TO_DEFAULT_OPSET(DynamicQuantizeLinear) { return std::make_unique<DynamicQuantizeLinear>(); };
REGISTER_TO_DEFAULT_OPSET(Cast) {
    return std::make_unique<Cast>((DataType)attr_int(node, "to", 1), attr_int(node, "saturate", 1));
};

}  // namespace lcml::onnx
