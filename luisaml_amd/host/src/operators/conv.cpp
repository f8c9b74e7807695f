// conv.cpp -- the ONNX Conv operator (2-D, NCHW) and its fused FP8 form.
//
// Conv follows the reference's Conv::apply (src/onnx/operators/conv.cpp:
// 115-207): attributes kernel_shape, strides, pads, dilations, group,
// auto_pad = NOTSET; only the begin pads enter the index arithmetic
// (conv.cpp:121) and the output size comes from the output tensor.
// FP8Conv is built by NetworkInstance's fusion pass from
// [x -> (Dynamic)QuantizeLinear -> DequantizeLinear] and
// DequantizeLinear(W_e4m3 constant, per-tensor or per-output-channel scale)
// into Conv [-> Relu/Gelu]: the activation is quantised straight into NHWC
// E4M3 and the convolution runs as an implicit-im2col GEMM on the matrix
// cores with the packed weight.
#include "common.h"

namespace lcml::onnx {
namespace {

using namespace ops;

struct ConvAttrs {
    int64_t kh, kw, sh, sw, ph, pw, dh, dw, group;
};

ConvAttrs conv_attrs(const Node &node, const char *op) {
    LCML_ASSERT(attr_string(node, "auto_pad", "NOTSET") == "NOTSET", "%s: only auto_pad=NOTSET is supported", op);
    auto ks = attr_ints(node, "kernel_shape", {});
    auto st = attr_ints(node, "strides", {1, 1});
    auto pd = attr_ints(node, "pads", {0, 0, 0, 0});
    auto dl = attr_ints(node, "dilations", {1, 1});
    LCML_ASSERT(st.size() == 2 && dl.size() == 2 && (pd.size() == 4 || pd.size() == 2),
                "%s: only 2-D convolution is supported", op);
    ConvAttrs a;
    a.kh = ks.size() == 2 ? ks[0] : 0;
    a.kw = ks.size() == 2 ? ks[1] : 0;
    a.sh = st[0]; a.sw = st[1];
    a.ph = pd[0]; a.pw = pd[1];
    a.dh = dl[0]; a.dw = dl[1];
    a.group = attr_int(node, "group", 1);
    return a;
}

// Conv(X [n,c,h,w], W [cout, c/group, kh, kw] [, B]) -> Y, all of one element
// type: float, or an fp8 type (FLOAT8E4M3FN / FLOAT8E5M2) as the reference
// also accepts (conv.cpp:65-70, 84-105: fp8 operands decoded, the result
// encoded back).  The fp8 form decodes X, W and B exactly to fp32, runs the
// fp32 convolution and encodes Y with the reference's CPU encoder; the
// reference accumulates fp8 convolutions in half precision and encodes with
// its half-precision device codec, so results can differ from it by the
// rounding of those half steps (the fp32 sum is the more accurate one).
class Conv : public StreamOperator {
    ConvAttrs a_;
    std::unique_ptr<DeviceBuffer> f32_;  // fp8 form: fp32 copies of X, W, B and Y
    size_t f32_bytes_ = 0;

public:
    explicit Conv(ConvAttrs a) : StreamOperator("Conv"), a_(a) {}
    void forward(std::span<std::reference_wrapper<ITensor>> inputs,
                 std::span<std::reference_wrapper<ITensor>> outputs) override {
        ITensor &X = inputs[0], &Wt = inputs[1], &Y = outputs[0];
        ITensor *B = inputs.size() > 2 ? &inputs[2].get() : nullptr;
        const int dt = fp8_path_dtype(X);
        LCML_ASSERT(dt != 0 && fp8_path_dtype(Wt) == dt && fp8_path_dtype(Y) == dt && (!B || fp8_path_dtype(*B) == dt),
                    "Conv: X, W, B and Y must all be float, FLOAT8E4M3FN or FLOAT8E5M2");
        LCML_ASSERT(X.ndim() == 4 && Wt.ndim() == 4 && Y.ndim() == 4, "Conv: only 2-D (NCHW) convolution");
        const int64_t kh = a_.kh ? a_.kh : Wt.shape(2), kw = a_.kw ? a_.kw : Wt.shape(3);
        LCML_ASSERT(Wt.shape(2) == kh && Wt.shape(3) == kw, "Conv: kernel_shape does not match W");
        const float *x = static_cast<const float *>(X.device_data());
        const float *w = static_cast<const float *>(Wt.device_data());
        const float *bias = B ? static_cast<const float *>(B->device_data()) : nullptr;
        float *y = static_cast<float *>(Y.device_data());
        if (dt != LCML_DTYPE_FLOAT) {
            const size_t nx = X.size(), nw = Wt.size(), nb = B ? B->size() : 0, ny = Y.size();
            const size_t need = (nx + nw + nb + ny) * sizeof(float);
            if (!f32_ || f32_bytes_ < need) {
                f32_ = std::make_unique<DeviceBuffer>(need);
                f32_bytes_ = need;
            }
            float *fx = static_cast<float *>(f32_->data()), *fw = fx + nx, *fb = fw + nw, *fy = fb + nb;
            check(lcml_fp8_cast(X.device_data(), dt, fx, LCML_DTYPE_FLOAT, (int64_t)nx, stream_), "Conv");
            check(lcml_fp8_cast(Wt.device_data(), dt, fw, LCML_DTYPE_FLOAT, (int64_t)nw, stream_), "Conv");
            if (B) check(lcml_fp8_cast(B->device_data(), dt, fb, LCML_DTYPE_FLOAT, (int64_t)nb, stream_), "Conv");
            x = fx;
            w = fw;
            bias = B ? fb : nullptr;
            y = fy;
        }
        check(lcml_fp8_conv2d_f32(x, w, bias, y, X.shape(0), X.shape(1), X.shape(2), X.shape(3), Wt.shape(0), kh, kw,
                                  a_.sh, a_.sw, a_.ph, a_.pw, a_.dh, a_.dw, a_.group, Y.shape(2), Y.shape(3),
                                  LCML_ACT_NONE, stream_),
              "Conv");
        if (dt != LCML_DTYPE_FLOAT)
            check(lcml_fp8_cast(y, LCML_DTYPE_FLOAT, Y.device_data(), dt, (int64_t)Y.size(), stream_), "Conv");
    }
};

// inputs: [X fp32, W packed, w_scale, (x_scale if a_mode == 1), (B if has_bias)]
// a_mode 1: static per-tensor activation scale; 2: dynamic (amax/448).
class FP8Conv : public StreamOperator {
    ConvAttrs a_;
    int a_mode_, has_bias_, act_;
    std::unique_ptr<DeviceBuffer> xq_, sx_, ws_;
    size_t xq_bytes_ = 0;

public:
    FP8Conv(ConvAttrs a, int a_mode, int has_bias, int act)
        : StreamOperator("FP8Conv"), a_(a), a_mode_(a_mode), has_bias_(has_bias), act_(act) {}
    void forward(std::span<std::reference_wrapper<ITensor>> inputs,
                 std::span<std::reference_wrapper<ITensor>> outputs) override {
        ITensor &X = inputs[0], &Y = outputs[0];
        auto *W = dynamic_cast<PackedWeightTensor *>(&inputs[1].get());
        LCML_ASSERT(W != nullptr, "FP8Conv: input 1 must be a packed weight");
        LCML_ASSERT(is_type<float>(X) && X.ndim() == 4 && Y.ndim() == 4, "FP8Conv: NCHW float input expected");
        size_t next = 3;
        ITensor *x_scale = a_mode_ == 1 ? &inputs[next++].get() : nullptr;
        const float *bias = has_bias_ ? static_cast<const float *>(inputs[next++].get().device_data()) : nullptr;
        const int64_t n = X.shape(0), c = X.shape(1), h = X.shape(2), w = X.shape(3);
        const size_t need = (size_t)(n * c * h * w);
        if (!xq_ || xq_bytes_ < need) {
            xq_ = std::make_unique<DeviceBuffer>(need);
            xq_bytes_ = need;
        }
        const float *x = static_cast<const float *>(X.device_data());
        uint8_t *xq = static_cast<uint8_t *>(xq_->data());
        const float *sx;
        if (a_mode_ == 1) {
            sx = static_cast<const float *>(x_scale->device_data());
            check(lcml_fp8_quantize_nhwc(x, xq, n, c, h, w, sx, nullptr, nullptr, stream_), "FP8Conv quantize");
        } else {
            if (!sx_) sx_ = std::make_unique<DeviceBuffer>(sizeof(float));
            if (!ws_) ws_ = std::make_unique<DeviceBuffer>(LCML_FP8_DYNAMIC_WORKSPACE_BYTES);
            check(lcml_fp8_quantize_nhwc(x, xq, n, c, h, w, nullptr, static_cast<float *>(sx_->data()), ws_->data(),
                                         stream_),
                  "FP8Conv quantize");
            sx = static_cast<const float *>(sx_->data());
        }
        check(lcml_fp8_conv2d(xq, sx, n, c, h, w, W->packed(), W->scale(), W->per_channel(), Y.shape(1), a_.kh, a_.kw,
                              a_.sh, a_.sw, a_.ph, a_.pw, a_.dh, a_.dw, a_.group, Y.shape(2), Y.shape(3), bias, act_,
                              Y.device_data(), out_dtype_code(Y, "FP8Conv"), LCML_KERNEL_AUTO, stream_),
              "FP8Conv");
    }
};

}  // namespace

REGISTER_TO_DEFAULT_OPSET(Conv) { return std::make_unique<Conv>(conv_attrs(node, "Conv")); };
REGISTER_TO_DEFAULT_OPSET(FP8Conv) {
    return std::make_unique<FP8Conv>(conv_attrs(node, "FP8Conv"), attr_int(node, "a_mode", 2),
                                     attr_int(node, "has_bias", 0), attr_int(node, "act", 0));
};

}  // namespace lcml::onnx
