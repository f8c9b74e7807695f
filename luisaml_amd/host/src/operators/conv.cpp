// conv.cpp -- the ONNX Conv operator (2-D, NCHW) and its fused FP8 form.
//
// Conv follows the reference's Conv::forward (src/onnx/operators/conv.cpp:
// 35-250): 1-D and 2-D; attributes kernel_shape, strides, pads, dilations,
// group (auto_pad is read and ignored, as there); only the begin pads enter
// the index arithmetic (conv.cpp:121, 213) and the output size comes from
// the output tensor.
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

// Attributes as written (kernel_shape, strides, pads, dilations, group;
// auto_pad is parsed and, as in the reference, not used: conv.cpp:257-275),
// resolved against the input rank at run time as the reference's
// Conv::forward does (conv.cpp:48-58): defaults 1 / 0, begin pads only.
// A 1-D convolution (X [n, c, l], W [cout, c/group, kl], conv.cpp:209-250)
// runs as the 2-D one over [n, c, 1, l] with a 1 x kl kernel: the same
// bytes, the same output positions and the same (tap, channel) order.
struct ConvAttrs {
    std::vector<int32_t> ks, st, pd, dl;
    int64_t group;
};

struct ConvGeom2D {
    int64_t kh, kw, sh, sw, ph, pw, dh, dw;
};

ConvAttrs conv_attrs(const Node &node) {
    return ConvAttrs{attr_ints(node, "kernel_shape", {}), attr_ints(node, "strides", {}), attr_ints(node, "pads", {}),
                     attr_ints(node, "dilations", {}), attr_int(node, "group", 1)};
}

// spatial = 1 or 2; wk = the weight's kernel extent(s) (kh, kw; kh = 1 for 1-D)
ConvGeom2D resolve(const ConvAttrs &a, int spatial, int64_t wkh, int64_t wkw, const char *op) {
    LCML_ASSERT(spatial == 1 || spatial == 2, "%s: only 1D and 2D convolution are supported.", op);
    auto pick = [&](const std::vector<int32_t> &v, size_t i, int64_t dflt) { return v.empty() ? dflt : (int64_t)v[i]; };
    const size_t S = (size_t)spatial;
    LCML_ASSERT((a.st.empty() || a.st.size() == S) && (a.dl.empty() || a.dl.size() == S) &&
                    (a.pd.empty() || a.pd.size() == 2 * S || a.pd.size() == S) && (a.ks.empty() || a.ks.size() == S),
                "%s: attribute lengths do not match %d spatial dimension(s)", op, spatial);
    ConvGeom2D g;
    if (spatial == 2) {
        g = {pick(a.ks, 0, wkh), pick(a.ks, 1, wkw), pick(a.st, 0, 1), pick(a.st, 1, 1),
             pick(a.pd, 0, 0), pick(a.pd, 1, 0), pick(a.dl, 0, 1), pick(a.dl, 1, 1)};
    } else {
        g = {1, pick(a.ks, 0, wkw), 1, pick(a.st, 0, 1), 0, pick(a.pd, 0, 0), 1, pick(a.dl, 0, 1)};
    }
    LCML_ASSERT(g.kh == wkh && g.kw == wkw, "%s: kernel_shape does not match W", op);
    return g;
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
    ConvAttrs attrs_;
    std::unique_ptr<DeviceBuffer> f32_;  // fp8 form: fp32 copies of X, W, B and Y
    size_t f32_bytes_ = 0;

public:
    explicit Conv(ConvAttrs a) : StreamOperator("Conv"), attrs_(std::move(a)) {}
    void forward(std::span<std::reference_wrapper<ITensor>> inputs,
                 std::span<std::reference_wrapper<ITensor>> outputs) override {
        ITensor &X = inputs[0], &Wt = inputs[1], &Y = outputs[0];
        ITensor *B = inputs.size() > 2 ? &inputs[2].get() : nullptr;
        const int dt = fp8_path_dtype(X);
        LCML_ASSERT(dt != 0 && fp8_path_dtype(Wt) == dt && fp8_path_dtype(Y) == dt && (!B || fp8_path_dtype(*B) == dt),
                    "Conv: X, W, B and Y must all be float, FLOAT8E4M3FN or FLOAT8E5M2");
        const int spatial = (int)X.ndim() - 2;
        LCML_ASSERT(Wt.ndim() == X.ndim() && Y.ndim() == X.ndim(), "Conv: X, W and Y ranks differ");
        const bool one_d = spatial == 1;
        const ConvGeom2D a_ = resolve(attrs_, spatial, one_d ? 1 : Wt.shape(2), Wt.shape(one_d ? 2 : 3), "Conv");
        const int64_t kh = a_.kh, kw = a_.kw;
        // [n, c, h, w] of the 2-D view
        const int64_t xh = one_d ? 1 : X.shape(2), xw = X.shape(one_d ? 2 : 3);
        const int64_t yh = one_d ? 1 : Y.shape(2), yw = Y.shape(one_d ? 2 : 3);
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
        check(lcml_fp8_conv2d_f32(x, w, bias, y, X.shape(0), X.shape(1), xh, xw, Wt.shape(0), kh, kw, a_.sh, a_.sw,
                                  a_.ph, a_.pw, a_.dh, a_.dw, attrs_.group, yh, yw, LCML_ACT_NONE, stream_),
              "Conv");
        if (dt != LCML_DTYPE_FLOAT)
            check(lcml_fp8_cast(y, LCML_DTYPE_FLOAT, Y.device_data(), dt, (int64_t)Y.size(), stream_), "Conv");
    }
};

// inputs: [X fp32, W packed, w_scale, (x_scale if a_mode == 1), (B if has_bias)]
// a_mode 1: static per-tensor activation scale; 2: dynamic (amax/448).
class FP8Conv : public StreamOperator {
    ConvAttrs attrs_;
    int a_mode_, has_bias_, act_;
    int kernel_;  // LCML_KERNEL_AUTO, or AUTO_FP8 (NetworkInstance::set_fp8_matrix_cores)
    std::unique_ptr<DeviceBuffer> xq_, sx_, ws_;
    size_t xq_bytes_ = 0;

public:
    FP8Conv(ConvAttrs a, int a_mode, int has_bias, int act, int kernel)
        : StreamOperator("FP8Conv"), attrs_(std::move(a)), a_mode_(a_mode), has_bias_(has_bias), act_(act),
          kernel_(kernel) {}
    void forward(std::span<std::reference_wrapper<ITensor>> inputs,
                 std::span<std::reference_wrapper<ITensor>> outputs) override {
        ITensor &X = inputs[0], &Y = outputs[0];
        auto *W = dynamic_cast<PackedWeightTensor *>(&inputs[1].get());
        LCML_ASSERT(W != nullptr, "FP8Conv: input 1 must be a packed weight");
        LCML_ASSERT(is_type<float>(X) && (X.ndim() == 4 || X.ndim() == 3) && Y.ndim() == X.ndim(),
                    "FP8Conv: NCHW / NCL float input expected");
        size_t next = 3;
        ITensor *x_scale = a_mode_ == 1 ? &inputs[next++].get() : nullptr;
        const float *bias = has_bias_ ? static_cast<const float *>(inputs[next++].get().device_data()) : nullptr;
        const bool one_d = X.ndim() == 3;
        // kernel_shape is set by the fusion pass from the weight: (kh, kw), or (kl) for 1-D
        const ConvGeom2D a_ = resolve(attrs_, one_d ? 1 : 2, one_d ? 1 : attrs_.ks.at(0), attrs_.ks.back(), "FP8Conv");
        const int64_t n = X.shape(0), c = X.shape(1), h = one_d ? 1 : X.shape(2), w = X.shape(one_d ? 2 : 3);
        const int64_t oh = one_d ? 1 : Y.shape(2), ow = Y.shape(one_d ? 2 : 3);
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
                              a_.sh, a_.sw, a_.ph, a_.pw, a_.dh, a_.dw, attrs_.group, oh, ow, bias, act_,
                              Y.device_data(), out_dtype_code(Y, "FP8Conv"), kernel_, stream_),
              "FP8Conv");
    }
};

}  // namespace

REGISTER_TO_DEFAULT_OPSET(Conv) { return std::make_unique<Conv>(conv_attrs(node)); };
REGISTER_TO_DEFAULT_OPSET(FP8Conv) {
    return std::make_unique<FP8Conv>(conv_attrs(node), attr_int(node, "a_mode", 2),
                                     attr_int(node, "has_bias", 0), attr_int(node, "act", 0),
                                     attr_int(node, "fp8_mfma", 0) ? LCML_KERNEL_AUTO_FP8 : LCML_KERNEL_AUTO);
};

}  // namespace lcml::onnx
