// Gemm, MatMul, Relu, Gelu and the fused FP8Linear.
//
// Gemm: Y = alpha * op(A) op(B) + beta * C with the reference's attributes
// and defaults (src/onnx/operators/gemm.cpp:365-385) and C broadcast rules
// (:81-103).  MatMul: 2-D B, A of any rank >= 1 (leading dims flattened into
// M), as the reference's 2-D path (src/onnx/operators/mat_mul.cpp:45-186).
// In an fp32 graph both run the plain fp32 kernel (same per-output fma
// order as the reference); in a QDQ graph the network's fusion pass has
// already replaced them, with their DequantizeLinear / QuantizeLinear
// neighbours and a following Relu/Gelu, by FP8Linear.
#include <vector>

#include "common.h"

namespace lcml::onnx {
namespace {

using namespace ops;

class Gemm : public StreamOperator {
    float alpha_, beta_;
    int transA_, transB_;

public:
    Gemm(float alpha, float beta, int transA, int transB)
        : StreamOperator("Gemm"), alpha_(alpha), beta_(beta), transA_(transA), transB_(transB) {}
    void forward(std::span<std::reference_wrapper<ITensor>> inputs,
                 std::span<std::reference_wrapper<ITensor>> outputs) override {
        LCML_ASSERT(inputs.size() >= 2 && inputs.size() <= 3 && outputs.size() == 1,
                    "Gemm requires 2 or 3 inputs and 1 output.");
        ITensor &A = inputs[0], &B = inputs[1], &Y = outputs[0];
        ITensor *C = inputs.size() == 3 ? &inputs[2].get() : nullptr;
        LCML_ASSERT(A.ndim() == 2 && B.ndim() == 2, "Gemm: A and B must be 2D tensors.");
        LCML_ASSERT(is_type<float>(A) && is_type<float>(B),
                    "Gemm: unfused operands must be float (FP8 weights reach Gemm through DequantizeLinear)");
        const int64_t M = transA_ ? A.shape(1) : A.shape(0), K = transA_ ? A.shape(0) : A.shape(1);
        const int64_t K2 = transB_ ? B.shape(1) : B.shape(0), N = transB_ ? B.shape(0) : B.shape(1);
        LCML_ASSERT(K == K2, "Gemm: inner dimensions mismatch (K=%lld vs %lld)", (long long)K, (long long)K2);
        LCML_ASSERT(Y.ndim() == 2 && Y.shape(0) == M && Y.shape(1) == N, "Gemm: Y shape mismatch");
        CArgs c = c_args(C);
        check(lcml_fp8_sgemm(M, N, K, static_cast<const float *>(A.device_data()), A.shape(1), transA_,
                             static_cast<const float *>(B.device_data()), B.shape(1), transB_, alpha_, c.ptr, c.ndim,
                             c.d0, c.d1, beta_, LCML_ACT_NONE, Y.device_data(), out_dtype_code(Y, "Gemm"), N, stream_),
              "Gemm");
    }
};

// MatMul with numpy semantics, as the reference (mat_mul.cpp:45-303): a 1-D
// A is one row and a 1-D B one column (both dropped from Y); batch
// dimensions are right-aligned and broadcast where they are 1.  A 2-D B
// (the linear-layer case) is one GEMM over all of A's rows; a batched B is
// one GEMM per output batch, each a sequential fma chain per output as the
// reference's own (B rows are not contiguous along k there either).
class MatMul : public StreamOperator {
public:
    MatMul() : StreamOperator("MatMul") {}
    void forward(std::span<std::reference_wrapper<ITensor>> inputs,
                 std::span<std::reference_wrapper<ITensor>> outputs) override {
        LCML_ASSERT(inputs.size() == 2 && outputs.size() == 1, "MatMul requires 2 inputs and 1 output.");
        ITensor &A = inputs[0], &B = inputs[1], &Y = outputs[0];
        LCML_ASSERT(is_type<float>(A) && is_type<float>(B), "MatMul: unfused operands must be float");
        const int an = (int)A.ndim(), bn = (int)B.ndim();
        LCML_ASSERT(an >= 1 && bn >= 1, "MatMul: operands must have at least one dimension");
        const int64_t K = A.shape(an - 1), M = an >= 2 ? A.shape(an - 2) : 1;
        const int64_t KB = bn >= 2 ? B.shape(bn - 2) : B.shape(0), N = bn >= 2 ? B.shape(bn - 1) : 1;
        LCML_ASSERT(KB == K, "MatMul: inner dimensions mismatch (K=%lld vs %lld)", (long long)K, (long long)KB);
        const int ydt = out_dtype_code(Y, "MatMul");
        const float *a = static_cast<const float *>(A.device_data());
        const float *b = static_cast<const float *>(B.device_data());
        char *y = static_cast<char *>(Y.device_data());
        const size_t esz = ydt == LCML_DTYPE_BFLOAT16 ? 2 : 4;
        if (bn <= 2) {  // every row of A against one B
            const int64_t rows = (int64_t)A.size() / K;
            LCML_ASSERT((int64_t)Y.size() == rows * N, "MatMul: output has %u elements, expected %lld", Y.size(),
                        (long long)(rows * N));
            check(lcml_fp8_sgemm(rows, N, K, a, K, 0, b, N, 0, 1.0f, nullptr, 0, 0, 0, 0.0f, LCML_ACT_NONE, y, ydt,
                                 N, stream_),
                  "MatMul");
            return;
        }
        // batch dimensions, right-aligned
        const int ab = an >= 2 ? an - 2 : 0, bb = bn - 2, nb = ab > bb ? ab : bb;
        std::vector<int64_t> ydim(nb), astr(nb, 0), bstr(nb, 0);
        int64_t sa = M * K, sb = K * N;
        for (int d = nb - 1; d >= 0; --d) {
            const int ai = d - (nb - ab), bi = d - (nb - bb);
            const int64_t ad = ai >= 0 ? A.shape(ai) : 1, bd = bi >= 0 ? B.shape(bi) : 1;
            LCML_ASSERT(ad == bd || ad == 1 || bd == 1, "MatMul: batch dimensions %lld and %lld do not broadcast",
                        (long long)ad, (long long)bd);
            ydim[d] = ad > bd ? ad : bd;
            if (ad > 1) astr[d] = sa;
            if (bd > 1) bstr[d] = sb;
            sa *= ad;
            sb *= bd;
        }
        int64_t batches = 1;
        for (int64_t v : ydim) batches *= v;
        LCML_ASSERT((int64_t)Y.size() == batches * M * N, "MatMul: output has %u elements, expected %lld", Y.size(),
                    (long long)(batches * M * N));
        std::vector<int64_t> idx(nb, 0);
        for (int64_t t = 0; t < batches; ++t) {
            int64_t ao = 0, bo = 0;
            for (int d = 0; d < nb; ++d) {
                ao += idx[d] * astr[d];
                bo += idx[d] * bstr[d];
            }
            check(lcml_fp8_sgemm(M, N, K, a + ao, K, 0, b + bo, N, 0, 1.0f, nullptr, 0, 0, 0, 0.0f, LCML_ACT_NONE,
                                 y + (size_t)(t * M * N) * esz, ydt, N, stream_),
                  "MatMul");
            for (int d = nb - 1; d >= 0 && ++idx[d] == ydim[d]; --d) idx[d] = 0;
        }
    }
};

class Activation : public StreamOperator {
    int act_;

public:
    Activation(const char *name, int act) : StreamOperator(name), act_(act) {}
    bool can_operate_inplace() const override { return true; }
    void forward(std::span<std::reference_wrapper<ITensor>> inputs,
                 std::span<std::reference_wrapper<ITensor>> outputs) override {
        ITensor &x = inputs[0], &y = outputs[0];
        LCML_ASSERT(is_type<float>(x) && is_type<float>(y), "%s: only float tensors are on the FP8 path",
                    get_name().c_str());
        LCML_ASSERT(x.size() == y.size(), "%s: input and output must have the same size.", get_name().c_str());
        check(lcml_fp8_activation(static_cast<const float *>(x.device_data()), static_cast<float *>(y.device_data()),
                                  x.size(), act_, stream_),
              get_name().c_str());
    }
};

// The fused QDQ linear built by NetworkInstance's fusion pass.
// inputs: [A, W packed, w_scale, (a_scale if a_mode == 1), (C if has_c)]
// a_mode 0: A fp32, W8A32 kernel; 1: A quantised with the static a_scale;
// 2: A quantised with its dynamic per-tensor scale (amax/448).
// trans_a: A is [K, M] (Gemm transA=1); the quantiser writes the [M, K]
// E4M3 copy as a transposing NCHW -> NHWC quantise of a [1, K, 1, M] view.
// wbatch: the batch dimensions of a batched MatMul weight [..., K, N] (empty
// for a 2-D weight): one GEMM per output batch, A's and W's batch dimensions
// right-aligned and broadcast where they are 1 (mat_mul.cpp:187-303); A is
// quantised once, per tensor, as the unfused DynamicQuantizeLinear does.
class FP8Linear : public StreamOperator {
    int a_mode_, has_c_, act_, trans_a_;
    float alpha_, beta_;
    std::vector<int32_t> wbatch_;
    int kernel_;  // LCML_KERNEL_AUTO, or AUTO_FP8 (NetworkInstance::set_fp8_matrix_cores)
    std::unique_ptr<DeviceBuffer> qa_, ws_, sx_;
    size_t qa_bytes_ = 0, ws_bytes_ = 0;

    uint8_t *qa_scratch(size_t need) {
        if (!qa_ || qa_bytes_ < need) {
            qa_ = std::make_unique<DeviceBuffer>(need);
            qa_bytes_ = need;
        }
        return static_cast<uint8_t *>(qa_->data());
    }
    void *dyn_workspace() {
        if (!ws_ || ws_bytes_ < (size_t)LCML_FP8_DYNAMIC_WORKSPACE_BYTES) {
            ws_ = std::make_unique<DeviceBuffer>((size_t)LCML_FP8_DYNAMIC_WORKSPACE_BYTES);
            ws_bytes_ = LCML_FP8_DYNAMIC_WORKSPACE_BYTES;
        }
        return ws_->data();
    }
    float *scale_slot() {
        if (!sx_) sx_ = std::make_unique<DeviceBuffer>(sizeof(float));
        return static_cast<float *>(sx_->data());
    }

    void forward_batched(ITensor &A, const PackedWeightTensor &W, ITensor *a_scale, ITensor &Y) {
        const int an = (int)A.ndim();
        const int64_t K = W.K(), N = W.N();
        LCML_ASSERT(an >= 2 && (int64_t)A.shape(an - 1) == K, "FP8Linear: A must be [..., M, K=%lld]", (long long)K);
        const int64_t M = A.shape(an - 2);
        const int ab = an - 2, bb = (int)wbatch_.size(), nb = ab > bb ? ab : bb;
        std::vector<int64_t> ydim(nb), astr(nb, 0), bstr(nb, 0);
        int64_t sa = M * K, sb = 1;  // A in elements, W in packed batches
        for (int d = nb - 1; d >= 0; --d) {
            const int ai = d - (nb - ab), bi = d - (nb - bb);
            const int64_t ad = ai >= 0 ? A.shape(ai) : 1, bd = bi >= 0 ? wbatch_[bi] : 1;
            LCML_ASSERT(ad == bd || ad == 1 || bd == 1, "FP8Linear: batch dimensions %lld and %lld do not broadcast",
                        (long long)ad, (long long)bd);
            ydim[d] = ad > bd ? ad : bd;
            if (ad > 1) astr[d] = sa;
            if (bd > 1) bstr[d] = sb;
            sa *= ad;
            sb *= bd;
        }
        LCML_ASSERT(sb == (int64_t)W.batches(), "FP8Linear: %u packed weights for %lld weight batches", W.batches(),
                    (long long)sb);
        int64_t batches = 1;
        for (int64_t v : ydim) batches *= v;
        LCML_ASSERT((int64_t)Y.size() == batches * M * N, "FP8Linear: output has %u elements, expected %lld", Y.size(),
                    (long long)(batches * M * N));
        const int ydt = out_dtype_code(Y, "FP8Linear");
        const size_t esz = ydt == LCML_DTYPE_BFLOAT16 ? 2 : 4;
        const float *a = static_cast<const float *>(A.device_data());
        char *y = static_cast<char *>(Y.device_data());
        const uint8_t *q = nullptr;
        const float *sa_dev = nullptr;
        if (a_mode_ != 0) {  // the whole activation once: E4M3 codes and one per-tensor scale
            uint8_t *qw = qa_scratch(A.size());
            if (a_mode_ == 1) {
                sa_dev = static_cast<const float *>(a_scale->device_data());
                check(lcml_fp8_quantize(a, qw, 1, 1, A.size(), sa_dev, stream_), "FP8Linear quantize");
            } else {
                float *sx = scale_slot();
                check(lcml_fp8_quantize_dynamic(a, qw, A.size(), sx, dyn_workspace(), stream_), "FP8Linear quantize");
                sa_dev = sx;
            }
            q = qw;
        }
        std::vector<int64_t> idx(nb, 0);
        for (int64_t t = 0; t < batches; ++t) {
            int64_t ao = 0, bo = 0;
            for (int d = 0; d < nb; ++d) {
                ao += idx[d] * astr[d];
                bo += idx[d] * bstr[d];
            }
            void *yt = y + (size_t)(t * M * N) * esz;
            if (a_mode_ == 0)
                check(lcml_fp8_gemm_w8a32(M, N, K, a + ao, K, W.packed(bo), W.scale(), W.per_channel(), alpha_, nullptr,
                                          0, 0, 0, beta_, act_, yt, ydt, N, stream_),
                      "FP8Linear");
            else
                check(lcml_fp8_gemm(M, N, K, q + ao, K, sa_dev, W.packed(bo), W.scale(), W.per_channel(), alpha_,
                                    nullptr, 0, 0, 0, beta_, act_, yt, ydt, N, kernel_, stream_),
                      "FP8Linear");
            for (int d = nb - 1; d >= 0 && ++idx[d] == ydim[d]; --d) idx[d] = 0;
        }
    }

public:
    FP8Linear(int a_mode, int has_c, int act, float alpha, float beta, int trans_a, std::vector<int32_t> wbatch,
              int kernel)
        : StreamOperator("FP8Linear"), a_mode_(a_mode), has_c_(has_c), act_(act), trans_a_(trans_a), alpha_(alpha),
          beta_(beta), wbatch_(std::move(wbatch)), kernel_(kernel) {}
    void forward(std::span<std::reference_wrapper<ITensor>> inputs,
                 std::span<std::reference_wrapper<ITensor>> outputs) override {
        ITensor &A = inputs[0], &Y = outputs[0];
        auto *W = dynamic_cast<PackedWeightTensor *>(&inputs[1].get());
        LCML_ASSERT(W != nullptr, "FP8Linear: input 1 must be a packed weight");
        LCML_ASSERT(is_type<float>(A), "FP8Linear: A must be float");
        size_t next = 3;
        ITensor *a_scale = a_mode_ == 1 ? &inputs[next++].get() : nullptr;
        ITensor *C = has_c_ ? &inputs[next++].get() : nullptr;
        if (!wbatch_.empty()) {
            LCML_ASSERT(!C && !trans_a_, "FP8Linear: a batched weight takes no C and no transA");
            forward_batched(A, *W, a_scale, Y);
            return;
        }
        const int64_t K = W->K(), N = W->N(), M = A.size() / K;
        LCML_ASSERT(M * K == (int64_t)A.size(), "FP8Linear: A has %u elements, not a multiple of K=%lld", A.size(),
                    (long long)K);
        LCML_ASSERT((int64_t)Y.size() == M * N, "FP8Linear: output size mismatch");
        CArgs c = c_args(C);
        const int ydt = out_dtype_code(Y, "FP8Linear");
        const float *a = static_cast<const float *>(A.device_data());
        LCML_ASSERT(!trans_a_ || (a_mode_ != 0 && A.ndim() == 2 && A.shape(0) == K),
                    "FP8Linear: transA needs a quantised [K, M] activation");
        if (trans_a_) {
            const size_t need = (size_t)(M * K);
            if (!qa_ || qa_bytes_ < need) {
                qa_ = std::make_unique<DeviceBuffer>(need);
                qa_bytes_ = need;
            }
            uint8_t *q = static_cast<uint8_t *>(qa_->data());
            const float *sa;
            if (a_mode_ == 1) {
                sa = static_cast<const float *>(a_scale->device_data());
                check(lcml_fp8_quantize_nhwc(a, q, 1, K, 1, M, sa, nullptr, nullptr, stream_), "FP8Linear quantize");
            } else {
                if (!sx_) sx_ = std::make_unique<DeviceBuffer>(sizeof(float));
                if (!ws_ || ws_bytes_ < (size_t)LCML_FP8_DYNAMIC_WORKSPACE_BYTES) {
                    ws_ = std::make_unique<DeviceBuffer>((size_t)LCML_FP8_DYNAMIC_WORKSPACE_BYTES);
                    ws_bytes_ = LCML_FP8_DYNAMIC_WORKSPACE_BYTES;
                }
                check(lcml_fp8_quantize_nhwc(a, q, 1, K, 1, M, nullptr, static_cast<float *>(sx_->data()), ws_->data(),
                                             stream_),
                      "FP8Linear quantize");
                sa = static_cast<const float *>(sx_->data());
            }
            check(lcml_fp8_gemm(M, N, K, q, K, sa, W->packed(), W->scale(), W->per_channel(), alpha_, c.ptr, c.ndim,
                                c.d0, c.d1, beta_, act_, Y.device_data(), ydt, N, kernel_, stream_),
                  "FP8Linear");
            return;
        }
        if (a_mode_ == 0) {
            check(lcml_fp8_gemm_w8a32(M, N, K, a, K, W->packed(), W->scale(), W->per_channel(), alpha_, c.ptr, c.ndim,
                                      c.d0, c.d1, beta_, act_, Y.device_data(), ydt, N, stream_),
                  "FP8Linear");
            return;
        }
        if (a_mode_ == 2) {
            // DynamicQuantizeLinear -> DQ -> Gemm in one call (one fused launch
            // for small M*K; otherwise quantise into the workspace + GEMM)
            // the size query assumes a 16-byte aligned A; a misaligned one
            // takes the two-step path (the MFMA kernel's size)
            const bool a16 = (reinterpret_cast<uintptr_t>(a) & 15) == 0;
            const int64_t ws =
                lcml_fp8_gemm_dynamic_workspace_bytes(M, K, a16 ? kernel_ : LCML_KERNEL_MFMA);
            if (ws > 0 && (!ws_ || ws_bytes_ < (size_t)ws)) {
                ws_ = std::make_unique<DeviceBuffer>((size_t)ws);
                ws_bytes_ = (size_t)ws;
            }
            check(lcml_fp8_gemm_dynamic(M, N, K, a, K, W->packed(), W->scale(), W->per_channel(), alpha_, c.ptr, c.ndim,
                                        c.d0, c.d1, beta_, act_, Y.device_data(), ydt, N, nullptr,
                                        ws > 0 ? ws_->data() : nullptr, ws, kernel_, stream_),
                  "FP8Linear");
            return;
        }
        // quantised activation scratch: M*K E4M3 bytes (16-byte aligned rows need K % 16 == 0)
        const size_t need = (size_t)(M * K);
        if (!qa_ || qa_bytes_ < need) {
            qa_ = std::make_unique<DeviceBuffer>(need);
            qa_bytes_ = need;
        }
        uint8_t *q = static_cast<uint8_t *>(qa_->data());
        const float *sa = static_cast<const float *>(a_scale->device_data());
        check(lcml_fp8_quantize(a, q, 1, 1, M * K, sa, stream_), "FP8Linear quantize");
        check(lcml_fp8_gemm(M, N, K, q, K, sa, W->packed(), W->scale(), W->per_channel(), alpha_, c.ptr, c.ndim, c.d0,
                            c.d1, beta_, act_, Y.device_data(), ydt, N, kernel_, stream_),
              "FP8Linear");
    }
};

}  // namespace

REGISTER_TO_DEFAULT_OPSET(Gemm) {
    return std::make_unique<Gemm>(attr_float(node, "alpha", 1.0f), attr_float(node, "beta", 1.0f),
                                  attr_int(node, "transA", 0), attr_int(node, "transB", 0));
};
REGISTER_TO_DEFAULT_OPSET(MatMul) { return std::make_unique<MatMul>(); };
REGISTER_TO_DEFAULT_OPSET(Relu) { return std::make_unique<Activation>("Relu", LCML_ACT_RELU); };
REGISTER_TO_DEFAULT_OPSET(Gelu) {
    std::string approx = attr_string(node, "approximate", "none");
    LCML_ASSERT(approx == "none" || approx == "tanh", "Gelu: unsupported approximate attribute: %s", approx.c_str());
    return std::make_unique<Activation>("Gelu", approx == "tanh" ? LCML_ACT_GELU_TANH : LCML_ACT_GELU_ERF);
};
REGISTER_TO_DEFAULT_OPSET(FP8Linear) {
    return std::make_unique<FP8Linear>(attr_int(node, "a_mode", 0), attr_int(node, "has_c", 0),
                                       attr_int(node, "act", 0), attr_float(node, "alpha", 1.0f),
                                       attr_float(node, "beta", 1.0f), attr_int(node, "trans_a", 0),
                                       attr_ints(node, "wbatch", {}),
                                       attr_int(node, "fp8_mfma", 0) ? LCML_KERNEL_AUTO_FP8 : LCML_KERNEL_AUTO);
};

}  // namespace lcml::onnx
