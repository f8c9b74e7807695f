// test_network.cpp -- GPU tests of the operator layer, in the manner of the
// reference's tests/onnx/test_onnx_inference.cpp, checked against the oracle
// (oracle/lcml_oracle.c, linked in as the reference arithmetic):
//   1. the reference's own fp32 MLP fixture (simple_mlp.onnx.json + weight
//      blob + input_ref/output_ref, tolerance 1e-3 as the reference uses);
//   2. the 3-layer FP8 MLP (784->256->128->10, batch 64, per-tensor E4M3
//      weights through DequantizeLinear, bias + Relu): fused into FP8Linear
//      nodes and unfused, both against the oracle;
//   3. static activation QDQ -> Gemm(transB=1, per-channel weights) -> Gelu;
//   4. DynamicQuantizeLinear -> DequantizeLinear -> MatMul(per-channel W);
//   5. standalone QuantizeLinear / DequantizeLinear / Cast, bit-exact;
//   6. error behaviour (dtype mismatch on bind, FP8 blob size rule);
//   7. DynamicQuantizeLinear -> DQ -> Conv(DQ(W), B) -> Relu, fused into
//      FP8Conv and op by op, against the oracle's direct conv;
//   8. an fp32 grouped / strided / dilated Conv;
//   9. E5M2 QuantizeLinear (saturate 1 and 0) / DequantizeLinear, Cast chains
//      FLOAT -> E5M2 -> E4M3 -> FLOAT, an E5M2 weight blob (4-byte padding);
//  10. Add / Sub / Mul / Div on FLOAT, E4M3 and E5M2 tensors with
//      broadcasting, and a DynamicQuantizeLinear zero-point output;
//  11. the device-buffer planner: a 9-node graph run with one planned arena
//      and with one allocation per intermediate, bit-identical outputs;
//  12. the FP8 QDQ MLP model file (tests/golden/fp8_mlp.*) loaded from disk,
//      fused (3 FP8Linear) and op by op, against its stored oracle output;
//  13. an E5M2 activation QDQ stays unfused in front of an E4M3 weight;
//  14. scalar (0-D) value_info of DynamicQuantizeLinear outputs;
//  15. one E4M3 weight behind two scales and two layouts;
//  16. Gemm(transA=1) with static and dynamic activation QDQ, fused;
//  17. 1-D Conv with auto_pad, fp32 and fused FP8.
//   usage: test_network <tests/golden dir>
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <sstream>
#include <string>
#include <vector>

#include <unistd.h>

#include "lcml_fp8.h"
#include "onnx/network_instance.h"

using namespace lcml::onnx;

extern "C" {
uint8_t orc_e4m3_from_float(float);
float orc_e4m3_to_float(uint8_t);
void orc_quantize(const float *, uint8_t *, int64_t, int64_t, int64_t, const float *);
void orc_dequantize(const uint8_t *, float *, int64_t, int64_t, int64_t, const float *);
float orc_amax(const float *, int64_t);
float orc_scale_from_amax(float);
void orc_gemm(int64_t, int64_t, int64_t, const float *, int, const float *, int, float, float, const float *, int,
              int64_t, int64_t, int, float *);
void orc_conv2d(const float *, const float *, const float *, float *, int64_t, int64_t, int64_t, int64_t, int64_t,
                int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t,
                int);
void orc_gemm_abs_bound(int64_t, int64_t, int64_t, const float *, int, const float *, int, float, float,
                        const float *, int, int64_t, int64_t, double *);
uint8_t orc_e5m2_from_float(float);
float orc_e5m2_to_float(uint8_t);
void orc_quantize_e5m2(const float *, uint8_t *, int64_t, int64_t, int64_t, const float *, int);
void orc_dequantize_e5m2(const uint8_t *, float *, int64_t, int64_t, int64_t, const float *);
void orc_fp8_binary(int, int, const void *, const int64_t *, int, const void *, const int64_t *, int, void *,
                    const int64_t *, int);
}

static int failures = 0;
#define CHECK(c)                                                                  \
    do {                                                                          \
        if (!(c)) {                                                               \
            std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #c);              \
            std::fflush(stdout);                                                  \
            ++failures;                                                           \
        }                                                                         \
    } while (0)

template <typename F>
static bool throws(F &&f) {
    try {
        f();
    } catch (const Error &) {
        return true;
    }
    return false;
}

// ---------------------------------------------------------------- data ----
struct Rng {
    uint64_t s;
    uint64_t next() {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    double uni() { return (next() >> 11) * (1.0 / 9007199254740992.0); }
    float normal(float std) {
        double u1 = 1.0 - uni(), u2 = uni();
        return (float)(std * std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
    }
};

static std::vector<float> normals(uint64_t seed, size_t n, float std) {
    Rng r{seed};
    std::vector<float> v(n);
    for (auto &x : v) x = r.normal(std);
    return v;
}

template <typename T>
static std::unique_ptr<NNTensor<T>> upload(const std::vector<T> &h, ITensor::shape_type shape) {
    auto t = make_device_tensor<T>(shape);
    if (!h.empty()) CHECK(hipMemcpy(t->data(), h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice) == hipSuccess);
    return t;
}

template <typename T>
static std::vector<T> download(const ITensor &t) {
    std::vector<T> h(t.size());
    CHECK(hipDeviceSynchronize() == hipSuccess);
    CHECK(hipMemcpy(h.data(), t.device_data(), h.size() * sizeof(T), hipMemcpyDeviceToHost) == hipSuccess);
    return h;
}

static std::string read_text(const std::string &p) {
    std::ifstream f(p, std::ios::binary);
    std::stringstream ss;
    ss << f.rdbuf();
    return ss.str();
}

// Weight blob builder: appends tensors at 4-byte aligned offsets, as the
// reference's exporter lays out data_offsets.
struct Blob {
    std::vector<uint8_t> bytes;
    std::pair<uint64_t, uint64_t> add(const void *p, size_t n, size_t padded) {
        uint64_t start = bytes.size();
        bytes.resize(start + padded, 0);
        std::memcpy(bytes.data() + start, p, n);
        return {start, start + padded};
    }
};

// Graph builder helpers.
static const Variable &var(Graph &g, const std::string &n, DataType dt, std::vector<size_t> shape) {
    return g.add_variable(Variable(n, dt, std::move(shape)));
}
static const Variable &blob_var(Graph &g, Blob &b, const std::string &n, DataType dt, std::vector<size_t> shape,
                                const void *data, size_t bytes) {
    size_t padded = dt == DataType::FLOAT8E4M3FN || dt == DataType::FLOAT8E5M2 ? (bytes + 3) / 4 * 4 : bytes;
    auto [s, e] = b.add(data, bytes, padded);
    return g.add_variable(Variable(n, dt, std::move(shape), {}, s, e));
}
static const Variable &raw_var(Graph &g, const std::string &n, DataType dt, std::vector<size_t> shape, const void *data,
                               size_t bytes) {
    return g.add_variable(Variable(n, dt, std::move(shape), std::string((const char *)data, bytes)));
}
static void node(Graph &g, const std::string &op, std::vector<std::string> ins, std::vector<std::string> outs,
                 std::vector<Attribute> attrs = {}) {
    Node n(op + "_" + outs[0], op);
    for (auto &i : ins) n.add_input(g.get_var(i));
    for (auto &o : outs) n.add_output(g.get_var(o));
    for (auto &a : attrs) n.set_attribute(std::move(a));
    g.add_node(std::move(n));
}

// |y - ref| <= tol * bound + atol, elementwise
static bool close(const std::vector<float> &y, const std::vector<float> &ref, const std::vector<double> &bound,
                  double tol, double atol, const char *what) {
    size_t bad = 0, first = 0;
    for (size_t i = 0; i < y.size(); ++i) {
        double d = std::fabs((double)y[i] - (double)ref[i]);
        if (!(d <= tol * bound[i] + atol)) {
            if (!bad) first = i;
            ++bad;
        }
    }
    if (bad)
        std::printf("  %s: %zu/%zu outside tolerance; first %zu: %.9g vs %.9g (bound %.3g)\n", what, bad, y.size(),
                    first, y[first], ref[first], bound[first]);
    return bad == 0;
}

// Per-element tolerance of one Gemm (transB = 1) + bias [+ Relu] layer of a
// chain checked against the oracle chain.  The layer may differ from the
// oracle's composition on the same inputs by 1e-4 * sum|a*b| (+|bias|)
// (fp32 summation order); the difference `carry` already in its inputs
// passes through |W| (Relu is 1-Lipschitz), and the device's own bound over
// its inputs exceeds the oracle's by at most carry * |W|:
//   t_l = 1e-4 * bound_l + (1 + 1e-4) * carry_{l-1} |W_l|^T,  carry_{-1} = 0.
// h: the layer's oracle input [B, K]; W: dequantised [N, K].
static std::vector<double> layer_tolerance(int B, int K, int N, const std::vector<float> &h, const float *W,
                                           const float *b, const std::vector<double> &carry) {
    std::vector<double> t((size_t)B * N);
    orc_gemm_abs_bound(B, N, K, h.data(), 0, W, 1, 1.0f, 1.0f, b, 1, N, 0, t.data());
    for (int m = 0; m < B; ++m)
        for (int n = 0; n < N; ++n) {
            double prop = 0.0;
            if (!carry.empty())
                for (int k = 0; k < K; ++k) prop += carry[(size_t)m * K + k] * std::fabs((double)W[(size_t)n * K + k]);
            t[(size_t)m * N + n] = 1e-4 * t[(size_t)m * N + n] + (1.0 + 1e-4) * prop;
        }
    return t;
}

// ------------------------------------------------------------- tests ----
static void test_reference_fixture(const std::string &golden) {
    std::printf("[1] reference fp32 MLP fixture\n");
    Model m = Model::load_from_json(read_text(golden + "/simple_mlp.onnx.json"));
    std::string blob = read_text(golden + "/simple_mlp.safetensors");
    std::string xin = read_text(golden + "/input_ref.bin"), yref = read_text(golden + "/output_ref.bin");
    DeviceBuffer wb(blob.size());
    CHECK(hipMemcpy(wb.data(), blob.data(), blob.size(), hipMemcpyHostToDevice) == hipSuccess);
    std::vector<float> x(784), want(10);
    std::memcpy(x.data(), xin.data(), 784 * 4);
    std::memcpy(want.data(), yref.data(), 40);
    auto xt = upload(x, {1, 784});
    auto yt = make_device_tensor<float>({1, 10});
    NetworkInstance net;
    net.set_model(std::move(m));
    net.set_warp_size(1);  // as the reference's inference test does (test_onnx_inference.cpp:177)
    net.set_weight_buffer(wb.data(), blob.size());
    net.set_input("input", *xt);
    net.set_output("output", *yt);
    // the execution log (network_instance.cpp:594-634 of the reference)
    const char *tmp = std::getenv("TMPDIR");
    const std::string log = std::string(tmp && *tmp ? tmp : "/tmp") + "/lcml_stats_" + std::to_string(getpid()) + ".md";
    std::remove(log.c_str());
    net.set_log_file(log);
    net.enable_logging(true);
    net.forward();
    net.enable_logging(false);
    net.forward();  // not logged
    auto y = download<float>(*yt);
    for (int i = 0; i < 10; ++i) {
        if (std::fabs(y[i] - want[i]) > 1e-3f) {
            std::printf("  MISMATCH at %d: GPU=%.6f Ref=%.6f\n", i, y[i], want[i]);
            ++failures;
        }
    }
    CHECK(net.warp_size() == 1 && !net.use_warp_optimization());
    CHECK(&net.get_inputs().at("input").get() == xt.get() && &net.get_outputs().at("output").get() == yt.get());
    CHECK(net.get_model().get_graph().get_nodes().size() == net.executed_op_types().size());
    const std::string text = read_text(log);
    std::remove(log.c_str());
    auto count = [&](const std::string &needle) {
        size_t n = 0;
        for (size_t p = text.find(needle); p != std::string::npos; p = text.find(needle, p + 1)) ++n;
        return n;
    };
    const size_t nodes = net.executed_op_types().size();
    CHECK(count("# Network Execution Log") == 1 && count("| Total Nodes | " + std::to_string(nodes) + " |") == 1);
    CHECK(count("### Node [") == nodes && count("**Kernels:** ") == nodes);
    CHECK(count("### Node [0/" + std::to_string(nodes - 1) + "]: Gemm") == 1);
    CHECK(count("- `input` : shape=[1, 784], dtype=FLOAT") == 1);
    CHECK(count("**Kernels:** lcml_fp8_sgemm") == 3 && count("**Kernels:** (none)") == 0);
}

static void test_fp8_mlp(bool fused) {
    std::printf("[2] FP8 MLP 784-256-128-10 batch 64, %s\n", fused ? "fused" : "unfused");
    const int B = 64, dims[4] = {784, 256, 128, 10};
    Graph g("mlp");
    Blob blob;
    std::vector<std::vector<float>> Wdq(3), bias(3);
    var(g, "x", DataType::FLOAT, {(size_t)B, 784});
    for (int l = 0; l < 3; ++l) {
        const int K = dims[l], N = dims[l + 1];
        auto w = normals(100 + l, (size_t)N * K, 0.05f);
        float s = orc_scale_from_amax(orc_amax(w.data(), w.size()));
        std::vector<uint8_t> q(w.size());
        orc_quantize(w.data(), q.data(), 1, 1, w.size(), &s);
        Wdq[l].resize(w.size());
        orc_dequantize(q.data(), Wdq[l].data(), 1, 1, q.size(), &s);
        bias[l] = normals(200 + l, N, 0.01f);
        std::string L = std::to_string(l);
        blob_var(g, blob, "W" + L, DataType::FLOAT8E4M3FN, {(size_t)N, (size_t)K}, q.data(), q.size());
        raw_var(g, "s" + L, DataType::FLOAT, {1}, &s, 4);
        blob_var(g, blob, "b" + L, DataType::FLOAT, {(size_t)N}, bias[l].data(), N * 4);
        var(g, "Wf" + L, DataType::FLOAT, {(size_t)N, (size_t)K});
        var(g, "y" + L, DataType::FLOAT, {(size_t)B, (size_t)N});
        node(g, "DequantizeLinear", {"W" + L, "s" + L}, {"Wf" + L});
        std::string in = l == 0 ? "x" : "h" + std::to_string(l - 1);
        node(g, "Gemm", {in, "Wf" + L, "b" + L}, {"y" + L},
             {Attribute{"transB", (int32_t)1}, Attribute{"alpha", 1.0f}, Attribute{"beta", 1.0f}});
        if (l < 2) {
            var(g, "h" + L, DataType::FLOAT, {(size_t)B, (size_t)N});
            node(g, "Relu", {"y" + L}, {"h" + L});
        }
    }
    g.add_input("x");
    g.add_output("y2");
    Model m(10, "test", "1");
    m.set_graph(std::move(g));
    DeviceBuffer wb(blob.bytes.size());
    CHECK(hipMemcpy(wb.data(), blob.bytes.data(), blob.bytes.size(), hipMemcpyHostToDevice) == hipSuccess);
    std::vector<float> x(B * 784);
    Rng r{7};
    for (auto &v : x) v = (float)r.uni();  // U(0,1)
    auto xt = upload(x, {(uint32_t)B, 784});
    auto yt = make_device_tensor<float>({(uint32_t)B, 10});
    NetworkInstance net;
    net.set_model(std::move(m));
    net.set_fusion(fused);
    net.set_weight_buffer(wb.data(), blob.bytes.size());
    net.set_input("x", *xt);
    net.set_output("y2", *yt);
    net.forward();
    auto y = download<float>(*yt);
    auto types = net.executed_op_types();
    if (fused) {
        CHECK(net.fused_linear_count() == 3 && types.size() == 3);
        for (auto &t : types) CHECK(t == "FP8Linear");
    } else {
        CHECK(types.size() == 8 && net.fused_linear_count() == 0);
    }
    // oracle chain, and the tolerance carried through it layer by layer
    std::vector<float> h = x;
    std::vector<double> tol;
    for (int l = 0; l < 3; ++l) {
        const int K = dims[l], N = dims[l + 1];
        std::vector<float> out((size_t)B * N);
        tol = layer_tolerance(B, K, N, h, Wdq[l].data(), bias[l].data(), tol);
        orc_gemm(B, N, K, h.data(), 0, Wdq[l].data(), 1, 1.0f, 1.0f, bias[l].data(), 1, N, 0, l < 2 ? 1 : 0,
                 out.data());
        h = std::move(out);
    }
    CHECK(close(y, h, tol, 1.0, 0.0, "mlp"));
}

// K % 16 != 0: E4M3 activation rows cannot take a 16-byte pitch, so the
// activation's Q/DQ pair stays and the fused node runs W8A32 on its output
static void test_static_qdq_gelu(int K = 256) {
    std::printf("[3] static QDQ activation -> Gemm(transB=1, per-channel) -> Gelu, K=%d\n", K);
    const int M = 64, N = 192;
    auto x = normals(31, (size_t)M * K, 1.0f), w = normals(32, (size_t)N * K, 0.02f), b = normals(33, N, 0.01f);
    float sx = orc_scale_from_amax(orc_amax(x.data(), x.size()));
    std::vector<float> sw(N);
    for (int n = 0; n < N; ++n) sw[n] = orc_scale_from_amax(orc_amax(w.data() + (size_t)n * K, K));
    std::vector<uint8_t> qw(w.size()), qx(x.size()), zp(1, 0);
    orc_quantize(w.data(), qw.data(), 1, N, K, sw.data());  // per-channel along axis 0 of [N, K]
    orc_quantize(x.data(), qx.data(), 1, 1, x.size(), &sx);
    Graph g("qdq");
    Blob blob;
    var(g, "x", DataType::FLOAT, {(size_t)M, (size_t)K});
    raw_var(g, "sx", DataType::FLOAT, {1}, &sx, 4);
    raw_var(g, "zx", DataType::FLOAT8E4M3FN, {1}, zp.data(), 1);
    blob_var(g, blob, "W", DataType::FLOAT8E4M3FN, {(size_t)N, (size_t)K}, qw.data(), qw.size());
    blob_var(g, blob, "sw", DataType::FLOAT, {(size_t)N}, sw.data(), N * 4);
    blob_var(g, blob, "b", DataType::FLOAT, {(size_t)N}, b.data(), N * 4);
    var(g, "xq", DataType::FLOAT8E4M3FN, {(size_t)M, (size_t)K});
    var(g, "xd", DataType::FLOAT, {(size_t)M, (size_t)K});
    var(g, "Wf", DataType::FLOAT, {(size_t)N, (size_t)K});
    var(g, "y", DataType::FLOAT, {(size_t)M, (size_t)N});
    var(g, "z", DataType::FLOAT, {(size_t)M, (size_t)N});
    node(g, "QuantizeLinear", {"x", "sx", "zx"}, {"xq"});
    node(g, "DequantizeLinear", {"xq", "sx", "zx"}, {"xd"});
    node(g, "DequantizeLinear", {"W", "sw"}, {"Wf"}, {Attribute{"axis", (int32_t)0}});
    node(g, "Gemm", {"xd", "Wf", "b"}, {"y"}, {Attribute{"transB", (int32_t)1}});
    node(g, "Gelu", {"y"}, {"z"});
    g.add_input("x");
    g.add_output("z");
    Model m(10, "test", "1");
    m.set_graph(std::move(g));
    DeviceBuffer wb(blob.bytes.size());
    CHECK(hipMemcpy(wb.data(), blob.bytes.data(), blob.bytes.size(), hipMemcpyHostToDevice) == hipSuccess);
    auto xt = upload(x, {(uint32_t)M, (uint32_t)K});
    auto zt = make_device_tensor<float>({(uint32_t)M, (uint32_t)N});
    NetworkInstance net;
    net.set_model(std::move(m));
    net.set_weight_buffer(wb.data(), blob.bytes.size());
    net.set_input("x", *xt);
    net.set_output("z", *zt);
    net.forward();
    auto z = download<float>(*zt);
    CHECK(net.fused_linear_count() == 1 && net.executed_op_types().size() == (K % 16 ? 3u : 1u));
    std::vector<float> A(x.size()), Bw(w.size()), ref((size_t)M * N);
    orc_dequantize(qx.data(), A.data(), 1, 1, qx.size(), &sx);
    orc_dequantize(qw.data(), Bw.data(), 1, N, K, sw.data());
    orc_gemm(M, N, K, A.data(), 0, Bw.data(), 1, 1.0f, 1.0f, b.data(), 1, N, 0, 2, ref.data());
    std::vector<double> bound((size_t)M * N);
    orc_gemm_abs_bound(M, N, K, A.data(), 0, Bw.data(), 1, 1.0f, 1.0f, b.data(), 1, N, 0, bound.data());
    // GELU: 1.13 x the summation-order bar plus twice the device's pinned
    // evaluation difference (8 * 2^-24 of the pre-activation, which the
    // bound dominates; tests/test_gpu_activation.py)
    CHECK(close(z, ref, bound, 1.13e-4 + 16.0 * 0x1p-24, 0.0, "static qdq gelu"));
}

static void test_dynamic_qdq_matmul(int K = 512) {
    std::printf("[4] DynamicQuantizeLinear -> DequantizeLinear -> MatMul(per-channel W[K,N]), K=%d\n", K);
    const int M = 16, N = 320;
    auto x = normals(41, (size_t)M * K, 1.0f), w = normals(42, (size_t)K * N, 0.02f);
    std::vector<float> sw(N, 0.0f);
    for (int k = 0; k < K; ++k)
        for (int n = 0; n < N; ++n) sw[n] = std::max(sw[n], std::fabs(w[(size_t)k * N + n]));
    for (auto &s : sw) s = orc_scale_from_amax(s);
    std::vector<uint8_t> qw(w.size());
    orc_quantize(w.data(), qw.data(), K, N, 1, sw.data());  // per-channel along axis 1 of [K, N]
    Graph g("dyn");
    Blob blob;
    var(g, "x", DataType::FLOAT, {(size_t)M, (size_t)K});
    blob_var(g, blob, "W", DataType::FLOAT8E4M3FN, {(size_t)K, (size_t)N}, qw.data(), qw.size());
    blob_var(g, blob, "sw", DataType::FLOAT, {(size_t)N}, sw.data(), N * 4);
    var(g, "xq", DataType::FLOAT8E4M3FN, {(size_t)M, (size_t)K});
    var(g, "xs", DataType::FLOAT, {1});
    var(g, "xz", DataType::FLOAT8E4M3FN, {1});
    var(g, "xd", DataType::FLOAT, {(size_t)M, (size_t)K});
    var(g, "Wf", DataType::FLOAT, {(size_t)K, (size_t)N});
    var(g, "y", DataType::FLOAT, {(size_t)M, (size_t)N});
    node(g, "DynamicQuantizeLinear", {"x"}, {"xq", "xs", "xz"});
    node(g, "DequantizeLinear", {"xq", "xs", "xz"}, {"xd"});
    node(g, "DequantizeLinear", {"W", "sw"}, {"Wf"}, {Attribute{"axis", (int32_t)1}});
    node(g, "MatMul", {"xd", "Wf"}, {"y"});
    g.add_input("x");
    g.add_output("y");
    Model m(10, "test", "1");
    m.set_graph(std::move(g));
    DeviceBuffer wb(blob.bytes.size());
    CHECK(hipMemcpy(wb.data(), blob.bytes.data(), blob.bytes.size(), hipMemcpyHostToDevice) == hipSuccess);
    {
        auto xt = upload(x, {(uint32_t)M, (uint32_t)K});
        auto yt = make_device_tensor<float>({(uint32_t)M, (uint32_t)N});
        NetworkInstance net;
        net.set_model(std::move(m));
        net.set_weight_buffer(wb.data(), blob.bytes.size());
        net.set_input("x", *xt);
        net.set_output("y", *yt);
        net.forward();
        auto y = download<float>(*yt);
        CHECK(net.fused_linear_count() == 1 && net.executed_op_types().size() == (K % 16 ? 3u : 1u));
        float sx = orc_scale_from_amax(orc_amax(x.data(), x.size()));
        std::vector<uint8_t> qx(x.size());
        orc_quantize(x.data(), qx.data(), 1, 1, x.size(), &sx);
        std::vector<float> A(x.size()), Bw(w.size()), ref((size_t)M * N);
        orc_dequantize(qx.data(), A.data(), 1, 1, qx.size(), &sx);
        orc_dequantize(qw.data(), Bw.data(), K, N, 1, sw.data());
        orc_gemm(M, N, K, A.data(), 0, Bw.data(), 0, 1.0f, 0.0f, nullptr, -1, 0, 0, 0, ref.data());
        std::vector<double> bound((size_t)M * N);
        orc_gemm_abs_bound(M, N, K, A.data(), 0, Bw.data(), 0, 1.0f, 0.0f, nullptr, -1, 0, 0, bound.data());
        CHECK(close(y, ref, bound, 1e-4, 0.0, "dynamic qdq matmul"));
    }
}

// DynamicQuantizeLinear -> DequantizeLinear -> Conv(DQ(W_e4m3, per-channel
// axis 0), B) -> Relu, fused into FP8Conv and op by op (fp32 Conv), both
// against the oracle's direct conv of the dequantised operands; then an fp32
// grouped Conv on its own.
static void test_qdq_conv(bool fused, int64_t G = 1) {
    std::printf("[7] DynamicQuantizeLinear -> DQ -> Conv(DQ(W), B, group %lld) -> Relu (%s)\n", (long long)G,
                fused ? "fused" : "op by op");
    const int64_t Nb = 2, C = 32 * G, H = 9, W = 11, CO = 24, KH = 3, KW = 3, OH = 9, OW = 11, CG = C / G;
    auto x = normals(71, (size_t)(Nb * C * H * W), 1.0f), w = normals(72, (size_t)(CO * CG * KH * KW), 0.05f);
    auto bias = normals(73, (size_t)CO, 0.01f);
    const int64_t kper = CG * KH * KW;
    std::vector<float> sw(CO, 0.0f);
    for (int64_t o = 0; o < CO; ++o)
        for (int64_t k = 0; k < kper; ++k) sw[o] = std::max(sw[o], std::fabs(w[o * kper + k]));
    for (auto &v : sw) v = orc_scale_from_amax(v);
    std::vector<uint8_t> qw(w.size());
    orc_quantize(w.data(), qw.data(), 1, CO, kper, sw.data());  // per output channel (axis 0)
    Graph g("conv");
    Blob blob;
    var(g, "x", DataType::FLOAT, {(size_t)Nb, (size_t)C, (size_t)H, (size_t)W});
    blob_var(g, blob, "W", DataType::FLOAT8E4M3FN, {(size_t)CO, (size_t)CG, (size_t)KH, (size_t)KW}, qw.data(),
             qw.size());
    blob_var(g, blob, "sw", DataType::FLOAT, {(size_t)CO}, sw.data(), CO * 4);
    blob_var(g, blob, "B", DataType::FLOAT, {(size_t)CO}, bias.data(), CO * 4);
    var(g, "xq", DataType::FLOAT8E4M3FN, {(size_t)Nb, (size_t)C, (size_t)H, (size_t)W});
    var(g, "xs", DataType::FLOAT, {1});
    var(g, "xz", DataType::FLOAT8E4M3FN, {1});
    var(g, "xd", DataType::FLOAT, {(size_t)Nb, (size_t)C, (size_t)H, (size_t)W});
    var(g, "Wf", DataType::FLOAT, {(size_t)CO, (size_t)CG, (size_t)KH, (size_t)KW});
    var(g, "c", DataType::FLOAT, {(size_t)Nb, (size_t)CO, (size_t)OH, (size_t)OW});
    var(g, "y", DataType::FLOAT, {(size_t)Nb, (size_t)CO, (size_t)OH, (size_t)OW});
    node(g, "DynamicQuantizeLinear", {"x"}, {"xq", "xs", "xz"});
    node(g, "DequantizeLinear", {"xq", "xs", "xz"}, {"xd"});
    node(g, "DequantizeLinear", {"W", "sw"}, {"Wf"}, {Attribute{"axis", (int32_t)0}});
    node(g, "Conv", {"xd", "Wf", "B"}, {"c"},
         {Attribute{"kernel_shape", std::vector<int32_t>{3, 3}}, Attribute{"pads", std::vector<int32_t>{1, 1, 1, 1}},
          Attribute{"group", (int32_t)G}});
    node(g, "Relu", {"c"}, {"y"});
    g.add_input("x");
    g.add_output("y");
    Model m(10, "test", "1");
    m.set_graph(std::move(g));
    DeviceBuffer wb(blob.bytes.size());
    CHECK(hipMemcpy(wb.data(), blob.bytes.data(), blob.bytes.size(), hipMemcpyHostToDevice) == hipSuccess);
    auto xt = upload(x, {(uint32_t)Nb, (uint32_t)C, (uint32_t)H, (uint32_t)W});
    auto yt = make_device_tensor<float>({(uint32_t)Nb, (uint32_t)CO, (uint32_t)OH, (uint32_t)OW});
    NetworkInstance net;
    net.set_model(std::move(m));
    net.set_fusion(fused);
    net.set_weight_buffer(wb.data(), blob.bytes.size());
    net.set_input("x", *xt);
    net.set_output("y", *yt);
    net.forward();
    auto y = download<float>(*yt);
    if (fused) CHECK(net.fused_linear_count() == 1 && net.executed_op_types().size() == 1 &&
                     net.executed_op_types()[0] == "FP8Conv");
    else CHECK(net.executed_op_types().size() == 5);
    float sx = orc_scale_from_amax(orc_amax(x.data(), x.size()));
    std::vector<uint8_t> qx(x.size());
    orc_quantize(x.data(), qx.data(), 1, 1, x.size(), &sx);
    std::vector<float> A(x.size()), Bw(w.size()), ref(y.size()), absA(x.size()), absB(w.size()), bnd(y.size());
    orc_dequantize(qx.data(), A.data(), 1, 1, qx.size(), &sx);
    orc_dequantize(qw.data(), Bw.data(), 1, CO, kper, sw.data());
    orc_conv2d(A.data(), Bw.data(), bias.data(), ref.data(), Nb, C, H, W, CO, KH, KW, 1, 1, 1, 1, 1, 1, G, OH, OW,
               LCML_ACT_RELU);
    for (size_t i = 0; i < A.size(); ++i) absA[i] = std::fabs(A[i]);
    for (size_t i = 0; i < Bw.size(); ++i) absB[i] = std::fabs(Bw[i]);
    std::vector<float> absb(bias.size());
    for (size_t i = 0; i < bias.size(); ++i) absb[i] = std::fabs(bias[i]);
    orc_conv2d(absA.data(), absB.data(), absb.data(), bnd.data(), Nb, C, H, W, CO, KH, KW, 1, 1, 1, 1, 1, 1, G, OH, OW,
               LCML_ACT_NONE);
    std::vector<double> bound(bnd.begin(), bnd.end());
    CHECK(close(y, ref, bound, 1e-4, 0.0, fused ? "fused qdq conv" : "qdq conv op by op"));
}

static void test_f32_grouped_conv() {
    std::printf("[8] fp32 Conv, group 2, stride 2, dilation 2\n");
    const int64_t Nb = 1, C = 8, H = 12, W = 10, CO = 6, KH = 3, KW = 3, G = 2;
    const int64_t OH = (H + 2 - 2 * (KH - 1) - 1) / 2 + 1, OW = (W + 2 - 2 * (KW - 1) - 1) / 2 + 1;
    auto x = normals(81, (size_t)(Nb * C * H * W), 1.0f), w = normals(82, (size_t)(CO * (C / G) * KH * KW), 0.3f);
    Graph g("conv32");
    Blob blob;
    var(g, "x", DataType::FLOAT, {(size_t)Nb, (size_t)C, (size_t)H, (size_t)W});
    blob_var(g, blob, "W", DataType::FLOAT, {(size_t)CO, (size_t)(C / G), (size_t)KH, (size_t)KW}, w.data(), w.size() * 4);
    var(g, "y", DataType::FLOAT, {(size_t)Nb, (size_t)CO, (size_t)OH, (size_t)OW});
    node(g, "Conv", {"x", "W"}, {"y"},
         {Attribute{"group", (int32_t)G}, Attribute{"strides", std::vector<int32_t>{2, 2}},
          Attribute{"dilations", std::vector<int32_t>{2, 2}}, Attribute{"pads", std::vector<int32_t>{1, 1, 1, 1}}});
    g.add_input("x");
    g.add_output("y");
    Model m(10, "test", "1");
    m.set_graph(std::move(g));
    DeviceBuffer wb(blob.bytes.size());
    CHECK(hipMemcpy(wb.data(), blob.bytes.data(), blob.bytes.size(), hipMemcpyHostToDevice) == hipSuccess);
    auto xt = upload(x, {(uint32_t)Nb, (uint32_t)C, (uint32_t)H, (uint32_t)W});
    auto yt = make_device_tensor<float>({(uint32_t)Nb, (uint32_t)CO, (uint32_t)OH, (uint32_t)OW});
    NetworkInstance net;
    net.set_model(std::move(m));
    net.set_weight_buffer(wb.data(), blob.bytes.size());
    net.set_input("x", *xt);
    net.set_output("y", *yt);
    net.forward();
    auto y = download<float>(*yt);
    std::vector<float> ref(y.size());
    orc_conv2d(x.data(), w.data(), nullptr, ref.data(), Nb, C, H, W, CO, KH, KW, 2, 2, 1, 1, 2, 2, G, OH, OW,
               LCML_ACT_NONE);
    std::vector<double> bound(y.size(), 0.0);
    for (size_t i = 0; i < ref.size(); ++i) bound[i] = std::fabs(ref[i]) + 1.0;
    CHECK(close(y, ref, bound, 1e-5, 0.0, "fp32 grouped conv"));
}

static void test_standalone_qdq_cast() {
    std::printf("[5] standalone QuantizeLinear / DequantizeLinear / Cast (bit-exact)\n");
    const int R = 8, C = 100;
    auto x = normals(51, (size_t)R * C, 3.0f);
    x[5] = INFINITY;
    x[6] = -INFINITY;
    x[7] = NAN;
    x[8] = -0.0f;
    std::vector<float> s(C);
    for (int c = 0; c < C; ++c) s[c] = 0.01f + 0.001f * c;
    Graph g("q");
    var(g, "x", DataType::FLOAT, {(size_t)R, (size_t)C});
    raw_var(g, "s", DataType::FLOAT, {(size_t)C}, s.data(), C * 4);
    var(g, "q", DataType::FLOAT8E4M3FN, {(size_t)R, (size_t)C});
    var(g, "d", DataType::FLOAT, {(size_t)R, (size_t)C});
    var(g, "c8", DataType::FLOAT8E4M3FN, {(size_t)R, (size_t)C});
    var(g, "cf", DataType::FLOAT, {(size_t)R, (size_t)C});
    node(g, "QuantizeLinear", {"x", "s"}, {"q"}, {Attribute{"axis", (int32_t)1}});
    node(g, "DequantizeLinear", {"q", "s"}, {"d"}, {Attribute{"axis", (int32_t)1}});
    node(g, "Cast", {"x"}, {"c8"}, {Attribute{"to", (int32_t)17}});
    node(g, "Cast", {"c8"}, {"cf"}, {Attribute{"to", (int32_t)1}});
    g.add_input("x");
    g.add_output("d");
    g.add_output("cf");
    Model m(10, "test", "1");
    m.set_graph(std::move(g));
    auto xt = upload(x, {(uint32_t)R, (uint32_t)C});
    auto dt = make_device_tensor<float>({(uint32_t)R, (uint32_t)C});
    auto ct = make_device_tensor<float>({(uint32_t)R, (uint32_t)C});
    NetworkInstance net;
    net.set_model(std::move(m));
    net.set_input("x", *xt);
    net.set_output("d", *dt);
    net.set_output("cf", *ct);
    net.forward();
    auto d = download<float>(*dt), cf = download<float>(*ct);
    std::vector<uint8_t> q(x.size());
    std::vector<float> dref(x.size());
    orc_quantize(x.data(), q.data(), R, C, 1, s.data());
    orc_dequantize(q.data(), dref.data(), R, C, 1, s.data());
    size_t bad = 0;
    for (size_t i = 0; i < x.size(); ++i) {
        bool same = std::isnan(dref[i]) ? std::isnan(d[i]) : std::memcmp(&d[i], &dref[i], 4) == 0;
        float cr = orc_e4m3_to_float(orc_e4m3_from_float(x[i]));
        bool same2 = std::isnan(cr) ? std::isnan(cf[i]) : std::memcmp(&cf[i], &cr, 4) == 0;
        bad += !same + !same2;
    }
    CHECK(bad == 0);
}

static void test_errors() {
    std::printf("[6] error behaviour\n");
    Graph g("e");
    Blob blob;
    std::vector<uint8_t> w(10, 1);
    float s = 1.0f;
    var(g, "x", DataType::FLOAT, {2, 5});
    // FP8 blob range of 10 bytes for 10 elements violates the ((n+3)/4)*4 rule
    auto [st, en] = blob.add(w.data(), 10, 10);
    g.add_variable(Variable("W", DataType::FLOAT8E4M3FN, {5, 2}, {}, st, en));
    raw_var(g, "s", DataType::FLOAT, {1}, &s, 4);
    var(g, "Wf", DataType::FLOAT, {5, 2});
    var(g, "y", DataType::FLOAT, {2, 2});
    node(g, "DequantizeLinear", {"W", "s"}, {"Wf"});
    node(g, "MatMul", {"x", "Wf"}, {"y"});
    g.add_input("x");
    g.add_output("y");
    Model m(10, "test", "1");
    m.set_graph(std::move(g));
    DeviceBuffer wb(16);
    auto xt = make_device_tensor<float>({2, 5});
    auto bad_y = make_device_tensor<FP8E4M3FN>({2, 2});
    auto yt = make_device_tensor<float>({2, 2});
    {
        NetworkInstance net;
        Model mm = Model::load_from_json(R"({"graph": {"input": [{"name": "x", "type": {"tensor_type": {"elem_type": "FLOAT", "shape": {"dim": [{"dim_value": "2"}, {"dim_value": "5"}]}}}}], "output": [{"name": "y", "type": {"tensor_type": {"elem_type": "FLOAT", "shape": {"dim": [{"dim_value": "2"}, {"dim_value": "5"}]}}}}], "node": [{"op_type": "Relu", "input": ["x"], "output": ["y"]}]}})");
        net.set_model(std::move(mm));
        net.set_input("x", *xt);
        net.set_output("y", *bad_y);  // FP8 tensor bound to a FLOAT output
        CHECK(throws([&] { net.forward(); }));
    }
    NetworkInstance net;
    net.set_model(std::move(m));
    net.set_fusion(false);
    net.set_weight_buffer(wb.data(), 16);
    net.set_input("x", *xt);
    net.set_output("y", *yt);
    CHECK(throws([&] { net.forward(); }));  // Weight buffer size mismatch
    // blocked quantisation (opset 21 block_size) is rejected, not silently run per-axis
    for (const char *op : {"QuantizeLinear", "DequantizeLinear"}) {
        bool q = op[0] == 'Q';
        Graph gb("b");
        var(gb, "x", q ? DataType::FLOAT : DataType::FLOAT8E4M3FN, {2, 64});
        raw_var(gb, "s", DataType::FLOAT, {2, 2}, std::vector<float>(4, 1.0f).data(), 16);
        var(gb, "y", q ? DataType::FLOAT8E4M3FN : DataType::FLOAT, {2, 64});
        node(gb, op, {"x", "s"}, {"y"}, {Attribute{"axis", (int32_t)1}, Attribute{"block_size", (int32_t)32}});
        gb.add_input("x");
        gb.add_output("y");
        Model mb(21, "test", "1");
        mb.set_graph(std::move(gb));
        auto xb = q ? make_device_tensor<float>({2, 64}) : nullptr;
        auto xq = q ? nullptr : make_device_tensor<FP8E4M3FN>({2, 64});
        auto yq = q ? make_device_tensor<FP8E4M3FN>({2, 64}) : nullptr;
        auto yb = q ? nullptr : make_device_tensor<float>({2, 64});
        CHECK(throws([&] {
            NetworkInstance nb;
            nb.set_model(std::move(mb));
            if (q) nb.set_input("x", *xb), nb.set_output("y", *yq);
            else nb.set_input("x", *xq), nb.set_output("y", *yb);
            nb.forward();
        }));
    }
}

static bool same_f32(float a, float b) { return std::isnan(b) ? std::isnan(a) : std::memcmp(&a, &b, 4) == 0; }

static void test_e5m2_qdq_cast() {
    std::printf("[9] E5M2 QuantizeLinear / DequantizeLinear, Cast chains, E5M2 weight blob (bit-exact)\n");
    const int R = 6, C = 37;
    auto x = normals(91, (size_t)R * C, 3000.0f);
    x[3] = INFINITY;
    x[4] = -INFINITY;
    x[5] = NAN;
    x[6] = -0.0f;
    x[7] = 2e5f;
    std::vector<float> s(C);
    for (int c = 0; c < C; ++c) s[c] = 0.5f + 0.01f * c;
    std::vector<uint8_t> w(7);  // an E5M2 constant of 7 elements in the blob: padded to 8 bytes
    for (int i = 0; i < 7; ++i) w[i] = (uint8_t)(0x30 + 5 * i);
    Blob blob;
    Graph g("e5");
    var(g, "x", DataType::FLOAT, {(size_t)R, (size_t)C});
    raw_var(g, "s", DataType::FLOAT, {(size_t)C}, s.data(), C * 4);
    var(g, "q1", DataType::FLOAT8E5M2, {(size_t)R, (size_t)C});
    var(g, "q0", DataType::FLOAT8E5M2, {(size_t)R, (size_t)C});
    var(g, "d1", DataType::FLOAT, {(size_t)R, (size_t)C});
    var(g, "c5", DataType::FLOAT8E5M2, {(size_t)R, (size_t)C});
    var(g, "c4", DataType::FLOAT8E4M3FN, {(size_t)R, (size_t)C});
    var(g, "cf", DataType::FLOAT, {(size_t)R, (size_t)C});
    blob_var(g, blob, "w", DataType::FLOAT8E5M2, {7}, w.data(), 7);
    var(g, "wf", DataType::FLOAT, {7});
    node(g, "QuantizeLinear", {"x", "s"}, {"q1"}, {Attribute{"axis", (int32_t)1}});
    node(g, "QuantizeLinear", {"x", "s"}, {"q0"}, {Attribute{"axis", (int32_t)1}, Attribute{"saturate", (int32_t)0}});
    node(g, "DequantizeLinear", {"q1", "s"}, {"d1"}, {Attribute{"axis", (int32_t)1}});
    node(g, "Cast", {"x"}, {"c5"}, {Attribute{"to", (int32_t)19}});
    node(g, "Cast", {"c5"}, {"c4"}, {Attribute{"to", (int32_t)17}});
    node(g, "Cast", {"c4"}, {"cf"}, {Attribute{"to", (int32_t)1}});
    node(g, "Cast", {"w"}, {"wf"}, {Attribute{"to", (int32_t)1}});
    g.add_input("x");
    for (const char *o : {"q1", "q0", "d1", "cf", "wf"}) g.add_output(o);
    Model m(10, "test", "1");
    m.set_graph(std::move(g));
    DeviceBuffer wb(blob.bytes.size());
    CHECK(hipMemcpy(wb.data(), blob.bytes.data(), blob.bytes.size(), hipMemcpyHostToDevice) == hipSuccess);
    auto xt = upload(x, {(uint32_t)R, (uint32_t)C});
    auto q1t = make_device_tensor<FP8E5M2>({(uint32_t)R, (uint32_t)C});
    auto q0t = make_device_tensor<FP8E5M2>({(uint32_t)R, (uint32_t)C});
    auto d1t = make_device_tensor<float>({(uint32_t)R, (uint32_t)C});
    auto cft = make_device_tensor<float>({(uint32_t)R, (uint32_t)C});
    auto wft = make_device_tensor<float>({7});
    NetworkInstance net;
    net.set_model(std::move(m));
    net.set_weight_buffer(static_cast<uint8_t *>(wb.data()), blob.bytes.size());
    net.set_input("x", *xt);
    net.set_output("q1", *q1t);
    net.set_output("q0", *q0t);
    net.set_output("d1", *d1t);
    net.set_output("cf", *cft);
    net.set_output("wf", *wft);
    net.forward();
    auto q1 = download<FP8E5M2>(*q1t), q0 = download<FP8E5M2>(*q0t);
    auto d1 = download<float>(*d1t), cf = download<float>(*cft), wf = download<float>(*wft);
    std::vector<uint8_t> r1(x.size()), r0(x.size());
    std::vector<float> rd(x.size());
    orc_quantize_e5m2(x.data(), r1.data(), R, C, 1, s.data(), 1);
    orc_quantize_e5m2(x.data(), r0.data(), R, C, 1, s.data(), 0);
    orc_dequantize_e5m2(r1.data(), rd.data(), R, C, 1, s.data());
    size_t bad = 0;
    for (size_t i = 0; i < x.size(); ++i) {
        bad += q1[i].bits != r1[i];
        bad += q0[i].bits != r0[i];
        bad += !same_f32(d1[i], rd[i]);
        bad += !same_f32(cf[i], orc_e4m3_to_float(orc_e4m3_from_float(orc_e5m2_to_float(orc_e5m2_from_float(x[i])))));
    }
    for (int i = 0; i < 7; ++i) bad += !same_f32(wf[i], orc_e5m2_to_float(w[i]));
    CHECK(bad == 0);
    CHECK(q0[3].bits == 0x7c && q1[3].bits == 0x7b);  // inf: kept by saturate=0, clamped by saturate=1
}

static void test_elementwise() {
    std::printf("[10] Add / Sub / Mul / Div on FLOAT, E4M3, E5M2 with broadcasting; DQL zero point\n");
    const char *ops[4] = {"Add", "Sub", "Mul", "Div"};
    uint64_t seed = 1;
    size_t bad = 0;
    for (int op = 0; op < 4; ++op) {
        for (DataType dt : {DataType::FLOAT, DataType::FLOAT8E4M3FN, DataType::FLOAT8E5M2}) {
            // a [3, 4, 5] with b [4, 1]: y [3, 4, 5]
            const std::vector<int64_t> sa = {3, 4, 5}, sb = {4, 1}, sy = {3, 4, 5};
            Graph g("ew");
            var(g, "a", dt, {3, 4, 5});
            var(g, "b", dt, {4, 1});
            var(g, "y", dt, {3, 4, 5});
            node(g, ops[op], {"a", "b"}, {"y"});
            g.add_input("a");
            g.add_input("b");
            g.add_output("y");
            Model m(10, "test", "1");
            m.set_graph(std::move(g));
            NetworkInstance net;
            net.set_model(std::move(m));
            const int code = (int)dt;
            if (dt == DataType::FLOAT) {
                auto a = normals(seed++, 60, 1.0f), b = normals(seed++, 4, 1.0f);
                b[1] = 0.0f;
                auto at = upload(a, {3, 4, 5});
                auto bt = upload(b, {4, 1});
                auto yt = make_device_tensor<float>({3, 4, 5});
                net.set_input("a", *at);
                net.set_input("b", *bt);
                net.set_output("y", *yt);
                net.forward();
                auto y = download<float>(*yt);
                std::vector<float> r(60);
                orc_fp8_binary(op, code, a.data(), sa.data(), 3, b.data(), sb.data(), 2, r.data(), sy.data(), 3);
                for (int i = 0; i < 60; ++i) bad += !same_f32(y[i], r[i]);
            } else {
                std::vector<uint8_t> a(60), b(4);
                for (int i = 0; i < 60; ++i) a[i] = (uint8_t)((i * 37 + op * 11 + seed) & 0xff);
                for (int i = 0; i < 4; ++i) b[i] = (uint8_t)((i * 101 + 7 * op) & 0xff);
                ++seed;
                auto run = [&]<typename T>() {
                    std::vector<T> ah(60), bh(4);
                    for (int i = 0; i < 60; ++i) ah[i].bits = a[i];
                    for (int i = 0; i < 4; ++i) bh[i].bits = b[i];
                    auto at = upload(ah, {3, 4, 5});
                    auto bt = upload(bh, {4, 1});
                    auto yt = make_device_tensor<T>({3, 4, 5});
                    net.set_input("a", *at);
                    net.set_input("b", *bt);
                    net.set_output("y", *yt);
                    net.forward();
                    auto y = download<T>(*yt);
                    std::vector<uint8_t> r(60);
                    orc_fp8_binary(op, code, a.data(), sa.data(), 3, b.data(), sb.data(), 2, r.data(), sy.data(), 3);
                    for (int i = 0; i < 60; ++i) bad += y[i].bits != r[i];
                };
                if (dt == DataType::FLOAT8E4M3FN) run.template operator()<FP8E4M3FN>();
                else run.template operator()<FP8E5M2>();
            }
        }
    }
    CHECK(bad == 0);
    // DynamicQuantizeLinear's y_zero_point output is written as 0
    Graph g("dq");
    var(g, "x", DataType::FLOAT, {2, 8});
    var(g, "y", DataType::FLOAT8E4M3FN, {2, 8});
    var(g, "s", DataType::FLOAT, {1});
    var(g, "z", DataType::FLOAT8E4M3FN, {1});
    node(g, "DynamicQuantizeLinear", {"x"}, {"y", "s", "z"});
    g.add_input("x");
    g.add_output("z");
    Model m(10, "test", "1");
    m.set_graph(std::move(g));
    auto xt = upload(normals(77, 16, 1.0f), {2, 8});
    auto zt = make_device_tensor<FP8E4M3FN>({1});
    std::vector<FP8E4M3FN> junk(1);
    junk[0].bits = 0x55;
    CHECK(hipMemcpy(zt->device_data(), junk.data(), 1, hipMemcpyHostToDevice) == hipSuccess);
    NetworkInstance net;
    net.set_model(std::move(m));
    net.set_input("x", *xt);
    net.set_output("z", *zt);
    net.forward();
    CHECK(download<FP8E4M3FN>(*zt)[0].bits == 0);
}

static void test_memory_planner() {
    std::printf("[11] intermediates in one planned arena vs one allocation each\n");
    const uint32_t R = 64, C = 1024;
    auto build = []() {
        Graph g("plan");
        const std::vector<size_t> sh = {64, 1024};
        var(g, "x", DataType::FLOAT, sh);
        float s = 0.05f;
        raw_var(g, "s", DataType::FLOAT, {1}, &s, 4);
        for (const char *n : {"a", "b", "d", "e", "f", "h", "y"}) var(g, n, DataType::FLOAT, sh);
        var(g, "q", DataType::FLOAT8E4M3FN, sh);
        var(g, "q5", DataType::FLOAT8E5M2, sh);
        node(g, "Add", {"x", "x"}, {"a"});
        node(g, "Mul", {"a", "x"}, {"b"});
        node(g, "QuantizeLinear", {"b", "s"}, {"q"});
        node(g, "DequantizeLinear", {"q", "s"}, {"d"});
        node(g, "Sub", {"d", "x"}, {"e"});
        node(g, "Relu", {"e"}, {"f"});
        node(g, "QuantizeLinear", {"f", "s"}, {"q5"});
        node(g, "DequantizeLinear", {"q5", "s"}, {"h"});
        node(g, "Add", {"h", "a"}, {"y"});  // a stays live across the whole graph
        g.add_input("x");
        g.add_output("y");
        Model m(10, "test", "1");
        m.set_graph(std::move(g));
        return m;
    };
    auto xt = upload(normals(111, (size_t)R * C, 1.0f), {R, C});
    std::vector<float> y[2];
    size_t arena = 0, unshared = 0, planned = 0;
    for (int mode = 0; mode < 2; ++mode) {
        auto yt = make_device_tensor<float>({R, C});
        NetworkInstance net;
        net.set_model(build());
        net.set_memory_planning(mode == 0);
        net.set_input("x", *xt);
        net.set_output("y", *yt);
        net.forward();
        net.forward();  // a second pass over the same arena
        y[mode] = download<float>(*yt);
        if (mode == 0) {
            arena = net.memory_plan().arena_bytes;
            unshared = net.memory_plan().unshared_bytes;
            planned = net.planned_intermediates();
        } else {
            CHECK(net.planned_intermediates() == 0);
        }
    }
    CHECK(planned == 8);
    CHECK(std::memcmp(y[0].data(), y[1].data(), y[0].size() * 4) == 0);
    // a is live throughout; the others chain: three fp32 slots (a plus two
    // alternating) hold every fp32 intermediate, the fp8 ones fit beside them
    std::printf("    arena %zu bytes for %zu bytes of intermediates\n", arena, unshared);
    CHECK(arena < unshared && arena <= (size_t)3 * R * C * 4 + (size_t)R * C);
}

// fp32 MatMul with numpy semantics (mat_mul.cpp:187-303): 1-D operands and
// right-aligned batch dimensions broadcast where they are 1; every output
// batch against the oracle's GEMM of the matching A and B slices.
// MatMul against a batched E4M3 weight [..., K, N] through DequantizeLinear
// (per-tensor or per-output-channel scale on the last axis), with a dynamic
// QDQ, a static QDQ or an fp32 activation: fused into one FP8Linear (one
// packed weight per batch, batch dimensions broadcast as mat_mul.cpp:187-303)
// and op by op, both against the oracle's per-batch Gemm of the dequantised
// operands.
static void test_batched_fp8_matmul(bool fused) {
    std::printf("[18] MatMul with a batched E4M3 weight, dynamic / static / fp32 activation (%s)\n",
                fused ? "fused" : "unfused");
    struct Case {
        std::vector<size_t> a, w, y;
        bool per_channel;
    };
    const size_t M = 5, K = 64, N = 48;
    const Case cases[] = {{{2, 3, M, K}, {3, K, N}, {2, 3, M, N}, true},
                          {{M, K}, {2, K, N}, {2, M, N}, false},
                          {{2, 1, M, K}, {1, 3, K, N}, {2, 3, M, N}, true}};
    auto count = [](const std::vector<size_t> &v) {
        size_t n = 1;
        for (size_t d : v) n *= d;
        return n;
    };
    int ci = 0;
    for (const Case &c : cases) {
        for (int mode = 0; mode < 3; ++mode) {  // 0: fp32 A, 1: static QDQ, 2: dynamic QDQ
            const size_t na = count(c.a), nw = count(c.w), wb = nw / (K * N);
            auto x = normals(300 + 10 * ci + mode, na, 1.0f), w = normals(400 + ci, nw, 0.05f);
            std::vector<float> sw(c.per_channel ? N : 1, 0.0f);
            for (size_t i = 0; i < nw; ++i) {
                float &m = sw[c.per_channel ? i % N : 0];
                m = std::max(m, std::fabs(w[i]));
            }
            for (auto &v : sw) v = orc_scale_from_amax(v);
            std::vector<uint8_t> qw(nw), zp(1, 0);
            if (c.per_channel)
                orc_quantize(w.data(), qw.data(), nw / N, N, 1, sw.data());  // axis = last
            else
                orc_quantize(w.data(), qw.data(), 1, 1, nw, sw.data());
            float sx = orc_scale_from_amax(orc_amax(x.data(), na));
            Graph g("bmm");
            Blob blob;
            var(g, "x", DataType::FLOAT, c.a);
            blob_var(g, blob, "W", DataType::FLOAT8E4M3FN, c.w, qw.data(), qw.size());
            blob_var(g, blob, "sw", DataType::FLOAT, {sw.size()}, sw.data(), sw.size() * 4);
            var(g, "Wf", DataType::FLOAT, c.w);
            var(g, "y", DataType::FLOAT, c.y);
            std::string a_in = "x";
            if (mode == 1) {
                raw_var(g, "sx", DataType::FLOAT, {1}, &sx, 4);
                raw_var(g, "zx", DataType::FLOAT8E4M3FN, {1}, zp.data(), 1);
                var(g, "xq", DataType::FLOAT8E4M3FN, c.a);
                var(g, "xd", DataType::FLOAT, c.a);
                node(g, "QuantizeLinear", {"x", "sx", "zx"}, {"xq"});
                node(g, "DequantizeLinear", {"xq", "sx", "zx"}, {"xd"});
                a_in = "xd";
            } else if (mode == 2) {
                var(g, "xq", DataType::FLOAT8E4M3FN, c.a);
                var(g, "xs", DataType::FLOAT, {1});
                var(g, "xz", DataType::FLOAT8E4M3FN, {1});
                var(g, "xd", DataType::FLOAT, c.a);
                node(g, "DynamicQuantizeLinear", {"x"}, {"xq", "xs", "xz"});
                node(g, "DequantizeLinear", {"xq", "xs", "xz"}, {"xd"});
                a_in = "xd";
            }
            if (c.per_channel)
                node(g, "DequantizeLinear", {"W", "sw"}, {"Wf"}, {Attribute{"axis", (int32_t)(c.w.size() - 1)}});
            else
                node(g, "DequantizeLinear", {"W", "sw"}, {"Wf"});
            node(g, "MatMul", {a_in, "Wf"}, {"y"});
            g.add_input("x");
            g.add_output("y");
            Model m(10, "test", "1");
            m.set_graph(std::move(g));
            DeviceBuffer wbuf(blob.bytes.size());
            CHECK(hipMemcpy(wbuf.data(), blob.bytes.data(), blob.bytes.size(), hipMemcpyHostToDevice) == hipSuccess);
            ITensor::shape_type as(c.a.begin(), c.a.end()), ys(c.y.begin(), c.y.end());
            auto xt = upload(x, as);
            auto yt = make_device_tensor<float>(ys);
            NetworkInstance net;
            net.set_model(std::move(m));
            net.set_fusion(fused);
            net.set_weight_buffer(wbuf.data(), blob.bytes.size());
            net.set_input("x", *xt);
            net.set_output("y", *yt);
            net.forward();
            auto y = download<float>(*yt);
            if (fused)
                CHECK(net.fused_linear_count() == 1 && net.executed_op_types() == std::vector<std::string>{"FP8Linear"});
            else
                CHECK(net.fused_linear_count() == 0);
            // oracle: the activation as the graph sees it, the dequantised weight, one Gemm per output batch
            std::vector<float> A(x), Bw(nw);
            if (mode != 0) {
                std::vector<uint8_t> qx(na);
                orc_quantize(x.data(), qx.data(), 1, 1, na, &sx);
                orc_dequantize(qx.data(), A.data(), 1, 1, na, &sx);
            }
            if (c.per_channel)
                orc_dequantize(qw.data(), Bw.data(), nw / N, N, 1, sw.data());
            else
                orc_dequantize(qw.data(), Bw.data(), 1, 1, nw, sw.data());
            std::vector<size_t> ab(c.a.begin(), c.a.end() - 2), bb(c.w.begin(), c.w.end() - 2);
            const size_t nb = std::max(ab.size(), bb.size());
            ab.insert(ab.begin(), nb - ab.size(), 1);
            bb.insert(bb.begin(), nb - bb.size(), 1);
            std::vector<size_t> yb(nb);
            size_t batches = 1;
            for (size_t d = 0; d < nb; ++d) batches *= (yb[d] = std::max(ab[d], bb[d]));
            CHECK(y.size() == batches * M * N && wb >= 1);
            std::vector<float> ref(y.size());
            std::vector<double> bound(y.size());
            for (size_t t = 0; t < batches; ++t) {
                size_t rem = t, ai = 0, bi = 0, am = 1, bm = 1;
                for (size_t d = nb; d-- > 0;) {
                    const size_t coord = rem % yb[d];
                    rem /= yb[d];
                    ai += (ab[d] == 1 ? 0 : coord) * am;
                    bi += (bb[d] == 1 ? 0 : coord) * bm;
                    am *= ab[d];
                    bm *= bb[d];
                }
                orc_gemm(M, N, K, A.data() + ai * M * K, 0, Bw.data() + bi * K * N, 0, 1.0f, 0.0f, nullptr, -1, 0, 0,
                         0, ref.data() + t * M * N);
                orc_gemm_abs_bound(M, N, K, A.data() + ai * M * K, 0, Bw.data() + bi * K * N, 0, 1.0f, 0.0f, nullptr,
                                   -1, 0, 0, bound.data() + t * M * N);
            }
            char what[64];
            std::snprintf(what, sizeof what, "batched fp8 matmul case %d mode %d", ci, mode);
            CHECK(close(y, ref, bound, 1e-4, 0.0, what));
        }
        ++ci;
    }
}

static void test_batched_matmul() {
    std::printf("[12] fp32 MatMul: batched, broadcast and 1-D operands\n");
    struct Case {
        std::vector<size_t> a, b, y;
    };
    const Case cases[] = {{{2, 3, 5, 7}, {3, 7, 4}, {2, 3, 5, 4}}, {{5, 8}, {2, 1, 8, 6}, {2, 1, 5, 6}},
                          {{7}, {3, 7, 4}, {3, 4}},                 {{2, 1, 5, 7}, {1, 3, 7, 4}, {2, 3, 5, 4}},
                          {{2, 5, 7}, {7}, {2, 5}},                  {{4, 9}, {9, 3}, {4, 3}}};
    int ci = 0;
    for (const Case &c : cases) {
        auto count = [](const std::vector<size_t> &v) {
            size_t n = 1;
            for (size_t d : v) n *= d;
            return n;
        };
        auto x = normals(120 + ci, count(c.a), 1.0f), w = normals(130 + ci, count(c.b), 1.0f);
        ++ci;
        Graph g("mm");
        Blob blob;
        var(g, "a", DataType::FLOAT, c.a);
        blob_var(g, blob, "B", DataType::FLOAT, c.b, w.data(), w.size() * 4);
        var(g, "y", DataType::FLOAT, c.y);
        node(g, "MatMul", {"a", "B"}, {"y"});
        g.add_input("a");
        g.add_output("y");
        Model m(10, "test", "1");
        m.set_graph(std::move(g));
        DeviceBuffer wb(blob.bytes.size());
        CHECK(hipMemcpy(wb.data(), blob.bytes.data(), blob.bytes.size(), hipMemcpyHostToDevice) == hipSuccess);
        ITensor::shape_type as(c.a.begin(), c.a.end()), ys(c.y.begin(), c.y.end());
        auto at = upload(x, as);
        auto yt = make_device_tensor<float>(ys);
        NetworkInstance net;
        net.set_model(std::move(m));
        net.set_weight_buffer(wb.data(), blob.bytes.size());
        net.set_input("a", *at);
        net.set_output("y", *yt);
        net.forward();
        auto y = download<float>(*yt);
        // reference: treat 1-D A as [1, K] and 1-D B as [K, 1]; pad batch dims on the left with 1
        const size_t K = c.a.back(), M = c.a.size() >= 2 ? c.a[c.a.size() - 2] : 1;
        const size_t N = c.b.size() >= 2 ? c.b.back() : 1;
        std::vector<size_t> ab(c.a.begin(), c.a.size() >= 2 ? c.a.end() - 2 : c.a.begin());
        std::vector<size_t> bb(c.b.begin(), c.b.size() >= 2 ? c.b.end() - 2 : c.b.begin());
        const size_t nb = std::max(ab.size(), bb.size());
        ab.insert(ab.begin(), nb - ab.size(), 1);
        bb.insert(bb.begin(), nb - bb.size(), 1);
        std::vector<size_t> yb(nb);
        size_t batches = 1;
        for (size_t d = 0; d < nb; ++d) batches *= (yb[d] = std::max(ab[d], bb[d]));
        CHECK(y.size() == batches * M * N);
        std::vector<float> ref(y.size());
        std::vector<double> bound(y.size());
        for (size_t t = 0; t < batches; ++t) {
            size_t rem = t, ai = 0, bi = 0, am = 1, bm = 1;
            for (size_t d = nb; d-- > 0;) {
                const size_t coord = rem % yb[d];
                rem /= yb[d];
                ai += (ab[d] == 1 ? 0 : coord) * am;
                bi += (bb[d] == 1 ? 0 : coord) * bm;
                am *= ab[d];
                bm *= bb[d];
            }
            orc_gemm(M, N, K, x.data() + ai * M * K, 0, w.data() + bi * K * N, 0, 1.0f, 0.0f, nullptr, -1, 0, 0, 0,
                     ref.data() + t * M * N);
            orc_gemm_abs_bound(M, N, K, x.data() + ai * M * K, 0, w.data() + bi * K * N, 0, 1.0f, 0.0f, nullptr, -1,
                               0, 0, bound.data() + t * M * N);
        }
        CHECK(close(y, ref, bound, 1e-5, 0.0, "batched matmul"));
    }
}

// Conv on fp8 tensors (the reference accepts FLOAT8E4M3FN / FLOAT8E5M2 X, W,
// B, Y: conv.cpp:65-105): Cast(x) -> Conv(x8, W8, B8) -> y8 -> Cast(float),
// against the oracle's fp32 conv of the decoded operands, encoded with the
// same CPU encoder.  Codes agree except, rarely, one step apart where the
// fp32 value sits next to a rounding midpoint and the summation orders
// differ in the last bit.
static void test_fp8_tensor_conv(bool e5m2) {
    std::printf("[13] Conv on %s tensors (decode, fp32 conv, encode)\n", e5m2 ? "FLOAT8E5M2" : "FLOAT8E4M3FN");
    const int64_t Nb = 2, C = 8, H = 9, W = 7, CO = 6, KH = 3, KW = 3, G = 2;
    const int64_t OH = H, OW = W;  // stride 1, pad 1
    const DataType dt = e5m2 ? DataType::FLOAT8E5M2 : DataType::FLOAT8E4M3FN;
    auto enc = [&](float v) { return e5m2 ? orc_e5m2_from_float(v) : orc_e4m3_from_float(v); };
    auto dec = [&](uint8_t c) { return e5m2 ? orc_e5m2_to_float(c) : orc_e4m3_to_float(c); };
    auto x = normals(140 + e5m2, (size_t)(Nb * C * H * W), 2.0f);
    auto wf = normals(142 + e5m2, (size_t)(CO * (C / G) * KH * KW), 0.5f);
    auto bf = normals(144 + e5m2, (size_t)CO, 0.5f);
    std::vector<uint8_t> w8(wf.size()), b8(bf.size());
    for (size_t i = 0; i < wf.size(); ++i) w8[i] = enc(wf[i]);
    for (size_t i = 0; i < bf.size(); ++i) b8[i] = enc(bf[i]);
    Graph g("conv8");
    Blob blob;
    var(g, "x", DataType::FLOAT, {(size_t)Nb, (size_t)C, (size_t)H, (size_t)W});
    var(g, "x8", dt, {(size_t)Nb, (size_t)C, (size_t)H, (size_t)W});
    blob_var(g, blob, "W8", dt, {(size_t)CO, (size_t)(C / G), (size_t)KH, (size_t)KW}, w8.data(), w8.size());
    blob_var(g, blob, "B8", dt, {(size_t)CO}, b8.data(), b8.size());
    var(g, "y8", dt, {(size_t)Nb, (size_t)CO, (size_t)OH, (size_t)OW});
    var(g, "y", DataType::FLOAT, {(size_t)Nb, (size_t)CO, (size_t)OH, (size_t)OW});
    node(g, "Cast", {"x"}, {"x8"}, {Attribute{"to", (int32_t)(e5m2 ? 19 : 17)}});
    node(g, "Conv", {"x8", "W8", "B8"}, {"y8"},
         {Attribute{"group", (int32_t)G}, Attribute{"pads", std::vector<int32_t>{1, 1, 1, 1}}});
    node(g, "Cast", {"y8"}, {"y"}, {Attribute{"to", (int32_t)1}});
    g.add_input("x");
    g.add_output("y");
    Model m(10, "test", "1");
    m.set_graph(std::move(g));
    DeviceBuffer wb(blob.bytes.size());
    CHECK(hipMemcpy(wb.data(), blob.bytes.data(), blob.bytes.size(), hipMemcpyHostToDevice) == hipSuccess);
    auto xt = upload(x, {(uint32_t)Nb, (uint32_t)C, (uint32_t)H, (uint32_t)W});
    auto yt = make_device_tensor<float>({(uint32_t)Nb, (uint32_t)CO, (uint32_t)OH, (uint32_t)OW});
    NetworkInstance net;
    net.set_model(std::move(m));
    net.set_weight_buffer(wb.data(), blob.bytes.size());
    net.set_input("x", *xt);
    net.set_output("y", *yt);
    net.forward();
    auto y = download<float>(*yt);
    std::vector<float> xd(x.size()), wd(wf.size()), bd(bf.size()), ref(y.size());
    for (size_t i = 0; i < x.size(); ++i) xd[i] = dec(enc(x[i]));
    for (size_t i = 0; i < wf.size(); ++i) wd[i] = dec(w8[i]);
    for (size_t i = 0; i < bf.size(); ++i) bd[i] = dec(b8[i]);
    orc_conv2d(xd.data(), wd.data(), bd.data(), ref.data(), Nb, C, H, W, CO, KH, KW, 1, 1, 1, 1, 1, 1, G, OH, OW,
               LCML_ACT_NONE);
    size_t exact = 0, near = 0, far = 0;
    for (size_t i = 0; i < y.size(); ++i) {
        const uint8_t want = enc(ref[i]), got = enc(y[i]);  // y holds decoded codes: re-encoding is exact
        if (want == got) {
            ++exact;
        } else if ((want & 0x80) == (got & 0x80) && std::abs((int)(want & 0x7f) - (int)(got & 0x7f)) == 1) {
            ++near;
        } else {
            ++far;
        }
    }
    std::printf("    %zu codes equal, %zu one step apart, %zu further\n", exact, near, far);
    CHECK(far == 0 && near * 200 <= y.size());
}

// Runs `m` on one fp32 input and returns the fp32 output (fusion on or off).
static std::vector<float> run_model(Model &&m, const void *blob, size_t blob_bytes, const std::string &in,
                                    const std::vector<float> &x, ITensor::shape_type xs, const std::string &out,
                                    ITensor::shape_type ys, bool fused, std::vector<std::string> *types = nullptr,
                                    size_t *fused_count = nullptr) {
    auto xt = upload(x, xs);
    auto yt = make_device_tensor<float>(ys);
    NetworkInstance net;
    net.set_model(std::move(m));
    net.set_fusion(fused);
    if (blob) net.set_weight_buffer(blob, blob_bytes);
    net.set_input(in, *xt);
    net.set_output(out, *yt);
    net.forward();
    if (types) *types = net.executed_op_types();
    if (fused_count) *fused_count = net.fused_linear_count();
    return download<float>(*yt);
}

static bool all_ops(const std::vector<std::string> &t, const char *op, size_t n) {
    return t.size() == n && std::all_of(t.begin(), t.end(), [&](const std::string &x) { return x == op; });
}

// The FP8 QDQ MLP model file written by tests/golden/write_fp8_mlp.cpp
// (ONNX-JSON + weight blob, E4M3 weights and zero points in the blob, 4-byte
// padded), loaded from disk and run fused (3 FP8Linear nodes: the blob zero
// points are recognised as zero) and op by op, against the oracle output
// stored with it; the tolerance is carried through the chain as in [2]
// (layer_tolerance).
static void test_fp8_mlp_from_file(const std::string &golden, bool fused) {
    std::printf("[12] FP8 QDQ MLP model file (fp8_mlp.onnx.json + blob), %s\n", fused ? "fused" : "op by op");
    std::string blob = read_text(golden + "/fp8_mlp.bin");
    std::string xin = read_text(golden + "/fp8_mlp_input.bin"), yref = read_text(golden + "/fp8_mlp_output.bin");
    CHECK(xin.size() == 64 * 784 * 4 && yref.size() == 64 * 10 * 4);
    Model m = Model::load_from_json(read_text(golden + "/fp8_mlp.onnx.json"));
    // host-side oracle chain for the bound: weights decoded from the blob
    const Graph &g = m.get_graph();
    const int dims[4] = {784, 256, 128, 10};
    std::vector<float> x(64 * 784), want(64 * 10);
    std::memcpy(x.data(), xin.data(), xin.size());
    std::memcpy(want.data(), yref.data(), yref.size());
    std::vector<float> h = x;
    std::vector<double> tol;
    for (int l = 0; l < 3; ++l) {
        const int K = dims[l], N = dims[l + 1];
        const std::string L = std::to_string(l);
        auto [ws, we] = g.get_var("net." + L + ".weight").get_buffer_range();
        auto [ss, se] = g.get_var("net." + L + ".weight_scale").get_buffer_range();
        auto [bs, be] = g.get_var("net." + L + ".bias").get_buffer_range();
        CHECK(we - ws == ((size_t)N * K + 3) / 4 * 4 && ws % 4 == 0 && se - ss == 4 && be - bs == (size_t)N * 4);
        float sc;
        std::memcpy(&sc, blob.data() + ss, 4);
        std::vector<float> wdq((size_t)N * K), b(N), out((size_t)64 * N);
        orc_dequantize(reinterpret_cast<const uint8_t *>(blob.data() + ws), wdq.data(), 1, 1, (int64_t)wdq.size(), &sc);
        std::memcpy(b.data(), blob.data() + bs, (size_t)N * 4);
        tol = layer_tolerance(64, K, N, h, wdq.data(), b.data(), tol);
        orc_gemm(64, N, K, h.data(), 0, wdq.data(), 1, 1.0f, 1.0f, b.data(), 1, N, 0, l < 2 ? 1 : 0, out.data());
        h = std::move(out);
    }
    CHECK(std::memcmp(h.data(), want.data(), want.size() * 4) == 0);  // the stored output is the oracle's
    DeviceBuffer wb(blob.size());
    CHECK(hipMemcpy(wb.data(), blob.data(), blob.size(), hipMemcpyHostToDevice) == hipSuccess);
    std::vector<std::string> types;
    size_t nf = 0;
    auto y = run_model(std::move(m), wb.data(), blob.size(), "input", x, {64, 784}, "output", {64, 10}, fused, &types,
                       &nf);
    if (fused) CHECK(nf == 3 && all_ops(types, "FP8Linear", 3));
    else CHECK(nf == 0 && types.size() == 8);
    CHECK(close(y, want, tol, 1.0, 0.0, "fp8 mlp from file"));
}

// An E5M2 activation Q -> DQ in front of a DQ(E4M3 weight) Gemm: the fused
// kernels quantise to E4M3, so the activation pair stays op by op (E5M2
// codes) and only the weight side fuses (W8A32 on the dequantised E5M2
// values); the result equals the unfused graph's within the GEMM bound.
static void test_e5m2_activation_stays_unfused() {
    std::printf("[13] E5M2 activation QDQ -> Gemm(DQ(E4M3 W)): activation pair not fused\n");
    const int M = 32, K = 256, N = 96;
    auto x = normals(131, (size_t)M * K, 1.0f), w = normals(132, (size_t)N * K, 0.05f);
    float sx = 0.01f, sw = orc_scale_from_amax(orc_amax(w.data(), w.size()));
    std::vector<uint8_t> qw(w.size()), z8(1, 0);
    orc_quantize(w.data(), qw.data(), 1, 1, (int64_t)qw.size(), &sw);
    auto build = [&]() {
        Graph g("e5m2act");
        var(g, "x", DataType::FLOAT, {(size_t)M, (size_t)K});
        raw_var(g, "sx", DataType::FLOAT, {1}, &sx, 4);
        raw_var(g, "zx", DataType::FLOAT8E5M2, {1}, z8.data(), 1);
        raw_var(g, "W", DataType::FLOAT8E4M3FN, {(size_t)N, (size_t)K}, qw.data(), qw.size());
        raw_var(g, "sw", DataType::FLOAT, {1}, &sw, 4);
        var(g, "xq", DataType::FLOAT8E5M2, {(size_t)M, (size_t)K});
        var(g, "xd", DataType::FLOAT, {(size_t)M, (size_t)K});
        var(g, "Wf", DataType::FLOAT, {(size_t)N, (size_t)K});
        var(g, "y", DataType::FLOAT, {(size_t)M, (size_t)N});
        node(g, "QuantizeLinear", {"x", "sx", "zx"}, {"xq"});
        node(g, "DequantizeLinear", {"xq", "sx", "zx"}, {"xd"});
        node(g, "DequantizeLinear", {"W", "sw"}, {"Wf"});
        node(g, "Gemm", {"xd", "Wf"}, {"y"}, {Attribute{"transB", (int32_t)1}});
        g.add_input("x");
        g.add_output("y");
        Model m(10, "test", "1");
        m.set_graph(std::move(g));
        return m;
    };
    std::vector<std::string> types;
    auto yf = run_model(build(), nullptr, 0, "x", x, {(uint32_t)M, (uint32_t)K}, "y", {(uint32_t)M, (uint32_t)N}, true,
                        &types);
    auto yu = run_model(build(), nullptr, 0, "x", x, {(uint32_t)M, (uint32_t)K}, "y", {(uint32_t)M, (uint32_t)N}, false);
    CHECK(types.size() == 3 && types[0] == "QuantizeLinear" && types[1] == "DequantizeLinear" &&
          types[2] == "FP8Linear");
    std::vector<uint8_t> qx(x.size());
    std::vector<float> A(x.size()), Bw(w.size()), ref((size_t)M * N);
    orc_quantize_e5m2(x.data(), qx.data(), 1, 1, (int64_t)x.size(), &sx, 1);
    orc_dequantize_e5m2(qx.data(), A.data(), 1, 1, (int64_t)qx.size(), &sx);
    orc_dequantize(qw.data(), Bw.data(), 1, 1, (int64_t)qw.size(), &sw);
    orc_gemm(M, N, K, A.data(), 0, Bw.data(), 1, 1.0f, 0.0f, nullptr, -1, 0, 0, 0, ref.data());
    std::vector<double> bound(ref.size());
    orc_gemm_abs_bound(M, N, K, A.data(), 0, Bw.data(), 1, 1.0f, 0.0f, nullptr, -1, 0, 0, bound.data());
    CHECK(close(yf, ref, bound, 1e-4, 0.0, "e5m2 activation, fused weight"));
    CHECK(close(yu, ref, bound, 1e-4, 0.0, "e5m2 activation, op by op"));
}

// A model file whose DynamicQuantizeLinear scale / zero-point outputs are
// declared as ONNX scalars (value_info without a dim list): they load as
// shape [1] (the reference's Variable::from_json, onnx.cpp:93-95) and the
// unfused graph runs through the planned arena.
static void test_scalar_value_info_unfused() {
    std::printf("[14] 0-D value_info (DynamicQuantizeLinear outputs) from JSON, unfused\n");
    const int M = 8, K = 64;
    auto x = normals(141, (size_t)M * K, 2.0f);
    const char *json = R"({
  "graph": {
    "node": [
      {"input": ["x"], "output": ["xq", "xs", "xz"], "name": "dq", "op_type": "DynamicQuantizeLinear"},
      {"input": ["xq", "xs", "xz"], "output": ["y"], "name": "dd", "op_type": "DequantizeLinear"}
    ],
    "name": "scalars",
    "input": [{"name": "x", "type": {"tensor_type": {"elem_type": "FLOAT",
               "shape": {"dim": [{"dim_value": "8"}, {"dim_value": "64"}]}}}}],
    "output": [{"name": "y", "type": {"tensor_type": {"elem_type": "FLOAT",
               "shape": {"dim": [{"dim_value": "8"}, {"dim_value": "64"}]}}}}],
    "value_info": [
      {"name": "xq", "type": {"tensor_type": {"elem_type": "FLOAT8E4M3FN",
               "shape": {"dim": [{"dim_value": "8"}, {"dim_value": "64"}]}}}},
      {"name": "xs", "type": {"tensor_type": {"elem_type": "FLOAT", "shape": {}}}},
      {"name": "xz", "type": {"tensor_type": {"elem_type": "FLOAT8E4M3FN"}}}
    ]
  }
})";
    Model m = Model::load_from_json(json);
    CHECK(m.get_graph().get_var("xs").get_shape() == std::vector<size_t>{1});
    CHECK(m.get_graph().get_var("xz").get_shape() == std::vector<size_t>{1});
    auto y = run_model(std::move(m), nullptr, 0, "x", x, {(uint32_t)M, (uint32_t)K}, "y", {(uint32_t)M, (uint32_t)K},
                       false);
    float s = orc_scale_from_amax(orc_amax(x.data(), x.size()));
    std::vector<uint8_t> q(x.size());
    std::vector<float> ref(x.size());
    orc_quantize(x.data(), q.data(), 1, 1, (int64_t)q.size(), &s);
    orc_dequantize(q.data(), ref.data(), 1, 1, (int64_t)q.size(), &s);
    CHECK(std::memcmp(y.data(), ref.data(), ref.size() * 4) == 0);
}

// One E4M3 weight W [64, 64] behind two DequantizeLinear nodes with
// different scales, feeding Gemm(transB=1) and MatMul (W read as [K, N]):
// each fused node packs its own (weight, scale, layout) copy.
static void test_tied_weight_two_layouts() {
    std::printf("[15] one E4M3 weight, two scales and two layouts\n");
    const int M = 16, D = 64;
    auto x = normals(151, (size_t)M * D, 1.0f), w = normals(152, (size_t)D * D, 0.05f);
    float s1 = orc_scale_from_amax(orc_amax(w.data(), w.size())), s2 = 2.5f * s1;
    std::vector<uint8_t> qw(w.size());
    orc_quantize(w.data(), qw.data(), 1, 1, (int64_t)qw.size(), &s1);
    Graph g("tied");
    var(g, "x", DataType::FLOAT, {(size_t)M, (size_t)D});
    raw_var(g, "W", DataType::FLOAT8E4M3FN, {(size_t)D, (size_t)D}, qw.data(), qw.size());
    raw_var(g, "s1", DataType::FLOAT, {1}, &s1, 4);
    raw_var(g, "s2", DataType::FLOAT, {1}, &s2, 4);
    var(g, "W1", DataType::FLOAT, {(size_t)D, (size_t)D});
    var(g, "W2", DataType::FLOAT, {(size_t)D, (size_t)D});
    var(g, "h", DataType::FLOAT, {(size_t)M, (size_t)D});
    var(g, "y", DataType::FLOAT, {(size_t)M, (size_t)D});
    node(g, "DequantizeLinear", {"W", "s1"}, {"W1"});
    node(g, "DequantizeLinear", {"W", "s2"}, {"W2"});
    node(g, "Gemm", {"x", "W1"}, {"h"}, {Attribute{"transB", (int32_t)1}});
    node(g, "MatMul", {"h", "W2"}, {"y"});
    g.add_input("x");
    g.add_output("y");
    Model m(10, "test", "1");
    m.set_graph(std::move(g));
    size_t nf = 0;
    auto y = run_model(std::move(m), nullptr, 0, "x", x, {(uint32_t)M, (uint32_t)D}, "y", {(uint32_t)M, (uint32_t)D},
                       true, nullptr, &nf);
    CHECK(nf == 2);
    std::vector<float> W1(w.size()), W2(w.size()), h((size_t)M * D), ref((size_t)M * D);
    orc_dequantize(qw.data(), W1.data(), 1, 1, (int64_t)qw.size(), &s1);
    orc_dequantize(qw.data(), W2.data(), 1, 1, (int64_t)qw.size(), &s2);
    orc_gemm(M, D, D, x.data(), 0, W1.data(), 1, 1.0f, 0.0f, nullptr, -1, 0, 0, 0, h.data());
    orc_gemm(M, D, D, h.data(), 0, W2.data(), 0, 1.0f, 0.0f, nullptr, -1, 0, 0, 0, ref.data());
    // two chained W8A32 layers: the first layer's error (within 1e-4 of its
    // bound) propagates, so the second bound sums (|h| + bound_h) |W2|
    std::vector<double> bound(ref.size()), bound_h(h.size());
    orc_gemm_abs_bound(M, D, D, x.data(), 0, W1.data(), 1, 1.0f, 0.0f, nullptr, -1, 0, 0, bound_h.data());
    std::vector<float> ah(h.size()), aw(W2.size());
    for (size_t i = 0; i < h.size(); ++i) ah[i] = std::fabs(h[i]) + (float)bound_h[i];
    for (size_t i = 0; i < W2.size(); ++i) aw[i] = std::fabs(W2[i]);
    orc_gemm_abs_bound(M, D, D, ah.data(), 0, aw.data(), 0, 1.0f, 0.0f, nullptr, -1, 0, 0, bound.data());
    CHECK(close(y, ref, bound, 1e-4, 0.0, "tied weight"));
}

// Gemm(transA=1): A is [K, M]; with a static or dynamic activation QDQ it
// fuses, the quantiser writing the transposed E4M3 copy.
static void test_gemm_trans_a(bool dynamic) {
    std::printf("[16] %s QDQ activation -> Gemm(transA=1, transB=1) fused\n", dynamic ? "dynamic" : "static");
    const int M = 48, K = 160, N = 80;
    auto xt = normals(161, (size_t)K * M, 1.0f), w = normals(162, (size_t)N * K, 0.05f), b = normals(163, N, 0.01f);
    float sx = orc_scale_from_amax(orc_amax(xt.data(), xt.size()));
    float sw = orc_scale_from_amax(orc_amax(w.data(), w.size()));
    std::vector<uint8_t> qw(w.size()), qx(xt.size()), z8(1, 0);
    orc_quantize(w.data(), qw.data(), 1, 1, (int64_t)qw.size(), &sw);
    orc_quantize(xt.data(), qx.data(), 1, 1, (int64_t)qx.size(), &sx);
    Graph g("transa");
    var(g, "x", DataType::FLOAT, {(size_t)K, (size_t)M});
    raw_var(g, "W", DataType::FLOAT8E4M3FN, {(size_t)N, (size_t)K}, qw.data(), qw.size());
    raw_var(g, "sw", DataType::FLOAT, {1}, &sw, 4);
    raw_var(g, "b", DataType::FLOAT, {(size_t)N}, b.data(), N * 4);
    var(g, "xq", DataType::FLOAT8E4M3FN, {(size_t)K, (size_t)M});
    var(g, "xd", DataType::FLOAT, {(size_t)K, (size_t)M});
    var(g, "Wf", DataType::FLOAT, {(size_t)N, (size_t)K});
    var(g, "y", DataType::FLOAT, {(size_t)M, (size_t)N});
    if (dynamic) {
        var(g, "xs", DataType::FLOAT, {1});
        var(g, "xz", DataType::FLOAT8E4M3FN, {1});
        node(g, "DynamicQuantizeLinear", {"x"}, {"xq", "xs", "xz"});
        node(g, "DequantizeLinear", {"xq", "xs", "xz"}, {"xd"});
    } else {
        raw_var(g, "xs", DataType::FLOAT, {1}, &sx, 4);
        raw_var(g, "xz", DataType::FLOAT8E4M3FN, {1}, z8.data(), 1);
        node(g, "QuantizeLinear", {"x", "xs", "xz"}, {"xq"});
        node(g, "DequantizeLinear", {"xq", "xs", "xz"}, {"xd"});
    }
    node(g, "DequantizeLinear", {"W", "sw"}, {"Wf"});
    node(g, "Gemm", {"xd", "Wf", "b"}, {"y"}, {Attribute{"transA", (int32_t)1}, Attribute{"transB", (int32_t)1}});
    g.add_input("x");
    g.add_output("y");
    Model m(10, "test", "1");
    m.set_graph(std::move(g));
    std::vector<std::string> types;
    auto y = run_model(std::move(m), nullptr, 0, "x", xt, {(uint32_t)K, (uint32_t)M}, "y", {(uint32_t)M, (uint32_t)N},
                       true, &types);
    CHECK(all_ops(types, "FP8Linear", 1));
    std::vector<float> A(xt.size()), Bw(w.size()), ref((size_t)M * N);
    orc_dequantize(qx.data(), A.data(), 1, 1, (int64_t)qx.size(), &sx);
    orc_dequantize(qw.data(), Bw.data(), 1, 1, (int64_t)qw.size(), &sw);
    orc_gemm(M, N, K, A.data(), 1, Bw.data(), 1, 1.0f, 1.0f, b.data(), 1, N, 0, 0, ref.data());
    std::vector<double> bound(ref.size());
    orc_gemm_abs_bound(M, N, K, A.data(), 1, Bw.data(), 1, 1.0f, 1.0f, b.data(), 1, N, 0, bound.data());
    CHECK(close(y, ref, bound, 1e-4, 0.0, "gemm transA"));
}

// 1-D Conv (X [n, c, l], W [cout, c, kl], conv.cpp:209-250) with an
// auto_pad attribute the reference parses and ignores: fp32 op by op, and
// with a dynamic activation QDQ fused into FP8Conv; both against the
// oracle's direct conv of the [n, c, 1, l] view.
static void test_conv1d(bool fused) {
    std::printf("[17] 1-D Conv (stride 2, pad 2, dilation 1, auto_pad SAME_UPPER ignored), %s\n",
                fused ? "DQ -> FP8Conv" : "fp32");
    const int64_t Nb = 2, C = 32, L = 40, CO = 24, KL = 5, S = 2, P = 2, OL = (L + 2 * P - KL) / S + 1;
    auto x = normals(171, (size_t)(Nb * C * L), 1.0f), w = normals(172, (size_t)(CO * C * KL), 0.05f);
    auto bias = normals(173, (size_t)CO, 0.01f);
    float sw = orc_scale_from_amax(orc_amax(w.data(), w.size()));
    std::vector<uint8_t> qw(w.size());
    orc_quantize(w.data(), qw.data(), 1, 1, (int64_t)qw.size(), &sw);
    std::vector<float> wd(w.size());
    orc_dequantize(qw.data(), wd.data(), 1, 1, (int64_t)qw.size(), &sw);
    Graph g("conv1d");
    var(g, "x", DataType::FLOAT, {(size_t)Nb, (size_t)C, (size_t)L});
    var(g, "y", DataType::FLOAT, {(size_t)Nb, (size_t)CO, (size_t)OL});
    raw_var(g, "B", DataType::FLOAT, {(size_t)CO}, bias.data(), CO * 4);
    std::vector<Attribute> attrs = {Attribute{"strides", std::vector<int32_t>{(int32_t)S}},
                                    Attribute{"pads", std::vector<int32_t>{(int32_t)P, (int32_t)P}},
                                    Attribute{"auto_pad", std::string("SAME_UPPER")},
                                    Attribute{"kernel_shape", std::vector<int32_t>{(int32_t)KL}}};
    std::vector<float> xin = x;
    if (fused) {
        raw_var(g, "W", DataType::FLOAT8E4M3FN, {(size_t)CO, (size_t)C, (size_t)KL}, qw.data(), qw.size());
        raw_var(g, "sw", DataType::FLOAT, {1}, &sw, 4);
        var(g, "xq", DataType::FLOAT8E4M3FN, {(size_t)Nb, (size_t)C, (size_t)L});
        var(g, "xs", DataType::FLOAT, {1});
        var(g, "xz", DataType::FLOAT8E4M3FN, {1});
        var(g, "xd", DataType::FLOAT, {(size_t)Nb, (size_t)C, (size_t)L});
        var(g, "Wf", DataType::FLOAT, {(size_t)CO, (size_t)C, (size_t)KL});
        node(g, "DynamicQuantizeLinear", {"x"}, {"xq", "xs", "xz"});
        node(g, "DequantizeLinear", {"xq", "xs", "xz"}, {"xd"});
        node(g, "DequantizeLinear", {"W", "sw"}, {"Wf"});
        node(g, "Conv", {"xd", "Wf", "B"}, {"y"}, attrs);
        float sx = orc_scale_from_amax(orc_amax(x.data(), x.size()));
        std::vector<uint8_t> qx(x.size());
        orc_quantize(x.data(), qx.data(), 1, 1, (int64_t)qx.size(), &sx);
        orc_dequantize(qx.data(), x.data(), 1, 1, (int64_t)qx.size(), &sx);  // x: the dequantised activation
    } else {
        raw_var(g, "W", DataType::FLOAT, {(size_t)CO, (size_t)C, (size_t)KL}, wd.data(), wd.size() * 4);
        node(g, "Conv", {"x", "W", "B"}, {"y"}, attrs);
    }
    g.add_input("x");
    g.add_output("y");
    Model m(10, "test", "1");
    m.set_graph(std::move(g));
    std::vector<std::string> types;
    auto y = run_model(std::move(m), nullptr, 0, "x", xin, {(uint32_t)Nb, (uint32_t)C, (uint32_t)L}, "y",
                       {(uint32_t)Nb, (uint32_t)CO, (uint32_t)OL}, true, &types);
    CHECK(fused ? all_ops(types, "FP8Conv", 1) : all_ops(types, "Conv", 1));
    std::vector<float> ref(y.size()), ax(x.size()), aw(wd.size()), ab(bias.size()), bnd(y.size());
    orc_conv2d(x.data(), wd.data(), bias.data(), ref.data(), Nb, C, 1, L, CO, 1, KL, 1, S, 0, P, 1, 1, 1, 1, OL,
               LCML_ACT_NONE);
    for (size_t i = 0; i < x.size(); ++i) ax[i] = std::fabs(x[i]);
    for (size_t i = 0; i < wd.size(); ++i) aw[i] = std::fabs(wd[i]);
    for (size_t i = 0; i < bias.size(); ++i) ab[i] = std::fabs(bias[i]);
    orc_conv2d(ax.data(), aw.data(), ab.data(), bnd.data(), Nb, C, 1, L, CO, 1, KL, 1, S, 0, P, 1, 1, 1, 1, OL,
               LCML_ACT_NONE);
    std::vector<double> bound(bnd.begin(), bnd.end());
    CHECK(close(y, ref, bound, 1e-4, 0.0, "conv1d"));
}

// NetworkInstance::set_fp8_matrix_cores: the fused FP8Linear runs gfx950's
// native FP8 MFMA kernels (LCML_KERNEL_AUTO_FP8).  Static QDQ (scale 1)
// activation -> MatMul(DQ(W), scale 1) with one row pattern 1, 2^-7 and one
// column pattern 1, 2^-7: the exact kernels return 1 + 2^-14, the FP8 MFMAs
// drop the product 14 binades below the largest (1.0), on the skinny (M = 1)
// and the tile (M = 1024) paths.  Then the dynamic QDQ MatMul on N(0,1) data
// against the oracle: the elementwise summation-order bound and relative
// Frobenius error < 3e-5 (the FP8-MFMA truncation), and not bit-identical to
// the exact network.
static std::vector<float> run_fp8_matmul(const std::vector<float> &x, const std::vector<uint8_t> &qw, int M, int K,
                                         int N, bool dynamic, bool fp8_mfma, const std::vector<float> &sw) {
    std::vector<uint8_t> zp(1, 0);
    const float one = 1.0f;
    Graph g("fp8mfma");
    Blob blob;
    var(g, "x", DataType::FLOAT, {(size_t)M, (size_t)K});
    blob_var(g, blob, "W", DataType::FLOAT8E4M3FN, {(size_t)K, (size_t)N}, qw.data(), qw.size());
    blob_var(g, blob, "sw", DataType::FLOAT, {(size_t)N}, sw.data(), N * 4);
    var(g, "xq", DataType::FLOAT8E4M3FN, {(size_t)M, (size_t)K});
    var(g, "xd", DataType::FLOAT, {(size_t)M, (size_t)K});
    var(g, "Wf", DataType::FLOAT, {(size_t)K, (size_t)N});
    var(g, "y", DataType::FLOAT, {(size_t)M, (size_t)N});
    if (dynamic) {
        var(g, "xs", DataType::FLOAT, {1});
        var(g, "xz", DataType::FLOAT8E4M3FN, {1});
        node(g, "DynamicQuantizeLinear", {"x"}, {"xq", "xs", "xz"});
    } else {
        raw_var(g, "xs", DataType::FLOAT, {1}, &one, 4);
        raw_var(g, "xz", DataType::FLOAT8E4M3FN, {1}, zp.data(), 1);
        node(g, "QuantizeLinear", {"x", "xs", "xz"}, {"xq"});
    }
    node(g, "DequantizeLinear", {"xq", "xs", "xz"}, {"xd"});
    node(g, "DequantizeLinear", {"W", "sw"}, {"Wf"}, {Attribute{"axis", (int32_t)1}});
    node(g, "MatMul", {"xd", "Wf"}, {"y"});
    g.add_input("x");
    g.add_output("y");
    Model m(10, "test", "1");
    m.set_graph(std::move(g));
    DeviceBuffer wb(blob.bytes.size());
    CHECK(hipMemcpy(wb.data(), blob.bytes.data(), blob.bytes.size(), hipMemcpyHostToDevice) == hipSuccess);
    auto xt = upload(x, {(uint32_t)M, (uint32_t)K});
    auto yt = make_device_tensor<float>({(uint32_t)M, (uint32_t)N});
    NetworkInstance net;
    net.set_fp8_matrix_cores(fp8_mfma);
    net.set_model(std::move(m));
    net.set_weight_buffer(wb.data(), blob.bytes.size());
    net.set_input("x", *xt);
    net.set_output("y", *yt);
    net.forward();
    CHECK(net.fused_linear_count() == 1 && net.executed_op_types().size() == 1u);
    return download<float>(*yt);
}

static void test_fp8_matrix_cores() {
    std::printf("[19] set_fp8_matrix_cores: fused FP8Linear on the native FP8 MFMA kernels\n");
    {
        const int K = 128, N = 64;
        std::vector<uint8_t> qw((size_t)K * N, 0);
        for (int n = 0; n < N; ++n) {
            qw[n] = 0x38;          // 1.0
            qw[(size_t)N + n] = 0x04;  // 2^-7
        }
        const std::vector<float> sw(N, 1.0f);
        for (int M : {1, 1024}) {
            std::vector<float> x((size_t)M * K, 0.0f);
            for (int r = 0; r < M; ++r) {
                x[(size_t)r * K] = 1.0f;
                x[(size_t)r * K + 1] = 0x1p-7f;
            }
            auto exact = run_fp8_matmul(x, qw, M, K, N, false, false, sw);
            auto fast = run_fp8_matmul(x, qw, M, K, N, false, true, sw);
            bool ok = true;
            for (size_t i = 0; i < exact.size(); ++i) ok &= exact[i] == 1.0f + 0x1p-14f && fast[i] == 1.0f;
            if (!ok) std::printf("  M=%d: expected 1 + 2^-14 (exact) and 1 (FP8 MFMA), got %a and %a\n", M,
                                 (double)exact[0], (double)fast[0]);
            CHECK(ok);
        }
    }
    {
        const int M = 512, K = 1024, N = 1024;
        auto x = normals(191, (size_t)M * K, 1.0f), w = normals(192, (size_t)K * N, 0.02f);
        std::vector<float> sw(N, 0.0f);
        for (int k = 0; k < K; ++k)
            for (int n = 0; n < N; ++n) sw[n] = std::max(sw[n], std::fabs(w[(size_t)k * N + n]));
        for (auto &s : sw) s = orc_scale_from_amax(s);
        std::vector<uint8_t> qw(w.size());
        orc_quantize(w.data(), qw.data(), K, N, 1, sw.data());
        auto exact = run_fp8_matmul(x, qw, M, K, N, true, false, sw);
        auto fast = run_fp8_matmul(x, qw, M, K, N, true, true, sw);
        float sx = orc_scale_from_amax(orc_amax(x.data(), x.size()));
        std::vector<uint8_t> qx(x.size());
        orc_quantize(x.data(), qx.data(), 1, 1, x.size(), &sx);
        std::vector<float> A(x.size()), Bw(w.size()), ref((size_t)M * N);
        orc_dequantize(qx.data(), A.data(), 1, 1, qx.size(), &sx);
        orc_dequantize(qw.data(), Bw.data(), K, N, 1, sw.data());
        orc_gemm(M, N, K, A.data(), 0, Bw.data(), 0, 1.0f, 0.0f, nullptr, -1, 0, 0, 0, ref.data());
        std::vector<double> bound((size_t)M * N);
        orc_gemm_abs_bound(M, N, K, A.data(), 0, Bw.data(), 0, 1.0f, 0.0f, nullptr, -1, 0, 0, bound.data());
        CHECK(close(exact, ref, bound, 1e-4, 0.0, "exact network"));
        CHECK(close(fast, ref, bound, 1e-4, 0.0, "FP8-MFMA network"));
        double num = 0, den = 0;
        for (size_t i = 0; i < ref.size(); ++i) {
            num += ((double)fast[i] - ref[i]) * ((double)fast[i] - ref[i]);
            den += (double)ref[i] * ref[i];
        }
        const double rel = std::sqrt(num / den);
        std::printf("  relative Frobenius error of the FP8-MFMA network: %.3g\n", rel);
        CHECK(rel < 3e-5);
        CHECK(exact != fast);
    }
}

int main(int argc, char **argv) {
    if (argc < 2) {
        std::printf("usage: test_network <golden dir>\n");
        return 2;
    }
    hipStream_t s;
    CHECK(hipStreamCreate(&s) == hipSuccess);
    try {
        test_reference_fixture(argv[1]);
        test_fp8_mlp(true);
        test_fp8_mlp(false);
        test_static_qdq_gelu();
        test_static_qdq_gelu(100);
        test_dynamic_qdq_matmul();
        test_dynamic_qdq_matmul(200);
        test_standalone_qdq_cast();
        test_qdq_conv(true);
        test_qdq_conv(false);
        test_qdq_conv(true, 2);
        test_f32_grouped_conv();
        test_batched_matmul();
        test_batched_fp8_matmul(true);
        test_batched_fp8_matmul(false);
        test_fp8_tensor_conv(false);
        test_fp8_tensor_conv(true);
        test_e5m2_qdq_cast();
        test_elementwise();
        test_memory_planner();
        test_fp8_mlp_from_file(argv[1], true);
        test_fp8_mlp_from_file(argv[1], false);
        test_e5m2_activation_stays_unfused();
        test_scalar_value_info_unfused();
        test_tied_weight_two_layouts();
        test_gemm_trans_a(false);
        test_gemm_trans_a(true);
        test_conv1d(false);
        test_conv1d(true);
        test_fp8_matrix_cores();
        test_errors();
    } catch (const Error &e) {
        std::printf("FAIL: uncaught error: %s\n", e.what());
        ++failures;
    }
    std::printf(failures ? "FAILED (%d)\n" : "PASS\n", failures);
    return failures ? 1 : 0;
}
