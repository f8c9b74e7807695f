// test_network.cpp -- GPU tests of the operator layer, in the manner of the
// reference's tests/onnx/test_onnx_inference.cpp, checked against the oracle
// (oracle/lcml_oracle.c, linked as the checker):
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
//   8. an fp32 grouped / strided / dilated Conv.
//   usage: test_network <tests/golden dir>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <sstream>
#include <string>
#include <vector>

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
    size_t padded = dt == DataType::FLOAT8E4M3FN ? (bytes + 3) / 4 * 4 : bytes;
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
    net.set_weight_buffer(wb.data(), blob.size());
    net.set_input("input", *xt);
    net.set_output("output", *yt);
    net.forward();
    auto y = download<float>(*yt);
    for (int i = 0; i < 10; ++i) {
        if (std::fabs(y[i] - want[i]) > 1e-3f) {
            std::printf("  MISMATCH at %d: GPU=%.6f Ref=%.6f\n", i, y[i], want[i]);
            ++failures;
        }
    }
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
    // oracle chain; the last layer's bound uses the oracle's own activations
    std::vector<float> h = x, ref;
    std::vector<double> bound;
    for (int l = 0; l < 3; ++l) {
        const int K = dims[l], N = dims[l + 1];
        std::vector<float> out((size_t)B * N);
        orc_gemm(B, N, K, h.data(), 0, Wdq[l].data(), 1, 1.0f, 1.0f, bias[l].data(), 1, N, 0, l < 2 ? 1 : 0,
                 out.data());
        if (l == 2) {
            bound.resize(out.size());
            orc_gemm_abs_bound(B, N, K, h.data(), 0, Wdq[l].data(), 1, 1.0f, 1.0f, bias[l].data(), 1, N, 0,
                               bound.data());
        }
        h = std::move(out);
    }
    ref = h;
    // earlier layers' fp32 reordering propagates: 1e-4 of the final bound plus 1e-5 absolute
    CHECK(close(y, ref, bound, 1e-4, 1e-5, "mlp"));
}

static void test_static_qdq_gelu() {
    std::printf("[3] static QDQ activation -> Gemm(transB=1, per-channel) -> Gelu\n");
    const int M = 64, K = 256, N = 192;
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
    CHECK(net.fused_linear_count() == 1 && net.executed_op_types().size() == 1);
    std::vector<float> A(x.size()), Bw(w.size()), ref((size_t)M * N);
    orc_dequantize(qx.data(), A.data(), 1, 1, qx.size(), &sx);
    orc_dequantize(qw.data(), Bw.data(), 1, N, K, sw.data());
    orc_gemm(M, N, K, A.data(), 0, Bw.data(), 1, 1.0f, 1.0f, b.data(), 1, N, 0, 2, ref.data());
    std::vector<double> bound((size_t)M * N);
    orc_gemm_abs_bound(M, N, K, A.data(), 0, Bw.data(), 1, 1.0f, 1.0f, b.data(), 1, N, 0, bound.data());
    CHECK(close(z, ref, bound, 1.13e-4, 1e-6, "static qdq gelu"));
}

static void test_dynamic_qdq_matmul() {
    std::printf("[4] DynamicQuantizeLinear -> DequantizeLinear -> MatMul(per-channel W[K,N])\n");
    const int M = 16, K = 512, N = 320;
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
        CHECK(net.fused_linear_count() == 1 && net.executed_op_types().size() == 1);
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
        test_dynamic_qdq_matmul();
        test_standalone_qdq_cast();
        test_qdq_conv(true);
        test_qdq_conv(false);
        test_qdq_conv(true, 2);
        test_f32_grouped_conv();
        test_errors();
    } catch (const Error &e) {
        std::printf("FAIL: uncaught error: %s\n", e.what());
        ++failures;
    }
    std::printf(failures ? "FAILED (%d)\n" : "PASS\n", failures);
    return failures ? 1 : 0;
}
