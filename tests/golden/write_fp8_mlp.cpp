// write_fp8_mlp.cpp -- writes the FP8 QDQ MLP fixture (the 3-layer MLP
// workload: Gemm 784->256 + Relu, Gemm 256->128 + Relu, Gemm 128->10, batch
// 64) as a model file, because the reference's exporter cannot emit FP8
// initializers (scripts/export_onnx.py:26-44):
//   fp8_mlp.onnx.json   ONNX-JSON (Model::save_to_json), torch Linear layout
//                       (Gemm transB=1), each weight behind
//                       DequantizeLinear(W_e4m3, scale, zero point)
//   fp8_mlp.bin         the raw weight blob its data_offsets index: E4M3
//                       weights (4-byte padded), fp32 per-tensor scales
//                       (amax / 448), E4M3 zero points (0), fp32 biases
//   fp8_mlp_input.bin   x [64, 784] fp32, U(0, 1)
//   fp8_mlp_output.bin  y [64, 10] fp32: the oracle's Gemm chain on the
//                       dequantised weights (the reference's fma order,
//                       src/onnx/operators/gemm.cpp:155-162)
// Weights N(0, 0.05), biases N(0, 0.01); seeded splitmix64 + Box-Muller.
// Needs no GPU.  usage: write_fp8_mlp <output dir>
#include <cmath>
#include <cstdio>
#include <fstream>
#include <string>
#include <vector>

#include "onnx/onnx.h"

using namespace lcml::onnx;

extern "C" {
void orc_quantize(const float *, uint8_t *, int64_t, int64_t, int64_t, const float *);
void orc_dequantize(const uint8_t *, float *, int64_t, int64_t, int64_t, const float *);
float orc_amax(const float *, int64_t);
float orc_scale_from_amax(float);
void orc_gemm(int64_t, int64_t, int64_t, const float *, int, const float *, int, float, float, const float *, int,
              int64_t, int64_t, int, float *);
}

namespace {

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

void write_file(const std::string &path, const void *p, size_t n) {
    std::ofstream f(path, std::ios::binary);
    f.write(static_cast<const char *>(p), (std::streamsize)n);
    if (!f) {
        std::fprintf(stderr, "cannot write %s\n", path.c_str());
        std::exit(1);
    }
}

}  // namespace

int main(int argc, char **argv) {
    if (argc != 2) {
        std::fprintf(stderr, "usage: %s <output dir>\n", argv[0]);
        return 2;
    }
    const std::string dir = argv[1];
    const size_t B = 64, dims[4] = {784, 256, 128, 10};
    Graph g("fp8_mlp");
    WeightBlobWriter blob;
    std::vector<std::vector<float>> wdq(3), bias(3);
    g.add_variable(Variable("input", DataType::FLOAT, {B, dims[0]}));
    for (int l = 0; l < 3; ++l) {
        const size_t K = dims[l], N = dims[l + 1];
        const std::string L = std::to_string(l);
        Rng rw{0x5eed0000ull + (uint64_t)l}, rb{0x5eed0100ull + (uint64_t)l};
        std::vector<float> w(N * K);
        for (auto &v : w) v = rw.normal(0.05f);
        bias[l].resize(N);
        for (auto &v : bias[l]) v = rb.normal(0.01f);
        const float s = orc_scale_from_amax(orc_amax(w.data(), (int64_t)w.size()));
        std::vector<uint8_t> q(w.size());
        orc_quantize(w.data(), q.data(), 1, 1, (int64_t)w.size(), &s);
        wdq[l].resize(w.size());
        orc_dequantize(q.data(), wdq[l].data(), 1, 1, (int64_t)q.size(), &s);
        const uint8_t zp = 0;
        g.add_variable(blob.add("net." + L + ".weight", DataType::FLOAT8E4M3FN, {N, K}, q.data(), q.size()));
        g.add_variable(blob.add("net." + L + ".weight_scale", DataType::FLOAT, {1}, &s, 4));
        g.add_variable(blob.add("net." + L + ".weight_zero_point", DataType::FLOAT8E4M3FN, {1}, &zp, 1));
        g.add_variable(blob.add("net." + L + ".bias", DataType::FLOAT, {N}, bias[l].data(), N * 4));
        g.add_variable(Variable("net." + L + ".weight_dq", DataType::FLOAT, {N, K}));
        const std::string y = l == 2 ? "output" : "linear_" + L;
        g.add_variable(Variable(y, DataType::FLOAT, {B, N}));
        Node dq("node_dequantize_" + L, "DequantizeLinear");
        dq.add_input(g.get_var("net." + L + ".weight"));
        dq.add_input(g.get_var("net." + L + ".weight_scale"));
        dq.add_input(g.get_var("net." + L + ".weight_zero_point"));
        dq.add_output(g.get_var("net." + L + ".weight_dq"));
        g.add_node(std::move(dq));
        Node gm("node_linear_" + L, "Gemm");
        gm.add_input(g.get_var(l == 0 ? "input" : "relu_" + std::to_string(l - 1)));
        gm.add_input(g.get_var("net." + L + ".weight_dq"));
        gm.add_input(g.get_var("net." + L + ".bias"));
        gm.add_output(g.get_var(y));
        gm.set_attribute(Attribute{"transA", (int32_t)0});
        gm.set_attribute(Attribute{"transB", (int32_t)1});
        gm.set_attribute(Attribute{"alpha", 1.0f});
        gm.set_attribute(Attribute{"beta", 1.0f});
        g.add_node(std::move(gm));
        if (l < 2) {
            g.add_variable(Variable("relu_" + L, DataType::FLOAT, {B, N}));
            Node r("node_relu_" + L, "Relu");
            r.add_input(g.get_var(y));
            r.add_output(g.get_var("relu_" + L));
            g.add_node(std::move(r));
        }
    }
    g.add_input("input");
    g.add_output("output");
    Model m(10, "luisaml_amd", "write_fp8_mlp");
    m.set_graph(std::move(g));

    std::vector<float> x(B * dims[0]);
    Rng rx{0x5eed0200ull};
    for (auto &v : x) v = (float)rx.uni();
    // the oracle's forward pass: Gemm(transB=1) + bias (+ Relu) per layer
    std::vector<float> h = x;
    for (int l = 0; l < 3; ++l) {
        const size_t K = dims[l], N = dims[l + 1];
        std::vector<float> out(B * N);
        orc_gemm((int64_t)B, (int64_t)N, (int64_t)K, h.data(), 0, wdq[l].data(), 1, 1.0f, 1.0f, bias[l].data(), 1,
                 (int64_t)N, 0, l < 2 ? 1 : 0, out.data());
        h = std::move(out);
    }
    const std::string json = m.save_to_json();
    write_file(dir + "/fp8_mlp.onnx.json", json.data(), json.size());
    write_file(dir + "/fp8_mlp.bin", blob.bytes().data(), blob.bytes().size());
    write_file(dir + "/fp8_mlp_input.bin", x.data(), x.size() * 4);
    write_file(dir + "/fp8_mlp_output.bin", h.data(), h.size() * 4);
    std::printf("wrote %s/fp8_mlp.{onnx.json,bin} (%zu blob bytes), input and output\n", dir.c_str(),
                blob.bytes().size());
    return 0;
}
