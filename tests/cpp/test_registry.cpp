// test_registry.cpp -- host-layer checks that need no GPU, in the manner of
// the reference's tests/onnx/test_onnx_import.cpp: the default operator set,
// JSON import of the reference's own MLP fixture, operator creation from
// the imported nodes, the tensor API and the error behaviour.
//   usage: test_registry <tests/golden dir>
#include <algorithm>
#include <concepts>
#include <cstdio>
#include <fstream>
#include <sstream>
#include <string>
#include <cstring>

#include "onnx/memory_planner.h"
#include "onnx/network_instance.h"
#include "onnx/onnx.h"
#include "onnx/tensor.h"

using namespace lcml::onnx;

static int failures = 0;
#define CHECK(c)                                                        \
    do {                                                                \
        if (!(c)) {                                                     \
            std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #c);    \
            ++failures;                                                 \
        }                                                               \
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

static std::string read_text(const std::string &path) {
    std::ifstream f(path);
    std::stringstream ss;
    ss << f.rdbuf();
    return ss.str();
}

int main(int argc, char **argv) {
    if (argc < 2) {
        std::printf("usage: test_registry <golden dir>\n");
        return 2;
    }
    const std::string golden = argv[1];
    auto &opset = OperatorSet::get_default();
    CHECK(opset.get_domain() == "default" && opset.get_version() == 21);
    for (const char *op : {"Gemm", "MatMul", "QuantizeLinear", "DequantizeLinear", "DynamicQuantizeLinear", "Cast",
                           "Relu", "Gelu", "FP8Linear", "Conv", "FP8Conv", "Add", "Sub", "Mul", "Div"})
        CHECK(opset.has_operator(op));

    // ---- device-buffer planner (host only) ----
    {
        // a chain: buffer i written by node i, read by node i+1 -> two slots
        std::vector<BufferRequest> chain;
        for (size_t i = 0; i < 6; ++i) chain.push_back({1000, i, i + 1});
        MemoryPlan p = plan_device_buffers(chain);
        CHECK(plan_is_valid(chain, p) && p.arena_bytes == 2 * 1024 && p.unshared_bytes == 6 * 1024);
        // all live at once -> no sharing
        std::vector<BufferRequest> all = {{300, 0, 5}, {5000, 1, 4}, {17, 2, 3}, {4096, 0, 3}};
        p = plan_device_buffers(all);
        CHECK(plan_is_valid(all, p) && p.arena_bytes == p.unshared_bytes);
        // a small buffer fits the gap a large one left
        std::vector<BufferRequest> gap = {{4096, 0, 1}, {4096, 2, 3}, {1024, 1, 2}, {8192, 0, 3}};
        p = plan_device_buffers(gap);
        CHECK(plan_is_valid(gap, p) && p.arena_bytes == 8192 + 4096 + 1024);
        // random graphs: always valid, never larger than no sharing, never
        // smaller than the peak of simultaneously live bytes
        uint64_t st = 12345;
        auto rnd = [&](uint64_t m) { st = st * 6364136223846793005ull + 1442695040888963407ull; return (st >> 33) % m; };
        for (int t = 0; t < 200; ++t) {
            std::vector<BufferRequest> r;
            const size_t nodes = 2 + rnd(30);
            for (size_t k = 0, nb = 1 + rnd(40); k < nb; ++k) {
                size_t a = rnd(nodes), b = a + rnd(nodes - a);
                r.push_back({1 + rnd(1 << 20), a, b});
            }
            p = plan_device_buffers(r);
            size_t peak = 0;
            for (size_t nd = 0; nd < nodes; ++nd) {
                size_t live = 0;
                for (auto &q : r)
                    if (q.first <= nd && nd <= q.last) live += (q.bytes + 255) / 256 * 256;
                peak = std::max(peak, live);
            }
            CHECK(plan_is_valid(r, p) && p.arena_bytes <= p.unshared_bytes && p.arena_bytes >= peak);
        }
    }
    CHECK(!opset.has_operator("NotAnOp"));
    Node bogus("n", "NotAnOp");
    CHECK(throws([&] { opset.create_operator("NotAnOp", bogus); }));
    // error messages: without arguments verbatim ('%' is not a conversion), with arguments formatted
    CHECK(lcml::onnx::format("x %s 100% %d") == "x %s 100% %d");
    CHECK(lcml::onnx::format("K=%d of %s", 7, "W") == "K=7 of W");
    try {
        LCML_ASSERT(false, "c % 4 != 0");
        CHECK(false);
    } catch (const lcml::onnx::Error &e) {
        CHECK(std::string(e.what()) == "c % 4 != 0");
    }

    // ---- import the reference's fixture graph ----
    Model m = Model::load_from_json(read_text(golden + "/simple_mlp.onnx.json"));
    const Graph &g = m.get_graph();
    CHECK(g.get_nodes().size() == 5);
    const char *ops[] = {"Gemm", "Relu", "Gemm", "Relu", "Gemm"};
    for (size_t i = 0; i < g.get_nodes().size() && i < 5; ++i) CHECK(g.get_nodes()[i].get_op_type() == ops[i]);
    CHECK(g.get_inputs().size() == 1 && g.get_inputs()[0].get().get_name() == "input");
    CHECK((g.get_inputs()[0].get().get_shape() == std::vector<size_t>{1, 784}));
    CHECK((g.get_outputs()[0].get().get_shape() == std::vector<size_t>{1, 10}));
    const Variable &w0 = g.get_var("net.0.weight");
    CHECK(w0.get_dtype() == DataType::FLOAT && w0.is_trainable_weight() && w0.is_constant());
    CHECK((w0.get_shape() == std::vector<size_t>{256, 784}));
    CHECK((w0.get_buffer_range() == std::pair<uint64_t, uint64_t>{1024, 803840}));
    const Node &gemm0 = g.get_nodes()[0];
    CHECK(attr_int(gemm0, "transB", 0) == 1 && attr_int(gemm0, "transA", 1) == 0);
    CHECK(attr_float(gemm0, "alpha", 0.f) == 1.0f && attr_float(gemm0, "beta", 0.f) == 1.0f);
    CHECK(!g.get_var("linear").is_constant() && !g.get_var("input").is_constant());
    for (const Node &n : g.get_nodes()) {
        auto op = opset.create_operator(n.get_op_type(), n);
        CHECK(op && op->get_name() == n.get_op_type() && !op->is_output_view(0, n));
    }

    // ---- attribute kinds and malformed graphs ----
    Model a = Model::load_from_json(R"({"ir_version": 10, "graph": {"name": "g",
        "input": [{"name": "x", "type": {"tensor_type": {"elem_type": "FLOAT", "shape": {"dim": [{"dim_value": "4"}]}}}}],
        "output": [{"name": "y", "type": {"tensor_type": {"elem_type": "FLOAT", "shape": {"dim": [{"dim_value": "4"}]}}}}],
        "node": [{"op_type": "Gelu", "input": ["x"], "output": ["y"],
                  "attribute": [{"name": "approximate", "s": "dGFuaA==", "type": "STRING"},
                                {"name": "ks", "ints": ["3", "3"], "type": "INTS"},
                                {"name": "fs", "floats": [0.5, 2], "type": "FLOATS"}]}]}})");
    const Node &gel = a.get_graph().get_nodes()[0];
    CHECK(attr_string(gel, "approximate", "") == "tanh");
    CHECK((gel.get_attribute("ks").get<AttributeType::INTS>() == std::vector<int32_t>{3, 3}));
    CHECK((gel.get_attribute("fs").get<AttributeType::FLOATS>() == std::vector<float>{0.5f, 2.0f}));
    CHECK(throws([&] { gel.get_attribute("missing"); }));
    CHECK(throws([&] { (void)gel.get_attribute("ks").get<AttributeType::FLOAT>(); }));
    CHECK(throws([] { Model::load_from_json(R"({"graph": {"node": [{"op_type": "NotAnOp", "input": [], "output": ["y"]}]}})"); }));
    CHECK(throws([] { Model::load_from_json(R"({"graph": {"node": [)"); }));
    CHECK(throws([] { Model::load_from_json(R"({"graph": {"initializer": [{"name": "w", "data_type": "BOGUS"}]}})"); }));
    {
        Model e = Model::load_from_json(R"({"graph": {"initializer": [{"name": "s", "data_type": "FLOAT", "raw_data": "AACAPw=="}]}})");
        const Variable &s = e.get_graph().get_var("s");
        CHECK((s.get_shape() == std::vector<size_t>{1}) && s.get_raw_data().size() == 4);  // shape [1] without dims
        float v;
        std::memcpy(&v, s.get_raw_data().data(), 4);
        CHECK(v == 1.0f);
    }

    // ---- the FP8 QDQ MLP model file (tests/golden/fp8_mlp.*) ----
    {
        const std::string text = read_text(golden + "/fp8_mlp.onnx.json");
        Model m = Model::load_from_json(text);
        const Graph &g = m.get_graph();
        const char *ops[] = {"DequantizeLinear", "Gemm", "Relu", "DequantizeLinear", "Gemm",
                             "Relu", "DequantizeLinear", "Gemm"};
        CHECK(g.get_nodes().size() == 8);
        for (size_t i = 0; i < g.get_nodes().size() && i < 8; ++i) CHECK(g.get_nodes()[i].get_op_type() == ops[i]);
        const size_t blob = read_text(golden + "/fp8_mlp.bin").size();
        const size_t K[3] = {784, 256, 128}, N[3] = {256, 128, 10};
        for (int l = 0; l < 3; ++l) {
            const std::string L = std::to_string(l);
            const Variable &w = g.get_var("net." + L + ".weight");
            const Variable &zp = g.get_var("net." + L + ".weight_zero_point");
            auto [s0, e0] = w.get_buffer_range();
            CHECK(w.get_dtype() == DataType::FLOAT8E4M3FN && w.is_constant() && w.is_trainable_weight());
            CHECK((w.get_shape() == std::vector<size_t>{N[l], K[l]}) && e0 - s0 == (N[l] * K[l] + 3) / 4 * 4);
            CHECK(s0 % 4 == 0 && e0 <= blob);
            auto [zs, ze] = zp.get_buffer_range();
            CHECK(zp.get_dtype() == DataType::FLOAT8E4M3FN && ze - zs == 4 && zs % 4 == 0);  // one byte, 4-byte padded
        }
        CHECK(g.get_inputs().size() == 1 && g.get_inputs()[0].get().get_name() == "input");
        CHECK(g.get_outputs().size() == 1 && g.get_outputs()[0].get().get_name() == "output");
        // the writer is the loader's inverse: the file reproduces byte for byte
        CHECK(m.save_to_json() == text);
        // and a weight blob writer pads FP8 ranges to 4 bytes at 4-byte offsets
        WeightBlobWriter wb;
        uint8_t five[5] = {1, 2, 3, 4, 5};
        float f = 2.0f;
        Variable a = wb.add("a", DataType::FLOAT8E4M3FN, {5}, five, 5);
        Variable b = wb.add("b", DataType::FLOAT, {1}, &f, 4);
        Variable c = wb.add("c", DataType::FLOAT8E5M2, {1}, five, 1);
        CHECK((a.get_buffer_range() == std::pair<uint64_t, uint64_t>{0, 8}));
        CHECK((b.get_buffer_range() == std::pair<uint64_t, uint64_t>{8, 12}));
        CHECK((c.get_buffer_range() == std::pair<uint64_t, uint64_t>{12, 16}));
        CHECK(wb.bytes().size() == 16 && wb.bytes()[5] == 0 && wb.bytes()[4] == 5);
        CHECK(throws([&] { wb.add("d", DataType::FLOAT, {3}, &f, 4); }));  // size does not match the shape
    }

    // ---- a scalar value_info (no dim list) loads as shape [1] ----
    {
        Model m = Model::load_from_json(R"({"graph": {"node": [
            {"input": ["x"], "output": ["q", "s", "z"], "op_type": "DynamicQuantizeLinear"}],
            "input": [{"name": "x", "type": {"tensor_type": {"elem_type": "FLOAT",
                       "shape": {"dim": [{"dim_value": "4"}]}}}}],
            "output": [{"name": "s", "type": {"tensor_type": {"elem_type": "FLOAT", "shape": {}}}}],
            "value_info": [{"name": "z", "type": {"tensor_type": {"elem_type": "FLOAT8E4M3FN"}}}]}})");
        CHECK((m.get_graph().get_var("s").get_shape() == std::vector<size_t>{1}));
        CHECK((m.get_graph().get_var("z").get_shape() == std::vector<size_t>{1}));
    }

    // ---- registration keeps the first factory of a name (onnx.h:358) ----
    {
        OperatorSet os("test", 1);
        os.register_operator("Op", [](const Node &) -> std::unique_ptr<Operator> { return nullptr; });
        bool second = false;
        os.register_operator("Op", [&](const Node &) -> std::unique_ptr<Operator> {
            second = true;
            return nullptr;
        });
        Node n("n", "Op");
        os.create_operator("Op", n);
        CHECK(!second);
    }

    // ---- tensor API (borrowed storage: no device allocation) ----
    float dummy[24];
    Tensor<float> t({2, 3, 4}, DeviceArray<float>(dummy, 0, 24));
    CHECK((t.strides() == ITensor::shape_type{12, 4, 1}) && t.ndim() == 3 && t.size() == 24);
    CHECK((t.unravel_index(17) == std::vector<uint32_t>{1, 1, 1}) && t.linear_index({1, 2, 3}) == 23);
    CHECK(t.element_type_name() == "float" && t.element_type_index() == refl::type_index_of<float>());
    CHECK(refl::type_index_of<float>() != refl::type_index_of<FP8E4M3FN>());
    CHECK(data_type_to_type_index(DataType::FLOAT8E4M3FN) == refl::type_index_of<FP8E4M3FN>());
    CHECK(!t.is_constant() && !t.is_view() && t.container().is_byte_buffer() && t.container().get_byte_offset() == 0);
    t.reshape({6, 4});
    CHECK((t.strides() == ITensor::shape_type{4, 1}));
    CHECK(throws([&] { Tensor<float> bad({5}, DeviceArray<float>(dummy, 0, 4)); }));
    int visited = 0;
    visit_type_index<NNTypeList>(refl::type_index_of<FP8E4M3FN>(), [&]<typename T>() {
        visited = std::is_same_v<T, FP8E4M3FN> ? 1 : -1;
    });
    CHECK(visited == 1);
    CHECK(throws([] { visit_type_index<NNTypeList>(12345, []<typename T>() {}); }));
    // set_name reaches the storage (tensor.h:128, 344-349 of the reference)
    t.set_name("activations");
    CHECK(t.container().name() == "activations");
    static_cast<const ITensor &>(t).set_name("renamed");
    CHECK(t.container().name() == "renamed");

    // ---- TensorTable: ownership, parent fallback, release, iteration ----
    {
        float d1[4], d2[4], d3[4];
        Tensor<float> ext({4}, DeviceArray<float>(d1, 0, 4));
        TensorTable parent, child;
        parent.own("w", std::make_unique<Tensor<float>>(ITensor::shape_type{4}, DeviceArray<float>(d2, 0, 4)));
        child.bind("x", ext);
        child.own("h", std::make_unique<Tensor<float>>(ITensor::shape_type{4}, DeviceArray<float>(d3, 0, 4)));
        CHECK(!child.contains("w") && child.parent() == nullptr);
        child.set_parent(&parent);
        CHECK(child.parent() == &parent && child.contains("w") && !child.contains_local("w"));
        CHECK(child.at("w").device_data() == d2 && &child.at("x") == &ext);
        const TensorTable &cc = child;
        CHECK(cc.at("h").device_data() == d3);
        CHECK(child.entry("x").is_borrowed() && child.entry("h").is_owned() && !child.entry("h").is_borrowed());
        CHECK(throws([&] { (void)child.entry("w"); }));          // entry() is local only
        CHECK(throws([&] { (void)child.at("missing"); }));
        CHECK(child.release_owned("x") == nullptr && child.contains_local("x"));  // borrowed stays
        auto h = child.release_owned("h");
        CHECK(h && h->device_data() == d3 && !child.contains("h") && child.size() == 1 && !child.empty());
        size_t n = 0;
        for (auto &[name, entry] : child) n += name == "x" && &entry.get() == &ext;
        CHECK(n == 1);
        child.clear();
        CHECK(child.empty() && child.contains("w"));  // the parent keeps its entries
    }

    // ---- the reference's engine and table members exist with compatible
    //      signatures (include/onnx/network_instance.h:185-230,
    //      tensor_table.h:97-214, tensor.h:128) ----
    {
        static_assert(requires(NetworkInstance &n, const NetworkInstance &cn, ITensor &t, Model m) {
            n.set_model(std::move(m));
            n.set_input("x", t);
            n.set_output("y", t);
            n.set_warp_size(1u);
            { cn.warp_size() } -> std::convertible_to<uint32_t>;
            { cn.use_warp_optimization() } -> std::same_as<bool>;
            n.set_use_cooperative_vector(true);
            { cn.use_cooperative_vector() } -> std::same_as<bool>;
            n.enable_logging(true);
            { cn.get_model() } -> std::same_as<const Model &>;
            cn.get_inputs().at("x").get();
            cn.get_outputs().at("y").get();
            { cn.get_tensor_table() } -> std::same_as<const TensorTable &>;
            n.forward();
        });
        static_assert(requires(TensorTable &tt, const TensorTable &ct, ITensor &t) {
            tt.set_parent(&tt);
            { ct.parent() } -> std::same_as<TensorTable *>;
            tt.bind("a", t);
            tt.own("b", std::unique_ptr<ITensor>{});
            { tt.at("a") } -> std::same_as<ITensor &>;
            { ct.at("a") } -> std::same_as<const ITensor &>;
            { ct.contains("a") } -> std::same_as<bool>;
            { ct.contains_local("a") } -> std::same_as<bool>;
            { tt.entry("a") } -> std::same_as<TensorEntry &>;
            { ct.entry("a") } -> std::same_as<const TensorEntry &>;
            { ct.size() } -> std::same_as<size_t>;
            { ct.empty() } -> std::same_as<bool>;
            tt.clear();
            { tt.release_owned("b") } -> std::same_as<std::unique_ptr<ITensor>>;
            tt.begin(); tt.end(); ct.begin(); ct.end(); ct.cbegin(); ct.cend();
        });
        static_assert(requires(TensorEntry &e, const TensorEntry &ce) {
            { ce.is_owned() } -> std::same_as<bool>;
            { ce.is_borrowed() } -> std::same_as<bool>;
            { e.get() } -> std::same_as<ITensor &>;
            { ce.get() } -> std::same_as<const ITensor &>;
            { e.release_owned() } -> std::same_as<std::unique_ptr<ITensor>>;
        });
        static_assert(requires(const ITensor &t) { t.set_name("n"); });
        NetworkInstance net;  // no device work until prepare()/forward()
        CHECK(net.warp_size() == 64 && net.use_warp_optimization() && !net.use_cooperative_vector());
        net.set_warp_size(1);
        net.set_use_cooperative_vector(true);
        CHECK(net.warp_size() == 1 && !net.use_warp_optimization() && net.use_cooperative_vector());
        float d[4];
        Tensor<float> a({4}, DeviceArray<float>(d, 0, 4)), b({4}, DeviceArray<float>(d, 0, 4));
        net.set_input("x", a);
        net.set_input("x", b);  // a later binding replaces the earlier one
        CHECK(net.get_inputs().size() == 1 && &net.get_inputs().at("x").get() == &b && net.get_outputs().empty());
        CHECK(net.get_tensor_table().empty() && net.log_file() == "./stats.md");
    }

    std::printf(failures ? "FAILED (%d)\n" : "PASS\n", failures);
    return failures ? 1 : 0;
}
