// onnx.h -- graph IR and operator registry of the host layer.
//
// Same shape as the reference's include/onnx/onnx.h: DataType numbering
// (31-60), Attribute / Variable / Node / Graph (103-336), and the operator
// registry OperatorSet with REGISTER_TO_DEFAULT_OPSET (338-385) whose
// default set is ("default", 21) (src/onnx/onnx.cpp:11-14).  Attributes are
// the scalar and list kinds the FP8 linear path uses (subgraph attributes
// belong to control-flow operators outside this path).
#pragma once

#include <cstdint>
#include <functional>
#include <map>
#include <memory>
#include <string>
#include <string_view>
#include <unordered_map>
#include <variant>
#include <vector>

#include "onnx/error.h"
#include "onnx/operator.h"

namespace lcml::onnx {

enum class DataType : int {
    UNDEFINED = 0,
    FLOAT = 1,
    UINT8 = 2,
    INT8 = 3,
    INT32 = 6,
    INT64 = 7,
    FLOAT16 = 10,
    DOUBLE = 11,
    BFLOAT16 = 16,
    FLOAT8E4M3FN = 17,
    FLOAT8E4M3FNUZ = 18,
    FLOAT8E5M2 = 19,
    FLOAT8E5M2FNUZ = 20,
};

std::string_view data_type_name(DataType dt);
DataType data_type_from_name(std::string_view name);  // "FLOAT", "FLOAT8E4M3FN", ...
size_t data_type_bytes(DataType dt);
refl::TypeIndex data_type_to_type_index(DataType dt);

enum class AttributeType : int { UNDEFINED = 0, FLOAT = 1, INT = 2, STRING = 3, FLOATS = 6, INTS = 7, STRINGS = 8 };

class Attribute : public std::variant<float, int32_t, std::string, std::vector<float>, std::vector<int32_t>,
                                      std::vector<std::string>> {
    using Base = std::variant<float, int32_t, std::string, std::vector<float>, std::vector<int32_t>,
                              std::vector<std::string>>;
    std::string name_;

public:
    Attribute() = default;
    template <typename T>
    Attribute(std::string name, T &&value) : Base(std::forward<T>(value)), name_(std::move(name)) {}
    const std::string &get_name() const { return name_; }

    static constexpr AttributeType type_of(const Attribute &a) {
        switch (a.index()) {
        case 0: return AttributeType::FLOAT;
        case 1: return AttributeType::INT;
        case 2: return AttributeType::STRING;
        case 3: return AttributeType::FLOATS;
        case 4: return AttributeType::INTS;
        case 5: return AttributeType::STRINGS;
        default: return AttributeType::UNDEFINED;
        }
    }
    static constexpr size_t index_of(AttributeType t) {
        switch (t) {
        case AttributeType::FLOAT: return 0;
        case AttributeType::INT: return 1;
        case AttributeType::STRING: return 2;
        case AttributeType::FLOATS: return 3;
        case AttributeType::INTS: return 4;
        case AttributeType::STRINGS: return 5;
        default: return ~size_t(0);
        }
    }
    template <AttributeType T>
    const auto &get() const {
        LCML_ASSERT(index() == index_of(T), "attribute %s: wrong kind", name_.c_str());
        return std::get<index_of(T)>(*this);
    }
};

class Variable {
    std::string name_;
    DataType dtype_ = DataType::UNDEFINED;
    std::vector<size_t> shape_;
    std::string raw_data_;
    uint64_t buffer_start_ = 0, buffer_end_ = 0;
    bool is_constant_ = false;

public:
    Variable() = default;
    Variable(std::string name, DataType dtype, std::vector<size_t> shape, std::string raw_data = {},
             uint64_t buffer_start = 0, uint64_t buffer_end = 0)
        : name_(std::move(name)), dtype_(dtype), shape_(std::move(shape)), raw_data_(std::move(raw_data)),
          buffer_start_(buffer_start), buffer_end_(buffer_end) {}
    void set_is_constant(bool v) { is_constant_ = v; }
    bool is_constant() const { return is_constant_; }
    const std::string &get_name() const { return name_; }
    DataType get_dtype() const { return dtype_; }
    const std::vector<size_t> &get_shape() const { return shape_; }
    const std::string &get_raw_data() const { return raw_data_; }
    bool has_data() const { return !raw_data_.empty() || is_trainable_weight(); }
    // weights stored in the external blob at [start, end) (onnx.h:204 of the reference)
    bool is_trainable_weight() const { return buffer_end_ > buffer_start_; }
    std::pair<uint64_t, uint64_t> get_buffer_range() const { return {buffer_start_, buffer_end_}; }
    size_t num_elements() const {
        size_t n = 1;
        for (auto d : shape_) n *= d;
        return n;
    }
};

class Graph;

class Node {
    std::string name_, op_type_;
    std::vector<std::reference_wrapper<const Variable>> inputs_, outputs_;
    std::map<std::string, Attribute, std::less<>> attributes_;

public:
    Node() = default;
    Node(std::string name, std::string op_type) : name_(std::move(name)), op_type_(std::move(op_type)) {}
    const std::string &get_name() const { return name_; }
    const std::string &get_op_type() const { return op_type_; }
    const std::vector<std::reference_wrapper<const Variable>> &get_inputs() const { return inputs_; }
    const std::vector<std::reference_wrapper<const Variable>> &get_outputs() const { return outputs_; }
    const std::map<std::string, Attribute, std::less<>> &get_attributes() const { return attributes_; }
    bool has_attribute(std::string_view n) const { return attributes_.find(n) != attributes_.end(); }
    void add_input(const Variable &v) { inputs_.emplace_back(v); }
    void add_output(const Variable &v) { outputs_.emplace_back(v); }
    void set_attribute(Attribute a) {
        std::string n = a.get_name();
        attributes_.insert_or_assign(std::move(n), std::move(a));
    }
    const Attribute &get_attribute(std::string_view n) const {
        auto it = attributes_.find(n);
        LCML_ASSERT(it != attributes_.end(), "Attribute not found: %.*s", (int)n.size(), n.data());
        return it->second;
    }
    const Attribute *try_get_attr(std::string_view n) const {
        auto it = attributes_.find(n);
        return it == attributes_.end() ? nullptr : &it->second;
    }
};

class Graph {
    std::string name_;
    // node-based map: references handed to Nodes stay valid on insertion
    std::unordered_map<std::string, Variable> variables_;
    std::vector<std::reference_wrapper<const Variable>> inputs_, outputs_;
    std::vector<Node> nodes_;

public:
    Graph() = default;
    explicit Graph(std::string name) : name_(std::move(name)) {}
    Graph(const Graph &) = delete;
    Graph &operator=(const Graph &) = delete;
    Graph(Graph &&) = default;
    Graph &operator=(Graph &&) = default;

    Variable &add_variable(Variable &&v) {
        std::string n = v.get_name();
        auto [it, ok] = variables_.emplace(n, std::move(v));
        LCML_ASSERT(ok, "duplicate variable %s", n.c_str());
        return it->second;
    }
    bool has_var(std::string_view name) const { return variables_.find(std::string(name)) != variables_.end(); }
    const Variable &get_var(std::string_view name) const {
        auto it = variables_.find(std::string(name));
        LCML_ASSERT(it != variables_.end(), "Variable not found: %.*s", (int)name.size(), name.data());
        return it->second;
    }
    void add_input(std::string_view name) { inputs_.emplace_back(get_var(name)); }
    void add_output(std::string_view name) { outputs_.emplace_back(get_var(name)); }
    void add_node(Node &&n) { nodes_.emplace_back(std::move(n)); }
    const std::string &get_name() const { return name_; }
    const std::unordered_map<std::string, Variable> &get_variables() const { return variables_; }
    const std::vector<std::reference_wrapper<const Variable>> &get_inputs() const { return inputs_; }
    const std::vector<std::reference_wrapper<const Variable>> &get_outputs() const { return outputs_; }
    const std::vector<Node> &get_nodes() const { return nodes_; }
    std::vector<Node> &mutable_nodes() { return nodes_; }
    // variables that no node produces are constants (src/onnx/onnx.cpp:38-48)
    void mark_constants();
};

class OperatorSet {
public:
    using Factory = std::function<std::unique_ptr<Operator>(const Node &)>;

private:
    std::string domain_;
    int64_t version_;
    std::unordered_map<std::string, Factory> factories_;

public:
    OperatorSet(std::string domain, int64_t version) : domain_(std::move(domain)), version_(version) {}
    const std::string &get_domain() const { return domain_; }
    int64_t get_version() const { return version_; }
    // the first registration of a name wins, as the reference's emplace
    // (include/onnx/onnx.h:358)
    void register_operator(std::string name, Factory f) { factories_.try_emplace(std::move(name), std::move(f)); }
    std::unique_ptr<Operator> create_operator(std::string_view name, const Node &node) const {
        auto it = factories_.find(std::string(name));
        LCML_ASSERT(it != factories_.end(), "Operator not found: %.*s", (int)name.size(), name.data());
        return it->second(node);
    }
    bool has_operator(std::string_view name) const { return factories_.find(std::string(name)) != factories_.end(); }
    std::vector<std::string> operator_names() const;

    static OperatorSet &get_default();

    struct RegHelper {
        std::string name;
        OperatorSet &opset;
        explicit RegHelper(std::string n, OperatorSet &o = OperatorSet::get_default()) : name(std::move(n)), opset(o) {}
        bool operator<<(Factory f) {
            opset.register_operator(std::move(name), std::move(f));
            return true;
        }
    };
};

// Static registration, as the reference's macro (onnx.h:382-384).  The
// library is linked as a shared object, so the registrars of every operator
// translation unit run at load time (the reference's static archive needed
// --whole-archive for the same effect).
#define REGISTER_TO_DEFAULT_OPSET(name)                                     \
    [[maybe_unused]] static bool _RegOp##name =                             \
        ::lcml::onnx::OperatorSet::RegHelper(#name) << [](                  \
            [[maybe_unused]] const ::lcml::onnx::Node &node) -> std::unique_ptr<::lcml::onnx::Operator>

class Model {
    int32_t ir_version_ = 0;
    std::string producer_name_, producer_version_;
    Graph graph_;
    OperatorSet *opset_ = &OperatorSet::get_default();

public:
    Model() = default;
    Model(int32_t ir, std::string producer, std::string version)
        : ir_version_(ir), producer_name_(std::move(producer)), producer_version_(std::move(version)) {}
    Model(Model &&) = default;
    Model &operator=(Model &&) = default;
    void set_graph(Graph &&g) {
        graph_ = std::move(g);
        graph_.mark_constants();
    }
    void set_opset(OperatorSet &o) { opset_ = &o; }
    const Graph &get_graph() const { return graph_; }
    Graph &mutable_graph() { return graph_; }
    OperatorSet &get_opset() const { return *opset_; }
    int32_t get_ir_version() const { return ir_version_; }
    const std::string &get_producer_name() const { return producer_name_; }
    const std::string &get_producer_version() const { return producer_version_; }
    // The ONNX-JSON text load_from_json reads back: the reference exporter's
    // format (snake_case keys, dtype names as strings, integers as strings,
    // blob initializers as data_offsets, scripts/export_onnx.py:26-173).
    // Initializers and value_info are written sorted by name, so the text
    // depends only on the graph.
    std::string save_to_json() const;

    // ONNX-JSON (protobuf JSON mapping) with initializers either base64
    // raw_data or data_offsets into an external weight blob
    // (src/onnx/onnx.cpp:87-125, 190-242 of the reference).
    static Model load_from_json(std::string_view json);
};

// Builds the external weight blob of a model file: each add() places the
// bytes at the next 4-byte aligned offset and returns the initializer
// Variable with its data_offsets.  FP8 tensors (FLOAT8E4M3FN / FLOAT8E5M2)
// take ((n + 3) / 4) * 4 bytes, zero padded, the size the loader requires
// of them (src/onnx/network_instance.cpp:222-224); every other type takes
// n * sizeof(element) bytes.
class WeightBlobWriter {
    std::vector<uint8_t> bytes_;

public:
    Variable add(std::string name, DataType dt, std::vector<size_t> shape, const void *data, size_t nbytes);
    const std::vector<uint8_t> &bytes() const { return bytes_; }
};

// Read a scalar/list attribute with a default.
inline float attr_float(const Node &n, std::string_view name, float def) {
    auto *a = n.try_get_attr(name);
    return a ? a->get<AttributeType::FLOAT>() : def;
}
inline int32_t attr_int(const Node &n, std::string_view name, int32_t def) {
    auto *a = n.try_get_attr(name);
    return a ? a->get<AttributeType::INT>() : def;
}
inline std::string attr_string(const Node &n, std::string_view name, std::string def) {
    auto *a = n.try_get_attr(name);
    return a ? a->get<AttributeType::STRING>() : def;
}
inline std::vector<int32_t> attr_ints(const Node &n, std::string_view name, std::vector<int32_t> def) {
    auto *a = n.try_get_attr(name);
    return a ? a->get<AttributeType::INTS>() : def;
}

}  // namespace lcml::onnx
