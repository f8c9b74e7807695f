// onnx.cpp -- data types, the default operator set and the ONNX-JSON loader.
//
// The loader reads the protobuf-JSON form the reference consumes
// (src/onnx/onnx.cpp:87-242): graph.node[] with op_type / input / output /
// attribute[] (INT values as strings, FLOAT as numbers, STRING as base64),
// graph.initializer[] with dims (strings), data_type (enum name) and either
// base64 raw_data or data_offsets [start, end) into an external weight blob
// (an initializer without dims is shape [1], :93-94), and graph.input /
// output / value_info with tensor_type shapes.
#include <cctype>
#include <cstdlib>
#include <cstring>
#include <unordered_set>

#include "onnx/onnx.h"

namespace lcml::onnx {

OperatorSet &OperatorSet::get_default() {
    static OperatorSet opset{"default", 21};
    return opset;
}

std::vector<std::string> OperatorSet::operator_names() const {
    std::vector<std::string> v;
    for (auto &kv : factories_) v.push_back(kv.first);
    return v;
}

namespace {
struct DTypeInfo {
    DataType dt;
    const char *name;
    size_t bytes;
};
const DTypeInfo kDTypes[] = {
    {DataType::FLOAT, "FLOAT", 4},          {DataType::UINT8, "UINT8", 1},
    {DataType::INT8, "INT8", 1},            {DataType::INT32, "INT32", 4},
    {DataType::INT64, "INT64", 8},          {DataType::FLOAT16, "FLOAT16", 2},
    {DataType::DOUBLE, "DOUBLE", 8},        {DataType::BFLOAT16, "BFLOAT16", 2},
    {DataType::FLOAT8E4M3FN, "FLOAT8E4M3FN", 1}, {DataType::FLOAT8E4M3FNUZ, "FLOAT8E4M3FNUZ", 1},
    {DataType::FLOAT8E5M2, "FLOAT8E5M2", 1},     {DataType::FLOAT8E5M2FNUZ, "FLOAT8E5M2FNUZ", 1},
};
}  // namespace

std::string_view data_type_name(DataType dt) {
    for (auto &d : kDTypes)
        if (d.dt == dt) return d.name;
    return "UNDEFINED";
}

DataType data_type_from_name(std::string_view name) {
    for (auto &d : kDTypes)
        if (name == d.name) return d.dt;
    LCML_ASSERT(false, "Unsupported ONNX DataType: %.*s", (int)name.size(), name.data());
    return DataType::UNDEFINED;
}

size_t data_type_bytes(DataType dt) {
    for (auto &d : kDTypes)
        if (d.dt == dt) return d.bytes;
    LCML_ASSERT(false, "Unsupported ONNX DataType: %d", (int)dt);
    return 0;
}

refl::TypeIndex data_type_to_type_index(DataType dt) {
    switch (dt) {
    case DataType::FLOAT: return refl::type_index_of<float>();
    case DataType::FLOAT8E4M3FN: return refl::type_index_of<FP8E4M3FN>();
    case DataType::FLOAT8E5M2: return refl::type_index_of<FP8E5M2>();
    case DataType::BFLOAT16: return refl::type_index_of<BFloat16>();
    case DataType::INT64: return refl::type_index_of<int64_t>();
    default: LCML_ASSERT(false, "Unsupported ONNX DataType on the FP8 path: %s", data_type_name(dt).data());
    }
    return 0;
}

void Graph::mark_constants() {
    std::unordered_set<std::string> produced;
    for (auto &n : nodes_)
        for (auto &o : n.get_outputs()) produced.insert(o.get().get_name());
    for (auto &kv : variables_) kv.second.set_is_constant(produced.find(kv.first) == produced.end());
    // graph inputs are runtime data, not constants
    for (auto &in : inputs_) variables_.at(in.get().get_name()).set_is_constant(false);
}

// ---------------------------------------------------------------- JSON ----

namespace {

struct JValue {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    double num = 0;
    bool b = false;
    std::string str;
    std::vector<JValue> arr;
    std::vector<std::pair<std::string, JValue>> obj;

    const JValue *get(std::string_view k) const {
        for (auto &kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
    const JValue &at(std::string_view k) const {
        auto *v = get(k);
        LCML_ASSERT(v, "JSON: missing key %.*s", (int)k.size(), k.data());
        return *v;
    }
    std::string as_string() const {
        if (kind == Str) return str;
        LCML_ASSERT(kind == Num, "JSON: expected string");
        char buf[64];
        std::snprintf(buf, sizeof buf, "%.17g", num);
        return buf;
    }
    double as_number() const {
        if (kind == Num) return num;
        LCML_ASSERT(kind == Str, "JSON: expected number");
        return std::strtod(str.c_str(), nullptr);
    }
    int64_t as_int() const {
        if (kind == Str) return std::strtoll(str.c_str(), nullptr, 10);
        LCML_ASSERT(kind == Num, "JSON: expected integer");
        return (int64_t)num;
    }
};

class JParser {
    std::string_view s_;
    size_t i_ = 0;

    void ws() {
        while (i_ < s_.size() && std::isspace((unsigned char)s_[i_])) ++i_;
    }
    char peek() {
        ws();
        LCML_ASSERT(i_ < s_.size(), "JSON: unexpected end of input");
        return s_[i_];
    }
    void expect(char c) {
        LCML_ASSERT(peek() == c, "JSON: expected '%c' at offset %zu", c, i_);
        ++i_;
    }
    std::string parse_string() {
        expect('"');
        std::string out;
        while (true) {
            LCML_ASSERT(i_ < s_.size(), "JSON: unterminated string");
            char c = s_[i_++];
            if (c == '"') break;
            if (c == '\\') {
                LCML_ASSERT(i_ < s_.size(), "JSON: bad escape");
                char e = s_[i_++];
                switch (e) {
                case 'n': out += '\n'; break;
                case 't': out += '\t'; break;
                case 'r': out += '\r'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'u': {
                    LCML_ASSERT(i_ + 4 <= s_.size(), "JSON: bad \\u escape");
                    unsigned cp = (unsigned)std::strtoul(std::string(s_.substr(i_, 4)).c_str(), nullptr, 16);
                    i_ += 4;
                    if (cp < 0x80) out += (char)cp;
                    else if (cp < 0x800) { out += (char)(0xC0 | (cp >> 6)); out += (char)(0x80 | (cp & 63)); }
                    else { out += (char)(0xE0 | (cp >> 12)); out += (char)(0x80 | ((cp >> 6) & 63)); out += (char)(0x80 | (cp & 63)); }
                    break;
                }
                default: out += e;
                }
            } else {
                out += c;
            }
        }
        return out;
    }

public:
    explicit JParser(std::string_view s) : s_(s) {}
    JValue parse() {
        JValue v;
        char c = peek();
        if (c == '{') {
            v.kind = JValue::Obj;
            ++i_;
            if (peek() == '}') { ++i_; return v; }
            while (true) {
                std::string k = parse_string();
                expect(':');
                v.obj.emplace_back(std::move(k), parse());
                if (peek() == ',') { ++i_; continue; }
                expect('}');
                break;
            }
        } else if (c == '[') {
            v.kind = JValue::Arr;
            ++i_;
            if (peek() == ']') { ++i_; return v; }
            while (true) {
                v.arr.push_back(parse());
                if (peek() == ',') { ++i_; continue; }
                expect(']');
                break;
            }
        } else if (c == '"') {
            v.kind = JValue::Str;
            v.str = parse_string();
        } else if (s_.compare(i_, 4, "true") == 0) { v.kind = JValue::Bool; v.b = true; i_ += 4; }
        else if (s_.compare(i_, 5, "false") == 0) { v.kind = JValue::Bool; i_ += 5; }
        else if (s_.compare(i_, 4, "null") == 0) { i_ += 4; }
        else {
            v.kind = JValue::Num;
            const char *b = s_.data() + i_;
            char *e = nullptr;
            v.num = std::strtod(b, &e);
            LCML_ASSERT(e != b, "JSON: bad value at offset %zu", i_);
            i_ += (size_t)(e - b);
        }
        return v;
    }
};

std::string base64_decode(std::string_view in) {
    auto val = [](char c) -> int {
        if (c >= 'A' && c <= 'Z') return c - 'A';
        if (c >= 'a' && c <= 'z') return c - 'a' + 26;
        if (c >= '0' && c <= '9') return c - '0' + 52;
        if (c == '+' || c == '-') return 62;
        if (c == '/' || c == '_') return 63;
        return -1;
    };
    std::string out;
    int bits = 0, acc = 0;
    for (char c : in) {
        int v = val(c);
        if (v < 0) continue;  // '=' padding and whitespace
        acc = (acc << 6) | v;
        bits += 6;
        if (bits >= 8) {
            bits -= 8;
            out += (char)((acc >> bits) & 0xFF);
        }
    }
    return out;
}

// A tensor type without a dim list (how ONNX writes a scalar, e.g. the
// y_scale / y_zero_point outputs of DynamicQuantizeLinear) has shape [1], as
// in the reference's Variable::from_json (src/onnx/onnx.cpp:93-95).
std::vector<size_t> shape_of_type(const JValue &type) {
    std::vector<size_t> shape;
    auto *tt = type.get("tensor_type");
    if (!tt) return shape;
    auto *sh = tt->get("shape");
    auto *dims = sh ? sh->get("dim") : nullptr;
    if (!dims || dims->arr.empty()) return {1};
    for (auto &d : dims->arr) {
        auto *dv = d.get("dim_value");
        LCML_ASSERT(dv, "graph variable with a symbolic dimension (static shapes are required)");
        shape.push_back((size_t)dv->as_int());
    }
    return shape;
}

Variable variable_from_json(const JValue &j) {
    std::string name = j.at("name").as_string();
    DataType dt = DataType::UNDEFINED;
    std::vector<size_t> shape;
    if (auto *t = j.get("type")) {
        if (auto *tt = t->get("tensor_type"))
            if (auto *et = tt->get("elem_type")) dt = et->kind == JValue::Str ? data_type_from_name(et->str) : (DataType)et->as_int();
        shape = shape_of_type(*t);
    }
    return Variable{std::move(name), dt, std::move(shape)};
}

Variable initializer_from_json(const JValue &j) {
    std::string name = j.at("name").as_string();
    const JValue &dtv = j.at("data_type");
    DataType dt = dtv.kind == JValue::Str ? data_type_from_name(dtv.str) : (DataType)dtv.as_int();
    std::vector<size_t> shape;
    if (auto *dims = j.get("dims")) {
        for (auto &d : dims->arr) shape.push_back((size_t)d.as_int());
    }
    if (shape.empty()) shape.push_back(1);  // a scalar initializer (onnx.cpp:107-108)
    if (auto *off = j.get("data_offsets")) {
        LCML_ASSERT(off->arr.size() == 2, "initializer %s: data_offsets needs [start, end]", name.c_str());
        return Variable{std::move(name), dt, std::move(shape), {}, (uint64_t)off->arr[0].as_int(),
                        (uint64_t)off->arr[1].as_int()};
    }
    std::string raw;
    if (auto *r = j.get("raw_data")) raw = base64_decode(r->as_string());
    return Variable{std::move(name), dt, std::move(shape), std::move(raw)};
}

Attribute attribute_from_json(const JValue &j) {
    std::string name = j.at("name").as_string();
    std::string type = j.at("type").as_string();
    if (type == "FLOAT") return Attribute{name, (float)j.at("f").as_number()};
    if (type == "INT") return Attribute{name, (int32_t)j.at("i").as_int()};
    if (type == "STRING") return Attribute{name, base64_decode(j.at("s").as_string())};
    if (type == "FLOATS") {
        std::vector<float> v;
        if (auto *a = j.get("floats"))
            for (auto &x : a->arr) v.push_back((float)x.as_number());
        return Attribute{name, std::move(v)};
    }
    if (type == "INTS") {
        std::vector<int32_t> v;
        if (auto *a = j.get("ints"))
            for (auto &x : a->arr) v.push_back((int32_t)x.as_int());
        return Attribute{name, std::move(v)};
    }
    if (type == "STRINGS") {
        std::vector<std::string> v;
        if (auto *a = j.get("strings"))
            for (auto &x : a->arr) v.push_back(base64_decode(x.as_string()));
        return Attribute{name, std::move(v)};
    }
    LCML_ASSERT(false, "attribute %s: unsupported type %s", name.c_str(), type.c_str());
    return {};
}

}  // namespace

Model Model::load_from_json(std::string_view json) {
    JValue root = JParser(json).parse();
    Model m((int32_t)(root.get("ir_version") ? root.at("ir_version").as_int() : 0),
            root.get("producer_name") ? root.at("producer_name").as_string() : "",
            root.get("producer_version") ? root.at("producer_version").as_string() : "");
    const JValue &gj = root.at("graph");
    Graph g(gj.get("name") ? gj.at("name").as_string() : "");
    if (auto *inits = gj.get("initializer"))
        for (auto &i : inits->arr) g.add_variable(initializer_from_json(i));
    auto add_vars = [&](const char *key) {
        if (auto *arr = gj.get(key))
            for (auto &v : arr->arr) {
                Variable var = variable_from_json(v);
                if (!g.has_var(var.get_name())) g.add_variable(std::move(var));
            }
    };
    add_vars("input");
    add_vars("output");
    add_vars("value_info");
    const OperatorSet &opset = m.get_opset();
    if (auto *nodes = gj.get("node")) {
        for (auto &nj : nodes->arr) {
            std::string op = nj.at("op_type").as_string();
            Node n(nj.get("name") ? nj.at("name").as_string() : "", op);
            LCML_ASSERT(opset.has_operator(op), "Operator not found: %s", op.c_str());
            if (auto *ins = nj.get("input"))
                for (auto &x : ins->arr) {
                    std::string vn = x.as_string();
                    if (vn.empty()) continue;  // omitted optional input
                    n.add_input(g.get_var(vn));
                }
            if (auto *outs = nj.get("output"))
                for (auto &x : outs->arr) {
                    std::string vn = x.as_string();
                    if (!g.has_var(vn)) g.add_variable(Variable{vn, DataType::UNDEFINED, {}});
                    n.add_output(g.get_var(vn));
                }
            if (auto *attrs = nj.get("attribute"))
                for (auto &a : attrs->arr) n.set_attribute(attribute_from_json(a));
            g.add_node(std::move(n));
        }
    }
    if (auto *arr = gj.get("input"))
        for (auto &v : arr->arr) {
            std::string n = v.at("name").as_string();
            // graph inputs that are also initializers are weights, not runtime inputs
            bool is_init = false;
            if (auto *inits = gj.get("initializer"))
                for (auto &i : inits->arr) is_init |= i.at("name").as_string() == n;
            if (!is_init) g.add_input(n);
        }
    if (auto *arr = gj.get("output"))
        for (auto &v : arr->arr) g.add_output(v.at("name").as_string());
    m.set_graph(std::move(g));
    return m;
}

}  // namespace lcml::onnx
