// onnx_writer.cpp -- Model::save_to_json and WeightBlobWriter: the writing
// side of the ONNX-JSON model format that Model::load_from_json reads.
//
// The reference's exporter (scripts/export_onnx.py:26-173) turns a protobuf
// ModelProto into this form with MessageToJson and cannot emit FP8 tensors
// (its dtype map stops at BFLOAT16, :26-44).  This writer produces the same
// key layout for any graph the loader accepts, FP8 initializers included, so
// FP8 QDQ models can be stored as files: the .onnx.json text plus the raw
// weight blob (no header) that data_offsets index.
#include <algorithm>
#include <cstdio>
#include <cstring>

#include "onnx/onnx.h"

namespace lcml::onnx {

Variable WeightBlobWriter::add(std::string name, DataType dt, std::vector<size_t> shape, const void *data,
                               size_t nbytes) {
    size_t n = 1;
    for (size_t d : shape) n *= d;
    const bool fp8 = dt == DataType::FLOAT8E4M3FN || dt == DataType::FLOAT8E5M2;
    const size_t want = fp8 ? n : n * data_type_bytes(dt);
    LCML_ASSERT(nbytes == want, "WeightBlobWriter: %s holds %zu bytes, its shape needs %zu", name.c_str(), nbytes,
                want);
    const size_t start = (bytes_.size() + 3) / 4 * 4;
    const size_t len = fp8 ? (n + 3) / 4 * 4 : nbytes;
    bytes_.resize(start + len, 0);
    if (nbytes) std::memcpy(bytes_.data() + start, data, nbytes);
    return Variable(std::move(name), dt, std::move(shape), {}, start, start + len);
}

namespace {

class JsonOut {
    std::string s_;
    int depth_ = 0;
    std::vector<bool> first_{true};

    void indent() {
        s_ += '\n';
        s_.append((size_t)depth_ * 2, ' ');
    }
    void sep() {
        if (!first_.back()) s_ += ',';
        first_.back() = false;
        if (depth_ > 0) indent();
    }

public:
    static std::string quote(std::string_view v) {
        std::string o = "\"";
        for (unsigned char c : v) {
            if (c == '"' || c == '\\') {
                o += '\\';
                o += (char)c;
            } else if (c < 0x20) {
                char buf[8];
                std::snprintf(buf, sizeof buf, "\\u%04x", c);
                o += buf;
            } else {
                o += (char)c;
            }
        }
        return o + "\"";
    }
    void open(char br, std::string_view key = {}) {
        sep();
        if (!key.empty()) s_ += quote(key) + ": ";
        s_ += br;
        ++depth_;
        first_.push_back(true);
    }
    void close(char br) {
        const bool empty = first_.back();
        first_.pop_back();
        --depth_;
        if (!empty) indent();
        s_ += br;
    }
    void raw(std::string_view key, const std::string &value) {  // value already JSON
        sep();
        if (!key.empty()) s_ += quote(key) + ": ";
        s_ += value;
    }
    void str(std::string_view key, std::string_view value) { raw(key, quote(value)); }
    std::string take() { return std::move(s_); }
};

std::string base64(std::string_view in) {
    static const char *tab = "ABCDEFGHIJKLMNOPQRSTUVWXYZabcdefghijklmnopqrstuvwxyz0123456789+/";
    std::string out;
    size_t i = 0;
    for (; i + 3 <= in.size(); i += 3) {
        const uint32_t v = ((uint8_t)in[i] << 16) | ((uint8_t)in[i + 1] << 8) | (uint8_t)in[i + 2];
        for (int k = 18; k >= 0; k -= 6) out += tab[(v >> k) & 63];
    }
    if (i + 1 == in.size()) {
        const uint32_t v = (uint8_t)in[i] << 16;
        out += tab[(v >> 18) & 63];
        out += tab[(v >> 12) & 63];
        out += "==";
    } else if (i + 2 == in.size()) {
        const uint32_t v = ((uint8_t)in[i] << 16) | ((uint8_t)in[i + 1] << 8);
        out += tab[(v >> 18) & 63];
        out += tab[(v >> 12) & 63];
        out += tab[(v >> 6) & 63];
        out += '=';
    }
    return out;
}

std::string num(double v) {
    char buf[32];
    std::snprintf(buf, sizeof buf, "%.9g", v);
    return buf;
}

void write_value_info(JsonOut &j, const Variable &v) {
    j.open('{');
    j.str("name", v.get_name());
    j.open('{', "type");
    j.open('{', "tensor_type");
    j.str("elem_type", data_type_name(v.get_dtype()));
    j.open('{', "shape");
    if (!v.get_shape().empty()) {
        j.open('[', "dim");
        for (size_t d : v.get_shape()) {
            j.open('{');
            j.str("dim_value", std::to_string(d));
            j.close('}');
        }
        j.close(']');
    }
    j.close('}');
    j.close('}');
    j.close('}');
    j.close('}');
}

void write_attribute(JsonOut &j, const Attribute &a) {
    j.open('{');
    j.str("name", a.get_name());
    switch (Attribute::type_of(a)) {
    case AttributeType::FLOAT:
        j.raw("f", num(a.get<AttributeType::FLOAT>()));
        j.str("type", "FLOAT");
        break;
    case AttributeType::INT:
        j.str("i", std::to_string(a.get<AttributeType::INT>()));
        j.str("type", "INT");
        break;
    case AttributeType::STRING:
        j.str("s", base64(a.get<AttributeType::STRING>()));
        j.str("type", "STRING");
        break;
    case AttributeType::FLOATS:
        j.open('[', "floats");
        for (float f : a.get<AttributeType::FLOATS>()) j.raw({}, num(f));
        j.close(']');
        j.str("type", "FLOATS");
        break;
    case AttributeType::INTS:
        j.open('[', "ints");
        for (int32_t i : a.get<AttributeType::INTS>()) j.str({}, std::to_string(i));
        j.close(']');
        j.str("type", "INTS");
        break;
    case AttributeType::STRINGS:
        j.open('[', "strings");
        for (auto &t : a.get<AttributeType::STRINGS>()) j.str({}, base64(t));
        j.close(']');
        j.str("type", "STRINGS");
        break;
    default: LCML_ASSERT(false, "attribute %s: unsupported kind", a.get_name().c_str());
    }
    j.close('}');
}

}  // namespace

std::string Model::save_to_json() const {
    const Graph &g = graph_;
    std::vector<const Variable *> inits, infos;
    std::vector<std::string> io;
    for (auto &v : g.get_inputs()) io.push_back(v.get().get_name());
    for (auto &v : g.get_outputs()) io.push_back(v.get().get_name());
    for (auto &[name, v] : g.get_variables()) {
        if (v.has_data()) inits.push_back(&v);
        else if (std::find(io.begin(), io.end(), name) == io.end() && v.get_dtype() != DataType::UNDEFINED &&
                 !v.get_shape().empty())
            infos.push_back(&v);
    }
    auto by_name = [](const Variable *a, const Variable *b) { return a->get_name() < b->get_name(); };
    std::sort(inits.begin(), inits.end(), by_name);
    std::sort(infos.begin(), infos.end(), by_name);

    JsonOut j;
    j.open('{');
    j.str("ir_version", std::to_string(ir_version_));
    j.str("producer_name", producer_name_);
    j.str("producer_version", producer_version_);
    j.open('{', "graph");
    j.open('[', "node");
    for (const Node &n : g.get_nodes()) {
        j.open('{');
        j.open('[', "input");
        for (auto &v : n.get_inputs()) j.str({}, v.get().get_name());
        j.close(']');
        j.open('[', "output");
        for (auto &v : n.get_outputs()) j.str({}, v.get().get_name());
        j.close(']');
        j.str("name", n.get_name());
        j.str("op_type", n.get_op_type());
        if (!n.get_attributes().empty()) {
            j.open('[', "attribute");
            for (auto &[k, a] : n.get_attributes()) write_attribute(j, a);
            j.close(']');
        }
        j.close('}');
    }
    j.close(']');
    j.str("name", g.get_name());
    j.open('[', "initializer");
    for (const Variable *v : inits) {
        j.open('{');
        j.open('[', "dims");
        for (size_t d : v->get_shape()) j.str({}, std::to_string(d));
        j.close(']');
        j.str("data_type", data_type_name(v->get_dtype()));
        j.str("name", v->get_name());
        if (v->is_trainable_weight()) {
            auto [s, e] = v->get_buffer_range();
            j.open('[', "data_offsets");
            j.raw({}, std::to_string(s));
            j.raw({}, std::to_string(e));
            j.close(']');
        } else {
            j.str("raw_data", base64(v->get_raw_data()));
        }
        j.close('}');
    }
    j.close(']');
    j.open('[', "input");
    for (auto &v : g.get_inputs()) write_value_info(j, v.get());
    j.close(']');
    j.open('[', "output");
    for (auto &v : g.get_outputs()) write_value_info(j, v.get());
    j.close(']');
    j.open('[', "value_info");
    for (const Variable *v : infos) write_value_info(j, *v);
    j.close(']');
    j.close('}');
    j.open('[', "opset_import");
    j.open('{');
    j.str("domain", "");
    j.str("version", std::to_string(opset_->get_version()));
    j.close('}');
    j.close(']');
    j.close('}');
    return j.take() + "\n";
}

}  // namespace lcml::onnx
