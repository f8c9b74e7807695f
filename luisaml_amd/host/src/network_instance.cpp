// network_instance.cpp -- binding, initializer tensors, QDQ fusion, weight
// packing and eager execution (see network_instance.h).
#include "onnx/network_instance.h"

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <unordered_map>
#include <unordered_set>

#include "lcml_fp8.h"

namespace lcml::onnx {

namespace {

ITensor::shape_type to_tensor_shape(const std::vector<size_t> &s) {
    ITensor::shape_type out;
    for (auto d : s) out.push_back((ITensor::size_type)d);
    return out;
}

void hip_check(hipError_t e, const char *what) {
    LCML_ASSERT(e == hipSuccess, "%s: %s", what, hipGetErrorString(e));
}

void lcml_check(int rc, const char *what) {
    LCML_ASSERT(rc == 0, "%s: %s", what, lcml_fp8_last_error());
}

}  // namespace

void NetworkInstance::set_model(Model &&m) {
    model_ = std::move(m);
    prepared_ = false;
    ops_.clear();
    table_.clear();
}

void NetworkInstance::set_weight_buffer(const void *device_blob, size_t bytes) {
    weight_buffer_ = static_cast<const uint8_t *>(device_blob);
    weight_bytes_ = bytes;
}

void NetworkInstance::set_input(std::string_view name, ITensor &t) {
    inputs_.insert_or_assign(std::string(name), std::ref(t));
}

void NetworkInstance::set_output(std::string_view name, ITensor &t) {
    outputs_.insert_or_assign(std::string(name), std::ref(t));
}

// Dtype and shape of an external tensor must match the graph variable
// (src/onnx/network_instance.cpp:40-69 of the reference).
void NetworkInstance::validate_and_bind(std::string_view role, const Variable &var, ITensor &t) {
    LCML_ASSERT(t.element_type_index() == data_type_to_type_index(var.get_dtype()),
                "%.*s '%s': element type %.*s does not match graph dtype %s", (int)role.size(), role.data(),
                var.get_name().c_str(), (int)t.element_type_name().size(), t.element_type_name().data(),
                data_type_name(var.get_dtype()).data());
    auto shape = to_tensor_shape(var.get_shape());
    if (!shape.empty()) {
        LCML_ASSERT(t.shape() == shape, "%.*s '%s': shape mismatch", (int)role.size(), role.data(),
                    var.get_name().c_str());
    }
    table_.bind(var.get_name(), t);
}

// Initializers (from raw_data or the weight blob) and intermediates
// (allocated from the variable's static shape), as create_tensor_for_var
// (src/onnx/network_instance.cpp:202-342).
void NetworkInstance::create_tensor_for_var(const Variable &var) {
    if (table_.contains(var.get_name())) return;
    const auto &name = var.get_name();
    const size_t n = var.num_elements();
    auto shape = to_tensor_shape(var.get_shape());
    visit_type_index<NNTypeList>(data_type_to_type_index(var.get_dtype()), [&]<typename T>() {
        if (var.is_trainable_weight()) {
            LCML_ASSERT(weight_buffer_ != nullptr, "Weight buffer not set but required for variable: %s",
                        name.c_str());
            auto [start, end] = var.get_buffer_range();
            LCML_ASSERT(end <= weight_bytes_, "variable %s: data_offsets beyond the weight buffer", name.c_str());
            if constexpr (std::is_same_v<T, FP8E4M3FN> || std::is_same_v<T, FP8E5M2>) {
                // FP8 blobs are 4-byte padded (network_instance.cpp:222-224)
                LCML_ASSERT(end - start == ((n + 3) / 4) * 4, "Weight buffer size mismatch for variable: %s",
                            name.c_str());
            } else {
                LCML_ASSERT(end - start == n * sizeof(T), "Weight buffer size mismatch for variable: %s",
                            name.c_str());
            }
            std::vector<uint8_t> host;
            if (end - start <= 4096) {  // small constants (scales, zero points) get a host copy
                host.resize(end - start);
                hip_check(hipMemcpy(host.data(), weight_buffer_ + start, end - start, hipMemcpyDeviceToHost),
                          "hipMemcpy");
            }
            table_.own(name, std::make_unique<ConstTensor<T>>(
                                 shape, DeviceArray<T>(const_cast<uint8_t *>(weight_buffer_), start, n),
                                 std::move(host)));
        } else if (!var.get_raw_data().empty()) {
            const auto &raw = var.get_raw_data();
            LCML_ASSERT(raw.size() == n * sizeof(T), "variable %s: raw_data holds %zu bytes, expected %zu",
                        name.c_str(), raw.size(), n * sizeof(T));
            DeviceArray<T> arr(n);
            hip_check(hipMemcpy(arr.data(), raw.data(), raw.size(), hipMemcpyHostToDevice), "hipMemcpy");
            table_.own(name, std::make_unique<ConstTensor<T>>(shape, std::move(arr),
                                                              std::vector<uint8_t>(raw.begin(), raw.end())));
        } else if (auto it = planned_.find(name); it != planned_.end()) {
            table_.own(name, std::make_unique<NNTensor<T>>(shape, DeviceArray<T>(arena_, it->second, n)));
        } else {
            LCML_ASSERT(!shape.empty() || n == 1, "variable %s has no static shape", name.c_str());
            table_.own(name, make_device_tensor<T>(shape));
        }
    });
}

// ------------------------------------------------------------------------
// QDQ fusion:  [x -> QuantizeLinear(s) -> DequantizeLinear(s)] or
// [x -> DynamicQuantizeLinear -> DequantizeLinear] or plain fp32 A, and
// DequantizeLinear(W_e4m3 constant, s_w) as B, into Gemm/MatMul, optionally
// followed by Relu/Gelu, become one FP8Linear node; the same with a quantised
// activation into Conv (4-D E4M3 weight, channels per group % 16 == 0)
// becomes one FP8Conv node.
// ------------------------------------------------------------------------
// An E4M3 zero point that is a constant holding only 0x00 bytes, embedded
// (raw_data) or in the weight blob (read back from the device; a zero point
// is one byte per scale entry, so at most a few KB).  Anything else -- another
// element type, a non-constant, a nonzero byte -- keeps the node unfused.
bool NetworkInstance::is_zero_e4m3_constant(const Variable &v) const {
    if (!v.is_constant() || v.get_dtype() != DataType::FLOAT8E4M3FN) return false;
    const size_t n = v.num_elements();
    auto zero = [](const uint8_t *p, size_t k) { return std::all_of(p, p + k, [](uint8_t c) { return c == 0; }); };
    const std::string &raw = v.get_raw_data();
    if (!raw.empty()) return raw.size() >= n && zero(reinterpret_cast<const uint8_t *>(raw.data()), n);
    if (!v.is_trainable_weight() || weight_buffer_ == nullptr) return false;
    auto [start, end] = v.get_buffer_range();
    if (end > weight_bytes_ || end - start < n || n > 65536) return false;
    std::vector<uint8_t> host(n);
    hip_check(hipMemcpy(host.data(), weight_buffer_ + start, n, hipMemcpyDeviceToHost), "hipMemcpy");
    return zero(host.data(), n);
}

void NetworkInstance::fuse_qdq_linear() {
    Graph &g = model_.mutable_graph();
    auto &nodes = g.mutable_nodes();
    std::unordered_map<std::string, size_t> producer;
    std::unordered_map<std::string, std::vector<size_t>> consumers;
    for (size_t i = 0; i < nodes.size(); ++i) {
        for (auto &o : nodes[i].get_outputs()) producer[o.get().get_name()] = i;
        for (auto &in : nodes[i].get_inputs()) consumers[in.get().get_name()].push_back(i);
    }
    std::unordered_set<std::string> graph_outputs;
    for (auto &o : g.get_outputs()) graph_outputs.insert(o.get().get_name());
    auto only_consumer = [&](const std::string &v, size_t who) {
        auto it = consumers.find(v);
        return it != consumers.end() && it->second.size() == 1 && it->second[0] == who && !graph_outputs.count(v);
    };
    auto prod = [&](const std::string &v) -> const Node * {
        auto it = producer.find(v);
        return it == producer.end() ? nullptr : &nodes[it->second];
    };
    auto prod_idx = [&](const std::string &v) { return producer.at(v); };

    // Activation side of node `who`'s input A: static QDQ (a_mode 1),
    // dynamic QDQ (2) or neither (0, A itself); the Q and DQ nodes to drop.
    struct ActQ {
        int a_mode = 0;
        const Variable *src = nullptr, *scale = nullptr;
        std::vector<size_t> drop;
    };
    auto match_act = [&](const Variable &A, size_t who) {
        ActQ r;
        r.src = &A;
        const Node *dqa = prod(A.get_name());
        if (!dqa || dqa->get_op_type() != "DequantizeLinear" || !only_consumer(A.get_name(), who)) return r;
        const Variable &qv = dqa->get_inputs()[0].get();
        // the fused kernels quantise to E4M3: an E5M2 or integer Q -> DQ stays
        // op by op (its own QuantizeLinear / DequantizeLinear semantics)
        if (qv.get_dtype() != DataType::FLOAT8E4M3FN) return r;
        const Node *q = prod(qv.get_name());
        // the DQ zero point is a constant 0, or DynamicQuantizeLinear's own (zero) output
        bool zp_ok = dqa->get_inputs().size() <= 2 || is_zero_e4m3_constant(dqa->get_inputs()[2].get()) ||
                     (q && q->get_op_type() == "DynamicQuantizeLinear" && q->get_outputs().size() > 2 &&
                      &q->get_outputs()[2].get() == &dqa->get_inputs()[2].get());
        if (!q || !zp_ok || !only_consumer(qv.get_name(), prod_idx(A.get_name())) ||
            dqa->get_inputs()[1].get().num_elements() != 1)
            return r;
        if (q->get_op_type() == "QuantizeLinear" && &q->get_inputs()[1].get() == &dqa->get_inputs()[1].get() &&
            (q->get_inputs().size() <= 2 || is_zero_e4m3_constant(q->get_inputs()[2].get())) &&
            attr_int(*q, "saturate", 1) == 1) {
            r.a_mode = 1;
            r.src = &q->get_inputs()[0].get();
            r.scale = &q->get_inputs()[1].get();
        } else if (q->get_op_type() == "DynamicQuantizeLinear" &&
                   &q->get_outputs()[1].get() == &dqa->get_inputs()[1].get()) {
            bool private_outputs = true;
            for (size_t o = 0; o < q->get_outputs().size(); ++o) {
                const auto &on = q->get_outputs()[o].get().get_name();
                if (graph_outputs.count(on)) private_outputs = false;
                auto it = consumers.find(on);
                if (it != consumers.end())
                    for (size_t c : it->second)
                        if (c != prod_idx(A.get_name())) private_outputs = false;
            }
            if (private_outputs) {
                r.a_mode = 2;
                r.src = &q->get_inputs()[0].get();
            }
        }
        if (r.a_mode) r.drop = {prod_idx(A.get_name()), prod_idx(qv.get_name())};
        return r;
    };
    // a Relu/Gelu that is the only consumer of `out` becomes the epilogue
    auto match_epilogue = [&](const Variable *&out, std::vector<size_t> &drop) {
        int act = LCML_ACT_NONE;
        auto cit = consumers.find(out->get_name());
        if (cit != consumers.end() && cit->second.size() == 1 && !graph_outputs.count(out->get_name())) {
            const Node &r = nodes[cit->second[0]];
            if (r.get_op_type() == "Relu") act = LCML_ACT_RELU;
            else if (r.get_op_type() == "Gelu")
                act = attr_string(r, "approximate", "none") == "tanh" ? LCML_ACT_GELU_TANH : LCML_ACT_GELU_ERF;
            if (act != LCML_ACT_NONE) {
                drop.push_back(cit->second[0]);
                out = &r.get_outputs()[0].get();
            }
        }
        return act;
    };
    // B = DequantizeLinear(W_e4m3 constant of rank `rank`, constant scale [, 0]) feeding only `who`
    auto match_weight = [&](const Variable &B, size_t who, size_t rank) -> const Node * {
        const Node *dqw = prod(B.get_name());
        if (!dqw || dqw->get_op_type() != "DequantizeLinear" || !only_consumer(B.get_name(), who)) return nullptr;
        const Variable &W = dqw->get_inputs()[0].get();
        if (W.get_dtype() != DataType::FLOAT8E4M3FN || !W.is_constant() || W.get_shape().size() != rank)
            return nullptr;
        if (!dqw->get_inputs()[1].get().is_constant()) return nullptr;
        if (dqw->get_inputs().size() > 2 && !is_zero_e4m3_constant(dqw->get_inputs()[2].get())) return nullptr;
        return dqw;
    };

    std::vector<bool> removed(nodes.size(), false);
    std::unordered_map<size_t, Node> replacement;
    for (size_t i = 0; i < nodes.size(); ++i) {
        const Node &n = nodes[i];
        if (n.get_op_type() == "Conv") {
            // ---- DQ(x) , DQ(W_e4m3 [cout, cin, kh, kw]) -> Conv [-> act] ----
            // 2-D, or 1-D as a 1 x kl kernel over [n, c, 1, l]; auto_pad is
            // ignored as in the reference (only `pads` enters, conv.cpp:257-275)
            const int group = attr_int(n, "group", 1);
            if (n.get_inputs().size() < 2 || group < 1) continue;
            const Variable &X = n.get_inputs()[0].get();
            const Variable &Bv = n.get_inputs()[1].get();
            const size_t rank = X.get_shape().size();
            if (rank != 3 && rank != 4) continue;
            const Node *dqw = match_weight(Bv, i, rank);
            if (!dqw) continue;
            const Variable &W = dqw->get_inputs()[0].get();
            const Variable &sw = dqw->get_inputs()[1].get();
            const auto &ws = W.get_shape();
            // cin: channels per group
            const size_t cout = ws[0], cin = ws[1], kh = rank == 4 ? ws[2] : 1, kw = ws[rank - 1];
            if (cin % 16 != 0 || cout % (size_t)group != 0) continue;
            if (sw.num_elements() != 1 && !(sw.num_elements() == cout && attr_int(*dqw, "axis", 1) == 0)) continue;
            if (X.get_shape()[1] != cin * (size_t)group) continue;
            ActQ aq = match_act(X, i);
            if (aq.a_mode == 0) continue;  // FP8 conv needs a quantised activation
            std::vector<size_t> drop = aq.drop;
            drop.push_back(prod_idx(Bv.get_name()));
            const Variable *out = &n.get_outputs()[0].get();
            const int act = match_epilogue(out, drop);
            std::string pname = W.get_name() + "::packed_conv::" + sw.get_name() + "::g" + std::to_string(group);
            if (!g.has_var(pname)) {
                Variable pv(pname, DataType::FLOAT8E4M3FN, {kh * kw * cin, cout});
                pv.set_is_constant(true);
                g.add_variable(std::move(pv));
            }
            Node f(n.get_name().empty() ? "fp8_conv" : n.get_name() + "::fp8", "FP8Conv");
            f.add_input(*aq.src);
            f.add_input(g.get_var(pname));
            f.add_input(sw);
            if (aq.a_mode == 1) f.add_input(*aq.scale);
            const bool has_bias = n.get_inputs().size() > 2;
            if (has_bias) f.add_input(n.get_inputs()[2].get());
            f.add_output(*out);
            for (const char *a : {"strides", "pads", "dilations", "group"})
                if (auto *at = n.try_get_attr(a)) f.set_attribute(*at);
            f.set_attribute(Attribute{"kernel_shape", rank == 4 ? std::vector<int32_t>{(int32_t)kh, (int32_t)kw}
                                                                 : std::vector<int32_t>{(int32_t)kw}});
            f.set_attribute(Attribute{"a_mode", (int32_t)aq.a_mode});
            f.set_attribute(Attribute{"has_bias", (int32_t)has_bias});
            f.set_attribute(Attribute{"act", (int32_t)act});
            f.set_attribute(Attribute{"fp8_mfma", (int32_t)fp8_mfma_});
            f.set_attribute(Attribute{"weight", W.get_name()});
            for (size_t d : drop) removed[d] = true;
            replacement.emplace(i, std::move(f));
            ++fused_count_;
            continue;
        }
        const bool gemm = n.get_op_type() == "Gemm", matmul = n.get_op_type() == "MatMul";
        if (!gemm && !matmul) continue;
        // transA = 1 (A is [K, M], gemm.cpp:35-40) fuses with a quantised
        // activation: the quantiser writes the transposed E4M3 copy
        const bool trans_a = gemm && attr_int(n, "transA", 0) != 0;
        const Variable &A = n.get_inputs()[0].get();
        const Variable &B = n.get_inputs()[1].get();
        // ---- B = DequantizeLinear(W_e4m3 constant, s_w [, 0]) ----
        // MatMul also takes a batched weight [..., K, N] (mat_mul.cpp:187-303):
        // one packed weight per batch, batch dimensions right-aligned and
        // broadcast against A's where they are 1
        const size_t wrank = matmul && B.get_shape().size() >= 3 ? B.get_shape().size() : 2;
        const Node *dqw = match_weight(B, i, wrank);
        if (!dqw) continue;
        const Variable &W = dqw->get_inputs()[0].get();
        const Variable &sw = dqw->get_inputs()[1].get();
        const bool w_is_nk = gemm && attr_int(n, "transB", 0) != 0;
        const auto &wsh = W.get_shape();
        const size_t N = w_is_nk ? wsh[0] : wsh[wrank - 1];
        const size_t K = w_is_nk ? wsh[1] : wsh[wrank - 2];
        const size_t nscale = sw.num_elements();
        if (nscale != 1) {
            int axis = attr_int(*dqw, "axis", 1);
            if (axis < 0) axis += (int)wrank;
            const int n_axis = w_is_nk ? 0 : (int)wrank - 1;
            if (axis != n_axis || nscale != N) continue;  // only per-output-channel scales fuse
        }
        if (A.get_shape().empty()) continue;
        std::vector<int32_t> wbatch;  // the weight's batch dimensions
        if (wrank > 2) {
            const auto &ash = A.get_shape();
            if (ash.size() < 2) continue;  // a 1-D A against a batched weight stays unfused
            const size_t ab = ash.size() - 2, bb = wrank - 2, nb = std::max(ab, bb);
            bool bcast = true;
            for (size_t d = 0; d < nb; ++d) {
                const size_t ad = d + ab >= nb ? ash[d + ab - nb] : 1, bd = d + bb >= nb ? wsh[d + bb - nb] : 1;
                bcast = bcast && (ad == bd || ad == 1 || bd == 1);
            }
            if (!bcast) continue;
            for (size_t d = 0; d < bb; ++d) wbatch.push_back((int32_t)wsh[d]);
        }
        if (trans_a ? (A.get_shape().size() != 2 || A.get_shape()[0] != K) : A.get_shape().back() != K) continue;
        // ---- A: static QDQ, dynamic QDQ, or fp32 ----
        ActQ aq = match_act(A, i);
        // E4M3 activation rows need a 16-byte pitch (K % 16 == 0); otherwise
        // the activation's Q/DQ nodes stay and the fused node runs W8A32 on
        // their (exactly representable) fp32 output
        if (aq.a_mode != 0 && K % 16 != 0) aq = ActQ{0, &A, nullptr, {}};
        if (trans_a && aq.a_mode == 0) continue;  // W8A32 reads A row-major: stays unfused
        const int a_mode = aq.a_mode;  // 0: fp32 (W8A32), 1: static scale, 2: dynamic per-tensor
        const Variable *a_src = aq.src, *a_scale = aq.scale;
        std::vector<size_t> drop = {prod_idx(B.get_name())};
        drop.insert(drop.end(), aq.drop.begin(), aq.drop.end());
        if (a_mode == 0 && A.get_dtype() != DataType::FLOAT) continue;
        // ---- epilogue activation ----
        const Variable *out = &n.get_outputs()[0].get();
        const int act = match_epilogue(out, drop);
        // ---- build the fused node ----
        // one packed copy per (weight, scale, layout): a weight shared by two
        // nodes through different DequantizeLinear scales or transB packs twice
        std::string pname = W.get_name() + "::packed::" + sw.get_name() + (w_is_nk ? "::nk" : "::kn");
        if (!g.has_var(pname)) {
            std::vector<size_t> pshape(wsh.begin(), wsh.end() - 2);  // batch dimensions, then [K, N]
            pshape.push_back(K);
            pshape.push_back(N);
            Variable pv(pname, DataType::FLOAT8E4M3FN, pshape);
            pv.set_is_constant(true);
            g.add_variable(std::move(pv));
        }
        Node f(n.get_name().empty() ? "fp8_linear" : n.get_name() + "::fp8", "FP8Linear");
        f.add_input(*a_src);
        f.add_input(g.get_var(pname));
        f.add_input(sw);
        if (a_mode == 1) f.add_input(*a_scale);
        const bool has_c = gemm && n.get_inputs().size() > 2;
        if (has_c) f.add_input(n.get_inputs()[2].get());
        f.add_output(*out);
        f.set_attribute(Attribute{"a_mode", (int32_t)a_mode});
        f.set_attribute(Attribute{"has_c", (int32_t)has_c});
        f.set_attribute(Attribute{"act", (int32_t)act});
        f.set_attribute(Attribute{"alpha", gemm ? attr_float(n, "alpha", 1.0f) : 1.0f});
        f.set_attribute(Attribute{"beta", gemm ? attr_float(n, "beta", 1.0f) : 1.0f});
        f.set_attribute(Attribute{"w_is_nk", (int32_t)w_is_nk});
        f.set_attribute(Attribute{"trans_a", (int32_t)trans_a});
        f.set_attribute(Attribute{"fp8_mfma", (int32_t)fp8_mfma_});
        f.set_attribute(Attribute{"weight", W.get_name()});
        if (!wbatch.empty()) f.set_attribute(Attribute{"wbatch", wbatch});
        for (size_t d : drop) removed[d] = true;
        replacement.emplace(i, std::move(f));
        ++fused_count_;
    }
    if (replacement.empty()) return;
    std::vector<Node> out;
    for (size_t i = 0; i < nodes.size(); ++i) {
        auto it = replacement.find(i);
        if (it != replacement.end()) out.push_back(std::move(it->second));
        else if (!removed[i]) out.push_back(std::move(nodes[i]));
    }
    nodes = std::move(out);
}

// Load-time packing of every fused weight: weights are laid out at model
// load in MFMA-fragment order, beside their fp32 scales.
void NetworkInstance::pack_weights() {
    for (const Node &n : model_.get_graph().get_nodes()) {
        const bool conv = n.get_op_type() == "FP8Conv";
        if (n.get_op_type() != "FP8Linear" && !conv) continue;
        const Variable &pv = n.get_inputs()[1].get();
        if (table_.contains(pv.get_name())) continue;
        const Variable &W = model_.get_graph().get_var(attr_string(n, "weight", ""));
        const Variable &sw = n.get_inputs()[2].get();
        create_tensor_for_var(W);
        create_tensor_for_var(sw);
        // [batch dimensions..., K, N]: one packed weight per batch
        const auto &psh = pv.get_shape();
        LCML_ASSERT(psh.size() >= 2, "%s: packed weight %s of rank %zu", n.get_op_type().c_str(),
                    pv.get_name().c_str(), psh.size());
        const uint32_t K = (uint32_t)psh[psh.size() - 2], N = (uint32_t)psh[psh.size() - 1];
        uint32_t batches = 1;
        for (size_t d = 0; d + 2 < psh.size(); ++d) batches *= (uint32_t)psh[d];
        const auto &ws = W.get_shape();
        const int64_t group = conv ? attr_int(n, "group", 1) : 1;
        // conv weights [cout, cin_g, kh, kw], or [cout, cin_g, kl] (1-D: kh = 1)
        const int64_t ckh = conv && ws.size() == 4 ? (int64_t)ws[2] : 1, ckw = conv ? (int64_t)ws.back() : 1;
        const size_t batch_bytes = (size_t)lcml_fp8_packed_weight_bytes(K, N);
        DeviceArray<uint8_t> packed(conv ? (size_t)lcml_fp8_packed_conv_weight_bytes(ws[0], ws[1], ckh, ckw, group)
                                         : batch_bytes * batches);
        ITensor &wt = table_.at(W.get_name());
        const uint8_t *wsrc = static_cast<const uint8_t *>(wt.device_data());
        if (conv)
            lcml_check(lcml_fp8_pack_conv_weight(wsrc, ws[0], ws[1], ckh, ckw, group, packed.data(), stream_),
                       "pack conv weight");
        else
            for (uint32_t b = 0; b < batches; ++b)
                lcml_check(lcml_fp8_pack_weight(wsrc + (size_t)b * K * N, K, N, attr_int(n, "w_is_nk", 0),
                                                packed.data() + b * batch_bytes, stream_),
                           "pack weight");
        ITensor &st = table_.at(sw.get_name());
        DeviceArray<float> scale(static_cast<float *>(st.device_data()), 0, st.size());
        table_.own(pv.get_name(), std::make_unique<PackedWeightTensor>(to_tensor_shape(psh), std::move(packed),
                                                                        std::move(scale)));
    }
}

// Intermediates (written by a node, not bound from outside, not constants)
// share one arena: each is live from its producer through its last reader
// in node order, and the planner lets disjoint live ranges share bytes.
void NetworkInstance::plan_intermediates() {
    planned_.clear();
    arena_.reset();
    plan_ = MemoryPlan{};
    if (!memory_planning_) return;
    const auto &nodes = model_.get_graph().get_nodes();
    std::unordered_map<std::string, size_t> index;
    std::vector<BufferRequest> reqs;
    std::vector<std::string> names;
    for (size_t i = 0; i < nodes.size(); ++i) {
        for (auto &in : nodes[i].get_inputs()) {
            auto it = index.find(in.get().get_name());
            if (it != index.end()) reqs[it->second].last = std::max(reqs[it->second].last, i);
        }
        for (auto &out : nodes[i].get_outputs()) {
            const Variable &v = out.get();
            if (table_.contains(v.get_name()) || v.is_trainable_weight() || !v.get_raw_data().empty()) continue;
            if (v.get_shape().empty() && v.num_elements() != 1) continue;  // no static shape: allocated on its own
            auto [it, fresh] = index.try_emplace(v.get_name(), reqs.size());
            if (fresh) {
                reqs.push_back({v.num_elements() * data_type_bytes(v.get_dtype()), i, i});
                names.push_back(v.get_name());
            } else {
                reqs[it->second].last = std::max(reqs[it->second].last, i);
            }
        }
    }
    if (reqs.empty()) return;
    plan_ = plan_device_buffers(reqs);
    LCML_ASSERT(plan_is_valid(reqs, plan_), "memory plan: overlapping live buffers");
    arena_ = std::make_shared<DeviceBuffer>(plan_.arena_bytes);
    for (size_t r = 0; r < reqs.size(); ++r) planned_[names[r]] = plan_.offsets[r];
}

void NetworkInstance::prepare() {
    Graph &g = model_.mutable_graph();
    g.mark_constants();
    fused_count_ = 0;
    if (fusion_) fuse_qdq_linear();
    table_.clear();
    for (auto &[name, t] : inputs_) validate_and_bind("input", g.get_var(name), t.get());
    for (auto &[name, t] : outputs_) validate_and_bind("output", g.get_var(name), t.get());
    pack_weights();
    plan_intermediates();
    for (const Node &n : g.get_nodes()) {
        for (auto &v : n.get_inputs()) create_tensor_for_var(v.get());
        for (auto &v : n.get_outputs()) create_tensor_for_var(v.get());
    }
    ops_.clear();
    for (const Node &n : g.get_nodes()) ops_.push_back(model_.get_opset().create_operator(n.get_op_type(), n));
    hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize");  // packing done before first use
    prepared_ = true;
}

void NetworkInstance::forward() {
    if (!prepared_) prepare();
    const Graph &g = model_.get_graph();
    for (auto &[name, t] : inputs_) table_.bind(name, t.get());
    for (auto &[name, t] : outputs_) table_.bind(name, t.get());
    const auto &nodes = g.get_nodes();
    if (enable_logging_) {
        log_graph();
        (void)lcml_fp8_kernel_trace();  // start each node's record empty
    }
    for (size_t i = 0; i < nodes.size(); ++i) {
        std::vector<std::reference_wrapper<ITensor>> ins, outs;
        for (auto &v : nodes[i].get_inputs()) ins.emplace_back(table_.at(v.get().get_name()));
        for (auto &v : nodes[i].get_outputs()) outs.emplace_back(table_.at(v.get().get_name()));
        ops_[i]->set_environment(*this, table_);
        ops_[i]->forward(ins, outs);
        if (enable_logging_) log_node(i, nodes[i], lcml_fp8_kernel_trace());
    }
}

namespace {

std::string shape_text(const std::vector<size_t> &shape) {
    std::string s = "[";
    for (size_t i = 0; i < shape.size(); ++i) s += (i ? ", " : "") + std::to_string(shape[i]);
    return s + "]";
}

// a markdown table cell: '|' escaped
std::string cell(std::string s) {
    for (size_t p = 0; (p = s.find('|', p)) != std::string::npos; p += 2) s.replace(p, 1, "\\|");
    return s;
}

std::string names(const std::vector<std::reference_wrapper<const Variable>> &vars) {
    std::string s;
    for (auto &v : vars) s += (s.empty() ? "" : ", ") + v.get().get_name();
    return s.empty() ? "(none)" : s;
}

}  // namespace

// The execution log's graph part, appended once per forward(): a summary
// table and one row per node (index, operator, inputs, outputs) of the graph
// as it executes, i.e. after QDQ fusion.
void NetworkInstance::log_graph() const {
    FILE *f = fopen(log_path_.c_str(), "a");
    if (!f) return;
    const Graph &g = model_.get_graph();
    const auto &nodes = g.get_nodes();
    fprintf(f, "\n# Network Execution Log\n\n## Summary\n\n| Metric | Value |\n|--------|-------|\n");
    fprintf(f, "| Total Nodes | %zu |\n| Graph Inputs | %zu |\n| Graph Outputs | %zu |\n| Variables | %zu |\n",
            nodes.size(), g.get_inputs().size(), g.get_outputs().size(), g.get_variables().size());
    fprintf(f, "| Fused FP8 nodes | %zu |\n| Warp size | %u |\n\n", fused_count_, warp_size_);
    fprintf(f, "## Nodes Detail\n\n| Index | Op Type | Inputs | Outputs |\n|-------|---------|--------|---------|\n");
    for (size_t i = 0; i < nodes.size(); ++i)
        fprintf(f, "| %zu | %s | %s | %s |\n", i, nodes[i].get_op_type().c_str(),
                cell(names(nodes[i].get_inputs())).c_str(), cell(names(nodes[i].get_outputs())).c_str());
    fprintf(f, "\n");
    fclose(f);
}

// One executed node: its inputs and outputs with shapes and dtypes, and the
// kernels its forward() launched (the C ABI's kernel trace).
void NetworkInstance::log_node(size_t i, const Node &n, const char *kernels) const {
    FILE *f = fopen(log_path_.c_str(), "a");
    if (!f) return;
    const size_t total = model_.get_graph().get_nodes().size();
    fprintf(f, "\n### Node [%zu/%zu]: %s\n\n**Inputs:**\n", i, total - 1, n.get_op_type().c_str());
    auto vars = [&](const std::vector<std::reference_wrapper<const Variable>> &vs) {
        for (auto &v : vs) {
            const std::string_view dt = data_type_name(v.get().get_dtype());
            fprintf(f, "- `%s` : shape=%s, dtype=%.*s\n", v.get().get_name().c_str(),
                    shape_text(v.get().get_shape()).c_str(), (int)dt.size(), dt.data());
        }
        if (vs.empty()) fprintf(f, "- (none)\n");
    };
    vars(n.get_inputs());
    fprintf(f, "\n**Outputs:**\n");
    vars(n.get_outputs());
    fprintf(f, "\n**Kernels:** %s\n\n---\n", kernels && *kernels ? kernels : "(none)");
    fclose(f);
}

std::vector<std::string> NetworkInstance::executed_op_types() const {
    std::vector<std::string> v;
    for (auto &n : model_.get_graph().get_nodes()) v.push_back(n.get_op_type());
    return v;
}

}  // namespace lcml::onnx
