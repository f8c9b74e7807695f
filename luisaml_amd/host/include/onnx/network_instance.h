// network_instance.h -- binds a Model to device memory and runs it.
//
// Follows the reference's NetworkInstance (include/onnx/network_instance.h:
// 38-299, src/onnx/network_instance.cpp): external inputs/outputs are bound
// by name with dtype/shape validation (validate_and_bind, :40-69), weights
// live in one device weight blob addressed by the initializers' data_offsets
// (create_tensor_for_var, :202-342, with the FP8 size rule
// ((n+3)/4)*4 at :222-224), operators come from the OperatorSet and run in
// node order after set_environment (:641-650).
//
// MI355X differences: forward() launches HIP kernels eagerly on one stream
// (no tracing); prepare() runs once and (1) fuses DequantizeLinear(W_fp8) ->
// Gemm/MatMul [-> Relu/Gelu], with QuantizeLinear/DynamicQuantizeLinear ->
// DequantizeLinear on the activation, into one FP8Linear node, and (2) packs
// every fused FP8 weight into MFMA panels once, at load time, and (3) plans
// one device arena for the intermediates by live range (memory_planner.h).
#pragma once

#include <unordered_map>

#include <hip/hip_runtime.h>

#include <memory>
#include <string>
#include <vector>

#include "onnx/memory_planner.h"
#include "onnx/onnx.h"
#include "onnx/tensor_table.h"

namespace lcml::onnx {

// E4M3 weight packed for the GEMM kernels (lcml_fp8_pack_weight) with its
// fp32 dequantisation scale (1 entry, or N for per-output-channel).
class PackedWeightTensor : public ITensor {
    DeviceArray<uint8_t> packed_;
    DeviceArray<float> scale_;
    uint32_t K_, N_, batches_;
    size_t batch_bytes_;

    static shape_type checked(shape_type shape) {
        LCML_ASSERT(shape.size() >= 2, "PackedWeightTensor: shape of rank %zu (needs [..., K, N])", shape.size());
        size_t n = 1;
        for (auto d : shape) n *= d;
        LCML_ASSERT(n <= 0xffffffffu, "PackedWeightTensor: %zu elements exceed the u32 size type", n);
        return shape;
    }

public:
    // shape [batch dims..., K, N]: prod(batch dims) packed [K, N] weights one
    // after another (a MatMul weight [..., K, N]; a Gemm or conv weight is
    // [K, N]); the scale is per tensor or per output channel, shared by every
    // batch.  size() counts every batch's elements, like the shape.
    PackedWeightTensor(shape_type shape, DeviceArray<uint8_t> packed, DeviceArray<float> scale)
        : ITensor(checked(std::move(shape))), packed_(std::move(packed)), scale_(std::move(scale)),
          K_(shape_[shape_.size() - 2]), N_(shape_.back()), batches_(1) {
        for (size_t d = 0; d + 2 < shape_.size(); ++d) batches_ *= shape_[d];
        batch_bytes_ = batches_ ? packed_.size() / batches_ : 0;
    }
    size_type size() const noexcept override { return (size_type)((size_t)batches_ * K_ * N_); }
    refl::TypeIndex element_type_index() const noexcept override { return refl::type_index_of<FP8E4M3FN>(); }
    std::string_view element_type_name() const noexcept override { return "FP8E4M3FN(packed)"; }
    bool is_constant() const noexcept override { return true; }
    void *device_data() const noexcept override { return packed_.data(); }
    uint32_t K() const { return K_; }
    uint32_t N() const { return N_; }
    uint32_t batches() const { return batches_; }
    const uint8_t *packed(size_t batch = 0) const { return packed_.data() + batch * batch_bytes_; }
    const float *scale() const { return scale_.data(); }
    bool per_channel() const { return scale_.size() > 1; }
};

class NetworkInstance {
public:
    using TensorRef = std::reference_wrapper<ITensor>;
    using ExternalTensorTable = std::unordered_map<std::string, TensorRef>;

private:
    // declared before the tensor table: the planned intermediates are views
    // into it (they also share its ownership)
    std::shared_ptr<DeviceBuffer> arena_;
    Model model_;
    TensorTable table_;
    std::vector<std::unique_ptr<Operator>> ops_;
    std::vector<size_t> node_order_;
    hipStream_t stream_ = nullptr;
    const uint8_t *weight_buffer_ = nullptr;  // device
    size_t weight_bytes_ = 0;
    bool fusion_ = true;
    bool fp8_mfma_ = false;
    bool memory_planning_ = true;
    bool prepared_ = false;
    MemoryPlan plan_;
    std::unordered_map<std::string, size_t> planned_;  // intermediate -> arena offset
    size_t fused_count_ = 0;
    ExternalTensorTable inputs_, outputs_;
    uint32_t warp_size_ = 64;
    bool use_cooperative_vector_ = false;
    bool enable_logging_ = false;
    std::string log_path_ = "./stats.md";

    void create_tensor_for_var(const Variable &var);
    void validate_and_bind(std::string_view role, const Variable &var, ITensor &t);
    void fuse_qdq_linear();
    void log_graph() const;
    void log_node(size_t i, const Node &n, const char *kernels) const;
    bool is_zero_e4m3_constant(const Variable &v) const;
    void pack_weights();
    void plan_intermediates();

public:
    NetworkInstance() = default;
    NetworkInstance(const NetworkInstance &) = delete;
    NetworkInstance &operator=(const NetworkInstance &) = delete;

    void set_model(Model &&m);
    const Model &model() const { return model_; }
    const Model &get_model() const { return model_; }
    void set_stream(hipStream_t s) { stream_ = s; }
    hipStream_t stream() const { return stream_; }
    // Device memory holding the initializers that carry data_offsets.
    void set_weight_buffer(const void *device_blob, size_t bytes);
    // bind an external tensor by name (a later binding of the same name
    // replaces the earlier one, as in the reference's insert_or_assign)
    void set_input(std::string_view name, ITensor &t);
    void set_output(std::string_view name, ITensor &t);
    const ExternalTensorTable &get_inputs() const { return inputs_; }
    const ExternalTensorTable &get_outputs() const { return outputs_; }
    // QDQ -> FP8Linear fusion (default on); off runs every node as written.
    void set_fusion(bool on) { fusion_ = on; }
    // Fused FP8Linear / FP8Conv nodes on gfx950's native FP8 matrix-core
    // instructions (LCML_KERNEL_AUTO_FP8: twice the large-GEMM rate, FP8-MFMA
    // precision) instead of the exact kernels (default off).  Set before
    // prepare(); no reference counterpart.
    void set_fp8_matrix_cores(bool on) { fp8_mfma_ = on; }
    // Intermediates share one arena by live range (default on); off gives
    // every intermediate its own allocation.
    void set_memory_planning(bool on) { memory_planning_ = on; }
    const MemoryPlan &memory_plan() const { return plan_; }
    size_t planned_intermediates() const { return planned_.size(); }
    // The reference's warp-width knob (network_instance.h:50-54, 215-217):
    // there it sizes the warp intrinsics of the traced kernel (<= 1 turns
    // them off for single-thread dispatch).  Here every operator launches its
    // own grid of 64-lane gfx950 wavefronts, so the value is recorded for
    // callers and operators that read it and changes no kernel choice.
    // Default 64, the wavefront width.
    void set_warp_size(uint32_t size) { warp_size_ = size; }
    uint32_t warp_size() const { return warp_size_; }
    bool use_warp_optimization() const { return warp_size_ > 1; }
    // The reference's CooperativeVector switch for Gemm (network_instance.h:
    // 220-225): recorded; the GEMMs always run on the matrix cores.
    void set_use_cooperative_vector(bool enable) { use_cooperative_vector_ = enable; }
    bool use_cooperative_vector() const { return use_cooperative_vector_; }
    // Execution log (network_instance.cpp:594-634 of the reference): each
    // forward() appends a markdown summary and node table, then one section
    // per executed node (inputs and outputs with shapes and dtypes, and the
    // kernels it launched) to ./stats.md, or to the file set_log_file names.
    void enable_logging(bool enable) { enable_logging_ = enable; }
    void set_log_file(std::string path) { log_path_ = std::move(path); }
    const std::string &log_file() const { return log_path_; }

    void prepare();
    void forward();
    size_t fused_linear_count() const { return fused_count_; }
    std::vector<std::string> executed_op_types() const;
    TensorTable &tensor_table() { return table_; }
    const TensorTable &get_tensor_table() const { return table_; }
};

}  // namespace lcml::onnx
