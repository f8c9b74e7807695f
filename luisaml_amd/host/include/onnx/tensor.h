// tensor.h -- the tensor API of the operator layer, with device storage.
//
// Mirrors the reference's ITensor / Tensor<T, Container> (include/onnx/
// tensor.h:24-359): u32 row-major shape and strides, element type index and
// name, is_constant / is_view, typed containers reached with
// static_cast<NNTensor<T>&> after a visit_type_index.  The container is a
// view of HIP device memory instead of a LuisaCompute ByteBuffer; like
// DynamicArray's byte-buffer mode (include/onnx/dynamic_array/
// dynamic_array.h:174-178, 289-313) it exposes is_byte_buffer(),
// get_byte_buffer() and get_byte_offset().  FP8 tensors are dense, one byte
// per element (fp8_data.h:25-43).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <functional>
#include <memory>
#include <numeric>
#include <span>
#include <string>
#include <string_view>
#include <vector>

#include "onnx/error.h"
#include "onnx/type_dispatch.h"

namespace lcml::onnx {

// Owned device allocation (freed with the last DeviceArray that views it).
class DeviceBuffer {
    void *ptr_ = nullptr;
    size_t bytes_ = 0;

public:
    explicit DeviceBuffer(size_t bytes) : bytes_(bytes) {
        if (bytes) {
            hipError_t e = hipMalloc(&ptr_, bytes);
            LCML_ASSERT(e == hipSuccess, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
        }
    }
    ~DeviceBuffer() {
        if (ptr_) (void)hipFree(ptr_);
    }
    DeviceBuffer(const DeviceBuffer &) = delete;
    DeviceBuffer &operator=(const DeviceBuffer &) = delete;
    void *data() const noexcept { return ptr_; }
    size_t bytes() const noexcept { return bytes_; }
};

// A typed view of device memory: either an owned buffer or borrowed memory
// (external inputs/outputs, the weight blob), plus a byte offset.
template <typename T>
class DeviceArray {
    std::shared_ptr<DeviceBuffer> owner_;
    void *base_ = nullptr;
    size_t byte_offset_ = 0;
    size_t count_ = 0;
    bool view_ = false;
    mutable std::string name_;

public:
    using value_type = T;
    static constexpr size_t elem_bytes = sizeof(T);

    DeviceArray() = default;
    // allocate count elements
    explicit DeviceArray(size_t count)
        : owner_(std::make_shared<DeviceBuffer>(count * elem_bytes)), count_(count) {
        base_ = owner_->data();
    }
    // borrow memory owned elsewhere
    DeviceArray(void *base, size_t byte_offset, size_t count, bool is_view = false)
        : base_(base), byte_offset_(byte_offset), count_(count), view_(is_view) {}
    // a region of a shared buffer (the planned arena of intermediates)
    DeviceArray(std::shared_ptr<DeviceBuffer> owner, size_t byte_offset, size_t count)
        : owner_(std::move(owner)), byte_offset_(byte_offset), count_(count), view_(true) {
        base_ = owner_->data();
    }
    // view of another array's storage
    DeviceArray(const DeviceArray &src, size_t elem_offset, size_t count)
        : owner_(src.owner_), base_(src.base_), byte_offset_(src.byte_offset_ + elem_offset * elem_bytes),
          count_(count), view_(true) {}

    size_t size() const noexcept { return count_; }
    // a debug name for the storage (ITensor::set_name forwards here); the
    // reference names its DynamicArray storage the same way
    void set_name(std::string_view name) const { name_ = name; }
    const std::string &name() const noexcept { return name_; }
    bool is_byte_buffer() const noexcept { return true; }
    void *get_byte_buffer() const noexcept { return base_; }
    size_t get_byte_offset() const noexcept { return byte_offset_; }
    bool is_view() const noexcept { return view_; }
    T *data() const noexcept { return reinterpret_cast<T *>(static_cast<char *>(base_) + byte_offset_); }
};

class ITensor {
public:
    using size_type = uint32_t;
    using shape_type = std::vector<size_type>;

protected:
    shape_type shape_;
    shape_type strides_;

    void compute_strides() {
        strides_.resize(shape_.size());
        if (shape_.empty()) return;
        strides_.back() = 1;
        for (int i = (int)shape_.size() - 2; i >= 0; --i) strides_[i] = strides_[i + 1] * shape_[i + 1];
    }
    ITensor() = default;
    explicit ITensor(shape_type shape) : shape_(std::move(shape)) { compute_strides(); }

public:
    virtual ~ITensor() = default;
    const shape_type &shape() const noexcept { return shape_; }
    const shape_type &strides() const noexcept { return strides_; }
    size_type ndim() const noexcept { return (size_type)shape_.size(); }
    size_type shape(size_type dim) const { return shape_[dim]; }
    bool empty() const noexcept { return shape_.empty(); }
    virtual size_type size() const noexcept = 0;
    virtual refl::TypeIndex element_type_index() const noexcept = 0;
    virtual std::string_view element_type_name() const noexcept = 0;
    // names the tensor's storage (reference tensor.h:128); no-op by default
    virtual void set_name(std::string_view) const noexcept {}
    virtual bool is_constant() const noexcept { return false; }
    virtual bool is_view() const noexcept { return false; }
    virtual bool is_local() const noexcept { return false; }
    // device address of element 0 (the container's byte buffer + offset)
    virtual void *device_data() const noexcept = 0;

    void reshape(const shape_type &new_shape) {
        shape_ = new_shape;
        compute_strides();
    }
    std::vector<size_type> unravel_index(size_type linear) const {
        std::vector<size_type> idx(shape_.size());
        for (size_t i = 0; i < shape_.size(); ++i) {
            idx[i] = linear / strides_[i];
            linear %= strides_[i];
        }
        return idx;
    }
    size_type linear_index(const std::vector<size_type> &idx) const {
        size_type l = 0;
        for (size_t i = 0; i < idx.size(); ++i) l += idx[i] * strides_[i];
        return l;
    }
};

template <typename T, typename Container = DeviceArray<T>>
class Tensor : public ITensor {
    Container data_;

public:
    using value_type = T;
    using container_type = Container;

    Tensor() = default;
    Tensor(shape_type shape, Container data) : ITensor(std::move(shape)), data_(std::move(data)) {
        size_type n = shape_.empty() ? 0 : std::accumulate(shape_.begin(), shape_.end(), size_type(1),
                                                             std::multiplies<size_type>());
        LCML_ASSERT(n == data_.size(), "Tensor: shape holds %u elements, container %zu", n, data_.size());
    }
    size_type size() const noexcept override { return (size_type)data_.size(); }
    refl::TypeIndex element_type_index() const noexcept override { return refl::type_index_of<T>(); }
    std::string_view element_type_name() const noexcept override { return type_name_v<T>; }
    bool is_view() const noexcept override { return data_.is_view(); }
    void *device_data() const noexcept override { return data_.data(); }
    // forwards to the container where it can hold a name (tensor.h:344-349)
    void set_name(std::string_view name) const noexcept override {
        if constexpr (requires { data_.set_name(name); }) {
            try {
                data_.set_name(name);
            } catch (...) {
            }
        }
    }
    Container &container() noexcept { return data_; }
    const Container &container() const noexcept { return data_; }
    T *data() const noexcept { return data_.data(); }
};

// Constant tensors (initializers) keep a host copy of their values, like the
// reference's ConstTensor (tensor.h:367-406).
template <typename T>
class ConstTensor : public Tensor<T> {
    std::vector<uint8_t> host_;

public:
    ConstTensor(ITensor::shape_type shape, DeviceArray<T> data, std::vector<uint8_t> host)
        : Tensor<T>(std::move(shape), std::move(data)), host_(std::move(host)) {}
    bool is_constant() const noexcept override { return true; }
    const std::vector<uint8_t> &const_data() const noexcept { return host_; }
};

template <typename T>
using NNTensor = Tensor<T, DeviceArray<T>>;

// Allocate a device tensor of the given element type and shape.
template <typename T>
std::unique_ptr<NNTensor<T>> make_device_tensor(const ITensor::shape_type &shape) {
    size_t n = 1;
    for (auto d : shape) n *= d;
    return std::make_unique<NNTensor<T>>(shape, DeviceArray<T>(n));
}

}  // namespace lcml::onnx
