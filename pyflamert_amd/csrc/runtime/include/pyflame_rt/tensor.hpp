// Host tensor of the runtime: shape, dtype and shared, 64-byte aligned,
// zero-initialised storage, or a non-owning view (the reference's Tensor,
// include/pyflame_rt/tensor.hpp:12-90, has the same interface).
#pragma once

#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "pyflame_rt/types.hpp"

namespace pyflame_rt {

class Tensor {
public:
    Tensor() = default;
    Tensor(const std::vector<int64_t>& shape, DType dtype);
    Tensor(void* data, const std::vector<int64_t>& shape, DType dtype);  // view
    Tensor(const Tensor& other);                                         // deep copy
    Tensor(Tensor&& other) noexcept;
    Tensor& operator=(const Tensor& other);
    Tensor& operator=(Tensor&& other) noexcept;
    ~Tensor() = default;

    const std::vector<int64_t>& shape() const { return shape_; }
    DType dtype() const { return dtype_; }
    size_t ndim() const { return shape_.size(); }
    int64_t num_elements() const { return shape_.empty() ? 0 : checked_product(shape_); }
    size_t size_bytes() const { return static_cast<size_t>(num_elements()) * dtype_size(dtype_); }

    void* data() { return data_; }
    const void* data() const { return data_; }
    template <class T> T* data_ptr() { return static_cast<T*>(data_); }
    template <class T> const T* data_ptr() const { return static_cast<const T*>(data_); }

    bool owns_data() const { return owned_ != nullptr; }
    bool is_valid() const { return data_ != nullptr; }
    Tensor clone() const { return Tensor(*this); }
    Tensor view() const { return Tensor(data_, shape_, dtype_); }
    void zero();
    Tensor reshape(const std::vector<int64_t>& new_shape) const;

private:
    void* data_ = nullptr;
    std::vector<int64_t> shape_;
    DType dtype_ = DType::Float32;
    std::shared_ptr<void> owned_;
};

}  // namespace pyflame_rt
