// Element types, shapes and tensor metadata of the runtime.  The DType
// values, names and sizes are those of the reference (include/pyflame_rt/
// types.hpp:48-113) because .pfm files store them as integers.
#pragma once

#include <cstdint>
#include <limits>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

namespace pyflame_rt {

inline int64_t checked_multiply(int64_t a, int64_t b) {
    if (a == 0 || b == 0) return 0;
    if (a < 0 || b < 0) throw std::invalid_argument("Negative dimensions not allowed in size calculation");
    if (a > std::numeric_limits<int64_t>::max() / b) throw std::overflow_error("Integer overflow in size calculation");
    return a * b;
}

inline int64_t checked_product(const std::vector<int64_t>& v) {
    int64_t r = 1;
    for (int64_t x : v) r = checked_multiply(r, x);
    return r;
}

enum class DType : uint8_t {
    Float32 = 0, Float16 = 1, BFloat16 = 2, Float64 = 3, Int64 = 4,
    Int32 = 5, Int16 = 6, Int8 = 7, UInt8 = 8, Bool = 9
};

inline bool validate_dtype_value(uint32_t v) { return v <= static_cast<uint32_t>(DType::Bool); }

inline size_t dtype_size(DType d) {
    switch (d) {
        case DType::Float32: case DType::Int32: return 4;
        case DType::Float16: case DType::BFloat16: case DType::Int16: return 2;
        case DType::Float64: case DType::Int64: return 8;
        case DType::Int8: case DType::UInt8: case DType::Bool: return 1;
    }
    throw std::invalid_argument("Unknown dtype");
}

inline std::string dtype_name(DType d) {
    static const char* names[] = {"float32", "float16", "bfloat16", "float64", "int64",
                                  "int32", "int16", "int8", "uint8", "bool"};
    const auto i = static_cast<uint32_t>(d);
    if (i > 9) throw std::invalid_argument("Unknown dtype");
    return names[i];
}

// nullopt marks a dynamic dimension.
using Shape = std::vector<std::optional<int64_t>>;

inline std::string shape_to_string(const Shape& s) {
    std::string r = "[";
    for (size_t i = 0; i < s.size(); ++i) {
        if (i) r += ", ";
        r += s[i] ? std::to_string(*s[i]) : "?";
    }
    return r + "]";
}

inline bool is_dynamic_shape(const Shape& s) {
    for (const auto& d : s)
        if (!d) return true;
    return false;
}

struct TensorInfo {
    std::string name;
    Shape shape;
    DType dtype = DType::Float32;
    TensorInfo() = default;
    TensorInfo(std::string n, Shape s, DType d) : name(std::move(n)), shape(std::move(s)), dtype(d) {}
    bool is_dynamic() const { return is_dynamic_shape(shape); }
};

// ONNX-Runtime-style argument descriptor returned by get_inputs/get_outputs.
struct NodeArg {
    std::string name;
    Shape shape;
    std::string type_str;
    static NodeArg from_tensor_info(const TensorInfo& i) {
        return {i.name, i.shape, "tensor(" + dtype_name(i.dtype) + ")"};
    }
};

enum class OptLevel : uint8_t { None = 0, Basic = 1, Extended = 2, All = 3 };

}  // namespace pyflame_rt
