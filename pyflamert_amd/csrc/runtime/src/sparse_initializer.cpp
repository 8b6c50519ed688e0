// SparseInitializer: structure checks and dense expansion (layout described
// in graph.hpp).
#include <cmath>
#include <cstring>

#include "pyflame_rt/errors.hpp"
#include "pyflame_rt/graph.hpp"
#include "pyflame_rt/pyflame_format.hpp"

namespace pyflame_rt {

int64_t SparseInitializer::nnz() const {
    if (format == Csr) return indptr.empty() ? 0 : indptr.back();
    int64_t n = 0;
    for (uint8_t v : values) n += v != 0;
    return n;
}

size_t SparseInitializer::stored_bytes() const {
    return indptr.size() * sizeof(int64_t) + indices.size() * sizeof(int32_t) + values.size() + positions.size() +
           scales.size() * sizeof(float);
}

void SparseInitializer::validate(const std::string& name) const {
    auto bad = [&](const std::string& why) { throw InvalidModelError("Sparse initializer '" + name + "': " + why); };
    if (rows < 0 || cols < 0) bad("negative dimension");
    if (rows > DeserializationLimits::MAX_DIMENSION_SIZE || cols > DeserializationLimits::MAX_DIMENSION_SIZE)
        bad("dimension too large");
    if (format == Csr) {
        if (dtype != DType::Float32 && dtype != DType::Int8) bad("CSR values must be float32 or int8");
        if ((int64_t)indptr.size() != rows + 1) bad("indptr must have rows + 1 entries");
        if (indptr[0] != 0) bad("indptr[0] must be 0");
        for (int64_t r = 0; r < rows; ++r)
            if (indptr[(size_t)r + 1] < indptr[(size_t)r]) bad("indptr must be non-decreasing");
        const int64_t n = indptr.back();
        if (n > DeserializationLimits::MAX_TOTAL_ELEMENTS) bad("too many nonzeros");
        if ((int64_t)indices.size() != n) bad("indices must have indptr[rows] entries");
        if ((int64_t)values.size() != n * (int64_t)dtype_size(dtype)) bad("values size does not match nnz");
        for (int64_t r = 0; r < rows; ++r)
            for (int64_t j = indptr[(size_t)r]; j < indptr[(size_t)r + 1]; ++j) {
                const int32_t c = indices[(size_t)j];
                if (c < 0 || c >= cols)
                    bad("column index " + std::to_string(c) + " out of range [0, " + std::to_string(cols) + ")");
                if (j > indptr[(size_t)r] && c <= indices[(size_t)j - 1])
                    bad("column indices must ascend within row " + std::to_string(r));
            }
        if (dtype == DType::Int8) {
            const size_t want1 = scale_axis == 0 ? (size_t)rows : (size_t)cols;
            if (scale_axis > 1) bad("scale_axis must be 0 or 1");
            if (scales.size() != 1 && scales.size() != want1)
                bad("int8 values need 1 scale or one per " + std::string(scale_axis ? "column" : "row"));
            for (float s : scales)
                if (!(s > 0.0f) || !std::isfinite(s)) bad("scales must be positive and finite");
        } else if (!scales.empty()) {
            bad("float32 values take no scales");
        }
        if (!positions.empty()) bad("CSR takes no positions");
    } else if (format == Nm24) {
        if (dtype != DType::Int8) bad("2:4 values must be int8");
        if (cols % 4) bad("2:4 needs cols divisible by 4");
        if ((int64_t)values.size() != rows * (cols / 2)) bad("2:4 values must be rows x cols/2");
        if ((int64_t)positions.size() != rows * (cols / 4)) bad("2:4 positions must be rows x cols/4");
        for (size_t g = 0; g < positions.size(); ++g) {
            const int p0 = positions[g] & 3, p1 = (positions[g] >> 2) & 3;
            if ((positions[g] >> 4) || p0 >= p1) bad("2:4 group " + std::to_string(g) + " has invalid positions");
        }
        if (!indptr.empty() || !indices.empty() || !scales.empty()) bad("2:4 takes no indptr, indices or scales");
    } else {
        bad("unknown sparse format " + std::to_string((uint32_t)format));
    }
}

Tensor SparseInitializer::to_dense() const {
    Tensor t({rows, cols}, logical_dtype());
    if (format == Csr) {
        float* d = t.data_ptr<float>();
        for (int64_t r = 0; r < rows; ++r)
            for (int64_t j = indptr[(size_t)r]; j < indptr[(size_t)r + 1]; ++j) {
                float v;
                if (dtype == DType::Float32) {
                    std::memcpy(&v, &values[(size_t)j * 4], 4);
                } else {
                    const int64_t c = indices[(size_t)j];
                    const float s = scales.size() == 1 ? scales[0] : scales[(size_t)(scale_axis ? c : r)];
                    v = (float)(int8_t)values[(size_t)j] * s;
                }
                d[r * cols + indices[(size_t)j]] = v;
            }
    } else {
        int8_t* d = static_cast<int8_t*>(t.data());
        const int64_t groups = cols / 4;
        for (int64_t r = 0; r < rows; ++r)
            for (int64_t g = 0; g < groups; ++g) {
                const uint8_t p = positions[(size_t)(r * groups + g)];
                const int8_t* v = reinterpret_cast<const int8_t*>(&values[(size_t)(r * groups + g) * 2]);
                d[r * cols + g * 4 + (p & 3)] = v[0];
                d[r * cols + g * 4 + ((p >> 2) & 3)] = v[1];
            }
    }
    return t;
}

}  // namespace pyflame_rt
