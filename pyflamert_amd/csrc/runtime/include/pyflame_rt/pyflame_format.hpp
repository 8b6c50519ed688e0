// Native model format .pfm, version 1 (src/io/pyflame_format.cpp:392-498 of
// the reference): magic "PFM\0", u32 version, graph name, inputs and outputs
// (name, u32 dtype, u64 ndim, i64 dims, -1 = dynamic), initializers (name,
// dtype, dims, u64 byte count + raw little-endian data), nodes (name, op,
// inputs, outputs, attributes typed 0 int64 / 1 float / 2 string /
// 3 int64[] / 4 float[] / 255 skipped).  Strings are u64 length + bytes.
//
// Version 2 (this runtime; the reference loader rejects it as an unsupported
// version, pyflame_format.cpp:406-409) appends after the nodes a section of
// sparse initializers (SparseInitializer, graph.hpp): u64 count, then per
// record name, u32 format (1 CSR, 2 2:4), u32 stored value dtype, i64 rows,
// i64 cols and
//   CSR: u64 nnz, u32 index width (2: uint16, 4: int32), indptr (rows + 1)
//        x int64, indices nnz x width, values nnz x dtype size, u32 scale
//        axis, u64 scale count, scales x float32;
//   2:4: values rows x cols/2 int8, positions rows x cols/4 bytes.
// A graph without sparse initializers is written as version 1.
#pragma once

#include <cstdint>
#include <memory>
#include <string>

#include "pyflame_rt/graph.hpp"

namespace pyflame_rt {

struct DeserializationLimits {
    static constexpr uint64_t MAX_STRING_SIZE = 10ULL * 1024 * 1024;
    static constexpr uint64_t MAX_TENSOR_DATA_SIZE = 4ULL * 1024 * 1024 * 1024;
    static constexpr uint64_t MAX_ARRAY_COUNT = 1000000;
    static constexpr uint64_t MAX_DIMS = 16;
    static constexpr uint64_t MAX_NODES = 1000000;
    static constexpr uint64_t MAX_ATTRIBUTES = 1000;
    static constexpr int64_t MAX_DIMENSION_SIZE = 100000000LL;
    static constexpr int64_t MAX_TOTAL_ELEMENTS = 1000000000LL;
};

class PyFlameFormat {
public:
    static constexpr char MAGIC[4] = {'P', 'F', 'M', '\0'};
    static constexpr uint32_t VERSION = 2;
    static std::unique_ptr<Graph> load(const std::string& path);
    static void save(const Graph& graph, const std::string& path);
};

// Dispatch on the file extension (".pfm" only), as src/io/loader.cpp:105-130.
std::unique_ptr<Graph> load_model(const std::string& path);
void save_model(const Graph& graph, const std::string& path);

}  // namespace pyflame_rt
