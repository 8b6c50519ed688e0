// Computational graph: nodes, graph inputs/outputs, named initializers, with
// the reference's size limits (include/pyflame_rt/graph.hpp:17-30), Kahn
// topological order and validation.  Besides the reference's dense
// initializers a graph holds sparse ones (SparseInitializer), which the
// reference's Graph has no slot for: its initializers are dense Tensors
// only, so a pruned weight is stored and counted against the limits at its
// dense size (graph.hpp:17-30, pyflame_format.cpp:168-176).
#pragma once

#include <functional>
#include <memory>
#include <optional>
#include <string>
#include <unordered_map>
#include <vector>

#include "pyflame_rt/node.hpp"
#include "pyflame_rt/tensor.hpp"
#include "pyflame_rt/types.hpp"

namespace pyflame_rt {

struct GraphLimits {
    size_t max_nodes = 100000;
    size_t max_initializers = 50000;
    size_t max_initializer_bytes = 4ULL * 1024 * 1024 * 1024;
};

// A pruned weight kept in compressed form.  The tensor it stands for is 2-D,
// rows x cols:
//  * Csr: row r holds (indices[j], value j) for j in [indptr[r], indptr[r+1]),
//    indices strictly ascending (the order to_sparse produces,
//    sparse_tensor.cpp:560-610, so storage order = ascending k).  Values are
//    Float32, or Int8 with symmetric scales: the logical tensor is then
//    Float32 with entry (float)q * scale (dequantize_tensor with zero point 0,
//    quant_ops.cpp:182-196), the scale taken per tensor (scales.size() == 1),
//    per row (scale_axis 0, rows scales) or per column (scale_axis 1, cols
//    scales).
//  * Nm24: an Int8 tensor whose every group of four consecutive columns holds
//    at most two nonzeros (NMSparsityPruning(2, 4), nm_sparsity.cpp:45-120);
//    values [rows, cols/2] are the two kept entries of each group and
//    positions [rows, cols/4] their column offsets in the group, pos0 | pos1 << 2
//    with pos0 < pos1 (an unused slot holds value 0).  No scales (the
//    QuantizedMatMul consuming it carries them as attributes).
struct SparseInitializer {
    enum Format : uint32_t { Csr = 1, Nm24 = 2 };
    Format format = Csr;
    DType dtype = DType::Float32;  // stored value type
    int64_t rows = 0, cols = 0;
    std::vector<int64_t> indptr;   // Csr: rows + 1
    std::vector<int32_t> indices;  // Csr: nnz
    std::vector<uint8_t> values;   // Csr: nnz values; Nm24: rows * cols / 2 int8
    std::vector<uint8_t> positions;  // Nm24: rows * cols / 4
    std::vector<float> scales;     // Csr Int8: 1, rows or cols
    uint32_t scale_axis = 0;

    int64_t nnz() const;
    DType logical_dtype() const { return format == Csr ? DType::Float32 : DType::Int8; }
    size_t stored_bytes() const;
    // Checks the structure (sizes, index ranges and order, positions, scales);
    // throws InvalidModelError naming the tensor.
    void validate(const std::string& name) const;
    // The dense tensor this record stands for.
    Tensor to_dense() const;
};

class Graph {
public:
    explicit Graph(std::string name = "", GraphLimits limits = {}) : name_(std::move(name)), limits_(limits) {}

    const std::string& name() const { return name_; }
    size_t num_nodes() const { return nodes_.size(); }
    void add_node(std::shared_ptr<Node> node);
    const Node* get_node(const std::string& name) const;
    const std::vector<std::shared_ptr<Node>>& nodes() const { return nodes_; }

    void add_input(const TensorInfo& i) { inputs_.push_back(i); }
    void add_output(const TensorInfo& o) { outputs_.push_back(o); }
    const std::vector<TensorInfo>& inputs() const { return inputs_; }
    const std::vector<TensorInfo>& outputs() const { return outputs_; }

    void add_initializer(const std::string& name, Tensor t);
    std::optional<std::reference_wrapper<const Tensor>> get_initializer(const std::string& name) const;
    const std::unordered_map<std::string, Tensor>& initializers() const { return initializers_; }
    bool has_initializer(const std::string& name) const {
        return initializers_.count(name) > 0 || sparse_.count(name) > 0;
    }
    size_t total_initializer_bytes() const { return init_bytes_; }

    // Sparse initializers count against max_initializers and, at their stored
    // size, against max_initializer_bytes.  A name is dense or sparse, not both.
    void add_sparse_initializer(const std::string& name, SparseInitializer s);
    const SparseInitializer* get_sparse_initializer(const std::string& name) const;
    const std::unordered_map<std::string, SparseInitializer>& sparse_initializers() const { return sparse_; }

    const std::string* get_producer(const std::string& tensor) const;
    std::vector<std::shared_ptr<Node>> topological_sort() const;
    std::vector<std::string> validate() const;

private:
    std::string name_;
    GraphLimits limits_;
    std::vector<std::shared_ptr<Node>> nodes_;
    std::unordered_map<std::string, std::shared_ptr<Node>> node_map_;
    std::vector<TensorInfo> inputs_, outputs_;
    std::unordered_map<std::string, Tensor> initializers_;
    std::unordered_map<std::string, SparseInitializer> sparse_;
    std::unordered_map<std::string, std::string> producers_;
    size_t init_bytes_ = 0;
};

}  // namespace pyflame_rt
