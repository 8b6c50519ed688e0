// Computational graph: nodes, graph inputs/outputs, named initializers, with
// the reference's size limits (include/pyflame_rt/graph.hpp:17-30), Kahn
// topological order and validation.
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
    bool has_initializer(const std::string& name) const { return initializers_.count(name) > 0; }
    size_t total_initializer_bytes() const { return init_bytes_; }

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
    std::unordered_map<std::string, std::string> producers_;
    size_t init_bytes_ = 0;
};

}  // namespace pyflame_rt
