// Execution backend interface (include/pyflame_rt/backend.hpp:14-43 of the
// reference): a backend runs a whole graph on a feed of named inputs.
#pragma once

#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "pyflame_rt/errors.hpp"
#include "pyflame_rt/graph.hpp"
#include "pyflame_rt/tensor.hpp"

namespace pyflame_rt {

class Backend {
public:
    virtual ~Backend() = default;
    virtual const std::string& name() const = 0;
    virtual bool supports_op(const std::string& op_type) const = 0;
    virtual std::vector<std::string> get_supported_ops() const = 0;
    virtual std::vector<Tensor> execute(const Graph& graph,
                                        const std::unordered_map<std::string, Tensor>& input_feed,
                                        const std::vector<std::string>& output_names = {}) = 0;
    // Names, ranks and fixed dimensions of the feed against the graph inputs
    // (src/backends/cpu/executor.cpp:150-212).
    void validate_inputs(const Graph& graph, const std::unordered_map<std::string, Tensor>& input_feed) const;
};

// "rocm" only: this runtime carries the MI355X backend.
std::unique_ptr<Backend> create_backend(const std::string& name, int num_threads = 0);

}  // namespace pyflame_rt
