// InferenceSession: load a .pfm model, validate, bind a backend, run
// (include/pyflame_rt/session.hpp:30-108 of the reference).  Graph passes and
// the quantizer of the reference are not part of this runtime; models are run
// as stored.
#pragma once

#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "pyflame_rt/backend.hpp"
#include "pyflame_rt/graph.hpp"
#include "pyflame_rt/options.hpp"

namespace pyflame_rt {

class InferenceSession {
public:
    explicit InferenceSession(const std::string& model_path, SessionOptions options = {},
                              std::vector<std::string> providers = {});
    ~InferenceSession();
    InferenceSession(const InferenceSession&) = delete;
    InferenceSession& operator=(const InferenceSession&) = delete;

    std::vector<Tensor> run(const std::vector<std::string>& output_names,
                            const std::unordered_map<std::string, Tensor>& input_feed,
                            const RunOptions& run_options = {});
    std::vector<NodeArg> get_inputs() const;
    std::vector<NodeArg> get_outputs() const;
    std::vector<std::string> get_providers() const;
    const Graph& graph() const { return *graph_; }
    Backend& backend() { return *backend_; }

private:
    void validate_inputs(const std::unordered_map<std::string, Tensor>& input_feed) const;
    SessionOptions options_;
    std::unique_ptr<Graph> graph_;
    std::unique_ptr<Backend> backend_;
};

}  // namespace pyflame_rt
