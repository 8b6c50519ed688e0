// InferenceSession (src/session.cpp:15-199 of the reference): options
// validation, .pfm load, graph validation, backend selection, run.  This
// runtime binds device "rocm" to RocmExecutor; the reference's other devices
// ("cpu", "wse*") are served by the reference runtime itself.
#include "pyflame_rt/session.hpp"

#include <unordered_set>

#include "../backends/rocm/rocm_executor.hpp"
#include "pyflame_rt/errors.hpp"
#include "pyflame_rt/pyflame_format.hpp"
#include "pyflame_rt/quantize.hpp"

namespace pyflame_rt {

InferenceSession::InferenceSession(const std::string& model_path, SessionOptions options,
                                   std::vector<std::string> /*providers*/)
    : options_(std::move(options)) {
    auto errors = options_.validate();
    if (!errors.empty()) {
        std::string msg = "Invalid session options:\n";
        for (const auto& e : errors) msg += "  - " + e + "\n";
        throw PyFlameRTError(msg);
    }
    graph_ = load_model(model_path);
    auto verr = graph_->validate();
    if (!verr.empty()) throw ValidationError(verr);
    // the reference applies quantization after the graph passes
    // (src/session.cpp:38-41)
    if (options_.quantization == "dynamic_int8") {
        graph_ = quantize_dynamic_int8(*graph_);
        verr = graph_->validate();
        if (!verr.empty()) throw ValidationError(verr);
    }
    if (options_.device != "rocm")
        throw PyFlameRTError("Device '" + options_.device +
                             "' is not provided by this runtime; it runs device='rocm' (MI355X)");
    backend_ = std::make_unique<RocmExecutor>(options_.rocm_device_id, options_.strict_math_mode,
                                              options_.rocm_math_mode, options_.optimization_level);
}

InferenceSession::~InferenceSession() = default;

void InferenceSession::validate_inputs(const std::unordered_map<std::string, Tensor>& feed) const {
    for (const auto& info : graph_->inputs()) {
        if (graph_->has_initializer(info.name)) continue;
        auto it = feed.find(info.name);
        if (it == feed.end()) throw PyFlameRTError("Missing required input '" + info.name + "'");
        if (it->second.dtype() != info.dtype)
            throw PyFlameRTError("Input '" + info.name + "' has dtype " + dtype_name(it->second.dtype()) +
                                 " but expected " + dtype_name(info.dtype));
        if (!info.is_dynamic()) {
            const auto& s = it->second.shape();
            if (s.size() != info.shape.size())
                throw PyFlameRTError("Input '" + info.name + "' has " + std::to_string(s.size()) +
                                     " dimensions but expected " + std::to_string(info.shape.size()));
            for (size_t i = 0; i < s.size(); ++i)
                if (info.shape[i] && *info.shape[i] != s[i])
                    throw PyFlameRTError("Input '" + info.name + "' dimension " + std::to_string(i) + " has size " +
                                         std::to_string(s[i]) + " but expected " + std::to_string(*info.shape[i]));
        }
    }
}

std::vector<Tensor> InferenceSession::run(const std::vector<std::string>& output_names,
                                          const std::unordered_map<std::string, Tensor>& input_feed,
                                          const RunOptions&) {
    validate_inputs(input_feed);
    if (!output_names.empty()) {
        std::unordered_set<std::string> valid;
        for (const auto& o : graph_->outputs()) valid.insert(o.name);
        for (const auto& n : output_names)
            if (!valid.count(n)) throw PyFlameRTError("Requested output '" + n + "' does not exist in graph");
    }
    return backend_->execute(*graph_, input_feed, output_names);
}

std::vector<NodeArg> InferenceSession::get_inputs() const {
    std::vector<NodeArg> r;
    for (const auto& i : graph_->inputs()) r.push_back(NodeArg::from_tensor_info(i));
    return r;
}

std::vector<NodeArg> InferenceSession::get_outputs() const {
    std::vector<NodeArg> r;
    for (const auto& o : graph_->outputs()) r.push_back(NodeArg::from_tensor_info(o));
    return r;
}

std::vector<std::string> InferenceSession::get_providers() const { return {"ROCMExecutionProvider"}; }

}  // namespace pyflame_rt
