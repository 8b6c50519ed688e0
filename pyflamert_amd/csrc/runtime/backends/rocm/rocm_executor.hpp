// RocmExecutor: the MI355X backend.  It runs a graph node by node like the
// reference's CPUExecutor (src/backends/cpu/executor.cpp:45-147): each node's
// kernel is looked up in the OperatorRegistry -- under "rocm::<OpType>" --
// and called through the unchanged OpFunc interface; exceptions become
// BackendError carrying the node name.
//
// Differences that make it a GPU backend:
//  * pruned weights (initializers feeding MatMul / Gemm / QuantizedMatMul)
//    are converted once, on the first run of a graph, into device-resident
//    CSR or 2:4-compressed operands kept by the executor per node; the rocm
//    kernels find them through RocmExecutor::current();
//  * inputs and initializers are not deep-copied on every run.
#pragma once

#include <memory>
#include <string>
#include <unordered_map>

#include "pfr_rocm.h"
#include "pyflame_rt/backend.hpp"
#include "pyflame_rt/registry.hpp"

namespace pyflame_rt {

class RocmExecutor : public Backend {
public:
    struct DeviceWeight {
        enum Kind { None, CsrB, CsrA, Sp24A } kind = None;
        pfr_csr* csr = nullptr;    // CsrB: CSR of op(B)^T; CsrA: CSR of A
        pfr_sp24* sp24 = nullptr;  // Sp24A: 2:4-compressed int8 A
    };

    explicit RocmExecutor(int device = 0, bool strict_math_mode = false, int math_mode = PFR_MODE_STRICT);
    ~RocmExecutor() override;

    const std::string& name() const override { return name_; }
    bool supports_op(const std::string& op_type) const override;
    std::vector<std::string> get_supported_ops() const override;
    std::vector<Tensor> execute(const Graph& graph, const std::unordered_map<std::string, Tensor>& input_feed,
                                const std::vector<std::string>& output_names = {}) override;

    // The executor running a graph on this thread (set during execute).
    static RocmExecutor* current();
    pfr_ctx* ctx() const { return ctx_; }
    int math_mode() const { return math_mode_; }
    const DeviceWeight* weight(const Node* node) const;

private:
    void prepare(const Graph& graph);
    void release_weights();

    std::string name_ = "rocm";
    pfr_ctx* ctx_ = nullptr;
    bool strict_math_mode_;
    int math_mode_;
    const Graph* prepared_for_ = nullptr;
    std::unordered_map<const Node*, DeviceWeight> weights_;
};

// Throws the C ABI's last error as std::invalid_argument / std::runtime_error.
void pfr_check(int status);

}  // namespace pyflame_rt
