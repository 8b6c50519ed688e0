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
//    kernels find them through RocmExecutor::current().  A sparse
//    initializer (a CSR or 2:4 record of a version-2 .pfm) is uploaded from
//    its compressed form, never expanded to a dense host tensor;
//  * inputs and initializers are not deep-copied on every run;
//  * from OptLevel::Basic up, a graph whose every node has a device kernel
//    (pruned Gemm / MatMul / 2:4 QuantizedMatMul, DynamicQuantizeLinear,
//    Relu, Softmax, Gelu, Add, LayerNormalization, per-tensor Quantize /
//    Dequantize / QuantizeLinear / DequantizeLinear) runs as a
//    device-resident plan:
//    graph inputs are copied to the GPU once per run, the remaining
//    initializers once per graph, activations stay in device buffers
//    between nodes, from OptLevel::Extended up a Gemm/MatMul whose only
//    consumer is a Relu or a Gelu runs with it fused into its epilogue (the
//    reference's Extended level adds operator fusion, types.hpp:119-124), and
//    only the requested outputs come back to the host.  Other graphs, and
//    OptLevel::None, run node by node through the host OpFuncs.
#pragma once

#include <memory>
#include <string>
#include <unordered_map>
#include <unordered_set>

#include "pfr_rocm.h"
#include "pyflame_rt/backend.hpp"
#include "pyflame_rt/registry.hpp"

namespace pyflame_rt {

// Output shape of a broadcasting binary op (math.cpp:39-64): shapes are
// right-aligned, each axis takes the larger extent; throws "<op>: shapes are
// not broadcastable" (math.cpp:154-158).
std::vector<int64_t> broadcast_shapes(const std::vector<int64_t>& a, const std::vector<int64_t>& b,
                                      const char* op);

// LayerNormalization's attributes and extents (nn.cpp:419-455): epsilon
// (1e-5), axis (-1) over a tensor of at least one dimension; the rows are
// the product of the dimensions before axis, the normalised extent that of
// the rest.  scale and bias must hold the normalised extent (the reference
// reads that many elements of each).
struct LayerNormExtent {
    int64_t outer, norm;
    float epsilon;
};
LayerNormExtent layernorm_extent(const std::vector<int64_t>& x_shape, int64_t scale_numel, int64_t bias_numel,
                                 const Node* node);

class RocmExecutor : public Backend {
public:
    struct DeviceWeight {
        enum Kind { None, CsrB, CsrA, Sp24A, Sp24B, DenseB, DenseA } kind = None;
        pfr_csr* csr = nullptr;    // CsrB: CSR of op(B)^T; CsrA: CSR of A
        pfr_sp24* sp24 = nullptr;  // Sp24A: 2:4-compressed int8 A; Sp24B: B^T (N x K), 2:4 along K
        float* dense = nullptr;    // DenseB: op(B), K x N row-major; DenseA: A, M x K row-major
        // the weight is the product's second operand (B)
        bool second() const { return kind == CsrB || kind == Sp24B || kind == DenseB; }
    };
    // A float32 initializer weight takes the sparse (CSR) path when at most
    // this fraction of its entries is nonzero, else the dense product.
    static constexpr double kSparseDensityGate = 0.5;

    // opt: None runs node by node through the OpFuncs; Basic adds the
    // device-resident plan; Extended and All also fuse Relu into products.
    explicit RocmExecutor(int device = 0, bool strict_math_mode = false, int math_mode = PFR_MODE_STRICT,
                          OptLevel opt = OptLevel::Extended);
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
    // True when the last run went through the device-resident plan.
    bool device_plan() const { return last_on_device_; }
    // Kernel launches of the plan (a fused pair counts once).
    size_t device_plan_steps() const { return plan_.size(); }
    // Prepared weights by device form: CSR, dense (above the density gate), 2:4.
    void weight_forms(int* csr, int* dense, int* sp24) const {
        *csr = *dense = *sp24 = 0;
        for (const auto& kv : weights_) {
            const auto k = kv.second.kind;
            if (k == DeviceWeight::CsrA || k == DeviceWeight::CsrB) ++*csr;
            else if (k == DeviceWeight::DenseA || k == DeviceWeight::DenseB) ++*dense;
            else if (k == DeviceWeight::Sp24A || k == DeviceWeight::Sp24B) ++*sp24;
        }
    }

private:
    DeviceWeight dense_initializer_weight(const Tensor& W, bool second, bool transB);
    // One kernel launch of the device plan.
    struct PlanStep {
        enum Op { Gemm, MatMulB, MatMulA, QMatMul, QMatMulT, Relu, Softmax, DynQuant, Gelu, Add, LayerNorm, Quant, Dequant } op;
        const Node* node;
        int act = 0;      // pfr_act of a following Relu/Gelu run in this step's epilogue
        std::string out;  // tensor the step writes (the activation's output when fused)
    };
    // A tensor held in device memory while a plan runs.
    struct DevTensor {
        void* p = nullptr;
        std::vector<int64_t> shape;
        DType dtype = DType::Float32;
    };
    struct DevBuf {
        void* p = nullptr;
        int64_t cap = 0;
    };

    void prepare(const Graph& graph);
    void prepare_sparse_views(const Graph& graph);
    void build_plan(const Graph& graph);
    // The weight operand's host-side tensor: a dense initializer, or for a
    // sparse one a data-less view with its logical shape and type.
    const Tensor& weight_tensor(const Graph& graph, const std::string& name) const;
    // A non-weight use of an initializer: the dense one, or a sparse one
    // expanded once (sparse_dense_).
    const Tensor& initializer_value(const Graph& graph, const std::string& name);
    void release_weights();
    void* device_buffer(const std::string& name, int64_t bytes);
    std::vector<Tensor> execute_plan(const Graph& graph, const std::unordered_map<std::string, Tensor>& input_feed,
                                     const std::vector<std::string>& names);

    std::string name_ = "rocm";
    pfr_ctx* ctx_ = nullptr;
    bool strict_math_mode_;
    int math_mode_;
    OptLevel opt_;
    const Graph* prepared_for_ = nullptr;
    std::unordered_map<const Node*, DeviceWeight> weights_;
    bool plan_ok_ = false;
    bool last_on_device_ = false;
    std::vector<PlanStep> plan_;
    std::unordered_set<std::string> fused_away_;           // product outputs a fused Relu consumes
    std::unordered_map<std::string, DevTensor> constants_;  // non-weight initializers, uploaded once
    std::unordered_map<std::string, DevBuf> bufs_;          // graph inputs and activations, by name
    std::unordered_map<std::string, Tensor> sparse_views_;  // sparse weights: shape-only views
    std::unordered_map<std::string, Tensor> sparse_dense_;  // sparse initializers used as plain tensors
};

// Throws the C ABI's last error as std::invalid_argument / std::runtime_error.
void pfr_check(int status);

}  // namespace pyflame_rt
