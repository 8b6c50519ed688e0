#include "rocm_executor.hpp"

#include <stdexcept>
#include <unordered_set>

#include "pyflame_rt/errors.hpp"

namespace pyflame_rt {

namespace {
thread_local RocmExecutor* t_current = nullptr;

struct CurrentGuard {
    RocmExecutor* prev;
    explicit CurrentGuard(RocmExecutor* e) : prev(t_current) { t_current = e; }
    ~CurrentGuard() { t_current = prev; }
};

bool is_f32_matrix(const Tensor& t) { return t.dtype() == DType::Float32 && t.ndim() == 2; }
}  // namespace

void pfr_check(int status) {
    if (status == PFR_OK) return;
    const std::string msg = pfr_last_error();
    if (status == PFR_ERR_INVALID_ARG) throw std::invalid_argument(msg);
    throw std::runtime_error(msg);
}

RocmExecutor::RocmExecutor(int device, bool strict_math_mode, int math_mode)
    : strict_math_mode_(strict_math_mode), math_mode_(math_mode) {
    const int st = pfr_rocm_init(device, &ctx_);
    if (st != PFR_OK) throw BackendError(std::string("cannot initialise ROCm device: ") + pfr_last_error());
}

RocmExecutor::~RocmExecutor() {
    release_weights();
    if (ctx_) pfr_rocm_destroy(ctx_);
}

void RocmExecutor::release_weights() {
    for (auto& kv : weights_) {
        if (kv.second.csr) pfr_csr_free(kv.second.csr);
        if (kv.second.sp24) pfr_sp24_free(kv.second.sp24);
    }
    weights_.clear();
    prepared_for_ = nullptr;
}

RocmExecutor* RocmExecutor::current() { return t_current; }

const RocmExecutor::DeviceWeight* RocmExecutor::weight(const Node* node) const {
    auto it = weights_.find(node);
    return it == weights_.end() ? nullptr : &it->second;
}

bool RocmExecutor::supports_op(const std::string& op_type) const {
    return OperatorRegistry::instance().has("rocm::" + op_type);
}

std::vector<std::string> RocmExecutor::get_supported_ops() const {
    std::vector<std::string> r;
    for (const auto& n : OperatorRegistry::instance().list_ops())
        if (n.rfind("rocm::", 0) == 0) r.push_back(n.substr(6));
    return r;
}

// Device operands for nodes whose weight is an initializer:
//  Gemm(A, W[, C])          W f32 2-D  -> CSR of op(W)^T
//  MatMul(A, W)             W f32 2-D  -> CSR of W^T
//  MatMul(W, B)             W f32 2-D, B an activation -> CSR of W
//  QuantizedMatMul(W, B)    W int8 2-D 2:4 along K, zero points 0
//                           -> 2:4 compressed, per-tensor scale a_scale
void RocmExecutor::prepare(const Graph& graph) {
    if (prepared_for_ == &graph) return;
    release_weights();
    for (const auto& n : graph.nodes()) {
        const auto& in = n->inputs();
        auto init = [&](size_t i) -> const Tensor* {
            if (i >= in.size()) return nullptr;
            auto t = graph.get_initializer(in[i]);
            return t ? &t->get() : nullptr;
        };
        DeviceWeight w;
        try {
            if (n->op_type() == "Gemm" && init(1) && is_f32_matrix(*init(1))) {
                const Tensor& B = *init(1);
                const bool tb = n->get_attr<int64_t>("transB", 0) != 0;
                pfr_check(pfr_csr_from_dense(ctx_, B.data_ptr<float>(), B.shape()[0], B.shape()[1], tb ? 0 : 1, 0.0f,
                                             &w.csr));
                w.kind = DeviceWeight::CsrB;
            } else if (n->op_type() == "MatMul" && init(1) && is_f32_matrix(*init(1))) {
                const Tensor& B = *init(1);
                pfr_check(pfr_csr_from_dense(ctx_, B.data_ptr<float>(), B.shape()[0], B.shape()[1], 1, 0.0f, &w.csr));
                w.kind = DeviceWeight::CsrB;
            } else if (n->op_type() == "MatMul" && init(0) && !init(1) && is_f32_matrix(*init(0))) {
                const Tensor& A = *init(0);
                pfr_check(pfr_csr_from_dense(ctx_, A.data_ptr<float>(), A.shape()[0], A.shape()[1], 0, 0.0f, &w.csr));
                w.kind = DeviceWeight::CsrA;
            } else if (n->op_type() == "QuantizedMatMul" && init(0) && init(0)->ndim() == 2 &&
                       (init(0)->dtype() == DType::Int8 || init(0)->dtype() == DType::UInt8) &&
                       n->get_attr<int64_t>("a_zero_point", 0) == 0 && n->get_attr<int64_t>("b_zero_point", 0) == 0) {
                const Tensor& A = *init(0);
                const float a_scale = n->get_attr<float>("a_scale", 1.0f);
                // UInt8 data is read as int8, as the reference kernel does
                // (src/backends/cpu/ops/quantized_ops.cpp:143-144).
                const int st = pfr_sp24_pack(ctx_, A.shape()[0], A.shape()[1], A.data(), PFR_I8, &a_scale, 1, &w.sp24);
                if (st == PFR_OK) w.kind = DeviceWeight::Sp24A;
            }
        } catch (const std::exception& e) {
            throw BackendError(std::string("preparing device weight: ") + e.what(), n->name());
        }
        if (w.kind != DeviceWeight::None) weights_[n.get()] = w;
    }
    prepared_for_ = &graph;
}

std::vector<Tensor> RocmExecutor::execute(const Graph& graph, const std::unordered_map<std::string, Tensor>& input_feed,
                                          const std::vector<std::string>& output_names) {
    validate_inputs(graph, input_feed);
    prepare(graph);
    CurrentGuard guard(this);
    std::unordered_map<std::string, const Tensor*> view;
    std::unordered_map<std::string, Tensor> produced;
    for (const auto& kv : input_feed) view[kv.first] = &kv.second;
    for (const auto& kv : graph.initializers())
        if (!view.count(kv.first)) view[kv.first] = &kv.second;
    auto& reg = OperatorRegistry::instance();
    for (const auto& node : graph.topological_sort()) {
        const OpFunc* op = reg.get("rocm::" + node->op_type());
        if (!op) throw UnsupportedOperatorError(node->op_type(), name_);
        std::vector<const Tensor*> ins;
        ins.reserve(node->inputs().size());
        for (const auto& nm : node->inputs()) {
            auto it = view.find(nm);
            if (it == view.end()) throw BackendError("Input tensor '" + nm + "' not found", node->name());
            ins.push_back(it->second);
        }
        OpContext octx{node.get(), strict_math_mode_};
        std::vector<Tensor> outs;
        try {
            outs = (*op)(ins, octx);
        } catch (const std::exception& e) {
            throw BackendError(e.what(), node->name());
        }
        if (outs.size() != node->outputs().size())
            throw BackendError("Operator returned " + std::to_string(outs.size()) + " outputs, expected " +
                                   std::to_string(node->outputs().size()),
                               node->name());
        for (size_t i = 0; i < outs.size(); ++i) {
            const std::string& nm = node->outputs()[i];
            produced[nm] = std::move(outs[i]);
            view[nm] = &produced[nm];
        }
    }
    std::vector<std::string> names = output_names;
    if (names.empty())
        for (const auto& o : graph.outputs()) names.push_back(o.name);
    std::vector<Tensor> results;
    for (const auto& nm : names) {
        auto it = produced.find(nm);
        if (it != produced.end()) {
            results.push_back(std::move(it->second));
            produced.erase(it);
            view.erase(nm);
            continue;
        }
        auto v = view.find(nm);
        if (v == view.end()) throw BackendError("Output tensor '" + nm + "' not found");
        results.push_back(v->second->clone());
    }
    return results;
}

std::unique_ptr<Backend> create_backend(const std::string& name, int /*num_threads*/) {
    if (name == "rocm") return std::make_unique<RocmExecutor>();
    throw UnsupportedFormatError(name, {"rocm"});
}

}  // namespace pyflame_rt
