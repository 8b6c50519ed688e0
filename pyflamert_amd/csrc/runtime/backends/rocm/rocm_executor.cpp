#include "rocm_executor.hpp"

#include <algorithm>
#include <cstring>
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

int64_t numel(const std::vector<int64_t>& shape) {
    int64_t n = 1;
    for (int64_t d : shape) n *= d;
    return n;
}

void need_f32(DType d, const char* what) {
    if (d != DType::Float32) throw std::invalid_argument(std::string(what) + " must be float32, got " + dtype_name(d));
}

// CSR of a sparse record's transpose (cols x rows); within each new row the
// source rows come in ascending order, so indices stay ascending.  A
// per-row scale becomes a per-column one and the reverse.
SparseInitializer csr_transpose(const SparseInitializer& s) {
    SparseInitializer t;
    t.format = SparseInitializer::Csr;
    t.dtype = s.dtype;
    t.rows = s.cols;
    t.cols = s.rows;
    t.scales = s.scales;
    t.scale_axis = s.scales.size() > 1 ? 1 - s.scale_axis : 0;
    const size_t es = dtype_size(s.dtype);
    const int64_t nnz = s.nnz();
    t.indptr.assign((size_t)t.rows + 1, 0);
    for (int64_t j = 0; j < nnz; ++j) ++t.indptr[(size_t)s.indices[(size_t)j] + 1];
    for (int64_t c = 0; c < t.rows; ++c) t.indptr[(size_t)c + 1] += t.indptr[(size_t)c];
    t.indices.resize((size_t)nnz);
    t.values.resize((size_t)nnz * es);
    std::vector<int64_t> next(t.indptr.begin(), t.indptr.end() - 1);
    for (int64_t r = 0; r < s.rows; ++r)
        for (int64_t j = s.indptr[(size_t)r]; j < s.indptr[(size_t)r + 1]; ++j) {
            const int64_t d = next[(size_t)s.indices[(size_t)j]]++;
            t.indices[(size_t)d] = (int32_t)r;
            std::memcpy(&t.values[(size_t)d * es], &s.values[(size_t)j * es], es);
        }
    return t;
}

// Uploads a CSR record (or, with transpose, its transpose) as a device
// weight whose rows are output channels.  int8 values keep the in-kernel
// dequantisation when their scale is per tensor or per device row; a scale
// along the reduction dimension is applied on the host instead, giving the
// same float weights RN((float)q * scale).
pfr_csr* upload_sparse_csr(pfr_ctx* ctx, const SparseInitializer& src, bool transpose) {
    SparseInitializer tmp;
    const SparseInitializer& s = transpose ? (tmp = csr_transpose(src)) : src;
    pfr_csr* w = nullptr;
    if (s.dtype == DType::Float32) {
        pfr_check(pfr_csr_upload_i32(ctx, s.rows, s.cols, s.nnz(), s.indptr.data(), s.indices.data(),
                                     s.values.data(), PFR_F32, nullptr, &w));
        return w;
    }
    if (s.scales.size() == 1 || s.scale_axis == 0) {
        std::vector<float> rs = s.scales.size() == 1 ? std::vector<float>((size_t)s.rows, s.scales[0]) : s.scales;
        pfr_check(pfr_csr_upload_i32(ctx, s.rows, s.cols, s.nnz(), s.indptr.data(), s.indices.data(),
                                     s.values.data(), PFR_I8, rs.data(), &w));
        return w;
    }
    std::vector<float> v((size_t)s.nnz());
    for (size_t j = 0; j < v.size(); ++j)
        v[j] = (float)(int8_t)s.values[j] * s.scales[(size_t)s.indices[j]];
    pfr_check(pfr_csr_upload_i32(ctx, s.rows, s.cols, s.nnz(), s.indptr.data(), s.indices.data(), v.data(),
                                 PFR_F32, nullptr, &w));
    return w;
}

// Waits for the context's stream when a plan run leaves early, so that no
// queued copy still reads a host input after execute returns.
struct StreamDrain {
    pfr_ctx* ctx;
    bool armed = true;
    ~StreamDrain() {
        if (armed) pfr_synchronize(ctx);
    }
};
}  // namespace

void pfr_check(int status) {
    if (status == PFR_OK) return;
    const std::string msg = pfr_last_error();
    if (status == PFR_ERR_INVALID_ARG) throw std::invalid_argument(msg);
    throw std::runtime_error(msg);
}

RocmExecutor::RocmExecutor(int device, bool strict_math_mode, int math_mode, OptLevel opt)
    : strict_math_mode_(strict_math_mode), math_mode_(math_mode), opt_(opt) {
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
        if (kv.second.dense) pfr_dev_free(ctx_, kv.second.dense);
    }
    weights_.clear();
    for (auto& kv : constants_) pfr_dev_free(ctx_, kv.second.p);
    constants_.clear();
    for (auto& kv : bufs_) pfr_dev_free(ctx_, kv.second.p);
    bufs_.clear();
    plan_.clear();
    fused_away_.clear();
    sparse_views_.clear();
    sparse_dense_.clear();
    plan_ok_ = false;
    prepared_for_ = nullptr;
}

const Tensor& RocmExecutor::weight_tensor(const Graph& graph, const std::string& name) const {
    auto t = graph.get_initializer(name);
    if (t) return t->get();
    auto it = sparse_views_.find(name);
    if (it == sparse_views_.end()) throw BackendError("Initializer '" + name + "' not found");
    return it->second;
}

const Tensor& RocmExecutor::initializer_value(const Graph& graph, const std::string& name) {
    auto t = graph.get_initializer(name);
    if (t) return t->get();
    auto it = sparse_dense_.find(name);
    if (it != sparse_dense_.end()) return it->second;
    const SparseInitializer* s = graph.get_sparse_initializer(name);
    if (!s) throw BackendError("Initializer '" + name + "' not found");
    return sparse_dense_.emplace(name, s->to_dense()).first->second;
}

// Shape-only views of the sparse initializers that feed a prepared weight
// slot (the OpFuncs read only the weight's shape and type; the values are on
// the device).
void RocmExecutor::prepare_sparse_views(const Graph& graph) {
    for (const auto& kv : weights_) {
        const Node* n = kv.first;
        const int slot = kv.second.second() ? 1 : 0;
        const std::string& nm = n->inputs()[(size_t)slot];
        const SparseInitializer* s = graph.get_sparse_initializer(nm);
        if (s && !sparse_views_.count(nm))
            sparse_views_.emplace(nm, Tensor(nullptr, {s->rows, s->cols}, s->logical_dtype()));
    }
}

void* RocmExecutor::device_buffer(const std::string& name, int64_t bytes) {
    DevBuf& b = bufs_[name];
    const int64_t need = std::max<int64_t>(bytes, 256);
    if (b.cap < need) {
        if (b.p) pfr_check(pfr_dev_free(ctx_, b.p));
        b.p = nullptr;
        b.cap = 0;
        pfr_check(pfr_dev_alloc(ctx_, need, &b.p));
        b.cap = need;
    }
    return b.p;
}

RocmExecutor* RocmExecutor::current() { return t_current; }

std::vector<int64_t> broadcast_shapes(const std::vector<int64_t>& a, const std::vector<int64_t>& b,
                                      const char* op) {
    const size_t nd = std::max(a.size(), b.size());
    std::vector<int64_t> out(nd);
    for (size_t i = 0; i < nd; ++i) {
        const int64_t da = i < a.size() ? a[a.size() - 1 - i] : 1;
        const int64_t db = i < b.size() ? b[b.size() - 1 - i] : 1;
        if (da != db && da != 1 && db != 1)
            throw std::invalid_argument(std::string(op) + ": shapes are not broadcastable");
        out[nd - 1 - i] = std::max(da, db);
    }
    return out;
}

LayerNormExtent layernorm_extent(const std::vector<int64_t>& x_shape, int64_t scale_numel, int64_t bias_numel,
                                 const Node* node) {
    const int64_t nd = (int64_t)x_shape.size();
    if (nd < 1)
        throw std::invalid_argument("LayerNormalization input must have at least 1 dimensions, got " +
                                    std::to_string(nd));
    LayerNormExtent e{1, 1, node->get_attr<float>("epsilon", 1e-5f)};
    int64_t axis = node->get_attr<int64_t>("axis", -1);
    if (axis < 0) axis += nd;
    if (axis < 0 || axis >= nd)
        throw std::invalid_argument("LayerNormalization: axis " + std::to_string(axis) + " out of range");
    for (int64_t i = 0; i < axis; ++i) e.outer *= x_shape[(size_t)i];
    for (int64_t i = axis; i < nd; ++i) e.norm *= x_shape[(size_t)i];
    if (scale_numel < e.norm || bias_numel < e.norm)
        throw std::invalid_argument("LayerNormalization: scale and bias need " + std::to_string(e.norm) +
                                    " elements, got " + std::to_string(scale_numel) + " and " +
                                    std::to_string(bias_numel));
    return e;
}

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
//  QuantizedMatMul(W, B)    W int8 2-D 2:4 along K, a_zero_point 0
//                           -> 2:4 compressed, per-tensor scale a_scale or
//                              per-channel a_scales
//  QuantizedMatMul(A, W)    A an activation, W int8 2-D (K x N, or N x K
//                           with transB = 1) 2:4 along K, b_zero_point 0
//                           -> 2:4 compressed W^T, per-tensor b_scale or
//                              per-output-column b_scales
namespace {
// The weight scales of a QuantizedMatMul: a_scales (one per row) when set,
// else the per-tensor a_scale.
std::vector<float> weight_scales(const Node& n, int64_t rows) {
    auto v = n.get_attr<std::vector<float>>("a_scales");
    if (v) {
        if ((int64_t)v->size() != rows)
            throw std::invalid_argument("QuantizedMatMul: a_scales has " + std::to_string(v->size()) +
                                        " entries for " + std::to_string(rows) + " rows");
        return *v;
    }
    return {n.get_attr<float>("a_scale", 1.0f)};
}

std::vector<float> weight_scales_b(const Node& n, int64_t cols) {
    auto v = n.get_attr<std::vector<float>>("b_scales");
    if (v) {
        if ((int64_t)v->size() != cols)
            throw std::invalid_argument("QuantizedMatMul: b_scales has " + std::to_string(v->size()) +
                                        " entries for " + std::to_string(cols) + " columns");
        return *v;
    }
    return {n.get_attr<float>("b_scale", 1.0f)};
}
}  // namespace

// The device form of a float32 initializer weight W (rows x cols) of a
// Gemm / MatMul: the product's second operand B (op(B) = W, or W^T with
// transB), or its first operand A.  The density gate picks the form:
// - at most kSparseDensityGate nonzero: a CSR (of op(B)^T, or of A) that
//   drops the zeros, with the dense kernels' non-finite rules switched on
//   (pfr_csr_dense_semantics) and NaN weights kept as stored entries, so
//   every result equals cpu_gemm / cpu_matmul on W;
// - denser: W itself for the dense product (op(B) made K x N row-major).
RocmExecutor::DeviceWeight RocmExecutor::dense_initializer_weight(const Tensor& W, bool second, bool transB) {
    const int64_t rows = W.shape()[0], cols = W.shape()[1];
    const float* d = W.data_ptr<float>();
    int64_t nnz = 0;
    bool nan = false;
    for (int64_t i = 0; i < rows * cols; ++i) {
        nnz += d[i] != 0.0f || d[i] != d[i];
        nan = nan || d[i] != d[i];
    }
    DeviceWeight w;
    const bool sparse = rows * cols == 0 || (double)nnz <= kSparseDensityGate * (double)(rows * cols);
    if (sparse) {
        // CSR rows: output features (op(B)^T) for B, rows of A for A
        const bool tr = second && !transB;  // B given K x N: its CSR is of W^T
        const int64_t M = tr ? cols : rows, K = tr ? rows : cols;
        auto at = [&](int64_t r, int64_t c) { return tr ? d[c * cols + r] : d[r * cols + c]; };
        if (!nan) {
            pfr_check(pfr_csr_from_dense(ctx_, d, rows, cols, tr ? 1 : 0, 0.0f, &w.csr));
        } else {  // to_sparse drops NaN (|NaN| > 0 fails); the dense kernels multiply it
            std::vector<int64_t> ip((size_t)M + 1, 0), ix;
            std::vector<float> v;
            ix.reserve((size_t)nnz);
            v.reserve((size_t)nnz);
            for (int64_t r = 0; r < M; ++r) {
                for (int64_t c = 0; c < K; ++c) {
                    const float x = at(r, c);
                    if (x != 0.0f || x != x) {
                        ix.push_back(c);
                        v.push_back(x);
                    }
                }
                ip[(size_t)r + 1] = (int64_t)ix.size();
            }
            pfr_check(pfr_csr_upload(ctx_, M, K, (int64_t)v.size(), ip.data(), ix.data(), v.data(), PFR_F32, nullptr,
                                     &w.csr));
        }
        w.kind = second ? DeviceWeight::CsrB : DeviceWeight::CsrA;
        pfr_check(pfr_csr_dense_semantics(w.csr));
        return w;
    }
    // dense: B as op(B) (K x N), A as is (M x K)
    std::vector<float> t;
    const float* src = d;
    if (second && transB) {  // B is N x K
        t.resize((size_t)(rows * cols));
        for (int64_t n = 0; n < rows; ++n)
            for (int64_t k = 0; k < cols; ++k) t[(size_t)(k * rows + n)] = d[n * cols + k];
        src = t.data();
    }
    void* p = nullptr;
    pfr_check(pfr_dev_alloc(ctx_, rows * cols * 4, &p));
    w.dense = static_cast<float*>(p);
    w.kind = second ? DeviceWeight::DenseB : DeviceWeight::DenseA;
    try {
        pfr_check(pfr_copy_to_device(ctx_, p, src, rows * cols * 4));
        pfr_check(pfr_synchronize(ctx_));
    } catch (...) {
        pfr_dev_free(ctx_, p);
        throw;
    }
    return w;
}

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
        auto sparse = [&](size_t i) -> const SparseInitializer* {
            return i < in.size() ? graph.get_sparse_initializer(in[i]) : nullptr;
        };
        auto csr_rec = [&](size_t i) { return sparse(i) && sparse(i)->format == SparseInitializer::Csr; };
        DeviceWeight w;
        try {
            // A CSR record stands for the zero-filled weight it was written
            // from, so its products keep the dense kernels' non-finite rules.
            if (n->op_type() == "Gemm" && csr_rec(1)) {
                // B stored K x N (transB 0) or N x K: the device weight is op(B)^T
                const bool tb = n->get_attr<int64_t>("transB", 0) != 0;
                w.csr = upload_sparse_csr(ctx_, *sparse(1), !tb);
                w.kind = DeviceWeight::CsrB;
                pfr_check(pfr_csr_dense_semantics(w.csr));
            } else if (n->op_type() == "MatMul" && csr_rec(1)) {
                w.csr = upload_sparse_csr(ctx_, *sparse(1), true);
                w.kind = DeviceWeight::CsrB;
                pfr_check(pfr_csr_dense_semantics(w.csr));
            } else if (n->op_type() == "MatMul" && csr_rec(0) && !init(1) && !sparse(1)) {
                w.csr = upload_sparse_csr(ctx_, *sparse(0), false);
                w.kind = DeviceWeight::CsrA;
                pfr_check(pfr_csr_dense_semantics(w.csr));
            } else if (n->op_type() == "QuantizedMatMul" && sparse(0) &&
                       sparse(0)->format == SparseInitializer::Nm24 && n->get_attr<int64_t>("a_zero_point", 0) == 0) {
                // expanded for the packer only; the record is 2:4 by construction
                const Tensor A = sparse(0)->to_dense();
                const std::vector<float> sc = weight_scales(*n, A.shape()[0]);
                pfr_check(pfr_sp24_pack(ctx_, A.shape()[0], A.shape()[1], A.data(), PFR_I8, sc.data(),
                                        (int64_t)sc.size(), &w.sp24));
                w.kind = DeviceWeight::Sp24A;
            } else if (n->op_type() == "Gemm" && init(1) && is_f32_matrix(*init(1))) {
                w = dense_initializer_weight(*init(1), true, n->get_attr<int64_t>("transB", 0) != 0);
            } else if (n->op_type() == "MatMul" && init(1) && is_f32_matrix(*init(1))) {
                w = dense_initializer_weight(*init(1), true, false);
            } else if (n->op_type() == "MatMul" && init(0) && !init(1) && is_f32_matrix(*init(0))) {
                w = dense_initializer_weight(*init(0), false, false);
            } else if (n->op_type() == "QuantizedMatMul" && !init(0) && !sparse(0) &&
                       ((sparse(1) && sparse(1)->format == SparseInitializer::Nm24) ||
                        (init(1) && init(1)->ndim() == 2 &&
                         (init(1)->dtype() == DType::Int8 || init(1)->dtype() == DType::UInt8))) &&
                       n->get_attr<int64_t>("b_zero_point", 0) == 0) {
                // the weight as the second operand: pack W^T (N x K), 2:4 along K
                const Tensor B = sparse(1) ? sparse(1)->to_dense() : init(1)->clone();
                const bool tb = n->get_attr<int64_t>("transB", 0) != 0;
                const int64_t Nn = tb ? B.shape()[0] : B.shape()[1], Kk = tb ? B.shape()[1] : B.shape()[0];
                std::vector<int8_t> wt((size_t)(Nn * Kk));
                const int8_t* src = static_cast<const int8_t*>(B.data());
                for (int64_t r = 0; r < Nn; ++r)
                    for (int64_t c = 0; c < Kk; ++c) wt[(size_t)(r * Kk + c)] = tb ? src[r * Kk + c] : src[c * Nn + r];
                const std::vector<float> sc = weight_scales_b(*n, Nn);
                const int st = pfr_sp24_pack(ctx_, Nn, Kk, wt.data(), PFR_I8, sc.data(), (int64_t)sc.size(), &w.sp24);
                if (st == PFR_OK) w.kind = DeviceWeight::Sp24B;
            } else if (n->op_type() == "QuantizedMatMul" && init(0) && init(0)->ndim() == 2 &&
                       (init(0)->dtype() == DType::Int8 || init(0)->dtype() == DType::UInt8) &&
                       n->get_attr<int64_t>("a_zero_point", 0) == 0) {
                const Tensor& A = *init(0);
                const std::vector<float> sc = weight_scales(*n, A.shape()[0]);
                // UInt8 data is read as int8, as the reference kernel does
                // (src/backends/cpu/ops/quantized_ops.cpp:143-144).
                const int st = pfr_sp24_pack(ctx_, A.shape()[0], A.shape()[1], A.data(), PFR_I8, sc.data(),
                                             (int64_t)sc.size(), &w.sp24);
                if (st == PFR_OK) w.kind = DeviceWeight::Sp24A;
            }
        } catch (const std::exception& e) {
            throw BackendError(std::string("preparing device weight: ") + e.what(), n->name());
        }
        if (w.kind != DeviceWeight::None) weights_[n.get()] = w;
    }
    prepare_sparse_views(graph);
    build_plan(graph);
    prepared_for_ = &graph;
}

// The device-resident plan: one step per node in topological order, each a
// device entry point; a product whose output feeds exactly one node, a Relu
// or a Gelu, and is not a graph output takes that activation into its
// epilogue (PFR_ACT_RELU / PFR_ACT_GELU: the same function of the same fp32
// value, so fusion changes no bit; the activation then runs at the
// product's position, which its single input allows).  Any node without a
// device kernel leaves plan_ok_ false.
void RocmExecutor::build_plan(const Graph& graph) {
    plan_.clear();
    fused_away_.clear();
    plan_ok_ = false;
    if (opt_ == OptLevel::None) return;
    const auto order = graph.topological_sort();
    std::unordered_map<std::string, int> uses;
    for (const auto& n : order)
        for (const auto& nm : n->inputs()) ++uses[nm];
    std::unordered_set<std::string> graph_outs;
    for (const auto& o : graph.outputs()) graph_outs.insert(o.name);

    std::vector<PlanStep> steps;
    for (const auto& np : order) {
        const Node* n = np.get();
        const std::string& op = n->op_type();
        const bool dynq = op == "DynamicQuantizeLinear" && n->inputs().size() == 1 && n->outputs().size() == 3;
        if (!dynq && n->outputs().size() != 1) return;
        const DeviceWeight* w = weight(n);
        PlanStep st{PlanStep::Relu, n, PFR_ACT_NONE, n->outputs()[0]};
        if (op == "Gemm" && w && (w->kind == DeviceWeight::CsrB || w->kind == DeviceWeight::DenseB))
            st.op = PlanStep::Gemm;
        else if (op == "MatMul" && w && (w->kind == DeviceWeight::CsrB || w->kind == DeviceWeight::DenseB))
            st.op = PlanStep::MatMulB;
        else if (op == "MatMul" && w && (w->kind == DeviceWeight::CsrA || w->kind == DeviceWeight::DenseA))
            st.op = PlanStep::MatMulA;
        else if (op == "QuantizedMatMul" && w && w->kind == DeviceWeight::Sp24A)
            st.op = PlanStep::QMatMul;
        else if (op == "QuantizedMatMul" && w && w->kind == DeviceWeight::Sp24B)
            st.op = PlanStep::QMatMulT;
        else if (op == "Relu" && n->inputs().size() == 1)
            st.op = PlanStep::Relu;
        else if (op == "Softmax" && n->inputs().size() == 1)
            st.op = PlanStep::Softmax;
        else if (op == "Gelu" && n->inputs().size() == 1)
            st.op = PlanStep::Gelu;
        else if (op == "Add" && n->inputs().size() == 2)
            st.op = PlanStep::Add;
        else if (op == "LayerNormalization" && n->inputs().size() == 3)
            st.op = PlanStep::LayerNorm;
        else if ((op == "Quantize" && n->inputs().size() == 1) ||
                 (op == "QuantizeLinear" && n->inputs().size() >= 2 && n->inputs().size() <= 3))
            st.op = PlanStep::Quant;
        else if ((op == "Dequantize" && n->inputs().size() == 1) ||
                 (op == "DequantizeLinear" && n->inputs().size() >= 2 && n->inputs().size() <= 3))
            st.op = PlanStep::Dequant;
        else if (dynq)
            st.op = PlanStep::DynQuant;
        else
            return;
        steps.push_back(st);
    }

    std::vector<bool> dropped(steps.size(), false);
    for (auto& st : steps) {
        if (opt_ == OptLevel::Basic) break;
        if (st.op != PlanStep::Gemm && st.op != PlanStep::MatMulB && st.op != PlanStep::MatMulA) continue;
        const std::string prod = st.out;
        if (uses[prod] != 1 || graph_outs.count(prod)) continue;
        for (size_t j = 0; j < steps.size(); ++j) {
            const bool relu = steps[j].op == PlanStep::Relu, gelu = steps[j].op == PlanStep::Gelu;
            if (dropped[j] || !(relu || gelu) || steps[j].node->inputs()[0] != prod) continue;
            st.act = relu ? PFR_ACT_RELU : PFR_ACT_GELU;
            st.out = steps[j].out;
            dropped[j] = true;
            fused_away_.insert(prod);
            break;
        }
    }

    // Initializers a step reads as an activation (biases, LayerNorm's scale
    // and bias, a constant operand of an elementwise step) go to the device
    // once; the pruned operand of a product is already a device weight.
    for (size_t i = 0; i < steps.size(); ++i) {
        if (dropped[i]) continue;
        const PlanStep& st = steps[i];
        const auto& in = st.node->inputs();
        const int weight_slot = (st.op == PlanStep::Gemm || st.op == PlanStep::MatMulB || st.op == PlanStep::QMatMulT)
                                    ? 1
                                : (st.op == PlanStep::MatMulA || st.op == PlanStep::QMatMul) ? 0
                                                                                             : -1;
        for (size_t k = 0; k < in.size(); ++k) {
            if ((int)k == weight_slot || constants_.count(in[k]) || !graph.has_initializer(in[k])) continue;
            const Tensor& src = initializer_value(graph, in[k]);
            DevTensor d;
            d.shape = src.shape();
            d.dtype = src.dtype();
            const int64_t bytes = (int64_t)src.size_bytes();
            pfr_check(pfr_dev_alloc(ctx_, std::max<int64_t>(bytes, 256), &d.p));
            constants_[in[k]] = d;
            if (bytes) pfr_check(pfr_copy_to_device(ctx_, d.p, src.data(), bytes));
        }
        plan_.push_back(st);
    }
    pfr_check(pfr_synchronize(ctx_));
    plan_ok_ = true;
}

// Runs the plan: graph inputs to the device, every step on the context's
// stream with no host round trip, requested outputs back.  Shape and dtype
// checks and their texts are those of the rocm:: OpFuncs.
std::vector<Tensor> RocmExecutor::execute_plan(const Graph& graph,
                                               const std::unordered_map<std::string, Tensor>& input_feed,
                                               const std::vector<std::string>& names) {
    StreamDrain drain{ctx_};
    std::unordered_map<std::string, DevTensor> live(constants_);
    std::vector<std::pair<const Node*, void*>> statuses;  // DynamicQuantizeLinear scale checks
    for (const auto& kv : input_feed) {
        const Tensor& t = kv.second;
        const int64_t bytes = (int64_t)t.size_bytes();
        DevTensor d;
        d.p = device_buffer(kv.first, bytes);
        d.shape = t.shape();
        d.dtype = t.dtype();
        if (bytes) pfr_check(pfr_copy_to_device(ctx_, d.p, t.data(), bytes));
        live[kv.first] = d;
    }

    for (const PlanStep& st : plan_) {
        const Node* n = st.node;
        const auto& in = n->inputs();
        auto act_in = [&](size_t i) -> const DevTensor& {
            auto it = live.find(in[i]);
            if (it == live.end()) throw BackendError("Input tensor '" + in[i] + "' not found", n->name());
            return it->second;
        };
        auto init_in = [&](size_t i) -> const Tensor& { return weight_tensor(graph, in[i]); };
        auto need_inputs = [&](size_t k, const char* op) {
            if (in.size() < k)
                throw std::invalid_argument(std::string(op) + ": expected at least " + std::to_string(k) +
                                            " inputs, got " + std::to_string(in.size()));
        };
        const int act = st.act;
        DevTensor out;
        out.dtype = DType::Float32;
        try {
            switch (st.op) {
            case PlanStep::Gemm: {
                // math.cpp:377-438; the same checks as rocm::Gemm.
                need_inputs(2, "Gemm");
                const DevTensor& A = act_in(0);
                const Tensor& B = init_in(1);
                const DevTensor* C = in.size() > 2 ? &act_in(2) : nullptr;
                if (A.shape.size() < 2 || B.ndim() < 2)
                    throw std::invalid_argument("Gemm input A/B must have at least 2 dimensions");
                need_f32(A.dtype, "Gemm input A");
                const float alpha = n->get_attr<float>("alpha", 1.0f);
                const float beta = n->get_attr<float>("beta", 1.0f);
                const int64_t ta = n->get_attr<int64_t>("transA", 0);
                const int64_t tb = n->get_attr<int64_t>("transB", 0);
                const int64_t M = ta ? A.shape[1] : A.shape[0];
                const int64_t Ka = ta ? A.shape[0] : A.shape[1];
                const int64_t Kb = tb ? B.shape()[1] : B.shape()[0];
                const int64_t N = tb ? B.shape()[0] : B.shape()[1];
                if (Ka != Kb)
                    throw std::invalid_argument("Gemm: incompatible dimensions - A has K=" + std::to_string(Ka) +
                                                ", B has K=" + std::to_string(Kb));
                const float* c = nullptr;
                int64_t c_size = 0;
                if (C && numel(C->shape) > 0) {
                    need_f32(C->dtype, "Gemm input C");
                    c = static_cast<const float*>(C->p);
                    c_size = numel(C->shape);
                }
                out.shape = {M, N};
                out.p = device_buffer(st.out, M * N * 4);
                const DeviceWeight* w = weight(n);
                if (w->kind == DeviceWeight::DenseB)
                    pfr_check(pfr_gemm_dense_dev(ctx_, static_cast<const float*>(A.p), M, Ka, (int)ta, w->dense, N, N,
                                                 alpha, beta, c, c_size, static_cast<float*>(out.p), N, act));
                else
                    pfr_check(pfr_gemm_csr_act_dev(ctx_, static_cast<const float*>(A.p), M, Ka, (int)ta, w->csr,
                                                   alpha, beta, c, c_size, static_cast<float*>(out.p), math_mode_,
                                                   act));
                break;
            }
            case PlanStep::MatMulB:
            case PlanStep::MatMulA: {
                // math.cpp:268-374; the same checks as rocm::MatMul.
                need_inputs(2, "MatMul");
                const bool wb = st.op == PlanStep::MatMulB;
                const std::vector<int64_t> as = wb ? act_in(0).shape : init_in(0).shape();
                const std::vector<int64_t> bs = wb ? init_in(1).shape() : act_in(1).shape;
                if (as.size() < 2 || bs.size() < 2)
                    throw std::invalid_argument("MatMul: inputs must have at least 2 dimensions");
                const int64_t Ka = as.back(), Kb = bs[bs.size() - 2];
                if (Ka != Kb)
                    throw std::invalid_argument("MatMul: incompatible dimensions - A has inner dim " +
                                                std::to_string(Ka) + ", B has inner dim " + std::to_string(Kb));
                if (wb) {
                    const DevTensor& A = act_in(0);
                    need_f32(A.dtype, "MatMul input A");
                    const int64_t N = bs[1];
                    out.shape.assign(as.begin(), as.end() - 1);
                    const int64_t rows = numel(out.shape);
                    out.shape.push_back(N);
                    out.p = device_buffer(st.out, rows * N * 4);
                    const DeviceWeight* w = weight(n);
                    if (w->kind == DeviceWeight::DenseB)
                        pfr_check(pfr_gemm_dense_dev(ctx_, static_cast<const float*>(A.p), rows, Ka, 0, w->dense, N, N,
                                                     1.0f, 1.0f, nullptr, 0, static_cast<float*>(out.p), N, act));
                    else
                        pfr_check(pfr_gemm_csr_act_dev(ctx_, static_cast<const float*>(A.p), rows, Ka, 0, w->csr,
                                                       1.0f, 1.0f, nullptr, 0, static_cast<float*>(out.p), math_mode_,
                                                       act));
                } else {
                    const DevTensor& B = act_in(1);
                    need_f32(B.dtype, "MatMul input B");
                    if (bs.size() != 2)
                        throw std::invalid_argument("MatMul: a pruned first operand needs a 2-D second operand");
                    const int64_t M = as[0], N = bs[1];
                    out.shape = {M, N};
                    out.p = device_buffer(st.out, M * N * 4);
                    const DeviceWeight* w = weight(n);
                    if (w->kind == DeviceWeight::DenseA)
                        pfr_check(pfr_gemm_dense_dev(ctx_, w->dense, M, Ka, 0, static_cast<const float*>(B.p), N, N,
                                                     1.0f, 1.0f, nullptr, 0, static_cast<float*>(out.p), N, act));
                    else
                        pfr_check(pfr_spmm_csr_act_dev(ctx_, w->csr, static_cast<const float*>(B.p), N, N,
                                                       static_cast<float*>(out.p), N, math_mode_, act));
                }
                break;
            }
            case PlanStep::QMatMul: {
                // quantized_ops.cpp:77-167; the same checks as rocm::QuantizedMatMul.
                need_inputs(2, "QuantizedMatMul");
                const Tensor& a = init_in(0);
                const DevTensor& b = act_in(1);
                if (b.dtype != DType::Int8 && b.dtype != DType::UInt8)
                    throw std::invalid_argument("QuantizedMatMul: input B must be Int8 or UInt8");
                if (b.shape.size() < 2)
                    throw std::invalid_argument("QuantizedMatMul: inputs must have at least 2 dimensions");
                const int64_t K = a.shape().back(), Kb = b.shape[b.shape.size() - 2];
                if (K != Kb)
                    throw std::invalid_argument("QuantizedMatMul: inner dimensions must match (got " +
                                                std::to_string(K) + " and " + std::to_string(Kb) + ")");
                if (b.shape.size() != 2)
                    throw std::runtime_error("QuantizedMatMul: the rocm backend needs a 2-D int8 initializer A that "
                                             "is 2:4 sparse along K, zero points 0, and a 2-D B");
                // two inputs: B's bytes as int8, scale and zero point attributes
                // (quantized_ops.cpp:87-90, :143-144); four: B's scale and zero
                // point as device tensors, uint8 B as uint8
                float b_scale = n->get_attr<float>("b_scale", 1.0f);
                int32_t b_zp = (int32_t)n->get_attr<int64_t>("b_zero_point", 0);
                const float* s_dev = nullptr;
                const uint8_t* z_dev = nullptr;
                pfr_dtype bdt = PFR_I8;
                if (in.size() >= 4) {
                    const DevTensor& s = act_in(2);
                    const DevTensor& z = act_in(3);
                    if (s.dtype != DType::Float32 || numel(s.shape) != 1)
                        throw std::invalid_argument("QuantizedMatMul: b_scale input must be one float32");
                    if ((z.dtype != DType::UInt8 && z.dtype != DType::Int8) || numel(z.shape) != 1)
                        throw std::invalid_argument("QuantizedMatMul: b_zero_point input must be one int8 or uint8");
                    s_dev = static_cast<const float*>(s.p);
                    if (z.dtype == DType::UInt8) {
                        z_dev = static_cast<const uint8_t*>(z.p);
                    } else {
                        int8_t zv = 0;
                        pfr_check(pfr_copy_to_host(ctx_, &zv, z.p, 1));
                        b_zp = zv;
                    }
                    bdt = b.dtype == DType::UInt8 ? PFR_U8 : PFR_I8;
                }
                const int64_t M = a.shape()[0], N = b.shape[1];
                out.shape = {M, N};
                out.p = device_buffer(st.out, M * N * 4);
                pfr_check(pfr_sp24_gemm_q_dev(ctx_, weight(n)->sp24, b.p, bdt, N, N, b_scale, b_zp, s_dev, z_dev,
                                              PFR_SP24_OUT_F32, 1.0f, 0, out.p, N));
                break;
            }
            case PlanStep::QMatMulT: {
                // the x . W form: A the activation, B the 2:4 weight (our
                // extension of quantized_ops.cpp:77-167 to a weight in the B
                // position, transB and per-column b_scales)
                need_inputs(2, "QuantizedMatMul");
                const DevTensor& a = act_in(0);
                if (a.dtype != DType::Int8 && a.dtype != DType::UInt8)
                    throw std::invalid_argument("QuantizedMatMul: input A must be Int8 or UInt8");
                const Tensor& b = init_in(1);
                const bool tb = n->get_attr<int64_t>("transB", 0) != 0;
                const int64_t Kb = tb ? b.shape()[1] : b.shape()[0], N = tb ? b.shape()[0] : b.shape()[1];
                if (a.shape.size() != 2)
                    throw std::runtime_error("QuantizedMatMul: the rocm backend needs a 2-D activation A with a 2:4 "
                                             "weight B");
                if (a.shape[1] != Kb)
                    throw std::invalid_argument("QuantizedMatMul: inner dimensions must match (got " +
                                                std::to_string(a.shape[1]) + " and " + std::to_string(Kb) + ")");
                float a_scale = n->get_attr<float>("a_scale", 1.0f);
                int32_t a_zp = (int32_t)n->get_attr<int64_t>("a_zero_point", 0);
                const float* s_dev = nullptr;
                const uint8_t* z_dev = nullptr;
                pfr_dtype adt = PFR_I8;
                if (in.size() >= 4) {
                    const DevTensor& s = act_in(2);
                    const DevTensor& z = act_in(3);
                    if (s.dtype != DType::Float32 || numel(s.shape) != 1)
                        throw std::invalid_argument("QuantizedMatMul: a_scale input must be one float32");
                    if ((z.dtype != DType::UInt8 && z.dtype != DType::Int8) || numel(z.shape) != 1)
                        throw std::invalid_argument("QuantizedMatMul: a_zero_point input must be one int8 or uint8");
                    s_dev = static_cast<const float*>(s.p);
                    if (z.dtype == DType::UInt8) {
                        z_dev = static_cast<const uint8_t*>(z.p);
                    } else {
                        int8_t zv = 0;
                        pfr_check(pfr_copy_to_host(ctx_, &zv, z.p, 1));
                        a_zp = zv;
                    }
                    adt = a.dtype == DType::UInt8 ? PFR_U8 : PFR_I8;
                }
                const int64_t T = a.shape[0];
                out.shape = {T, N};
                out.p = device_buffer(st.out, std::max<int64_t>(T * N, 1) * 4);
                pfr_check(pfr_sp24_gemm_qt_dev(ctx_, weight(n)->sp24, a.p, adt, T, Kb, a_scale, a_zp, s_dev, z_dev,
                                               static_cast<float*>(out.p), N));
                break;
            }
            case PlanStep::DynQuant: {
                // quantized_ops.cpp:251-278; outputs y (uint8), scale [1], zero point [1]
                const DevTensor& x = act_in(0);
                if (x.dtype != DType::Float32)
                    throw std::invalid_argument("DynamicQuantizeLinear: input must be Float32");
                const int64_t cnt = numel(x.shape);
                const auto& outs = n->outputs();
                DevTensor sc, zp;
                sc.p = device_buffer(outs[1], 4);
                sc.shape = {1};
                sc.dtype = DType::Float32;
                zp.p = device_buffer(outs[2], 1);
                zp.shape = {1};
                zp.dtype = DType::UInt8;
                out.p = device_buffer(st.out, cnt);
                out.shape = x.shape;
                out.dtype = DType::UInt8;
                // the status word (a non-finite scale) sits after the scale
                void* status = device_buffer(std::string("\x01status:") + n->name(), 4);
                pfr_check(pfr_dynamic_quantize_linear_dev(ctx_, static_cast<const float*>(x.p), cnt,
                                                          static_cast<uint8_t*>(out.p), static_cast<float*>(sc.p),
                                                          static_cast<uint8_t*>(zp.p), static_cast<int32_t*>(status)));
                statuses.push_back({n, status});
                live[outs[1]] = sc;
                live[outs[2]] = zp;
                break;
            }
            case PlanStep::Relu: {
                // activation.cpp:45-60.
                const DevTensor& x = act_in(0);
                need_f32(x.dtype, "Relu input");
                out.shape = x.shape;
                out.p = device_buffer(st.out, numel(x.shape) * 4);
                pfr_check(pfr_relu_dev(ctx_, static_cast<const float*>(x.p), numel(x.shape),
                                       static_cast<float*>(out.p)));
                break;
            }
            case PlanStep::Softmax: {
                // activation.cpp:157-237.
                const DevTensor& x = act_in(0);
                need_f32(x.dtype, "Softmax input");
                int64_t axis = n->get_attr<int64_t>("axis", -1);
                const int64_t nd = (int64_t)x.shape.size();
                if (axis < -nd || axis >= nd)
                    throw std::invalid_argument("Softmax: axis " + std::to_string(axis) + " out of range for " +
                                                std::to_string(nd) + "-D input");
                if (axis < 0) axis += nd;
                int64_t outer = 1, inner = 1;
                for (int64_t i = 0; i < axis; ++i) outer *= x.shape[i];
                for (int64_t i = axis + 1; i < nd; ++i) inner *= x.shape[i];
                out.shape = x.shape;
                out.p = device_buffer(st.out, numel(x.shape) * 4);
                pfr_check(pfr_softmax_dev(ctx_, static_cast<const float*>(x.p), outer, x.shape[axis], inner,
                                          static_cast<float*>(out.p)));
                break;
            }
            case PlanStep::Gelu: {
                // activation.cpp:239-259.
                const DevTensor& x = act_in(0);
                need_f32(x.dtype, "Gelu input");
                out.shape = x.shape;
                out.p = device_buffer(st.out, numel(x.shape) * 4);
                pfr_check(pfr_gelu_dev(ctx_, static_cast<const float*>(x.p), numel(x.shape),
                                       static_cast<float*>(out.p)));
                break;
            }
            case PlanStep::Add: {
                // math.cpp:150-226.
                const DevTensor& a = act_in(0);
                const DevTensor& b = act_in(1);
                need_f32(a.dtype, "Add input A");
                need_f32(b.dtype, "Add input B");
                out.shape = broadcast_shapes(a.shape, b.shape, "Add");
                out.p = device_buffer(st.out, std::max<int64_t>(numel(out.shape), 1) * 4);
                pfr_check(pfr_add_dev(ctx_, static_cast<const float*>(a.p), a.shape.data(), (int)a.shape.size(),
                                      static_cast<const float*>(b.p), b.shape.data(), (int)b.shape.size(),
                                      static_cast<float*>(out.p)));
                break;
            }
            case PlanStep::Quant:
            case PlanStep::Dequant: {
                // quantized_ops.cpp:35-70, :284-347: per-tensor parameters from
                // attributes or from the first elements of the scale and zero
                // point inputs (read back when a node produced them)
                const bool q = st.op == PlanStep::Quant;
                const bool lin = n->op_type().size() > 8 && n->op_type().compare(n->op_type().size() - 6, 6, "Linear") == 0;
                const DevTensor& x = act_in(0);
                float scale = n->get_attr<float>("scale", 1.0f);
                int32_t zp = (int32_t)n->get_attr<int64_t>("zero_point", 0);
                auto first_bytes = [&](size_t i, void* dst, size_t bytes) {
                    if (graph.has_initializer(in[i])) {
                        std::memcpy(dst, initializer_value(graph, in[i]).data(), bytes);
                    } else {
                        pfr_check(pfr_copy_to_host(ctx_, dst, act_in(i).p, (int64_t)bytes));
                    }
                };
                auto in_dtype = [&](size_t i) {
                    return graph.has_initializer(in[i]) ? initializer_value(graph, in[i]).dtype() : act_in(i).dtype;
                };
                auto in_numel = [&](size_t i) {
                    return graph.has_initializer(in[i]) ? initializer_value(graph, in[i]).num_elements()
                                                        : numel(act_in(i).shape);
                };
                if (lin) {
                    if (in_dtype(1) != DType::Float32 || in_numel(1) < 1)
                        throw std::invalid_argument(n->op_type() + ": scale must be a float32 tensor");
                    first_bytes(1, &scale, 4);
                    zp = 0;
                    if (in.size() > 2 && in_numel(2) >= 1) {
                        if (in_dtype(2) == DType::Int8) {
                            int8_t v;
                            first_bytes(2, &v, 1);
                            zp = v;
                        } else if (in_dtype(2) == DType::UInt8) {
                            uint8_t v;
                            first_bytes(2, &v, 1);
                            zp = v;
                        }
                    }
                }
                out.shape = x.shape;
                const int64_t cnt = numel(x.shape);
                if (q) {
                    const bool u8 = n->get_attr<std::string>(lin ? "output_dtype" : "dtype", "int8") == "uint8";
                    const pfr_dtype dt = u8 ? PFR_U8 : PFR_I8;
                    pfr_check(pfr_quantize_linear_dev(ctx_, nullptr, 0, scale, zp, dt, nullptr));  // parameter checks
                    if (x.dtype != DType::Float32)
                        throw std::invalid_argument("quantize_tensor: input must be Float32, got " + dtype_name(x.dtype));
                    out.dtype = u8 ? DType::UInt8 : DType::Int8;
                    out.p = device_buffer(st.out, std::max<int64_t>(cnt, 1));
                    pfr_check(pfr_quantize_linear_dev(ctx_, static_cast<const float*>(x.p), cnt, scale, zp, dt, out.p));
                } else {
                    const pfr_dtype dt =
                        x.dtype == DType::Int8 ? PFR_I8 : (x.dtype == DType::UInt8 ? PFR_U8 : PFR_F32);
                    out.dtype = DType::Float32;
                    out.p = device_buffer(st.out, std::max<int64_t>(cnt, 1) * 4);
                    pfr_check(pfr_dequantize_linear_dev(ctx_, x.p, dt, cnt, scale, zp, static_cast<float*>(out.p)));
                }
                break;
            }
            case PlanStep::LayerNorm: {
                // nn.cpp:419-478.
                const DevTensor& x = act_in(0);
                const DevTensor& sc = act_in(1);
                const DevTensor& bi = act_in(2);
                need_f32(x.dtype, "LayerNormalization input");
                need_f32(sc.dtype, "LayerNormalization scale");
                need_f32(bi.dtype, "LayerNormalization bias");
                const LayerNormExtent e = layernorm_extent(x.shape, numel(sc.shape), numel(bi.shape), n);
                out.shape = x.shape;
                out.p = device_buffer(st.out, numel(x.shape) * 4);
                pfr_check(pfr_layernorm_dev(ctx_, static_cast<const float*>(x.p), e.outer, e.norm,
                                            static_cast<const float*>(sc.p), static_cast<const float*>(bi.p),
                                            e.epsilon, static_cast<float*>(out.p)));
                break;
            }
            }
        } catch (const BackendError&) {
            throw;
        } catch (const std::exception& e) {
            throw BackendError(e.what(), n->name());
        }
        live[st.out] = out;
    }

    std::vector<Tensor> results;
    results.reserve(names.size());
    for (const auto& nm : names) {
        auto it = live.find(nm);
        if (it == live.end() && graph.has_initializer(nm)) {
            results.push_back(initializer_value(graph, nm).clone());  // a weight asked for as an output
            continue;
        }
        if (it == live.end()) throw BackendError("Output tensor '" + nm + "' not found");
        const DevTensor& d = it->second;
        Tensor t(d.shape, d.dtype);
        const int64_t bytes = (int64_t)t.size_bytes();
        try {
            if (bytes) pfr_check(pfr_copy_to_host(ctx_, t.data(), d.p, bytes));
        } catch (const std::exception& e) {
            throw BackendError(e.what());
        }
        results.push_back(std::move(t));
    }
    pfr_check(pfr_synchronize(ctx_));
    drain.armed = false;
    for (const auto& ns : statuses) {
        int32_t status = 0;
        pfr_check(pfr_copy_to_host(ctx_, &status, ns.second, 4));
        if (status)
            throw BackendError("QuantParams::per_tensor: scale must be positive and finite", ns.first->name());
    }
    return results;
}

std::vector<Tensor> RocmExecutor::execute(const Graph& graph, const std::unordered_map<std::string, Tensor>& input_feed,
                                          const std::vector<std::string>& output_names) {
    validate_inputs(graph, input_feed);
    prepare(graph);
    CurrentGuard guard(this);
    std::vector<std::string> names = output_names;
    if (names.empty())
        for (const auto& o : graph.outputs()) names.push_back(o.name);
    bool on_device = plan_ok_;
    for (const auto& nm : names)
        if (fused_away_.count(nm)) on_device = false;  // an intermediate the fused plan never writes
    last_on_device_ = on_device;
    if (on_device) return execute_plan(graph, input_feed, names);

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
        const DeviceWeight* w = weight(node.get());
        const int wslot = !w ? -1 : (w->second() ? 1 : 0);
        for (size_t i = 0; i < node->inputs().size(); ++i) {
            const std::string& nm = node->inputs()[i];
            auto it = view.find(nm);
            if (it == view.end() && graph.get_sparse_initializer(nm)) {
                // the prepared weight slot gets the shape-only view, any other
                // use the expanded tensor
                ins.push_back((int)i == wslot ? &sparse_views_.at(nm) : &initializer_value(graph, nm));
                continue;
            }
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
        if (v != view.end()) {
            results.push_back(v->second->clone());
        } else if (graph.get_sparse_initializer(nm)) {
            results.push_back(initializer_value(graph, nm).clone());
        } else {
            throw BackendError("Output tensor '" + nm + "' not found");
        }
    }
    return results;
}

std::unique_ptr<Backend> create_backend(const std::string& name, int /*num_threads*/) {
    if (name == "rocm") return std::make_unique<RocmExecutor>();
    throw UnsupportedFormatError(name, {"rocm"});
}

}  // namespace pyflame_rt
