// The dynamic int8 rewrite of 2:4-pruned MatMul(W, X), MatMul(X, W) and
// Gemm(X, W[, b]) nodes (declared in quantize.hpp).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <unordered_map>

#include "pyflame_rt/errors.hpp"
#include "pyflame_rt/quantize.hpp"

namespace pyflame_rt {

namespace {

// Per-row symmetric int8 parameters and values of a rows x cols weight, as
// compute_dynamic_params_per_channel(W, axis 0, Int8, symmetric) and the
// per-channel quantize_tensor compute them on the reference's x86 build.
void quantize_rows(const float* w, int64_t rows, int64_t cols, std::vector<float>& scales, std::vector<int8_t>& q) {
    scales.assign((size_t)rows, 1.0f);
    q.assign((size_t)(rows * cols), 0);
    for (int64_t r = 0; r < rows; ++r) {
        const float* row = w + r * cols;
        float mn = std::numeric_limits<float>::max(), mx = std::numeric_limits<float>::lowest();
        for (int64_t c = 0; c < cols; ++c)
            if (std::isfinite(row[c])) {
                mn = std::min(mn, row[c]);
                mx = std::max(mx, row[c]);
            }
        if (mn > mx) mn = mx = 0.0f;  // no finite value (quant_ops.cpp:366-372)
        float s = 1.0f;
        if (!(std::abs(mx - mn) < 1e-8f)) {  // quant_params.cpp:78-82
            s = std::max(std::abs(mn), std::abs(mx)) / 127.0f;
            if (s < 1e-10f) s = 1e-10f;
        }
        if (!(s > 0.0f) || !std::isfinite(s))
            throw std::invalid_argument("quantize_tensor: invalid scale for channel " + std::to_string(r));
        scales[(size_t)r] = s;
        const float inv = 1.0f / s;
        for (int64_t c = 0; c < cols; ++c) {
            const float v = std::round(row[c] * inv);
            // static_cast<int32_t> as x86 executes it: the integer indefinite
            // value for NaN and out-of-range results
            const int32_t i = (v >= -2147483648.0f && v < 2147483648.0f) ? (int32_t)v : INT32_MIN;
            q[(size_t)(r * cols + c)] = (int8_t)std::clamp(i, -128, 127);
        }
    }
}

bool at_most_two_per_four(const float* w, int64_t rows, int64_t cols) {
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t g = 0; g < cols; g += 4) {
            int nz = 0;
            for (int64_t c = g; c < std::min(g + 4, cols); ++c) nz += w[r * cols + c] != 0.0f;
            if (nz > 2) return false;
        }
    return true;
}

SparseInitializer nm24_record(const std::vector<int8_t>& q, int64_t rows, int64_t cols) {
    SparseInitializer s;
    s.format = SparseInitializer::Nm24;
    s.dtype = DType::Int8;
    s.rows = rows;
    s.cols = cols;
    const int64_t groups = cols / 4;
    s.values.assign((size_t)(rows * groups * 2), 0);
    s.positions.assign((size_t)(rows * groups), 0);
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t g = 0; g < groups; ++g) {
            const int8_t* v = &q[(size_t)(r * cols + 4 * g)];
            int pos[2], n = 0;
            for (int i = 0; i < 4 && n < 2; ++i)
                if (v[i] != 0) pos[n++] = i;
            for (int i = 0; i < 4 && n < 2; ++i)  // pad with the lowest unused offsets
                if (v[i] == 0 && (n == 0 || pos[0] != i)) pos[n++] = i;
            if (pos[0] > pos[1]) std::swap(pos[0], pos[1]);
            s.values[(size_t)((r * groups + g) * 2)] = (uint8_t)v[pos[0]];
            s.values[(size_t)((r * groups + g) * 2 + 1)] = (uint8_t)v[pos[1]];
            s.positions[(size_t)(r * groups + g)] = (uint8_t)(pos[0] | (pos[1] << 2));
        }
    return s;
}

// A float weight initializer (dense, or a CSR record expanded) as a 2-D
// float32 tensor, or null.
const Tensor* float_weight(const Graph& g, const std::string& name, Tensor& keep) {
    if (auto t = g.get_initializer(name)) {
        const Tensor* w = &t->get();
        return w->dtype() == DType::Float32 && w->ndim() == 2 && w->shape()[0] > 0 && w->shape()[1] > 0 ? w : nullptr;
    }
    if (const SparseInitializer* s = g.get_sparse_initializer(name))
        if (s->format == SparseInitializer::Csr) {
            keep = s->to_dense();
            return keep.dtype() == DType::Float32 && keep.shape()[0] > 0 && keep.shape()[1] > 0 ? &keep : nullptr;
        }
    return nullptr;
}

std::string fresh(const Graph& g, const std::unordered_map<std::string, int>& taken, const std::string& base) {
    std::string n = base;
    for (int i = 1; taken.count(n) || g.has_initializer(n); ++i) n = base + "_" + std::to_string(i);
    return n;
}

}  // namespace

std::unique_ptr<Graph> quantize_dynamic_int8(const Graph& g, QuantizeStats* stats) {
    QuantizeStats st;
    std::unordered_map<std::string, int> uses, names;  // tensor uses; every tensor / node name in the graph
    for (const auto& n : g.nodes()) {
        names[n->name()] = 1;
        for (const auto& t : n->inputs()) ++uses[t], names[t] = 1;
        for (const auto& t : n->outputs()) names[t] = 1;
    }
    for (const auto& i : g.inputs()) names[i.name] = 1;
    for (const auto& o : g.outputs()) names[o.name] = 1;

    auto out = std::make_unique<Graph>(g.name());
    for (const auto& i : g.inputs()) out->add_input(i);
    for (const auto& o : g.outputs()) out->add_output(o);

    std::unordered_map<std::string, int> consumed;  // float weights replaced, by name
    std::vector<std::shared_ptr<Node>> nodes;
    for (const auto& np : g.nodes()) {
        const Node& n = *np;
        bool done = false;
        if (n.op_type() == "MatMul" && n.inputs().size() == 2 && n.outputs().size() == 1 &&
            !g.has_initializer(n.inputs()[1])) {
            const std::string& wn = n.inputs()[0];
            Tensor dense;
            const Tensor* w = nullptr;
            if (auto t = g.get_initializer(wn)) {
                w = &t->get();
            } else if (const SparseInitializer* s = g.get_sparse_initializer(wn)) {
                if (s->format == SparseInitializer::Csr) {
                    dense = s->to_dense();
                    w = &dense;
                }
            }
            if (w && w->dtype() == DType::Float32 && w->ndim() == 2 && w->shape()[0] > 0 && w->shape()[1] > 0 &&
                at_most_two_per_four(w->data_ptr<float>(), w->shape()[0], w->shape()[1])) {
                const int64_t rows = w->shape()[0], cols = w->shape()[1];
                std::vector<float> scales;
                std::vector<int8_t> q;
                quantize_rows(w->data_ptr<float>(), rows, cols, scales, q);
                const std::string base = n.name();
                const std::string wq = fresh(g, names, wn + "_int8");
                names[wq] = 1;
                if (cols % 4 == 0) {
                    SparseInitializer rec = nm24_record(q, rows, cols);
                    st.int8_bytes += (int64_t)rec.stored_bytes();
                    out->add_sparse_initializer(wq, std::move(rec));
                } else {
                    Tensor t({rows, cols}, DType::Int8);
                    std::memcpy(t.data(), q.data(), q.size());
                    st.int8_bytes += (int64_t)q.size();
                    out->add_initializer(wq, std::move(t));
                }
                st.int8_bytes += 4 * rows;
                st.float_bytes += 4 * rows * cols;
                std::vector<std::string> qo;
                for (const char* suffix : {"_quantized", "_scale", "_zero_point"}) {
                    qo.push_back(fresh(g, names, n.inputs()[1] + "/" + base + suffix));
                    names[qo.back()] = 1;
                }
                const std::string dq_name = fresh(g, names, base + "_quantize_input");
                names[dq_name] = 1;
                nodes.push_back(std::make_shared<Node>(dq_name, "DynamicQuantizeLinear",
                                                       std::vector<std::string>{n.inputs()[1]}, qo));
                auto qmm = std::make_shared<Node>(base, "QuantizedMatMul",
                                                  std::vector<std::string>{wq, qo[0], qo[1], qo[2]}, n.outputs());
                qmm->set_attr("a_scales", scales);
                qmm->set_attr("a_zero_point", (int64_t)0);
                nodes.push_back(qmm);
                ++consumed[wn];
                ++st.rewritten;
                done = true;
            }
        }
        // The x . W form: MatMul(X, W) with W K x N, or Gemm(X, W[, b]) with
        // transA 0, alpha 1, beta 1 and a bias of N floats; W 2:4 along K.
        // The weight goes in as W^T (N x K, transB = 1) with per-output-column
        // scales; a Gemm bias becomes an Add (Gemm's bias modulo is numpy
        // broadcasting for a bias of N elements).
        const bool mm = n.op_type() == "MatMul" && n.inputs().size() == 2;
        const bool gm = n.op_type() == "Gemm" && (n.inputs().size() == 2 || n.inputs().size() == 3) &&
                        n.get_attr<int64_t>("transA", 0) == 0 && n.get_attr<float>("alpha", 1.0f) == 1.0f &&
                        (n.inputs().size() == 2 || n.get_attr<float>("beta", 1.0f) == 1.0f);
        if (!done && (mm || gm) && n.outputs().size() == 1 && !g.has_initializer(n.inputs()[0]) &&
            !g.get_sparse_initializer(n.inputs()[0])) {
            const std::string& wn = n.inputs()[1];
            Tensor keep;
            const Tensor* w = float_weight(g, wn, keep);
            const bool tb = gm && n.get_attr<int64_t>("transB", 0) != 0;
            const Tensor* bias = nullptr;
            if (w && gm && n.inputs().size() == 3) {
                auto c = g.get_initializer(n.inputs()[2]);
                const int64_t N = tb ? w->shape()[0] : w->shape()[1];
                if (c && c->get().dtype() == DType::Float32 && c->get().num_elements() == N &&
                    (c->get().ndim() == 1 || (c->get().ndim() == 2 && c->get().shape()[0] == 1)))
                    bias = &c->get();
                else
                    w = nullptr;  // another bias shape: left as it is
            }
            if (w) {
                const int64_t N = tb ? w->shape()[0] : w->shape()[1], K = tb ? w->shape()[1] : w->shape()[0];
                std::vector<float> wt((size_t)(N * K));  // W^T, N x K
                const float* src = w->data_ptr<float>();
                for (int64_t r = 0; r < N; ++r)
                    for (int64_t c = 0; c < K; ++c) wt[(size_t)(r * K + c)] = tb ? src[r * K + c] : src[c * N + r];
                if (at_most_two_per_four(wt.data(), N, K)) {
                    std::vector<float> scales;
                    std::vector<int8_t> q;
                    quantize_rows(wt.data(), N, K, scales, q);
                    const std::string base = n.name();
                    const std::string wq = fresh(g, names, wn + "_int8_t");
                    names[wq] = 1;
                    if (K % 4 == 0) {
                        SparseInitializer rec = nm24_record(q, N, K);
                        st.int8_bytes += (int64_t)rec.stored_bytes();
                        out->add_sparse_initializer(wq, std::move(rec));
                    } else {
                        Tensor t({N, K}, DType::Int8);
                        std::memcpy(t.data(), q.data(), q.size());
                        st.int8_bytes += (int64_t)q.size();
                        out->add_initializer(wq, std::move(t));
                    }
                    st.int8_bytes += 4 * N;
                    st.float_bytes += 4 * N * K;
                    std::vector<std::string> qo;
                    for (const char* suffix : {"_quantized", "_scale", "_zero_point"}) {
                        qo.push_back(fresh(g, names, n.inputs()[0] + "/" + base + suffix));
                        names[qo.back()] = 1;
                    }
                    const std::string dq_name = fresh(g, names, base + "_quantize_input");
                    names[dq_name] = 1;
                    nodes.push_back(std::make_shared<Node>(dq_name, "DynamicQuantizeLinear",
                                                           std::vector<std::string>{n.inputs()[0]}, qo));
                    std::vector<std::string> qmm_out = n.outputs();
                    if (bias) {
                        qmm_out = {fresh(g, names, n.outputs()[0] + "/" + base + "_product")};
                        names[qmm_out[0]] = 1;
                    }
                    auto qmm = std::make_shared<Node>(bias ? fresh(g, names, base + "_product") : base,
                                                      "QuantizedMatMul",
                                                      std::vector<std::string>{qo[0], wq, qo[1], qo[2]}, qmm_out);
                    names[qmm->name()] = 1;
                    qmm->set_attr("b_scales", scales);
                    qmm->set_attr("b_zero_point", (int64_t)0);
                    qmm->set_attr("transB", (int64_t)1);
                    nodes.push_back(qmm);
                    if (bias) {
                        nodes.push_back(std::make_shared<Node>(base, "Add",
                                                               std::vector<std::string>{qmm_out[0], n.inputs()[2]},
                                                               n.outputs()));
                    }
                    ++consumed[wn];
                    ++st.rewritten;
                    done = true;
                }
            }
        }
        if (!done) nodes.push_back(std::make_shared<Node>(n));
    }
    // initializers, less the float weights whose every use was rewritten
    for (const auto& kv : g.initializers())
        if (!(consumed.count(kv.first) && consumed[kv.first] == uses[kv.first])) out->add_initializer(kv.first, kv.second.clone());
    for (const auto& kv : g.sparse_initializers())
        if (!(consumed.count(kv.first) && consumed[kv.first] == uses[kv.first]))
            out->add_sparse_initializer(kv.first, kv.second);
    for (auto& n : nodes) out->add_node(n);
    if (stats) *stats = st;
    return out;
}

}  // namespace pyflame_rt
