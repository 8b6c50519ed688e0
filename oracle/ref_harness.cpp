// ref_harness.cpp -- extern "C" shims over the REFERENCE's own kernel
// functions, compiled together with the reference sources (oracle/Makefile,
// target ref) into oracle/_ref/libpfr_ref.so.
//
// TEST INFRASTRUCTURE ONLY.  It is used to write golden vectors
// (tests/golden/make_golden.py) and, where present, as the CPU baseline of
// bench.py.  Only this file is ours; the reference sources are compiled where
// they lie and never copied.
#include "pyflame_rt/graph.hpp"
#include "pyflame_rt/node.hpp"
#include "pyflame_rt/registry.hpp"
#include "pyflame_rt/tensor.hpp"
#include "pyflame_rt/pruning/pruning.hpp"
#include "pyflame_rt/pruning/sparse_tensor.hpp"
#include "pyflame_rt/quantization/half_types.hpp"
#include "pyflame_rt/quantization/quant_ops.hpp"
#include "pyflame_rt/quantization/quant_params.hpp"
#include "backends/cpu/executor.hpp"
#include "io/pyflame_format.hpp"

#include <chrono>
#include <cstring>
#include <exception>
#include <memory>
#include <string>

using namespace pyflame_rt;
namespace q = pyflame_rt::quantization;
namespace pr = pyflame_rt::pruning;

namespace {
thread_local std::string g_err;

Tensor make_f32(const float* p, std::vector<int64_t> shape) {
    Tensor t(shape, DType::Float32);
    if (t.size_bytes()) std::memcpy(t.data(), p, t.size_bytes());
    return t;
}

Tensor make_raw(const void* p, std::vector<int64_t> shape, DType dt) {
    Tensor t(shape, dt);
    if (t.size_bytes()) std::memcpy(t.data(), p, t.size_bytes());
    return t;
}

template <class F>
int guard(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}
}  // namespace

extern "C" {

const char* ref_last_error() { return g_err.c_str(); }

// Run a registered CPU op (MatMul / Gemm / Relu / Softmax / QuantizedMatMul)
// on explicit inputs.  Attributes come as parallel arrays (float then int).
int ref_run_op(const char* op_type, int n_in, const void* const* in_data,
               const int* in_dtype, const int64_t* const* in_shape,
               const int* in_ndim, int n_fattr, const char* const* fattr_names,
               const float* fattr_vals, int n_iattr,
               const char* const* iattr_names, const int64_t* iattr_vals,
               void* out, int64_t out_bytes, int64_t* out_shape,
               int* out_ndim) {
    return guard([&] {
        std::vector<Tensor> ins;
        std::vector<std::string> in_names;
        for (int i = 0; i < n_in; ++i) {
            std::vector<int64_t> sh(in_shape[i], in_shape[i] + in_ndim[i]);
            ins.push_back(make_raw(in_data[i], sh, static_cast<DType>(in_dtype[i])));
            in_names.push_back("in" + std::to_string(i));
        }
        Node node("n0", op_type, in_names, {"out"});
        for (int i = 0; i < n_fattr; ++i) node.set_attr(fattr_names[i], fattr_vals[i]);
        for (int i = 0; i < n_iattr; ++i) node.set_attr(iattr_names[i], iattr_vals[i]);
        const OpFunc* fn = OperatorRegistry::instance().get(op_type);
        if (!fn) throw std::runtime_error("op not registered");
        std::vector<const Tensor*> ptrs;
        for (auto& t : ins) ptrs.push_back(&t);
        OpContext ctx{&node, false};
        auto res = (*fn)(ptrs, ctx);
        const Tensor& r = res.at(0);
        if ((int64_t)r.size_bytes() > out_bytes) throw std::runtime_error("output buffer too small");
        if (r.size_bytes()) std::memcpy(out, r.data(), r.size_bytes());
        *out_ndim = (int)r.ndim();
        for (size_t d = 0; d < r.ndim(); ++d) out_shape[d] = r.shape()[d];
    });
}

// to_sparse(dense, threshold, CSR) then sparse_matmul / sparse_matvec.
// Pass indptr == nullptr to query nnz into *nnz_out only.
int ref_to_sparse_csr(const float* dense, int64_t rows, int64_t cols,
                      float threshold, int64_t* indptr, int64_t* indices,
                      float* values, int64_t* nnz_out) {
    return guard([&] {
        Tensor d = make_f32(dense, {rows, cols});
        pr::SparseTensor s = pr::to_sparse(d, threshold, pr::SparseFormat::CSR);
        *nnz_out = (int64_t)s.nnz();
        if (!indptr) return;
        std::memcpy(indptr, s.indptr().data(), sizeof(int64_t) * s.indptr().size());
        std::memcpy(indices, s.indices().data(), sizeof(int64_t) * s.indices().size());
        std::memcpy(values, s.values().data(), sizeof(float) * s.values().size());
    });
}

int ref_sparse_matmul(int64_t m, int64_t k, int64_t n, const int64_t* indptr,
                      const int64_t* indices, const float* values, int64_t nnz,
                      const float* b, int b_is_1d, float* out) {
    return guard([&] {
        std::vector<int64_t> ip(indptr, indptr + m + 1), ix(indices, indices + nnz);
        std::vector<float> vv(values, values + nnz);
        pr::SparseTensor s = pr::SparseTensor::from_csr({m, k}, ip, ix, vv);
        Tensor bt = b_is_1d ? make_f32(b, {k}) : make_f32(b, {k, n});
        Tensor r = pr::sparse_matmul(s, bt);
        std::memcpy(out, r.data(), r.size_bytes());
    });
}

// Wall time of the reference's sparse_matmul on a prebuilt SparseTensor and
// input Tensor: one warm-up call, then `reps` timed calls (ns each).  The last
// result goes to out.  Single thread, as the reference runs.
int ref_time_sparse_matmul(int64_t m, int64_t k, int64_t n, const int64_t* indptr,
                           const int64_t* indices, const float* values, int64_t nnz,
                           const float* b, int reps, int64_t* ns, float* out) {
    return guard([&] {
        std::vector<int64_t> ip(indptr, indptr + m + 1), ix(indices, indices + nnz);
        std::vector<float> vv(values, values + nnz);
        pr::SparseTensor s = pr::SparseTensor::from_csr({m, k}, ip, ix, vv);
        Tensor bt = make_f32(b, {k, n});
        Tensor r = pr::sparse_matmul(s, bt);
        for (int i = 0; i < reps; ++i) {
            auto t0 = std::chrono::steady_clock::now();
            r = pr::sparse_matmul(s, bt);
            auto t1 = std::chrono::steady_clock::now();
            ns[i] = std::chrono::duration_cast<std::chrono::nanoseconds>(t1 - t0).count();
        }
        std::memcpy(out, r.data(), r.size_bytes());
    });
}

// The same for the reference's sparse_matvec (x of k floats).
int ref_time_sparse_matvec(int64_t m, int64_t k, const int64_t* indptr, const int64_t* indices,
                           const float* values, int64_t nnz, const float* x, int reps, int64_t* ns,
                           float* out) {
    return guard([&] {
        std::vector<int64_t> ip(indptr, indptr + m + 1), ix(indices, indices + nnz);
        std::vector<float> vv(values, values + nnz);
        pr::SparseTensor s = pr::SparseTensor::from_csr({m, k}, ip, ix, vv);
        Tensor xt = make_f32(x, {k});
        Tensor r = pr::sparse_matvec(s, xt);
        for (int i = 0; i < reps; ++i) {
            auto t0 = std::chrono::steady_clock::now();
            r = pr::sparse_matvec(s, xt);
            auto t1 = std::chrono::steady_clock::now();
            ns[i] = std::chrono::duration_cast<std::chrono::nanoseconds>(t1 - t0).count();
        }
        std::memcpy(out, r.data(), r.size_bytes());
    });
}

int ref_sparse_matvec(int64_t m, int64_t k, const int64_t* indptr,
                      const int64_t* indices, const float* values, int64_t nnz,
                      const float* x, float* out) {
    return guard([&] {
        std::vector<int64_t> ip(indptr, indptr + m + 1), ix(indices, indices + nnz);
        std::vector<float> vv(values, values + nnz);
        pr::SparseTensor s = pr::SparseTensor::from_csr({m, k}, ip, ix, vv);
        Tensor r = pr::sparse_matvec(s, make_f32(x, {k}));
        std::memcpy(out, r.data(), r.size_bytes());
    });
}

int ref_apply_mask(const float* t, const float* mask, int64_t n, float* out) {
    return guard([&] {
        Tensor r = pr::apply_mask(make_f32(t, {n}), make_f32(mask, {n}));
        std::memcpy(out, r.data(), r.size_bytes());
    });
}

int ref_magnitude_mask(const float* w, int64_t rows, int64_t cols,
                       float sparsity, float* mask) {
    return guard([&] {
        pr::MagnitudePruning p;
        auto m = p.compute_mask("w", make_f32(w, {rows, cols}), sparsity);
        std::memcpy(mask, m.mask.data(), m.mask.size_bytes());
    });
}

int ref_nm_mask(const float* w, int64_t total, int64_t n, int64_t m,
                float* mask) {
    return guard([&] {
        pr::NMSparsityPruning p((size_t)n, (size_t)m);
        auto r = p.compute_mask("w", make_f32(w, {total}), 0.5f);
        std::memcpy(mask, r.mask.data(), r.mask.size_bytes());
    });
}

int ref_params_from_minmax(float mn, float mx, int qdtype, int symmetric,
                           float* scale, int32_t* zp) {
    return guard([&] {
        auto p = q::QuantParams::compute_from_minmax(mn, mx, static_cast<DType>(qdtype), symmetric != 0);
        *scale = p.scales[0];
        *zp = p.zero_points[0];
    });
}

int ref_dynamic_params(const float* x, int64_t count, int qdtype,
                       int symmetric, float* scale, int32_t* zp) {
    return guard([&] {
        Tensor t = count ? make_f32(x, {count}) : Tensor(std::vector<int64_t>{0}, DType::Float32);
        auto p = q::compute_dynamic_params(t, static_cast<DType>(qdtype), symmetric != 0);
        *scale = p.scales[0];
        *zp = p.zero_points[0];
    });
}

int ref_dynamic_params_per_channel(const float* x, int64_t outer,
                                   int64_t channels, int64_t inner,
                                   int qdtype, int symmetric, float* scales,
                                   int32_t* zps) {
    return guard([&] {
        auto p = q::compute_dynamic_params_per_channel(
            make_f32(x, {outer, channels, inner}), 1, static_cast<DType>(qdtype), symmetric != 0);
        std::memcpy(scales, p.scales.data(), sizeof(float) * p.scales.size());
        std::memcpy(zps, p.zero_points.data(), sizeof(int32_t) * p.zero_points.size());
    });
}

int ref_quantize(const float* x, int64_t outer, int64_t channels,
                 int64_t inner, const float* scales, const int32_t* zps,
                 int qdtype, void* out) {
    return guard([&] {
        DType dt = static_cast<DType>(qdtype);
        q::QuantParams p;
        Tensor t;
        if (channels == 0) {
            p = q::QuantParams::per_tensor(scales[0], zps[0], dt);
            t = make_f32(x, {outer * inner});
        } else {
            p = q::QuantParams::per_channel(std::vector<float>(scales, scales + channels),
                                            std::vector<int32_t>(zps, zps + channels), 1, dt);
            t = make_f32(x, {outer, channels, inner});
        }
        Tensor r = q::quantize_tensor(t, p);
        std::memcpy(out, r.data(), r.size_bytes());
    });
}

int ref_dequantize(const void* qd, int qdtype, int64_t outer, int64_t channels,
                   int64_t inner, const float* scales, const int32_t* zps,
                   float* out) {
    return guard([&] {
        DType dt = static_cast<DType>(qdtype);
        q::QuantParams p;
        Tensor t;
        if (channels == 0) {
            p = q::QuantParams::per_tensor(scales[0], zps[0], dt);
            t = make_raw(qd, {outer * inner}, dt);
        } else {
            p = q::QuantParams::per_channel(std::vector<float>(scales, scales + channels),
                                            std::vector<int32_t>(zps, zps + channels), 1, dt);
            t = make_raw(qd, {outer, channels, inner}, dt);
        }
        Tensor r = q::dequantize_tensor(t, p);
        std::memcpy(out, r.data(), r.size_bytes());
    });
}

// quantization::quantized_matmul, optionally requantized with per-tensor
// output params (out is int8/uint8 then, float otherwise).
int ref_quantized_matmul(const void* a, int a_dtype, const void* b,
                         int b_dtype, int64_t M, int64_t K, int64_t N,
                         float a_scale, int32_t a_zp, float b_scale,
                         int32_t b_zp, int requant, float out_scale,
                         int32_t out_zp, int out_dtype, void* out) {
    return guard([&] {
        DType adt = static_cast<DType>(a_dtype), bdt = static_cast<DType>(b_dtype);
        auto ap = q::QuantParams::per_tensor(a_scale, a_zp, adt);
        auto bp = q::QuantParams::per_tensor(b_scale, b_zp, bdt);
        Tensor at = make_raw(a, {M, K}, adt), bt = make_raw(b, {K, N}, bdt);
        Tensor r;
        if (requant) {
            auto op = q::QuantParams::per_tensor(out_scale, out_zp, static_cast<DType>(out_dtype));
            r = q::quantized_matmul(at, ap, bt, bp, &op);
        } else {
            r = q::quantized_matmul(at, ap, bt, bp, nullptr);
        }
        std::memcpy(out, r.data(), r.size_bytes());
    });
}

uint16_t ref_bf16_from_float(float v) { return q::BFloat16::from_float(v).bits; }

// Bulk conversion through float_to_bf16 (half_types.cpp:196-200); values go
// by pointer so signalling NaN payloads reach the reference untouched.
void ref_f32_to_bf16(const float* in, uint16_t* out, int64_t n) {
    std::vector<q::BFloat16> tmp((size_t)n);
    q::float_to_bf16(in, tmp.data(), (size_t)n);
    for (int64_t i = 0; i < n; ++i) out[i] = tmp[(size_t)i].bits;
}
float ref_bf16_to_float(uint16_t b) { return q::BFloat16(b).to_float(); }

// Build Gemm(x,W1,b1)->Relu->Gemm(.,W2,b2)->Softmax(axis=-1) with the
// reference Graph and save it with the reference .pfm writer.
int ref_save_mlp_pfm(const char* path, int64_t batch, int64_t d_in,
                     int64_t d_hid, int64_t d_out, const float* w1,
                     const float* b1, const float* w2, const float* b2) {
    return guard([&] {
        Graph g("mlp");
        g.add_input(TensorInfo("x", {batch, d_in}, DType::Float32));
        g.add_output(TensorInfo("y", {batch, d_out}, DType::Float32));
        g.add_initializer("fc1.weight", make_f32(w1, {d_in, d_hid}));
        g.add_initializer("fc1.bias", make_f32(b1, {d_hid}));
        g.add_initializer("fc2.weight", make_f32(w2, {d_hid, d_out}));
        g.add_initializer("fc2.bias", make_f32(b2, {d_out}));
        auto n1 = std::make_shared<Node>("gemm1", "Gemm",
            std::vector<std::string>{"x", "fc1.weight", "fc1.bias"}, std::vector<std::string>{"h1"});
        n1->set_attr("alpha", 1.0f);
        n1->set_attr("beta", 1.0f);
        n1->set_attr("transA", int64_t(0));
        n1->set_attr("transB", int64_t(0));
        auto n2 = std::make_shared<Node>("relu1", "Relu",
            std::vector<std::string>{"h1"}, std::vector<std::string>{"a1"});
        auto n3 = std::make_shared<Node>("gemm2", "Gemm",
            std::vector<std::string>{"a1", "fc2.weight", "fc2.bias"}, std::vector<std::string>{"z2"});
        auto n4 = std::make_shared<Node>("softmax", "Softmax",
            std::vector<std::string>{"z2"}, std::vector<std::string>{"y"});
        n4->set_attr("axis", int64_t(-1));
        g.add_node(n1);
        g.add_node(n2);
        g.add_node(n3);
        g.add_node(n4);
        PyFlameFormat::save(g, path);
    });
}

// Load a .pfm with the reference loader and run it with CPUExecutor.
// Returns the element count of the first graph output in *n_out.
int ref_run_pfm(const char* path, const char* input_name, const float* x,
                const int64_t* shape, int ndim, float* out, int64_t cap,
                int64_t* n_out) {
    return guard([&] {
        auto g = PyFlameFormat::load(path);
        std::unordered_map<std::string, Tensor> feed;
        feed[input_name] = make_f32(x, std::vector<int64_t>(shape, shape + ndim));
        CPUExecutor ex;
        auto outs = ex.execute(*g, feed);
        const Tensor& r = outs.at(0);
        *n_out = r.num_elements();
        if (r.num_elements() > cap) throw std::runtime_error("output buffer too small");
        std::memcpy(out, r.data(), r.size_bytes());
    });
}

// Load a .pfm with the reference loader once, then time `reps` calls of
// CPUExecutor::execute on it (each call's wall time in ns into times_ns):
// what a session's run() costs once its graph is loaded.
int ref_time_pfm(const char* path, const char* input_name, const float* x, const int64_t* shape, int ndim,
                 int reps, int64_t* times_ns) {
    return guard([&] {
        auto g = PyFlameFormat::load(path);
        std::unordered_map<std::string, Tensor> feed;
        feed[input_name] = make_f32(x, std::vector<int64_t>(shape, shape + ndim));
        CPUExecutor ex;
        for (int i = 0; i < reps; ++i) {
            const auto t0 = std::chrono::steady_clock::now();
            auto outs = ex.execute(*g, feed);
            const auto t1 = std::chrono::steady_clock::now();
            times_ns[i] = std::chrono::duration_cast<std::chrono::nanoseconds>(t1 - t0).count();
        }
    });
}

}  // extern "C"
