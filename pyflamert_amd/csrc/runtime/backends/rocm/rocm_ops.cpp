// The rocm:: kernels registered in the OperatorRegistry.  Each is an OpFunc
// with the reference's calling convention: borrowed host inputs in, owning
// host outputs out, synchronous.  The arithmetic runs on the GPU through the
// C ABI; shapes, attributes and error texts follow the reference kernels
// (src/backends/cpu/ops/math.cpp:150-226 and :268-438, quantized_ops.cpp:
// 77-167 and :251-278, activation.cpp:45-60, :157-237 and :239-259,
// nn.cpp:419-478; per-tensor Quantize / Dequantize / QuantizeLinear /
// DequantizeLinear, quantized_ops.cpp:35-70 and :284-347).
#include <algorithm>
#include <stdexcept>
#include <string>

#include "pyflame_rt/errors.hpp"
#include "rocm_executor.hpp"

namespace pyflame_rt {
namespace {

RocmExecutor& exec() {
    RocmExecutor* e = RocmExecutor::current();
    if (!e) throw std::runtime_error("rocm kernel called outside RocmExecutor::execute");
    return *e;
}

void need_inputs(const std::vector<const Tensor*>& in, size_t n, const char* op) {
    if (in.size() < n)
        throw std::invalid_argument(std::string(op) + ": expected at least " + std::to_string(n) + " inputs, got " +
                                    std::to_string(in.size()));
}

void need_f32(const Tensor& t, const char* what) {
    if (t.dtype() != DType::Float32)
        throw std::invalid_argument(std::string(what) + " must be float32, got " + dtype_name(t.dtype()));
}

// Device memory for one call's staged host operands.
struct DevScratch {
    pfr_ctx* ctx;
    void* p = nullptr;
    DevScratch(pfr_ctx* c, int64_t bytes) : ctx(c) { pfr_check(pfr_dev_alloc(c, std::max<int64_t>(bytes, 4), &p)); }
    ~DevScratch() {
        if (p) pfr_dev_free(ctx, p);
    }
    DevScratch(const DevScratch&) = delete;
    DevScratch& operator=(const DevScratch&) = delete;
    float* f() const { return static_cast<float*>(p); }
};

// The dense product (a weight above the density gate) on host operands:
// Y[M, N] = alpha * op(A) . B + beta * C with one of A, B the device weight.
void dense_host(pfr_ctx* ctx, const float* A, bool a_dev, int64_t M, int64_t K, int ta, const float* B, bool b_dev,
                int64_t N, float alpha, float beta, const float* C, int64_t c_size, float* Y) {
    DevScratch da(ctx, a_dev ? 0 : M * K * 4), db(ctx, b_dev ? 0 : K * N * 4), dc(ctx, c_size * 4), dy(ctx, M * N * 4);
    if (!a_dev) pfr_check(pfr_copy_to_device(ctx, da.p, A, M * K * 4));
    if (!b_dev) pfr_check(pfr_copy_to_device(ctx, db.p, B, K * N * 4));
    if (C && c_size) pfr_check(pfr_copy_to_device(ctx, dc.p, C, c_size * 4));
    pfr_check(pfr_gemm_dense_dev(ctx, a_dev ? A : da.f(), M, K, ta, b_dev ? B : db.f(), N, N, alpha, beta,
                                 C && c_size ? dc.f() : nullptr, c_size, dy.f(), N, PFR_ACT_NONE));
    pfr_check(pfr_copy_to_host(ctx, Y, dy.p, M * N * 4));
}

// MatMul with one pruned, initializer operand (math.cpp:268-374 semantics).
std::vector<Tensor> rocm_matmul(const std::vector<const Tensor*>& in, const OpContext& ctx) {
    need_inputs(in, 2, "MatMul");
    RocmExecutor& ex = exec();
    const auto* w = ex.weight(ctx.node);
    const Tensor& a = *in[0];
    const Tensor& b = *in[1];
    if (a.ndim() < 2 || b.ndim() < 2) throw std::invalid_argument("MatMul: inputs must have at least 2 dimensions");
    const int64_t Ka = a.shape().back(), Kb = b.shape()[b.ndim() - 2];
    if (Ka != Kb)
        throw std::invalid_argument("MatMul: incompatible dimensions - A has inner dim " + std::to_string(Ka) +
                                    ", B has inner dim " + std::to_string(Kb));
    using DW = RocmExecutor::DeviceWeight;
    if (w && (w->kind == DW::CsrB || w->kind == DW::DenseB)) {
        // A [..., M, K] (broadcast over the batch dims) x W [K, N]: rows flatten.
        need_f32(a, "MatMul input A");
        const int64_t N = b.shape()[1];
        std::vector<int64_t> os(a.shape().begin(), a.shape().end() - 1);
        os.push_back(N);
        Tensor out(os, DType::Float32);
        const int64_t rows = a.num_elements() / Ka;
        if (w->kind == DW::DenseB)
            dense_host(ex.ctx(), a.data_ptr<float>(), false, rows, Ka, 0, w->dense, true, N, 1.0f, 1.0f, nullptr, 0,
                       out.data_ptr<float>());
        else
            pfr_check(pfr_gemm_csr(ex.ctx(), a.data_ptr<float>(), rows, Ka, 0, w->csr, 1.0f, 1.0f, nullptr, 0,
                                   out.data_ptr<float>(), ex.math_mode()));
        return {std::move(out)};
    }
    if (w && (w->kind == DW::CsrA || w->kind == DW::DenseA)) {
        need_f32(b, "MatMul input B");
        if (b.ndim() != 2) throw std::invalid_argument("MatMul: a pruned first operand needs a 2-D second operand");
        const int64_t M = a.shape()[0], N = b.shape()[1];
        Tensor out({M, N}, DType::Float32);
        if (w->kind == DW::DenseA)
            dense_host(ex.ctx(), w->dense, true, M, Ka, 0, b.data_ptr<float>(), false, N, 1.0f, 1.0f, nullptr, 0,
                       out.data_ptr<float>());
        else
            pfr_check(pfr_spmm_csr(ex.ctx(), w->csr, b.data_ptr<float>(), N, out.data_ptr<float>(), ex.math_mode()));
        return {std::move(out)};
    }
    throw std::runtime_error("MatMul: neither operand is a float32 2-D initializer; the rocm backend runs "
                             "pruned-weight products only");
}

// Gemm with a pruned initializer B (math.cpp:377-438 semantics).
std::vector<Tensor> rocm_gemm(const std::vector<const Tensor*>& in, const OpContext& ctx) {
    need_inputs(in, 2, "Gemm");
    RocmExecutor& ex = exec();
    const auto* w = ex.weight(ctx.node);
    const Tensor& A = *in[0];
    const Tensor& B = *in[1];
    const Tensor* C = in.size() > 2 ? in[2] : nullptr;
    if (A.ndim() < 2 || B.ndim() < 2) throw std::invalid_argument("Gemm input A/B must have at least 2 dimensions");
    if (!w || (w->kind != RocmExecutor::DeviceWeight::CsrB && w->kind != RocmExecutor::DeviceWeight::DenseB))
        throw std::runtime_error("Gemm: B is not a float32 2-D initializer; the rocm backend runs pruned-weight "
                                 "products only");
    need_f32(A, "Gemm input A");
    const float alpha = ctx.node->get_attr<float>("alpha", 1.0f);
    const float beta = ctx.node->get_attr<float>("beta", 1.0f);
    const int64_t ta = ctx.node->get_attr<int64_t>("transA", 0);
    const int64_t tb = ctx.node->get_attr<int64_t>("transB", 0);
    const int64_t M = ta ? A.shape()[1] : A.shape()[0];
    const int64_t Ka = ta ? A.shape()[0] : A.shape()[1];
    const int64_t Kb = tb ? B.shape()[1] : B.shape()[0];
    const int64_t N = tb ? B.shape()[0] : B.shape()[1];
    if (Ka != Kb)
        throw std::invalid_argument("Gemm: incompatible dimensions - A has K=" + std::to_string(Ka) +
                                    ", B has K=" + std::to_string(Kb));
    Tensor out({M, N}, DType::Float32);
    const float* c = nullptr;
    int64_t c_size = 0;
    if (C && C->num_elements() > 0) {
        need_f32(*C, "Gemm input C");
        c = C->data_ptr<float>();
        c_size = C->num_elements();
    }
    if (w->kind == RocmExecutor::DeviceWeight::DenseB)
        dense_host(ex.ctx(), A.data_ptr<float>(), false, M, Ka, (int)ta, w->dense, true, N, alpha, beta, c, c_size,
                   out.data_ptr<float>());
    else
        pfr_check(pfr_gemm_csr(ex.ctx(), A.data_ptr<float>(), M, Ka, (int)ta, w->csr, alpha, beta, c, c_size,
                               out.data_ptr<float>(), ex.math_mode()));
    return {std::move(out)};
}

// QuantizedMatMul with a 2:4 int8 initializer A (quantized_ops.cpp:77-167):
// out = (float)acc * (a_scale * b_scale), acc = sum_k A[m, k] (B[k, n] -
// b_zero_point), int32 accumulation.  With two inputs B's bytes are read as
// int8 whatever its type, as the reference kernel reads them
// (quantized_ops.cpp:143-144), and b_scale / b_zero_point are attributes.
// With four inputs (what the dynamic int8 rewrite emits) B's scale and zero
// point are the tensors in[2] and in[3], and a uint8 B is read as uint8
// (quantization::quantized_matmul, quant_ops.cpp:468-490).  A per-channel
// float-vector attribute a_scales replaces a_scale.
std::vector<Tensor> rocm_qmatmul(const std::vector<const Tensor*>& in, const OpContext& ctx) {
    need_inputs(in, 2, "QuantizedMatMul");
    RocmExecutor& ex = exec();
    const auto* w = ex.weight(ctx.node);
    const Tensor& a = *in[0];
    const Tensor& b = *in[1];
    if ((a.dtype() != DType::Int8 && a.dtype() != DType::UInt8))
        throw std::invalid_argument("QuantizedMatMul: input A must be Int8 or UInt8");
    if ((b.dtype() != DType::Int8 && b.dtype() != DType::UInt8))
        throw std::invalid_argument("QuantizedMatMul: input B must be Int8 or UInt8");
    if (a.ndim() < 2 || b.ndim() < 2)
        throw std::invalid_argument("QuantizedMatMul: inputs must have at least 2 dimensions");
    if (w && w->kind == RocmExecutor::DeviceWeight::Sp24B) {
        // the x . W form: the activation is A, the 2:4 weight B (K x N, or
        // N x K with transB = 1), per-column b_scales
        const bool tb = ctx.node->get_attr<int64_t>("transB", 0) != 0;
        const int64_t Kb = tb ? b.shape()[1] : b.shape()[0], N = tb ? b.shape()[0] : b.shape()[1];
        if (a.ndim() != 2)
            throw std::runtime_error("QuantizedMatMul: the rocm backend needs a 2-D activation A with a 2:4 weight B");
        if (a.shape()[1] != Kb)
            throw std::invalid_argument("QuantizedMatMul: inner dimensions must match (got " +
                                        std::to_string(a.shape()[1]) + " and " + std::to_string(Kb) + ")");
        float a_scale = ctx.node->get_attr<float>("a_scale", 1.0f);
        int64_t a_zp = ctx.node->get_attr<int64_t>("a_zero_point", 0);
        pfr_dtype adt = PFR_I8;
        if (in.size() >= 4) {
            const Tensor& s = *in[2];
            const Tensor& z = *in[3];
            if (s.dtype() != DType::Float32 || s.num_elements() != 1)
                throw std::invalid_argument("QuantizedMatMul: a_scale input must be one float32");
            if ((z.dtype() != DType::UInt8 && z.dtype() != DType::Int8) || z.num_elements() != 1)
                throw std::invalid_argument("QuantizedMatMul: a_zero_point input must be one int8 or uint8");
            a_scale = s.data_ptr<float>()[0];
            a_zp = z.dtype() == DType::UInt8 ? (int64_t) static_cast<const uint8_t*>(z.data())[0]
                                             : (int64_t) static_cast<const int8_t*>(z.data())[0];
            adt = a.dtype() == DType::UInt8 ? PFR_U8 : PFR_I8;
        }
        const int64_t T = a.shape()[0];
        Tensor out({T, N}, DType::Float32);
        pfr_check(pfr_sp24_gemm_qt(ex.ctx(), w->sp24, a.data(), adt, T, a_scale, (int32_t)a_zp, out.data_ptr<float>()));
        return {std::move(out)};
    }
    const int64_t K = a.shape().back(), Kb = b.shape()[b.ndim() - 2];
    if (K != Kb)
        throw std::invalid_argument("QuantizedMatMul: inner dimensions must match (got " + std::to_string(K) +
                                    " and " + std::to_string(Kb) + ")");
    if (!w || w->kind != RocmExecutor::DeviceWeight::Sp24A || b.ndim() != 2)
        throw std::runtime_error("QuantizedMatMul: the rocm backend needs a 2-D int8 initializer A that is 2:4 "
                                 "sparse along K, zero points 0, and a 2-D B");
    float b_scale = ctx.node->get_attr<float>("b_scale", 1.0f);
    int64_t b_zp = ctx.node->get_attr<int64_t>("b_zero_point", 0);
    pfr_dtype bdt = PFR_I8;
    if (in.size() >= 4) {
        const Tensor& s = *in[2];
        const Tensor& z = *in[3];
        if (s.dtype() != DType::Float32 || s.num_elements() != 1)
            throw std::invalid_argument("QuantizedMatMul: b_scale input must be one float32");
        if ((z.dtype() != DType::UInt8 && z.dtype() != DType::Int8) || z.num_elements() != 1)
            throw std::invalid_argument("QuantizedMatMul: b_zero_point input must be one int8 or uint8");
        b_scale = s.data_ptr<float>()[0];
        b_zp = z.dtype() == DType::UInt8 ? (int64_t) static_cast<const uint8_t*>(z.data())[0]
                                         : (int64_t) static_cast<const int8_t*>(z.data())[0];
        bdt = b.dtype() == DType::UInt8 ? PFR_U8 : PFR_I8;
    }
    const int64_t M = a.shape()[0], N = b.shape()[1];
    Tensor out({M, N}, DType::Float32);
    pfr_check(pfr_sp24_gemm_q(ex.ctx(), w->sp24, b.data(), bdt, N, b_scale, (int32_t)b_zp, PFR_SP24_OUT_F32, 1.0f, 0,
                              out.data()));
    return {std::move(out)};
}

// DynamicQuantizeLinear (quantized_ops.cpp:251-278): uint8 tensor, scale
// [1] float32, zero point [1] uint8.
std::vector<Tensor> rocm_dynamic_quantize_linear(const std::vector<const Tensor*>& in, const OpContext&) {
    need_inputs(in, 1, "DynamicQuantizeLinear");
    const Tensor& x = *in[0];
    if (x.dtype() != DType::Float32) throw std::invalid_argument("DynamicQuantizeLinear: input must be Float32");
    Tensor y(x.shape(), DType::UInt8), s({1}, DType::Float32), z({1}, DType::UInt8);
    pfr_check(pfr_dynamic_quantize_linear(exec().ctx(), x.data_ptr<float>(), x.num_elements(),
                                          static_cast<uint8_t*>(y.data()), s.data_ptr<float>(),
                                          static_cast<uint8_t*>(z.data())));
    return {std::move(y), std::move(s), std::move(z)};
}

std::vector<Tensor> rocm_relu(const std::vector<const Tensor*>& in, const OpContext&) {
    need_inputs(in, 1, "Relu");
    const Tensor& x = *in[0];
    need_f32(x, "Relu input");
    Tensor out(x.shape(), x.dtype());
    pfr_check(pfr_relu(exec().ctx(), x.data_ptr<float>(), x.num_elements(), out.data_ptr<float>()));
    return {std::move(out)};
}

std::vector<Tensor> rocm_softmax(const std::vector<const Tensor*>& in, const OpContext& ctx) {
    need_inputs(in, 1, "Softmax");
    const Tensor& x = *in[0];
    need_f32(x, "Softmax input");
    int64_t axis = ctx.node->get_attr<int64_t>("axis", -1);
    const int64_t nd = (int64_t)x.ndim();
    if (axis < -nd || axis >= nd)
        throw std::invalid_argument("Softmax: axis " + std::to_string(axis) + " out of range for " +
                                    std::to_string(nd) + "-D input");
    if (axis < 0) axis += nd;
    int64_t outer = 1, inner = 1;
    for (int64_t i = 0; i < axis; ++i) outer *= x.shape()[i];
    for (int64_t i = axis + 1; i < nd; ++i) inner *= x.shape()[i];
    Tensor out(x.shape(), x.dtype());
    pfr_check(pfr_softmax(exec().ctx(), x.data_ptr<float>(), outer, x.shape()[axis], inner, out.data_ptr<float>()));
    return {std::move(out)};
}

// Gelu (activation.cpp:239-259).
std::vector<Tensor> rocm_gelu(const std::vector<const Tensor*>& in, const OpContext&) {
    need_inputs(in, 1, "Gelu");
    const Tensor& x = *in[0];
    need_f32(x, "Gelu input");
    Tensor out(x.shape(), x.dtype());
    pfr_check(pfr_gelu(exec().ctx(), x.data_ptr<float>(), x.num_elements(), out.data_ptr<float>()));
    return {std::move(out)};
}

// Add with broadcasting (math.cpp:150-226).
std::vector<Tensor> rocm_add(const std::vector<const Tensor*>& in, const OpContext&) {
    need_inputs(in, 2, "Add");
    const Tensor& a = *in[0];
    const Tensor& b = *in[1];
    need_f32(a, "Add input A");
    need_f32(b, "Add input B");
    Tensor out(broadcast_shapes(a.shape(), b.shape(), "Add"), DType::Float32);
    pfr_check(pfr_add(exec().ctx(), a.data_ptr<float>(), a.shape().data(), (int)a.ndim(), b.data_ptr<float>(),
                      b.shape().data(), (int)b.ndim(), out.data_ptr<float>()));
    return {std::move(out)};
}

// LayerNormalization (nn.cpp:419-478).
std::vector<Tensor> rocm_layernorm(const std::vector<const Tensor*>& in, const OpContext& ctx) {
    need_inputs(in, 3, "LayerNormalization");
    const Tensor& x = *in[0];
    const Tensor& scale = *in[1];
    const Tensor& bias = *in[2];
    need_f32(x, "LayerNormalization input");
    need_f32(scale, "LayerNormalization scale");
    need_f32(bias, "LayerNormalization bias");
    const LayerNormExtent e = layernorm_extent(x.shape(), scale.num_elements(), bias.num_elements(), ctx.node);
    Tensor out(x.shape(), x.dtype());
    pfr_check(pfr_layernorm(exec().ctx(), x.data_ptr<float>(), e.outer, e.norm, scale.data_ptr<float>(),
                            bias.data_ptr<float>(), e.epsilon, out.data_ptr<float>()));
    return {std::move(out)};
}

// Per-tensor quantize and dequantize (quantized_ops.cpp:35-70, :284-347):
// the parameters from attributes (Quantize, Dequantize) or from the first
// element of the scale and zero-point inputs (QuantizeLinear,
// DequantizeLinear; a zero point that is not int8 or uint8 counts as 0, as
// there).  The scale input must be float32 here (the reference reads its
// bytes as a float whatever its type).
float scale_input(const Tensor& s, const char* op) {
    if (s.dtype() != DType::Float32 || s.num_elements() < 1)
        throw std::invalid_argument(std::string(op) + ": scale must be a float32 tensor");
    return s.data_ptr<float>()[0];
}

int32_t zero_point_input(const std::vector<const Tensor*>& in) {
    if (in.size() < 3 || in[2] == nullptr || in[2]->num_elements() < 1) return 0;
    if (in[2]->dtype() == DType::Int8) return static_cast<const int8_t*>(in[2]->data())[0];
    if (in[2]->dtype() == DType::UInt8) return static_cast<const uint8_t*>(in[2]->data())[0];
    return 0;
}

Tensor quantize_call(const Tensor& x, float scale, int32_t zp, DType out) {
    // QuantParams::per_tensor validates first, then quantize_tensor the input
    pfr_check(pfr_quantize_linear(exec().ctx(), nullptr, 0, scale, zp, out == DType::UInt8 ? PFR_U8 : PFR_I8, nullptr));
    if (x.dtype() != DType::Float32)
        throw std::invalid_argument("quantize_tensor: input must be Float32, got " + dtype_name(x.dtype()));
    Tensor y(x.shape(), out);
    pfr_check(pfr_quantize_linear(exec().ctx(), x.data_ptr<float>(), x.num_elements(), scale, zp,
                                  out == DType::UInt8 ? PFR_U8 : PFR_I8, y.data()));
    return y;
}

Tensor dequantize_call(const Tensor& x, float scale, int32_t zp) {
    const pfr_dtype dt = x.dtype() == DType::Int8 ? PFR_I8 : (x.dtype() == DType::UInt8 ? PFR_U8 : PFR_F32);
    Tensor y(x.shape(), DType::Float32);
    pfr_check(pfr_dequantize_linear(exec().ctx(), x.data(), dt, x.num_elements(), scale, zp, y.data_ptr<float>()));
    return y;
}

DType quant_dtype_attr(const OpContext& ctx, const char* key) {
    return ctx.node->get_attr<std::string>(key, "int8") == "uint8" ? DType::UInt8 : DType::Int8;
}

std::vector<Tensor> rocm_quantize(const std::vector<const Tensor*>& in, const OpContext& ctx) {
    need_inputs(in, 1, "Quantize");
    const float scale = ctx.node->get_attr<float>("scale", 1.0f);
    const int32_t zp = (int32_t)ctx.node->get_attr<int64_t>("zero_point", 0);
    return {quantize_call(*in[0], scale, zp, quant_dtype_attr(ctx, "dtype"))};
}

std::vector<Tensor> rocm_dequantize(const std::vector<const Tensor*>& in, const OpContext& ctx) {
    need_inputs(in, 1, "Dequantize");
    const float scale = ctx.node->get_attr<float>("scale", 1.0f);
    const int32_t zp = (int32_t)ctx.node->get_attr<int64_t>("zero_point", 0);
    return {dequantize_call(*in[0], scale, zp)};
}

std::vector<Tensor> rocm_quantize_linear(const std::vector<const Tensor*>& in, const OpContext& ctx) {
    need_inputs(in, 2, "QuantizeLinear");
    return {quantize_call(*in[0], scale_input(*in[1], "QuantizeLinear"), zero_point_input(in),
                          quant_dtype_attr(ctx, "output_dtype"))};
}

std::vector<Tensor> rocm_dequantize_linear(const std::vector<const Tensor*>& in, const OpContext&) {
    need_inputs(in, 2, "DequantizeLinear");
    return {dequantize_call(*in[0], scale_input(*in[1], "DequantizeLinear"), zero_point_input(in))};
}

struct RocmOpsRegistrar {
    RocmOpsRegistrar() {
        auto& r = OperatorRegistry::instance();
        r.register_op("rocm::MatMul", rocm_matmul);
        r.register_op("rocm::Gemm", rocm_gemm);
        r.register_op("rocm::QuantizedMatMul", rocm_qmatmul);
        r.register_op("rocm::DynamicQuantizeLinear", rocm_dynamic_quantize_linear);
        r.register_op("rocm::Relu", rocm_relu);
        r.register_op("rocm::Softmax", rocm_softmax);
        r.register_op("rocm::Gelu", rocm_gelu);
        r.register_op("rocm::Add", rocm_add);
        r.register_op("rocm::LayerNormalization", rocm_layernorm);
        r.register_op("rocm::Quantize", rocm_quantize);
        r.register_op("rocm::Dequantize", rocm_dequantize);
        r.register_op("rocm::QuantizeLinear", rocm_quantize_linear);
        r.register_op("rocm::DequantizeLinear", rocm_dequantize_linear);
    }
};
RocmOpsRegistrar registrar;

}  // namespace
}  // namespace pyflame_rt
