// Dynamic int8 quantization of a graph's 2:4-pruned products, the rewrite the
// reference's Quantizer intends (src/quantization/quantizer.cpp:28-34 maps
// MatMul to QuantizedMatMul; :342-371 renames the node and attaches
// scales[0] only) made to run: weights per output channel, activations per
// tensor at run time.
#pragma once

#include <memory>

#include "pyflame_rt/graph.hpp"

namespace pyflame_rt {

struct QuantizeStats {
    int rewritten = 0;        // MatMul nodes turned into DynamicQuantizeLinear + QuantizedMatMul
    int64_t float_bytes = 0;  // their float32 weights
    int64_t int8_bytes = 0;   // the int8 weights and scales that replace them
};

// Every MatMul(W, X) whose W is a float32 2-D initializer (dense, or a CSR
// record) with at most two nonzeros in each group of four consecutive
// columns, and whose X is not an initializer, becomes
//   DynamicQuantizeLinear(X) -> (X_q uint8, X_scale, X_zero_point)
//   QuantizedMatMul(W_q, X_q, X_scale, X_zero_point)   a_scales = per-row scales
// with W_q the symmetric per-row int8 quantization of W
// (compute_dynamic_params_per_channel, quant_ops.cpp:321-381, with
// QuantParams::compute_per_channel, quant_params.cpp:57-106, then
// quantize_tensor's per-channel branch, quant_ops.cpp:56-124), stored as a
// 2:4 record when its width is a multiple of 4.
//
// The x . W form -- MatMul(X, W) with W K x N, and Gemm(X, W[, b]) with
// transA 0, alpha 1, beta 1 and a bias of N floats (W N x K when transB) --
// whose W is 2:4 along K becomes
//   DynamicQuantizeLinear(X) -> (X_q, X_scale, X_zero_point)
//   QuantizedMatMul(X_q, W_q^T, X_scale, X_zero_point)  transB = 1,
//                                           b_scales = per-output-column
//   Add(product, b)                         (Gemm with a bias)
// with W_q^T (N x K) the per-column quantization of W.  Other nodes are
// copied.
std::unique_ptr<Graph> quantize_dynamic_int8(const Graph& g, QuantizeStats* stats = nullptr);

}  // namespace pyflame_rt
