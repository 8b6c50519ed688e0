/*
 * pfr_oracle.h -- CPU restatement of PyFlameRT's pruned-weight MatMul/Gemm
 * path, used ONLY as the test checker and as the CPU baseline in bench.py.
 *
 * TEST INFRASTRUCTURE: nothing in the product (pyflamert_amd/) links, loads
 * or calls this library.  The product path runs on the GPU or fails.
 *
 * Every function restates one reference function line-for-line in its
 * numerics (loop order, rounding points, casts); the reference file:line is
 * given on each declaration.  Compiled with -std=c11 -O3 -ffp-contract=off
 * and no -march, like the reference's Release build (GCC, ISO mode, x86-64
 * baseline: SSE arithmetic, no FMA).
 *
 * Parity pinning (details in tests/test_oracle_*.py):
 *   - golden vectors written by the compiled reference (tests/golden/);
 *   - the reference's own known-answer test (test_executor.cpp:162-208);
 *   - closed forms and brute force on tiny inputs.
 * No function here is left "parity unpinned".
 */
#ifndef PFR_ORACLE_H
#define PFR_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* DType codes, same values as the reference's enum (types.hpp:48-59). */
enum { ORC_F32 = 0, ORC_BF16 = 2, ORC_I32 = 5, ORC_I8 = 7, ORC_U8 = 8 };

/* ---- dense fp32 (src/backends/cpu/ops/math.cpp) ------------------------- */

/* cpu_matmul, math.cpp:268-374.  a: [batch_a, M, K], b: [batch_b, K, N];
 * batch_a and batch_b are equal or one of them is 1 (broadcast, :339-371).
 * out: [max(batch_a, batch_b), M, N].  Returns 0, or -1 on bad batch. */
int orc_matmul_f32(const float* a, const float* b, float* out,
                   int64_t batch_a, int64_t batch_b,
                   int64_t M, int64_t K, int64_t N);

/* cpu_gemm, math.cpp:377-438.  A is [M,K] (transA=0) or [K,M]; B is [K,N]
 * (transB=0) or [N,K].  c may be NULL (no bias) or hold c_size elements,
 * added as beta*c[i % c_size] over the flat output (:427-435). */
void orc_gemm_f32(const float* A, const float* B, const float* c,
                  int64_t c_size, float* out, int64_t M, int64_t K, int64_t N,
                  float alpha, float beta, int transA, int transB);

/* ---- CSR (src/pruning/sparse_tensor.cpp) -------------------------------- */

/* sparse_matmul CSR branch, sparse_tensor.cpp:473-519: out [m, n]. */
void orc_csr_spmm_f32(int64_t m, int64_t k, int64_t n, const int64_t* indptr,
                      const int64_t* indices, const float* values,
                      const float* b, float* out);

/* sparse_matvec CSR branch, sparse_tensor.cpp:521-554: out [m]. */
void orc_csr_spmv_f32(int64_t m, int64_t k, const int64_t* indptr,
                      const int64_t* indices, const float* values,
                      const float* x, float* out);

/* to_sparse(dense, threshold, CSR), sparse_tensor.cpp:560-610.
 * Call with indices == NULL to get nnz only.  Keeps |v| > threshold. */
int64_t orc_to_sparse_csr(const float* dense, int64_t rows, int64_t cols,
                          float threshold, int64_t* indptr, int64_t* indices,
                          float* values);

/* apply_mask, sparse_tensor.cpp:616-631. */
void orc_apply_mask(const float* t, const float* mask, int64_t n, float* out);

/* ---- mask producers (src/pruning/) -------------------------------------- */

/* MagnitudePruning::compute_mask, magnitude_pruning.cpp:22-102. */
int orc_magnitude_mask(const float* w, int64_t n, float sparsity, float* mask);

/* NMSparsityPruning::compute_mask, nm_sparsity.cpp:45-120, with the group
 * selection done by a restatement of libstdc++ (GCC 11.4) std::partial_sort
 * so that ties resolve identically. */
int orc_nm_mask(const float* w, int64_t total, int64_t n, int64_t m,
                float* mask);

/* ---- quantization (src/quantization/) ----------------------------------- */

/* QuantParams::compute_from_minmax, quant_params.cpp:14-55. */
int orc_params_from_minmax(float min_val, float max_val, int qdtype,
                           int symmetric, float* scale, int32_t* zp);

/* compute_dynamic_params, quant_ops.cpp:288-322. */
int orc_dynamic_params(const float* x, int64_t count, int qdtype,
                       int symmetric, float* scale, int32_t* zp);

/* compute_dynamic_params_per_channel, quant_ops.cpp:324-381, which calls
 * QuantParams::compute_per_channel, quant_params.cpp:57-106. */
int orc_dynamic_params_per_channel(const float* x, int64_t outer,
                                   int64_t channels, int64_t inner,
                                   int qdtype, int symmetric, float* scales,
                                   int32_t* zps);

/* quantize_tensor, quant_ops.cpp:15-127.  Per-tensor when channels == 0
 * (scales[0], zps[0]); per-channel over [outer, channels, inner] otherwise.
 * out is int8 or uint8 by qdtype.  Returns -1 on an invalid scale. */
int orc_quantize(const float* x, int64_t outer, int64_t channels,
                 int64_t inner, const float* scales, const int32_t* zps,
                 int qdtype, void* out);

/* dequantize_tensor, quant_ops.cpp:129-214 (same layout convention). */
int orc_dequantize(const void* q, int qdtype, int64_t outer, int64_t channels,
                   int64_t inner, const float* scales, const int32_t* zps,
                   float* out);

/* quantization::quantized_matmul, quant_ops.cpp:387-506 (int64 accumulator,
 * per-tensor scales[0], float output).  a: [batch, M, K], b: [batch, K, N]. */
int orc_quantized_matmul(const void* a, int a_dtype, const void* b,
                         int b_dtype, int64_t batch, int64_t M, int64_t K,
                         int64_t N, float a_scale, float b_scale, int32_t a_zp,
                         int32_t b_zp, float* out);

/* The per-output-channel generalisation of quant_ops.cpp:435 used for
 * per-channel weights: out[i,j] = (float)acc * (a_scales[i] * b_scale).
 * With all a_scales equal it is orc_quantized_matmul (tested). */
void orc_quantized_matmul_rowscale(const int8_t* a, const int8_t* b,
                                   int64_t M, int64_t K, int64_t N,
                                   const float* a_scales, float b_scale,
                                   float* out);

/* Exact int32 accumulators of the int8 product (no scaling), i-k-j. */
void orc_int8_matmul_acc(const int8_t* a, const int8_t* b, int64_t M,
                         int64_t K, int64_t N, int32_t* acc);

/* cpu_quantized_matmul, quantized_ops.cpp:77-167 (int32 accumulator; UInt8
 * data is read as int8, :143-144). */
void orc_cpu_quantized_matmul(const int8_t* a, const int8_t* b, int64_t batch,
                              int64_t M, int64_t K, int64_t N, float a_scale,
                              float b_scale, int64_t a_zp, int64_t b_zp,
                              float* out);

/* ---- bf16 (src/quantization/half_types.cpp) ----------------------------- */

uint16_t orc_bf16_from_float(float v);  /* half_types.cpp:132-174 */
float orc_bf16_to_float(uint16_t b);    /* half_types.cpp:176-181 */
void orc_f32_to_bf16(const float* in, uint16_t* out, int64_t n);
void orc_bf16_to_f32(const uint16_t* in, float* out, int64_t n);

/* ---- neighbours on the MLP graph (src/backends/cpu/ops/activation.cpp) --- */

void orc_relu(const float* x, int64_t n, float* out);   /* :45-60 */
/* cpu_gelu, activation.cpp:239-259 (tanh approximation, libm tanhf). */
void orc_gelu(const float* x, int64_t n, float* out);
/* cpu_layernorm, nn.cpp:419-490: x viewed as [outer, norm] (norm = the
 * product of the dimensions from axis on), sequential mean and variance,
 * out = scale[i] * (x - mean) * inv_std + bias[i]. */
void orc_layernorm(const float* x, int64_t outer, int64_t norm, const float* scale,
                   const float* bias, float epsilon, float* out);
/* cpu_add (math.cpp:150-224 binary_elementwise with +): numpy-style
 * broadcasting of a [a_nd dims] and b [b_nd dims] to out [out_nd dims]. */
int orc_add(const float* a, const int64_t* a_shape, int a_nd, const float* b,
            const int64_t* b_shape, int b_nd, float* out, int64_t* out_shape,
            int* out_nd);
void orc_softmax(const float* x, int64_t outer, int64_t axis_size,
                 int64_t inner, float* out);            /* :157-237 */

#ifdef __cplusplus
}
#endif
#endif
