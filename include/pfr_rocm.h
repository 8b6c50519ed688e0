/*
 * pfr_rocm.h -- C ABI of the MI355X (gfx950) kernels for PyFlameRT's
 * pruned-weight MatMul/Gemm path.
 *
 * This is the boundary a `src/backends/rocm` backend inside PyFlameRT binds
 * to.  Plain pointers and sizes only; no exceptions cross it.  Every function
 * returns PFR_OK (0) or an error code; pfr_last_error() then describes the
 * failure (thread-local).  Functions whose pointer arguments are documented
 * as "host" copy in and out and synchronise before returning, matching the
 * synchronous OpFunc contract of the reference
 * (include/pyflame_rt/registry.hpp:26-29, src/backends/cpu/executor.cpp:106).
 * The *_dev variants take device pointers, enqueue on the context's stream
 * and do not synchronise.
 *
 * Numerics (defined by the reference CPU kernels):
 *   PFR_MODE_STRICT  fp32 results bit-identical to cpu_matmul / cpu_gemm /
 *                    sparse_matmul (math.cpp:268-438, sparse_tensor.cpp:473-554):
 *                    each output is the ascending-k sequence of separately
 *                    rounded products and sums, bias added last.
 *   PFR_MODE_FAST    fused multiply-add (one rounding per term) in an order
 *                    the kernel chooses (wave-parallel partial sums; the
 *                    column-slice kernel also takes a row's terms in an order
 *                    that spreads its LDS reads over the banks); close to,
 *                    not equal to, the reference.
 *   int8 paths       int32 accumulators and requantised int8 bit-exact to
 *                    quantized_matmul + quantize_tensor (quant_ops.cpp:387-506,
 *                    :15-127).
 */
#ifndef PFR_ROCM_H
#define PFR_ROCM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PFR_OK 0
#define PFR_ERR_INVALID_ARG 1 /* maps to std::invalid_argument in the OpFunc */
#define PFR_ERR_HIP 2         /* HIP runtime error; text from hipGetErrorString */
#define PFR_ERR_UNSUPPORTED 3 /* shape/dtype not handled by any kernel */
#define PFR_ERR_NO_DEVICE 4

/* Element types; the values are those of pyflame_rt::DType (types.hpp:48-59). */
typedef enum pfr_dtype {
    PFR_F32 = 0,
    PFR_BF16 = 2,
    PFR_I32 = 5,
    PFR_I8 = 7,
    PFR_U8 = 8
} pfr_dtype;

typedef enum pfr_mode { PFR_MODE_STRICT = 0, PFR_MODE_FAST = 1 } pfr_mode;

/* Activation fused into a product's epilogue (after the bias). */
typedef enum pfr_act {
    PFR_ACT_NONE = 0,
    PFR_ACT_RELU = 1, /* cpu_relu, activation.cpp:45-60: std::max(0.0f, v) */
    PFR_ACT_GELU = 2  /* cpu_gelu, activation.cpp:239-259: tanh approximation
                         (device tanhf: within a few ulp of the reference) */
} pfr_act;

typedef struct pfr_ctx pfr_ctx;   /* one device + one stream + scratch */
typedef struct pfr_csr pfr_csr;   /* device-resident CSR weight */
typedef struct pfr_sp24 pfr_sp24; /* device-resident 2:4 compressed weight */

/* ---- context ------------------------------------------------------------ */

/* Text of the last error on this thread ("" if none). */
const char* pfr_last_error(void);
int pfr_device_count(int* count);
/* Bind to `device`, create a stream.  Replaces the CPU-only backend choice of
 * InferenceSession::select_backend (src/session.cpp:67-95). */
int pfr_rocm_init(int device, pfr_ctx** out);
int pfr_rocm_destroy(pfr_ctx* ctx);
/* The hipStream_t the context enqueues on (as void*), and a way to replace
 * it with a caller-owned stream.  NULL is the device's null stream, as in
 * HIP; the context's own stream is whatever pfr_ctx_get_stream returned
 * right after pfr_rocm_init. */
int pfr_ctx_get_stream(pfr_ctx* ctx, void** stream);
int pfr_ctx_set_stream(pfr_ctx* ctx, void* stream);
int pfr_synchronize(pfr_ctx* ctx);

/* Device buffers for callers that keep activations on the GPU between
 * nodes (the executor's device-resident plan; the reference's Tensor storage,
 * src/tensor.cpp:31-49, is host memory only).  pfr_copy_to_device enqueues
 * on the context's stream (the host source must stay valid until the stream
 * reaches the copy, e.g. until a later pfr_copy_to_host or
 * pfr_synchronize); pfr_copy_to_host waits for the stream.  pfr_dev_free
 * waits for the stream before freeing. */
int pfr_dev_alloc(pfr_ctx* ctx, int64_t bytes, void** out);
int pfr_dev_free(pfr_ctx* ctx, void* p);
int pfr_copy_to_device(pfr_ctx* ctx, void* dst, const void* src, int64_t bytes);
int pfr_copy_to_host(pfr_ctx* ctx, void* dst, const void* src, int64_t bytes);

/* ---- CSR weights (reference: pruning::SparseTensor, sparse_tensor.hpp:19-132) */

/* Upload an M x K CSR matrix given as the reference's SparseTensor stores it
 * (indptr/indices int64, sparse_tensor.hpp:124-126; values float).  Indices
 * are range-checked (the check from_csr leaves out, sparse_tensor.cpp:39-49
 * is never called) and must ascend within a row.  values_dtype is PFR_F32 or
 * PFR_I8; for PFR_I8, row_scales[M] are the per-output-channel scales of a
 * symmetric weight (dequantised value = (float)q * row_scales[m],
 * quant_ops.cpp:182-196).  Host pointers. */
int pfr_csr_upload(pfr_ctx* ctx, int64_t M, int64_t K, int64_t nnz,
                   const int64_t* indptr, const int64_t* indices,
                   const void* values, pfr_dtype values_dtype,
                   const float* row_scales, pfr_csr** out);
/* pfr_csr_upload with int32 column indices: the form a sparse .pfm record
 * keeps in memory (no reference counterpart; the reference has no sparse
 * on-disk form, pyflame_format.cpp:168-176), uploaded without widening. */
int pfr_csr_upload_i32(pfr_ctx* ctx, int64_t M, int64_t K, int64_t nnz,
                       const int64_t* indptr, const int32_t* indices,
                       const void* values, pfr_dtype values_dtype,
                       const float* row_scales, pfr_csr** out);
/* Build the CSR of a dense, zero-filled pruned weight the way
 * to_sparse(dense, threshold, CSR) does (sparse_tensor.cpp:560-610: keeps
 * |v| > threshold, columns ascending).  dense is rows x cols, row-major,
 * host.  With transpose != 0 the CSR is of dense^T (cols x rows): the form a
 * Gemm/MatMul weight in the B position needs, so each output column's terms
 * stay in ascending k. */
int pfr_csr_from_dense(pfr_ctx* ctx, const float* dense, int64_t rows,
                       int64_t cols, int transpose, float threshold,
                       pfr_csr** out);
/* pfr_csr_from_dense for a weight already on the device, with the pruning
 * mask optionally applied on the way: the CSR of op(dense * mask), where
 * dense * mask is apply_mask (sparse_tensor.cpp:616-631; mask may be NULL)
 * and op transposes when transpose != 0, keeping |v| > threshold with
 * columns ascending as to_sparse does (sparse_tensor.cpp:560-610).  dense
 * and mask are rows x cols, row-major, device.  The nonzeros are found,
 * compacted and laid out on the device; only per-row counts come back to
 * the host (to plan the layouts), so the handle equals what
 * pfr_csr_from_dense builds from the same weight, and every product gives
 * bit-identical results with either.  Runs on the context's stream and
 * returns when the handle is complete.  At most 2^24 rows of op(dense). */
int pfr_csr_from_dense_dev(pfr_ctx* ctx, const float* dense, int64_t rows,
                           int64_t cols, int transpose, float threshold,
                           const float* mask, pfr_csr** out);
/* Give the handle the dense kernels' treatment of non-finite activations
 * (cpu_matmul / cpu_gemm, math.cpp:268-438, on the zero-filled weight), for
 * a CSR that stands in for a dense initializer: those kernels multiply every
 * activation by every weight, so an inf or NaN activation meets the zeros
 * the CSR does not store (inf * 0 = NaN), which sparse_matmul
 * (sparse_tensor.cpp:473-519) skips.  Builds a bitmap of the stored entries
 * (M x ceil(K / 64) words); from then on every product through the handle
 * is followed by a fix-up pass over the activations that writes NaN (through
 * the bias and activation epilogue) where an inf activation meets an
 * unstored weight or a NaN activation meets any weight of an output.  For
 * finite activations results are unchanged.  Idempotent. */
int pfr_csr_dense_semantics(pfr_csr* w);
int pfr_csr_info(const pfr_csr* w, int64_t* M, int64_t* K, int64_t* nnz);
/* Device bytes the handle holds: the CSR itself (row pointers, columns as
 * uint16 when K <= 65536 and int32 otherwise, values, row scales), the
 * row-block table, the merge-path partition and every derived copy built so
 * far.  The sliced-ELL copy (float32 weights, N >= 16; one in storage order
 * for the strict mode, one reordered for the fast mode, sharing their slab
 * tables), the row-chain copy (strict, N <= 8) and the nnz-balanced copy
 * (fast, N <= 8) are built by the
 * first product through the handle that would use one: that call plans on
 * the host, allocates, fills on the device and synchronizes the handle's
 * stream.  While that stream is being captured into a graph, and in
 * pfr_gemm_csr_act_noalloc_dev, nothing is built and a product without its
 * copy runs a kernel that reads the CSR in place (same results in strict
 * mode, the fast mode's own rounding otherwise), so run each kind of
 * product once before capture.  No counterpart in the reference (its
 * weights are host memory); for footprint reports. */
int pfr_csr_device_bytes(const pfr_csr* w, int64_t* bytes);
int pfr_csr_free(pfr_csr* w);

/* ---- CSR products --------------------------------------------------------- */

/* Y[M,N] = W[M,K] . X[K,N] (row-major, host).  N == 1 is the SpMV of
 * sparse_matvec (sparse_tensor.cpp:521-554).  Replaces sparse_matmul
 * (sparse_tensor.cpp:473-519) and MatMul with a pruned first operand
 * (math.cpp:268-374).  For int8 values each term uses the dequantised
 * weight RN((float)q * row_scales[m]) (dequantize_tensor with zero point 0,
 * quant_ops.cpp:182-196), so the result equals dequantize-then-sparse_matmul
 * bit for bit in strict mode. */
int pfr_spmm_csr(pfr_ctx* ctx, const pfr_csr* W, const float* X, int64_t N,
                 float* Y, int mode);
/* Device variant.  X rows are ldx floats apart, Y rows ldy floats apart
 * (ldx, ldy >= N). */
int pfr_spmm_csr_dev(pfr_ctx* ctx, const pfr_csr* W, const float* X,
                     int64_t N, int64_t ldx, float* Y, int64_t ldy, int mode);

/* pfr_spmm_csr_dev with an activation fused into the epilogue: the node
 * pair MatMul(W, X) -> Relu (math.cpp:268-374 then activation.cpp:45-60) in
 * one pass, bit-identical to the two nodes in strict mode. */
int pfr_spmm_csr_act_dev(pfr_ctx* ctx, const pfr_csr* W, const float* X,
                         int64_t N, int64_t ldx, float* Y, int64_t ldy,
                         int mode, int act);

/* Gemm with the weight in the B position (cpu_gemm, math.cpp:377-438):
 *   Y[Mb, Nf] = alpha * op(A)[Mb, K] . B[K, Nf] + beta * C[(i*Nf+j) % c_size]
 * where BT is the CSR of op(B)^T (Nf x K, from pfr_csr_from_dense with
 * transpose = !transB).  A is Mb x K (transA == 0) or K x Mb, host.  C may be
 * NULL (c_size ignored).  MatMul(X, W) with a pruned W is the case alpha = 1,
 * C = NULL (math.cpp:327-333). */
int pfr_gemm_csr(pfr_ctx* ctx, const float* A, int64_t Mb, int64_t K,
                 int transA, const pfr_csr* BT, float alpha, float beta,
                 const float* C, int64_t c_size, float* Y, int mode);
/* Device variant (A, C, Y device pointers, all contiguous). */
int pfr_gemm_csr_dev(pfr_ctx* ctx, const float* A, int64_t Mb, int64_t K,
                     int transA, const pfr_csr* BT, float alpha, float beta,
                     const float* C, int64_t c_size, float* Y, int mode);

/* pfr_gemm_csr_dev with an activation fused after the bias: the node pair
 * Gemm -> Relu (math.cpp:377-438 then activation.cpp:45-60) in one pass,
 * bit-identical to the two nodes in strict mode. */
int pfr_gemm_csr_act_dev(pfr_ctx* ctx, const float* A, int64_t Mb, int64_t K,
                         int transA, const pfr_csr* BT, float alpha, float beta,
                         const float* C, int64_t c_size, float* Y, int mode,
                         int act);

/* Allocation-free form of pfr_gemm_csr_act_dev.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, results and errors, except that it builds
 * none of the handle's derived copies (see pfr_csr_device_bytes): a product
 * whose copy the handle does not hold yet runs a kernel that reads the CSR
 * in place (bit-identical in strict mode, the fast mode's own rounding
 * otherwise), and that the copy of
 * op(A)^T that the product reads (made when transA == 0 or alpha != 1) is
 * staged in a fixed per-device workspace of 4,194,304 floats (16 MiB)
 * instead of the context's grow-only buffer; K * Mb beyond that is
 * PFR_ERR_INVALID_ARG, reported before anything is enqueued.  Calls no
 * hipMalloc or hipFree.  Every call on a GPU shares that GPU's workspace:
 * calls that overlap on one GPU (other streams or contexts) race; calls on
 * one stream are ordered. */
int pfr_gemm_csr_act_noalloc_dev(pfr_ctx* ctx, const float* A, int64_t Mb, int64_t K,
                                 int transA, const pfr_csr* BT, float alpha, float beta,
                                 const float* C, int64_t c_size, float* Y, int mode,
                                 int act);

/* ---- Dense products (weights above the sparse path's density gate) -------- */

/* cpu_gemm / cpu_matmul (math.cpp:268-438) on dense float32 operands:
 *   Y[i, j] = act(sum_k (alpha * op(A)[i, k]) * B[k, j] + beta * C[(i*N + j) % c_size])
 * op(A) = A (M x K) or, with transA, A^T (A is K x M); B is K x N with row
 * stride ldb; Y rows are ldy floats apart; C may be NULL.  Each output sums
 * its terms in ascending k from +0 with separate multiply and add, as the
 * reference loops do, so results are bit-identical to cpu_gemm (and, with
 * alpha = 1 and no C, to cpu_matmul), non-finite values included.  act as
 * in pfr_spmm_csr_act_dev.  Device pointers, the context's stream. */
int pfr_gemm_dense_dev(pfr_ctx* ctx, const float* A, int64_t M, int64_t K,
                       int transA, const float* B, int64_t N, int64_t ldb,
                       float alpha, float beta, const float* C, int64_t c_size,
                       float* Y, int64_t ldy, int act);

/* ---- 2:4 structured weights (sparse MFMA, gfx950 smfmac) ------------------- */

/* Pack a dense M x K weight that is 2:4 sparse along K (every group of four
 * consecutive k holds at most two nonzeros: what NMSparsityPruning(2, 4)
 * produces, nm_sparsity.cpp:45-120) into the compressed operand layout of
 * the gfx950 sparse MFMA: kept values + 2-bit positions, pre-arranged in
 * per-lane register order.  W is host, int8 (dtype PFR_I8, the output of
 * quantize_tensor) or bf16 bits (PFR_BF16).  w_scales holds n_scales = 1
 * (per-tensor, the reference's QuantParams::scales[0]) or M (per output
 * channel) symmetric scales; only used by the int8 float/requant outputs.
 * Fails with PFR_ERR_INVALID_ARG naming the first group with > 2 nonzeros. */
int pfr_sp24_pack(pfr_ctx* ctx, int64_t M, int64_t K, const void* W,
                  pfr_dtype dtype, const float* w_scales, int64_t n_scales,
                  pfr_sp24** out);
/* pfr_sp24_pack for a weight already on the device (W device, w_scales
 * host): the same layout, written by device kernels, so the weight never
 * crosses to the host; the 2:4 check runs on the device and reports the
 * first offending group in the same words.  Returns when the handle is
 * complete. */
int pfr_sp24_pack_dev(pfr_ctx* ctx, int64_t M, int64_t K, const void* W,
                      pfr_dtype dtype, const float* w_scales, int64_t n_scales,
                      pfr_sp24** out);
int pfr_sp24_info(const pfr_sp24* w, int64_t* M, int64_t* K, pfr_dtype* dtype);
int pfr_sp24_free(pfr_sp24* w);

/* Output form of the int8 2:4 GEMM. */
typedef enum pfr_sp24_out {
    PFR_SP24_OUT_I32 = 0,  /* raw int32 accumulators (exact) */
    PFR_SP24_OUT_F32 = 1,  /* (float)acc * (w_scale[m] * x_scale)
                              (quant_ops.cpp:435, :467) */
    PFR_SP24_OUT_I8 = 2    /* the float above requantised per tensor:
                              clamp(round(f * (1/out_scale)) + out_zp,
                              -128, 127) (quant_ops.cpp:500-503 -> :42-47) */
} pfr_sp24_out;

/* Y[M, N] = W[M, K] . X[K, N] with int8 X (row-major, zero-point 0) and
 * int32 accumulation: quantization::quantized_matmul
 * (quant_ops.cpp:387-506) with a 2:4 weight.  Host pointers; Y is int32,
 * float or int8 per out_kind. */
int pfr_sp24_gemm_i8(pfr_ctx* ctx, const pfr_sp24* W, const int8_t* X,
                     int64_t N, float x_scale, int out_kind, float out_scale,
                     int32_t out_zp, void* Y);
/* Device variant.  X is K x N row-major with row stride ldx; Y row stride
 * ldy (elements). */
int pfr_sp24_gemm_i8_dev(pfr_ctx* ctx, const pfr_sp24* W, const int8_t* X,
                         int64_t N, int64_t ldx, float x_scale, int out_kind,
                         float out_scale, int32_t out_zp, void* Y,
                         int64_t ldy);

/* The int8 2:4 GEMM with the activation as (Dynamic)QuantizeLinear leaves
 * it: int8 (x_dtype PFR_I8) or uint8 (PFR_U8) with a zero point:
 *   acc[m, n] = sum_k W[m, k] * (X[k, n] - zero_point)   (exact, int32)
 * then out_kind as above with x_scale: quantization::quantized_matmul
 * (quant_ops.cpp:387-506, which reads uint8 as uint8) with a per-channel
 * weight scale.  The scale and zero point are host values, or (_dev, when
 * x_scale_dev / x_zero_point_dev are non-NULL) device scalars such as the
 * outputs of pfr_dynamic_quantize_linear_dev on the same stream.  K < 2^17.
 * Host form: X and Y host pointers, X rows N apart. */
int pfr_sp24_gemm_q(pfr_ctx* ctx, const pfr_sp24* W, const void* X, pfr_dtype x_dtype,
                    int64_t N, float x_scale, int32_t x_zero_point, int out_kind,
                    float out_scale, int32_t out_zp, void* Y);
int pfr_sp24_gemm_q_dev(pfr_ctx* ctx, const pfr_sp24* W, const void* X, pfr_dtype x_dtype,
                        int64_t N, int64_t ldx, float x_scale, int32_t x_zero_point,
                        const float* x_scale_dev, const uint8_t* x_zero_point_dev,
                        int out_kind, float out_scale, int32_t out_zp, void* Y,
                        int64_t ldy);

/* The x . W form (the layout a Linear layer exports): Y[T, M] (float) =
 * X[T, K] . W^T with the packed 2:4 weight W[M, K] as the second operand of
 * QuantizedMatMul (quantization::quantized_matmul, quant_ops.cpp:387-506,
 * with the operands' roles swapped: per output column m the product is
 * (float) sum_k (x[t, k] - x_zero_point) * w[m, k] * (x_scale * w_scale[m])),
 * bit-exact.  X is row-major int8 or uint8 (ldx >= K), Y row-major (ldy >=
 * M); scale and zero point from host values or device scalars, as in
 * pfr_sp24_gemm_q_dev.  Host pointers: pfr_sp24_gemm_qt. */
int pfr_sp24_gemm_qt(pfr_ctx* ctx, const pfr_sp24* W, const void* X, pfr_dtype x_dtype,
                     int64_t T, float x_scale, int32_t x_zero_point, float* Y);
int pfr_sp24_gemm_qt_dev(pfr_ctx* ctx, const pfr_sp24* W, const void* X, pfr_dtype x_dtype,
                         int64_t T, int64_t ldx, float x_scale, int32_t x_zero_point,
                         const float* x_scale_dev, const uint8_t* x_zero_point_dev,
                         float* Y, int64_t ldy);

/* Y[M, N] (float) = W[M, K] . X[K, N] with bf16 operands and fp32
 * accumulation: cpu_gemm on bf16-rounded operands
 * (half_types.cpp:132-174 then math.cpp:377-438), within the bf16
 * tolerance (summation order differs).  X is bf16 bits, row-major. */
int pfr_sp24_gemm_bf16(pfr_ctx* ctx, const pfr_sp24* W, const uint16_t* X,
                       int64_t N, float* Y);
int pfr_sp24_gemm_bf16_dev(pfr_ctx* ctx, const pfr_sp24* W,
                           const uint16_t* X, int64_t N, int64_t ldx,
                           float* Y, int64_t ldy);

/* ---- graph neighbours kept on the device ---------------------------------- */

/* Relu, activation.cpp:45-60 (bit-exact).  Host pointers; _dev: device. */
int pfr_relu(pfr_ctx* ctx, const float* x, int64_t n, float* y);
int pfr_relu_dev(pfr_ctx* ctx, const float* x, int64_t n, float* y);
/* Softmax over the middle extent of x viewed as [outer, axis, inner],
 * activation.cpp:157-237 (same order and special cases; device expf). */
int pfr_softmax(pfr_ctx* ctx, const float* x, int64_t outer, int64_t axis,
                int64_t inner, float* y);
int pfr_softmax_dev(pfr_ctx* ctx, const float* x, int64_t outer, int64_t axis,
                    int64_t inner, float* y);
/* Gelu, cpu_gelu (activation.cpp:239-259): 0.5 x (1 + tanh(sqrt(2/pi)
 * (x + 0.044715 x^3))) with the device tanhf (a few ulp from the CPU). */
int pfr_gelu(pfr_ctx* ctx, const float* x, int64_t n, float* y);
int pfr_gelu_dev(pfr_ctx* ctx, const float* x, int64_t n, float* y);
/* Add with numpy broadcasting (cpu_add, math.cpp:150-224), bit-exact; at
 * most 8 dimensions.  y has the broadcast shape; shapes that do not
 * broadcast give PFR_ERR_INVALID_ARG. */
int pfr_add(pfr_ctx* ctx, const float* a, const int64_t* a_shape, int a_ndim,
            const float* b, const int64_t* b_shape, int b_ndim, float* y);
int pfr_add_dev(pfr_ctx* ctx, const float* a, const int64_t* a_shape, int a_ndim,
                const float* b, const int64_t* b_shape, int b_ndim, float* y);
/* LayerNormalization over the trailing `norm` elements of each of `outer`
 * rows (cpu_layer_norm, nn.cpp:419-490): sequential mean and variance in the
 * reference's order, y = scale * (x - mean) * (1 / sqrt(var + epsilon)) +
 * bias; bit-exact.  scale and bias hold `norm` floats. */
int pfr_layernorm(pfr_ctx* ctx, const float* x, int64_t outer, int64_t norm,
                  const float* scale, const float* bias, float epsilon, float* y);
int pfr_layernorm_dev(pfr_ctx* ctx, const float* x, int64_t outer, int64_t norm,
                      const float* scale, const float* bias, float epsilon, float* y);

/* ---- per-tensor quantize / dequantize ------------------------------------ */

/* QuantizeLinear and Quantize (cpu_quantize_linear, quantized_ops.cpp:284-315;
 * cpu_quantize, :35-55): quantize_tensor with per-tensor parameters
 * (quant_ops.cpp:15-57): q = clamp((int32) round(x * (1 / scale)) + zero_point)
 * to int8 (out_dtype PFR_I8) or uint8 (PFR_U8); bit-exact.  scale must be
 * positive and finite (QuantParams::per_tensor, quant_params.hpp:60-82).
 * Host pointers; _dev: device pointers, no synchronisation. */
int pfr_quantize_linear(pfr_ctx* ctx, const float* x, int64_t n, float scale,
                        int32_t zero_point, pfr_dtype out_dtype, void* y);
int pfr_quantize_linear_dev(pfr_ctx* ctx, const float* x, int64_t n, float scale,
                            int32_t zero_point, pfr_dtype out_dtype, void* y);
/* DequantizeLinear and Dequantize (cpu_dequantize_linear, :321-347;
 * cpu_dequantize, :57-70): dequantize_tensor per tensor (quant_ops.cpp:
 * 129-157): y = ((float) q - (float) zero_point) * scale; q int8 or uint8. */
int pfr_dequantize_linear(pfr_ctx* ctx, const void* q, pfr_dtype q_dtype, int64_t n,
                          float scale, int32_t zero_point, float* y);
int pfr_dequantize_linear_dev(pfr_ctx* ctx, const void* q, pfr_dtype q_dtype, int64_t n,
                              float scale, int32_t zero_point, float* y);

/* ---- dynamic activation quantization -------------------------------------- */

/* DynamicQuantizeLinear (cpu_dynamic_quantize_linear, quantized_ops.cpp:
 * 251-278): uint8 asymmetric per-tensor parameters from the finite minimum
 * and maximum of x (compute_dynamic_params, quant_ops.cpp:288-327, and
 * QuantParams::compute_from_minmax, quant_params.cpp:14-55), then y =
 * clamp((int)round(x * (1 / scale)) + zero_point, 0, 255) (quantize_tensor,
 * quant_ops.cpp:15-47).  Bit-exact.  Host pointers: y[n], *scale,
 * *zero_point; a non-finite scale fails with PFR_ERR_INVALID_ARG
 * ("QuantParams::per_tensor: scale must be positive and finite").  _dev:
 * device pointers, and (nullable) a device int32 *status that becomes 1 in
 * that case, 0 otherwise. */
int pfr_dynamic_quantize_linear(pfr_ctx* ctx, const float* x, int64_t n, uint8_t* y,
                                float* scale, uint8_t* zero_point);
int pfr_dynamic_quantize_linear_dev(pfr_ctx* ctx, const float* x, int64_t n, uint8_t* y,
                                    float* scale, uint8_t* zero_point, int32_t* status);

/* ---- pruning masks (session-time producers, on the GPU) -------------------- */

/* MagnitudePruning::compute_mask (magnitude_pruning.cpp:22-102): mask[i] =
 * 1.0f where |w[i]| exceeds the element at index min(floor((double)n * s),
 * n - 1) of the ascending sort of |w|; then elements equal to that value
 * are restored (set to 1) in flat order while more than (size_t)((float)n *
 * s) zeros remain.  s <= 0 gives all ones, s >= 1 all zeros; n == 0 with
 * 0 < s < 1 is PFR_ERR_INVALID_ARG ("Cannot prune empty weight tensor").
 * Bit-identical to the reference for NaN-free weights.  A NaN weight gets
 * mask 0 and counts among the zeros, as the reference's comparisons make
 * it; its place in the sort, which the reference's std::sort leaves
 * unspecified, is taken above +inf.
 * Host pointers; _dev: device pointers on the context's stream. */
int pfr_magnitude_mask(pfr_ctx* ctx, const float* w, int64_t n, float sparsity, float* mask);
int pfr_magnitude_mask_dev(pfr_ctx* ctx, const float* w, int64_t n, float sparsity, float* mask);
/* NMSparsityPruning::compute_mask (nm_sparsity.cpp:45-120): in every group
 * of m consecutive elements (flat order) mask = 1.0f for the n largest |w|,
 * ties broken as the reference's std::partial_sort breaks them; a last
 * partial group of g elements keeps ceil((float)(g * n) / m).  0 < n <= m <=
 * 16.  Host pointers; _dev: device pointers. */
int pfr_nm_mask(pfr_ctx* ctx, const float* w, int64_t total, int n, int m, float* mask);
int pfr_nm_mask_dev(pfr_ctx* ctx, const float* w, int64_t total, int n, int m, float* mask);
/* apply_mask (sparse_tensor.cpp:616-631): out[i] = w[i] * mask[i], one fp32
 * multiply per element (NaN or inf facing a 0 mask gives NaN, as there).
 * Host pointers; _dev: device pointers on the context's stream (out may be
 * w). */
int pfr_apply_mask(pfr_ctx* ctx, const float* w, const float* mask, int64_t n, float* out);
int pfr_apply_mask_dev(pfr_ctx* ctx, const float* w, const float* mask, int64_t n, float* out);

#ifdef __cplusplus
}
#endif
#endif
