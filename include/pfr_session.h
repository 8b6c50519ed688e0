/*
 * pfr_session.h -- C ABI of the runtime that runs .pfm models on the
 * MI355X backend: InferenceSession (include/pyflame_rt/session.hpp:30-108 of
 * the reference) behind plain pointers, for bindings (ctypes here; the
 * reference's pybind11 session binding, bindings/session_bind.cpp:13-92, is
 * the C++-side equivalent).  Errors: nonzero status, text from
 * pfr_session_last_error(); the status names the exception class the C++
 * runtime raised.
 */
#ifndef PFR_SESSION_H
#define PFR_SESSION_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PFR_S_OK 0
#define PFR_S_INVALID_MODEL 10   /* InvalidModelError */
#define PFR_S_VALIDATION 11      /* ValidationError */
#define PFR_S_UNSUPPORTED_OP 12  /* UnsupportedOperatorError */
#define PFR_S_INPUT 13           /* InputError / ShapeMismatchError */
#define PFR_S_BACKEND 14         /* BackendError */
#define PFR_S_RUNTIME 15         /* PyFlameRTError (other) */
#define PFR_S_FORMAT 16          /* UnsupportedFormatError */
#define PFR_S_OTHER 17           /* any other exception */

typedef struct pfr_session pfr_session;

const char* pfr_session_last_error(void);
/* device: "rocm" (other reference devices are rejected by this runtime).
 * math_mode: 0 strict (bit-exact fp32), 1 fast (FMA).
 * optimization_level: the reference's OptLevel (types.hpp:119-124).  0 None
 * runs node by node through the rocm:: OpFuncs; 1 Basic runs the
 * device-resident plan; 2 Extended (the reference's default) and 3 All add
 * operator fusion (Relu into the preceding pruned product).
 * quantization: NULL or "" for none; "dynamic_int8" rewrites every MatMul(W,
 * X) with a float 2:4-pruned initializer W into DynamicQuantizeLinear(X) +
 * QuantizedMatMul(per-row int8 W, ...) (the reference's QuantMode::
 * DynamicInt8 with per-channel weights). */
int pfr_session_create(const char* model_path, const char* device, int strict_math_mode, int math_mode,
                       int device_id, int optimization_level, const char* quantization,
                       pfr_session** out);
int pfr_session_destroy(pfr_session* s);
int pfr_session_io_count(pfr_session* s, int* n_inputs, int* n_outputs);
/* Name, DType code and shape (-1 = dynamic, at most 16 dims) of input or
 * output `index`.  name stays valid for the session's lifetime. */
int pfr_session_io_info(pfr_session* s, int is_output, int index, const char** name, int* dtype,
                        int64_t* shape, int* ndim);
/* Run with host tensors; outputs (all graph outputs, or the named ones) are
 * kept in the session until the next run. */
int pfr_session_run(pfr_session* s, int n_inputs, const char* const* names, const void* const* data,
                    const int* dtypes, const int64_t* const* shapes, const int* ndims, int n_outputs,
                    const char* const* output_names, int* n_results);
int pfr_session_result(pfr_session* s, int index, int* dtype, int64_t* shape, int* ndim, const void** data);
/* Backend identity and the op types it runs ("rocm::" kernels), newline
 * separated into buf (NUL-terminated, truncated to cap). */
int pfr_session_supported_ops(pfr_session* s, char* buf, int64_t cap);
/* After a run: *device_resident = 1 when the model runs as a device-resident
 * plan (graph inputs copied to the GPU once, activations kept there between
 * nodes, a Relu that is a product's only consumer fused into the product),
 * with *steps its kernel launches; 0 and 0 when it runs node by node. */
int pfr_session_device_plan(pfr_session* s, int* device_resident, int* steps);
/* After a run: how many Gemm / MatMul / QuantizedMatMul weights went to the
 * device as CSR (float32 initializers with at most half their entries
 * nonzero, and CSR records), as dense matrices (denser float32
 * initializers), and as 2:4 int8.  No reference counterpart (the CPU
 * backend keeps every weight as it is). */
int pfr_session_weight_forms(pfr_session* s, int* csr, int* dense, int* sp24);

/* Host-side model utilities (no device needed).  pfr_model_describe loads
 * and validates a .pfm with this runtime's loader and writes a JSON summary
 * (name, inputs, outputs, initializers with dtype/shape/nnz, nodes in
 * topological order with attributes) into buf; *needed gets the full size.
 * pfr_model_resave loads in_path and writes it back with this runtime's
 * writer (initializers and attributes in name order). */
int pfr_model_describe(const char* path, char* buf, int64_t cap, int64_t* needed);
/* The quantization rewrite offline: load in_path, apply mode ("dynamic_int8",
 * as the session option does), write out_path (version 2 when it adds 2:4
 * records); *rewritten (nullable) gets the number of MatMul nodes replaced. */
int pfr_model_quantize(const char* in_path, const char* out_path, const char* mode, int* rewritten);
int pfr_model_resave(const char* in_path, const char* out_path);

#ifdef __cplusplus
}
#endif
#endif
