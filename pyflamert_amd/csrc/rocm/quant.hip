// Per-tensor QuantizeLinear / DequantizeLinear (and the Quantize /
// Dequantize ops, which take the same parameters from attributes), and
// DynamicQuantizeLinear on the GPU (cpu_dynamic_quantize_linear,
// quantized_ops.cpp:251-278): per-tensor uint8 asymmetric parameters from
// the data, then the quantized tensor.
//   params  compute_dynamic_params(x, UInt8, symmetric = false)
//           (quant_ops.cpp:288-327): min and max over the finite elements;
//           none finite, or an empty tensor: scale 1, zero point 0; else
//           compute_from_minmax (quant_params.cpp:14-55): |max - min| <
//           1e-8 gives scale 1, zero point 0; otherwise scale = (max - min) /
//           255, zero point = clamp(0 - (int)round(min / scale), 0, 255),
//           scale floored at 1e-10; a non-finite scale is the error of
//           QuantParams::per_tensor (quant_params.hpp:60-82).
//   values  quantize_tensor (quant_ops.cpp:15-47): inv = 1 / scale,
//           q = (int)round(x * inv) + zero point, clamped to [0, 255].
// The reduction order of min and max cannot change them except for the sign
// of a zero, which does not reach the parameters (max - min, round(min /
// scale) and the comparisons are the same for +0 and -0), so a parallel
// reduction gives the reference's parameters exactly.
#include <cfloat>
#include <cmath>

#include "common.hpp"

#pragma clang fp contract(off)

namespace {

constexpr int kRedThreads = 256;
constexpr int kRedBlocks = 1024;  // partial min/max pairs

struct DqlState {
    float part_min[kRedBlocks];
    float part_max[kRedBlocks];
};

// min and max over the finite values of `v`
__device__ __forceinline__ void dql_take(float v, float& mn, float& mx) {
    if (isfinite(v)) {
        mn = v < mn ? v : mn;
        mx = mx < v ? v : mx;
    }
}

// min and max over a block's threads' values (all threads call it)
__device__ __forceinline__ void dql_block_reduce(float& mn, float& mx, float* smin, float* smax) {
    smin[threadIdx.x] = mn;
    smax[threadIdx.x] = mx;
    __syncthreads();
    for (int off = kRedThreads / 2; off > 0; off >>= 1) {
        if (threadIdx.x < off) {
            const float a = smin[threadIdx.x + off], b = smax[threadIdx.x + off];
            smin[threadIdx.x] = a < smin[threadIdx.x] ? a : smin[threadIdx.x];
            smax[threadIdx.x] = smax[threadIdx.x] < b ? b : smax[threadIdx.x];
        }
        __syncthreads();
    }
    mn = smin[0];
    mx = smax[0];
}

// Pass 1 of DynamicQuantizeLinear: each block's min and max over the finite
// values (float4 loads when x is 16-byte aligned).
template <bool VEC>
__global__ __launch_bounds__(kRedThreads) void k_dql_minmax(const float* __restrict__ x, int64_t n,
                                                             DqlState* __restrict__ st) {
    __shared__ float smin[kRedThreads], smax[kRedThreads];
    float mn = FLT_MAX, mx = -FLT_MAX;
    const int64_t stride = (int64_t)gridDim.x * kRedThreads;
    int64_t i = (int64_t)blockIdx.x * kRedThreads + threadIdx.x;
    if constexpr (VEC) {
        const float4* x4 = reinterpret_cast<const float4*>(x);
        const int64_t n4 = n / 4;
        for (; i < n4; i += stride) {
            const float4 v = x4[i];
            dql_take(v.x, mn, mx);
            dql_take(v.y, mn, mx);
            dql_take(v.z, mn, mx);
            dql_take(v.w, mn, mx);
        }
        i = 4 * n4 + (int64_t)blockIdx.x * kRedThreads + threadIdx.x;  // the last n % 4
    }
    for (; i < n; i += stride) dql_take(x[i], mn, mx);
    dql_block_reduce(mn, mx, smin, smax);
    if (threadIdx.x == 0) {
        st->part_min[blockIdx.x] = mn;
        st->part_max[blockIdx.x] = mx;
    }
}

__device__ __forceinline__ uint32_t dql_q(float v, float inv, int32_t zp) {
    int32_t q = (int32_t)((uint32_t)pfr::f2i_trunc_x86(roundf(v * inv)) + (uint32_t)zp);
    return (uint32_t)(q < 0 ? 0 : (q > 255 ? 255 : q));
}

// Pass 2: every block reduces the nparts partials to the parameters (block 0
// also writes them to the op's scale and zero-point outputs and the status),
// then quantizes its share of x: four values per thread (one float4 in, four
// bytes out) when x and y allow it.  nparts == 0 (an empty tensor) gives
// scale 1 and zero point 0.  status (optional): 0, or 1 when the scale is
// not finite (the error QuantParams::per_tensor raises).
template <bool VEC>
__global__ __launch_bounds__(kRedThreads) void k_dql_quant(const float* __restrict__ x, int64_t n, int nparts,
                                                           const DqlState* __restrict__ st, uint8_t* __restrict__ y,
                                                           float* __restrict__ scale_out, uint8_t* __restrict__ zp_out,
                                                           int32_t* status) {
    __shared__ float smin[kRedThreads], smax[kRedThreads];
    float mn = FLT_MAX, mx = -FLT_MAX;
    for (int i = threadIdx.x; i < nparts; i += kRedThreads) {
        const float a = st->part_min[i], b = st->part_max[i];
        mn = a < mn ? a : mn;
        mx = mx < b ? b : mx;
    }
    dql_block_reduce(mn, mx, smin, smax);
    float scale = 1.0f;
    int32_t zp = 0;
    if (nparts > 0 && !(mn > mx) && !(fabsf(mx - mn) < 1e-8f)) {
        scale = (mx - mn) / 255.0f;
        zp = (int32_t)(0u - (uint32_t)pfr::f2i_trunc_x86(roundf(mn / scale)));  // x86 wraps
        zp = zp < 0 ? 0 : (zp > 255 ? 255 : zp);
        if (scale < 1e-10f) scale = 1e-10f;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        if (status) *status = (scale > 0.0f && isfinite(scale)) ? 0 : 1;
        *scale_out = scale;
        *zp_out = (uint8_t)zp;
    }
    const float inv = 1.0f / scale;
    const int64_t stride = (int64_t)gridDim.x * kRedThreads;
    int64_t i = (int64_t)blockIdx.x * kRedThreads + threadIdx.x;
    if constexpr (VEC) {
        const int64_t n4 = n / 4;
        for (; i < n4; i += stride) {
            const float4 v = reinterpret_cast<const float4*>(x)[i];
            reinterpret_cast<uint32_t*>(y)[i] =
                dql_q(v.x, inv, zp) | dql_q(v.y, inv, zp) << 8 | dql_q(v.z, inv, zp) << 16 | dql_q(v.w, inv, zp) << 24;
        }
        i = 4 * n4 + (int64_t)blockIdx.x * kRedThreads + threadIdx.x;
    }
    for (; i < n; i += stride) y[i] = (uint8_t)dql_q(x[i], inv, zp);
}

// Per-tensor quantize (quantize_tensor, quant_ops.cpp:15-57): inv = 1 /
// scale, q = (int32) round(x * inv) + zero point (x86 conversion and
// wrapping add), clamped to [-128, 127] or [0, 255].
template <bool U8>
__global__ __launch_bounds__(256) void k_quantize(const float* __restrict__ x, int64_t n, float inv, int32_t zp,
                                                  void* __restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    int32_t q = (int32_t)((uint32_t)pfr::f2i_trunc_x86(roundf(x[i] * inv)) + (uint32_t)zp);
    if (U8) {
        q = q < 0 ? 0 : (q > 255 ? 255 : q);
        static_cast<uint8_t*>(y)[i] = (uint8_t)q;
    } else {
        q = q < -128 ? -128 : (q > 127 ? 127 : q);
        static_cast<int8_t*>(y)[i] = (int8_t)q;
    }
}

// Per-tensor dequantize (dequantize_tensor, quant_ops.cpp:129-157):
// ((float) q - (float) zero point) * scale.
template <bool U8>
__global__ __launch_bounds__(256) void k_dequantize(const void* __restrict__ q, int64_t n, float scale, float zpf,
                                                    float* __restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float v = U8 ? (float)static_cast<const uint8_t*>(q)[i] : (float)static_cast<const int8_t*>(q)[i];
    y[i] = (v - zpf) * scale;
}

// QuantParams::per_tensor (quant_params.hpp:60-82): the checks and texts.
void per_tensor_checks(float scale, pfr_dtype dt) {
    if (!(scale > 0.0f) || !std::isfinite(scale))
        throw pfr::Error(PFR_ERR_INVALID_ARG, "QuantParams::per_tensor: scale must be positive and finite");
    if (dt != PFR_I8 && dt != PFR_U8)
        throw pfr::Error(PFR_ERR_INVALID_ARG, "QuantParams::per_tensor: dtype must be Int8 or UInt8");
}

void quantize_dev(pfr_ctx* ctx, const float* x, int64_t n, float scale, int32_t zp, pfr_dtype dt, void* y) {
    pfr::require(n >= 0, "negative element count");
    per_tensor_checks(scale, dt);
    if (n == 0) return;
    pfr::require(x && y, "null x/y");
    const float inv = 1.0f / scale;
    const dim3 grid((unsigned)((n + 255) / 256));
    if (dt == PFR_U8) hipLaunchKernelGGL(k_quantize<true>, grid, dim3(256), 0, ctx->stream, x, n, inv, zp, y);
    else hipLaunchKernelGGL(k_quantize<false>, grid, dim3(256), 0, ctx->stream, x, n, inv, zp, y);
    PFR_HIP(hipGetLastError());
}

void dequantize_dev(pfr_ctx* ctx, const void* q, pfr_dtype dt, int64_t n, float scale, int32_t zp, float* y) {
    pfr::require(n >= 0, "negative element count");
    per_tensor_checks(scale, dt);  // the parameters are built before dequantize_tensor runs
    if (n == 0) return;
    pfr::require(q && y, "null q/y");
    const dim3 grid((unsigned)((n + 255) / 256));
    if (dt == PFR_U8)
        hipLaunchKernelGGL(k_dequantize<true>, grid, dim3(256), 0, ctx->stream, q, n, scale, (float)zp, y);
    else
        hipLaunchKernelGGL(k_dequantize<false>, grid, dim3(256), 0, ctx->stream, q, n, scale, (float)zp, y);
    PFR_HIP(hipGetLastError());
}

void dql_dev(pfr_ctx* ctx, const float* x, int64_t n, uint8_t* y, float* scale, uint8_t* zp, int32_t* status) {
    pfr::require(n >= 0, "negative element count");
    pfr::require(scale && zp, "null scale/zero-point output");
    pfr::require(n == 0 || (x && y), "null x/y");
    DqlState* st = static_cast<DqlState*>(ctx->scratch[4].ensure(sizeof(DqlState)));
    hipStream_t q = ctx->stream;
    const bool vx = n > 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
    const bool vy = vx && (reinterpret_cast<uintptr_t>(y) & 3) == 0;
    const int64_t per = vx ? 4 * kRedThreads : kRedThreads;  // elements per block and pass
    const int nparts = n == 0 ? 0 : (int)std::min<int64_t>(kRedBlocks, (n + per - 1) / per);
    if (nparts) {
        if (vx) hipLaunchKernelGGL(k_dql_minmax<true>, dim3(nparts), dim3(kRedThreads), 0, q, x, n, st);
        else hipLaunchKernelGGL(k_dql_minmax<false>, dim3(nparts), dim3(kRedThreads), 0, q, x, n, st);
    }
    // the quantize pass: about a block per CU-slot, each reducing the
    // partials (nparts x 8 B from L2) before its share of x
    const int qb = (int)std::max<int64_t>(1, std::min<int64_t>(512, (n + 4 * kRedThreads - 1) / (4 * kRedThreads)));
    if (vy)
        hipLaunchKernelGGL(k_dql_quant<true>, dim3(qb), dim3(kRedThreads), 0, q, x, n, nparts, st, y, scale, zp, status);
    else
        hipLaunchKernelGGL(k_dql_quant<false>, dim3(qb), dim3(kRedThreads), 0, q, x, n, nparts, st, y, scale, zp, status);
    PFR_HIP(hipGetLastError());
}

}  // namespace

extern "C" {

int pfr_dynamic_quantize_linear_dev(pfr_ctx* ctx, const float* x, int64_t n, uint8_t* y, float* scale,
                                    uint8_t* zero_point, int32_t* status) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        dql_dev(ctx, x, n, y, scale, zero_point, status);
    });
}

int pfr_quantize_linear_dev(pfr_ctx* ctx, const float* x, int64_t n, float scale, int32_t zero_point,
                            pfr_dtype out_dtype, void* y) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        quantize_dev(ctx, x, n, scale, zero_point, out_dtype, y);
    });
}

int pfr_quantize_linear(pfr_ctx* ctx, const float* x, int64_t n, float scale, int32_t zero_point,
                        pfr_dtype out_dtype, void* y) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        pfr::require(n >= 0, "negative element count");
        per_tensor_checks(scale, out_dtype);
        if (n == 0) return;
        pfr::require(x && y, "null x/y");
        float* dx = static_cast<float*>(ctx->scratch[0].ensure((size_t)n * 4));
        void* dy = ctx->scratch[2].ensure((size_t)n);
        PFR_HIP(hipMemcpyAsync(dx, x, (size_t)n * 4, hipMemcpyHostToDevice, ctx->stream));
        quantize_dev(ctx, dx, n, scale, zero_point, out_dtype, dy);
        PFR_HIP(hipMemcpyAsync(y, dy, (size_t)n, hipMemcpyDeviceToHost, ctx->stream));
        PFR_HIP(hipStreamSynchronize(ctx->stream));
    });
}

int pfr_dequantize_linear_dev(pfr_ctx* ctx, const void* q, pfr_dtype q_dtype, int64_t n, float scale,
                              int32_t zero_point, float* y) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        dequantize_dev(ctx, q, q_dtype, n, scale, zero_point, y);
    });
}

int pfr_dequantize_linear(pfr_ctx* ctx, const void* q, pfr_dtype q_dtype, int64_t n, float scale,
                          int32_t zero_point, float* y) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        pfr::require(n >= 0, "negative element count");
        per_tensor_checks(scale, q_dtype);
        if (n == 0) return;
        pfr::require(q && y, "null q/y");
        void* dq = ctx->scratch[0].ensure((size_t)n);
        float* dy = static_cast<float*>(ctx->scratch[2].ensure((size_t)n * 4));
        PFR_HIP(hipMemcpyAsync(dq, q, (size_t)n, hipMemcpyHostToDevice, ctx->stream));
        dequantize_dev(ctx, dq, q_dtype, n, scale, zero_point, dy);
        PFR_HIP(hipMemcpyAsync(y, dy, (size_t)n * 4, hipMemcpyDeviceToHost, ctx->stream));
        PFR_HIP(hipStreamSynchronize(ctx->stream));
    });
}

int pfr_dynamic_quantize_linear(pfr_ctx* ctx, const float* x, int64_t n, uint8_t* y, float* scale,
                                uint8_t* zero_point) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        pfr::require(n >= 0, "negative element count");
        pfr::require(scale && zero_point, "null scale/zero-point output");
        pfr::require(n == 0 || (x && y), "null x/y");
        float* dx = static_cast<float*>(ctx->scratch[0].ensure((size_t)n * 4 + 4));
        uint8_t* dy = static_cast<uint8_t*>(ctx->scratch[2].ensure((size_t)n + 64));
        float* dscale = reinterpret_cast<float*>(dy + ((n + 15) / 16) * 16);
        int32_t* dstatus = reinterpret_cast<int32_t*>(dscale + 1);
        uint8_t* dzp = reinterpret_cast<uint8_t*>(dstatus + 1);
        if (n) PFR_HIP(hipMemcpyAsync(dx, x, (size_t)n * 4, hipMemcpyHostToDevice, ctx->stream));
        dql_dev(ctx, dx, n, dy, dscale, dzp, dstatus);
        int32_t status = 0;
        PFR_HIP(hipMemcpyAsync(&status, dstatus, 4, hipMemcpyDeviceToHost, ctx->stream));
        PFR_HIP(hipStreamSynchronize(ctx->stream));
        if (status)
            throw pfr::Error(PFR_ERR_INVALID_ARG, "QuantParams::per_tensor: scale must be positive and finite");
        if (n) PFR_HIP(hipMemcpyAsync(y, dy, (size_t)n, hipMemcpyDeviceToHost, ctx->stream));
        PFR_HIP(hipMemcpyAsync(scale, dscale, 4, hipMemcpyDeviceToHost, ctx->stream));
        PFR_HIP(hipMemcpyAsync(zero_point, dzp, 1, hipMemcpyDeviceToHost, ctx->stream));
        PFR_HIP(hipStreamSynchronize(ctx->stream));
    });
}

}  // extern "C"
