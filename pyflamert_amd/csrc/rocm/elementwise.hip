// Neighbours of the pruned MatMul/Gemm on the MLP graph: Relu and Softmax,
// so a device="rocm" session keeps every node on the GPU.
//   Relu     out = std::max(0.0f, x)  (activation.cpp:45-60): (0 < x) ? x : +0
//   Softmax  activation.cpp:157-237: max with std::max semantics (NaN never
//            replaces the running max), exp(x - max), sequential sum, divide;
//            all -inf (or zero sum) rows become uniform 1/n.  exp is the
//            device expf, so results match the CPU within a few ulp, not bit
//            for bit.
#include <cmath>

#include "common.hpp"

#pragma clang fp contract(off)

namespace {

__global__ __launch_bounds__(256) void k_relu(const float* __restrict__ x, int64_t n, float* __restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) {
        const float v = x[i];
        y[i] = (0.0f < v) ? v : 0.0f;
    }
}

__global__ __launch_bounds__(256) void k_softmax(const float* __restrict__ x, int64_t outer, int64_t axis,
                                                 int64_t inner, float* __restrict__ y) {
    const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (r >= outer * inner) return;
    const int64_t o = r / inner, in = r % inner;
    const float* xp = x + o * axis * inner + in;
    float* yp = y + o * axis * inner + in;
    float mx = -INFINITY;
    for (int64_t a = 0; a < axis; ++a) {
        const float v = xp[a * inner];
        mx = (mx < v) ? v : mx;
    }
    const float uniform = 1.0f / (float)axis;
    if (isinf(mx) && mx < 0.0f) {
        for (int64_t a = 0; a < axis; ++a) yp[a * inner] = uniform;
        return;
    }
    float sum = 0.0f;
    for (int64_t a = 0; a < axis; ++a) {
        const float e = expf(xp[a * inner] - mx);
        yp[a * inner] = e;
        sum = sum + e;
    }
    if (sum == 0.0f) {
        for (int64_t a = 0; a < axis; ++a) yp[a * inner] = uniform;
        return;
    }
    for (int64_t a = 0; a < axis; ++a) yp[a * inner] = yp[a * inner] / sum;
}

void relu_dev(pfr_ctx* ctx, const float* x, int64_t n, float* y) {
    pfr::require(n >= 0, "negative element count");
    if (n == 0) return;
    pfr::require(x && y, "null x/y");
    hipLaunchKernelGGL(k_relu, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, ctx->stream, x, n, y);
    PFR_HIP(hipGetLastError());
}

void softmax_dev(pfr_ctx* ctx, const float* x, int64_t outer, int64_t axis, int64_t inner, float* y) {
    pfr::require(outer >= 0 && axis >= 0 && inner >= 0, "negative softmax extent");
    const int64_t rows = outer * inner;
    if (rows == 0 || axis == 0) return;
    pfr::require(x && y, "null x/y");
    hipLaunchKernelGGL(k_softmax, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, ctx->stream, x, outer, axis,
                       inner, y);
    PFR_HIP(hipGetLastError());
}

// Host-pointer form: stage, run, copy back, synchronise.
template <class F>
void host_call(pfr_ctx* ctx, const float* x, size_t n, float* y, F&& f) {
    if (n == 0) return;
    pfr::require(x && y, "null x/y");
    float* dx = static_cast<float*>(ctx->scratch[0].ensure(n * 4));
    float* dy = static_cast<float*>(ctx->scratch[2].ensure(n * 4));
    PFR_HIP(hipMemcpyAsync(dx, x, n * 4, hipMemcpyHostToDevice, ctx->stream));
    f(dx, dy);
    PFR_HIP(hipMemcpyAsync(y, dy, n * 4, hipMemcpyDeviceToHost, ctx->stream));
    PFR_HIP(hipStreamSynchronize(ctx->stream));
}

}  // namespace

extern "C" {

int pfr_relu_dev(pfr_ctx* ctx, const float* x, int64_t n, float* y) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        relu_dev(ctx, x, n, y);
    });
}

int pfr_relu(pfr_ctx* ctx, const float* x, int64_t n, float* y) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        pfr::require(n >= 0, "negative element count");
        host_call(ctx, x, (size_t)n, y, [&](float* dx, float* dy) { relu_dev(ctx, dx, n, dy); });
    });
}

int pfr_softmax_dev(pfr_ctx* ctx, const float* x, int64_t outer, int64_t axis, int64_t inner, float* y) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        softmax_dev(ctx, x, outer, axis, inner, y);
    });
}

int pfr_softmax(pfr_ctx* ctx, const float* x, int64_t outer, int64_t axis, int64_t inner, float* y) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        pfr::require(outer >= 0 && axis >= 0 && inner >= 0, "negative softmax extent");
        host_call(ctx, x, (size_t)(outer * axis * inner), y,
                  [&](float* dx, float* dy) { softmax_dev(ctx, dx, outer, axis, inner, dy); });
    });
}

}  // extern "C"
