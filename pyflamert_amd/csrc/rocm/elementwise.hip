// Neighbours of the pruned MatMul/Gemm on the MLP and BERT-shaped graphs,
// so a device="rocm" session keeps every node on the GPU.
//   Relu       out = std::max(0.0f, x)  (activation.cpp:45-60): (0 < x) ? x : +0
//   Softmax    activation.cpp:157-237: max with std::max semantics (NaN never
//              replaces the running max), exp(x - max), sequential sum,
//              divide; all -inf (or zero sum) rows become uniform 1/n.  exp
//              is the device expf, so results match the CPU within a few
//              ulp, not bit for bit.
//   Gelu       activation.cpp:239-259 (pfr::gelu; device tanhf, a few ulp).
//   Add        math.cpp:150-224: numpy-style broadcasting, bit-exact.
//   LayerNorm  nn.cpp:419-490: per row a sequential mean and variance in one
//              thread (the reference's summation order), then
//              scale * (x - mean) * inv_std + bias; bit-exact.
#include <cmath>
#include <cstring>
#include <vector>

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

__global__ __launch_bounds__(256) void k_gelu(const float* __restrict__ x, int64_t n, float* __restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) y[i] = pfr::gelu(x[i]);
}

__global__ __launch_bounds__(256) void k_zero(int64_t n, float* __restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) y[i] = 0.0f;
}

// Broadcast iteration space: up to kAddDims output dimensions, innermost
// first, after size-1 dimensions are dropped and dimensions that both
// operands walk contiguously (or both broadcast) are merged.
constexpr int kAddDims = 8;
struct AddShape {
    int nd;
    int64_t out[kAddDims];
    int64_t sa[kAddDims];  // element stride of a along each dimension (0 when broadcast)
    int64_t sb[kAddDims];
};

template <int ND>
__global__ __launch_bounds__(256) void k_add(const float* __restrict__ a, const float* __restrict__ b, int64_t n,
                                             AddShape sh, float* __restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    int64_t ia, ib;
    if (ND == 1) {
        ia = i * sh.sa[0];
        ib = i * sh.sb[0];
    } else {
        int64_t rem = i;
        ia = 0;
        ib = 0;
#pragma unroll
        for (int d = 0; d < ND; ++d) {
            const int64_t idx = d == ND - 1 ? rem : rem % sh.out[d];
            rem /= sh.out[d];
            ia += idx * sh.sa[d];
            ib += idx * sh.sb[d];
        }
    }
    y[i] = a[ia] + b[ib];
}

// LayerNormalization with the rows staged in LDS: the block loads `rows`
// rows coalesced, one lane per row then runs the reference's sequential
// mean and variance over its LDS row (same operations in the same order as
// nn.cpp:457-470), and the whole block writes the normalised rows.  LDS:
// rows * stride floats (stride a multiple of 4, padded by 4 so the lanes'
// 16-byte reads fall in different banks), then the rows' means and inverse
// standard deviations.
constexpr int kLnThreads = 256;
constexpr int kLnLdsFloats = 16384;  // 64 KiB
__global__ __launch_bounds__(kLnThreads) void k_layernorm_lds(const float* __restrict__ x, int64_t outer, int norm,
                                                              int stride, int rpb, const float* __restrict__ scale,
                                                              const float* __restrict__ bias, float eps,
                                                              float* __restrict__ y) {
    extern __shared__ float lds[];
    float* stat = lds + rpb * stride;
    const int64_t r0 = (int64_t)blockIdx.x * rpb;
    const int rows = (int)(outer - r0 < rpb ? outer - r0 : rpb);
    for (int j = 0; j < rows; ++j) {
        const float* xr = x + (r0 + j) * norm;
        for (int i = threadIdx.x; i < norm; i += kLnThreads) lds[j * stride + i] = xr[i];
    }
    __syncthreads();
    if ((int)threadIdx.x < rows) {
        const float* row = lds + threadIdx.x * stride;
        // in element order, 32 at a time: the next 32 are read from LDS into
        // the other register set while the current 32 are added, so the
        // dependent adds do not wait on each read
        const int n32 = norm & ~31;
        auto rd = [&](int i, float4* v) {
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = *reinterpret_cast<const float4*>(row + i + 4 * k);
        };
        float4 va[8], vb[8];
        float mean = 0.0f;
        auto add_sum = [&](const float4* v) {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                mean = mean + v[k].x;
                mean = mean + v[k].y;
                mean = mean + v[k].z;
                mean = mean + v[k].w;
            }
        };
        if (n32) rd(0, va);
        for (int i = 0; i < n32; i += 64) {
            if (i + 32 < n32) rd(i + 32, vb);
            add_sum(va);
            if (i + 32 >= n32) break;
            if (i + 64 < n32) rd(i + 64, va);
            add_sum(vb);
        }
        for (int i = n32; i < norm; ++i) mean = mean + row[i];
        mean = mean / (float)norm;
        float var = 0.0f;
        auto add_var = [&](const float4* v) {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const float d0 = v[k].x - mean, d1 = v[k].y - mean, d2 = v[k].z - mean, d3 = v[k].w - mean;
                var = var + d0 * d0;
                var = var + d1 * d1;
                var = var + d2 * d2;
                var = var + d3 * d3;
            }
        };
        if (n32) rd(0, va);
        for (int i = 0; i < n32; i += 64) {
            if (i + 32 < n32) rd(i + 32, vb);
            add_var(va);
            if (i + 32 >= n32) break;
            if (i + 64 < n32) rd(i + 64, va);
            add_var(vb);
        }
        for (int i = n32; i < norm; ++i) {
            const float d = row[i] - mean;
            var = var + d * d;
        }
        var = var / (float)norm;
        stat[threadIdx.x] = mean;
        stat[rpb + threadIdx.x] = 1.0f / sqrtf(var + eps);
    }
    __syncthreads();
    for (int j = 0; j < rows; ++j) {
        const float mean = stat[j], inv_std = stat[rpb + j];
        float* yr = y + (r0 + j) * norm;
        for (int i = threadIdx.x; i < norm; i += kLnThreads)
            yr[i] = scale[i] * (lds[j * stride + i] - mean) * inv_std + bias[i];
    }
}

// One thread per row, straight from global memory: rows too long for LDS.
__global__ __launch_bounds__(64) void k_layernorm(const float* __restrict__ x, int64_t outer, int64_t norm,
                                                  const float* __restrict__ scale, const float* __restrict__ bias,
                                                  float eps, float* __restrict__ y) {
    const int64_t r = (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (r >= outer) return;
    const float* xr = x + r * norm;
    float mean = 0.0f;
    for (int64_t i = 0; i < norm; ++i) mean = mean + xr[i];
    mean = mean / (float)norm;
    float var = 0.0f;
    for (int64_t i = 0; i < norm; ++i) {
        const float d = xr[i] - mean;
        var = var + d * d;
    }
    var = var / (float)norm;
    const float inv_std = 1.0f / sqrtf(var + eps);
    float* yr = y + r * norm;
    for (int64_t i = 0; i < norm; ++i) yr[i] = scale[i] * (xr[i] - mean) * inv_std + bias[i];
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

void gelu_dev(pfr_ctx* ctx, const float* x, int64_t n, float* y) {
    pfr::require(n >= 0, "negative element count");
    if (n == 0) return;
    pfr::require(x && y, "null x/y");
    hipLaunchKernelGGL(k_gelu, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, ctx->stream, x, n, y);
    PFR_HIP(hipGetLastError());
}

// Output shape of a + b; throws the reference's text when not broadcastable.
// sh (optional) receives the coalesced iteration space.
std::vector<int64_t> add_shape(const int64_t* as, int an, const int64_t* bs, int bn, AddShape* sh) {
    pfr::require(an >= 0 && bn >= 0 && an <= kAddDims && bn <= kAddDims, "Add: at most 8 dimensions");
    const int nd = an > bn ? an : bn;
    std::vector<int64_t> out((size_t)nd);
    int64_t sa = 1, sb = 1;
    if (sh) sh->nd = 0;
    for (int k = nd - 1; k >= 0; --k) {  // innermost first
        const int64_t da = k - (nd - an) >= 0 ? as[k - (nd - an)] : 1;
        const int64_t db = k - (nd - bn) >= 0 ? bs[k - (nd - bn)] : 1;
        pfr::require(da >= 0 && db >= 0, "Add: negative dimension");
        if (da != db && da != 1 && db != 1) throw pfr::Error(PFR_ERR_INVALID_ARG, "Add: shapes are not broadcastable");
        const int64_t o = da > db ? da : db;  // math.cpp:54-64: 0 against 1 gives 1
        out[(size_t)k] = o;
        if (sh && o != 1) {
            const int64_t ea = da == 1 ? 0 : sa, eb = db == 1 ? 0 : sb;
            const int c = sh->nd - 1;
            if (c >= 0 && ea == sh->sa[c] * sh->out[c] && eb == sh->sb[c] * sh->out[c]) {
                sh->out[c] *= o;  // continues the inner dimension for both operands
            } else {
                sh->out[sh->nd] = o;
                sh->sa[sh->nd] = ea;
                sh->sb[sh->nd] = eb;
                ++sh->nd;
            }
        }
        sa *= da;
        sb *= db;
    }
    if (sh && sh->nd == 0) {  // a single element
        sh->nd = 1;
        sh->out[0] = 1;
        sh->sa[0] = sh->sb[0] = 0;
    }
    return out;
}

void add_dev(pfr_ctx* ctx, const float* a, const int64_t* as, int an, const float* b, const int64_t* bs, int bn,
             float* y) {
    AddShape sh;
    const std::vector<int64_t> out = add_shape(as, an, bs, bn, &sh);
    int64_t n = 1, na = 1, nb = 1;
    for (int64_t d : out) n *= d;
    for (int i = 0; i < an; ++i) na *= as[i];
    for (int i = 0; i < bn; ++i) nb *= bs[i];
    if (n == 0) return;
    pfr::require(y, "null y");
    if (na == 0 || nb == 0) {  // math.cpp:170-173: the new, zeroed output (tensor.cpp:47)
        hipLaunchKernelGGL(k_zero, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, ctx->stream, n, y);
        PFR_HIP(hipGetLastError());
        return;
    }
    pfr::require(a && b, "null a/b");
    const dim3 grid((unsigned)((n + 255) / 256));
    switch (sh.nd) {
#define PFR_ADD_CASE(D) \
    case D: hipLaunchKernelGGL(k_add<D>, grid, dim3(256), 0, ctx->stream, a, b, n, sh, y); break;
        PFR_ADD_CASE(1)
        PFR_ADD_CASE(2)
        PFR_ADD_CASE(3)
        PFR_ADD_CASE(4)
        PFR_ADD_CASE(5)
        PFR_ADD_CASE(6)
        PFR_ADD_CASE(7)
        PFR_ADD_CASE(8)
#undef PFR_ADD_CASE
        default: throw pfr::Error(PFR_ERR_UNSUPPORTED, "Add: bad iteration space");
    }
    PFR_HIP(hipGetLastError());
}

void layernorm_dev(pfr_ctx* ctx, const float* x, int64_t outer, int64_t norm, const float* scale,
                   const float* bias, float eps, float* y) {
    pfr::require(outer >= 0 && norm >= 0, "negative layer-norm extent");
    if (outer == 0 || norm == 0) return;
    pfr::require(x && scale && bias && y, "null x/scale/bias/y");
    const int64_t stride = ((norm + 3) & ~(int64_t)3) + 4;
    const int64_t fit = kLnLdsFloats / (stride + 2);  // rows whose staging fits the LDS budget
    if (fit >= 1) {
        // about 1024 rows in flight per launch: rows run their sequential
        // sums on as many SIMDs as possible
        int64_t rpb = (outer + 1023) / 1024;
        rpb = rpb < 1 ? 1 : (rpb > 16 ? 16 : rpb);
        rpb = rpb > fit ? fit : rpb;
        const int64_t blocks = (outer + rpb - 1) / rpb;
        pfr::require(blocks <= 0x7fffffff, "layer-norm row count too large");
        const size_t lds = (size_t)(rpb * stride + 2 * rpb) * sizeof(float);
        hipLaunchKernelGGL(k_layernorm_lds, dim3((unsigned)blocks), dim3(kLnThreads), lds, ctx->stream, x, outer,
                           (int)norm, (int)stride, (int)rpb, scale, bias, eps, y);
    } else {
        hipLaunchKernelGGL(k_layernorm, dim3((unsigned)((outer + 63) / 64)), dim3(64), 0, ctx->stream, x, outer,
                           norm, scale, bias, eps, y);
    }
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

int pfr_gelu_dev(pfr_ctx* ctx, const float* x, int64_t n, float* y) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        gelu_dev(ctx, x, n, y);
    });
}

int pfr_gelu(pfr_ctx* ctx, const float* x, int64_t n, float* y) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        pfr::require(n >= 0, "negative element count");
        host_call(ctx, x, (size_t)n, y, [&](float* dx, float* dy) { gelu_dev(ctx, dx, n, dy); });
    });
}

int pfr_add_dev(pfr_ctx* ctx, const float* a, const int64_t* a_shape, int a_ndim, const float* b,
                const int64_t* b_shape, int b_ndim, float* y) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        add_dev(ctx, a, a_shape, a_ndim, b, b_shape, b_ndim, y);
    });
}

int pfr_add(pfr_ctx* ctx, const float* a, const int64_t* a_shape, int a_ndim, const float* b, const int64_t* b_shape,
            int b_ndim, float* y) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        const std::vector<int64_t> out = add_shape(a_shape, a_ndim, b_shape, b_ndim, nullptr);
        int64_t n = 1, na = 1, nb = 1;
        for (int64_t d : out) n *= d;
        for (int i = 0; i < a_ndim; ++i) na *= a_shape[i];
        for (int i = 0; i < b_ndim; ++i) nb *= b_shape[i];
        if (n == 0) return;
        pfr::require(y, "null y");
        if (na == 0 || nb == 0) {  // math.cpp:170-173: the new, zeroed output (tensor.cpp:47)
            std::memset(y, 0, (size_t)n * 4);
            return;
        }
        pfr::require(a && b, "null a/b");
        float* da = static_cast<float*>(ctx->scratch[0].ensure((size_t)na * 4));
        float* db = static_cast<float*>(ctx->scratch[1].ensure((size_t)nb * 4));
        float* dy = static_cast<float*>(ctx->scratch[2].ensure((size_t)n * 4));
        PFR_HIP(hipMemcpyAsync(da, a, (size_t)na * 4, hipMemcpyHostToDevice, ctx->stream));
        PFR_HIP(hipMemcpyAsync(db, b, (size_t)nb * 4, hipMemcpyHostToDevice, ctx->stream));
        add_dev(ctx, da, a_shape, a_ndim, db, b_shape, b_ndim, dy);
        PFR_HIP(hipMemcpyAsync(y, dy, (size_t)n * 4, hipMemcpyDeviceToHost, ctx->stream));
        PFR_HIP(hipStreamSynchronize(ctx->stream));
    });
}

int pfr_layernorm_dev(pfr_ctx* ctx, const float* x, int64_t outer, int64_t norm, const float* scale,
                      const float* bias, float epsilon, float* y) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        layernorm_dev(ctx, x, outer, norm, scale, bias, epsilon, y);
    });
}

int pfr_layernorm(pfr_ctx* ctx, const float* x, int64_t outer, int64_t norm, const float* scale, const float* bias,
                  float epsilon, float* y) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        pfr::require(outer >= 0 && norm >= 0, "negative layer-norm extent");
        const size_t n = (size_t)(outer * norm);
        if (n == 0) return;
        pfr::require(x && scale && bias && y, "null x/scale/bias/y");
        float* dx = static_cast<float*>(ctx->scratch[0].ensure(n * 4));
        float* dp = static_cast<float*>(ctx->scratch[1].ensure((size_t)norm * 8));
        float* dy = static_cast<float*>(ctx->scratch[2].ensure(n * 4));
        PFR_HIP(hipMemcpyAsync(dx, x, n * 4, hipMemcpyHostToDevice, ctx->stream));
        PFR_HIP(hipMemcpyAsync(dp, scale, (size_t)norm * 4, hipMemcpyHostToDevice, ctx->stream));
        PFR_HIP(hipMemcpyAsync(dp + norm, bias, (size_t)norm * 4, hipMemcpyHostToDevice, ctx->stream));
        layernorm_dev(ctx, dx, outer, norm, dp, dp + norm, epsilon, dy);
        PFR_HIP(hipMemcpyAsync(y, dy, n * 4, hipMemcpyDeviceToHost, ctx->stream));
        PFR_HIP(hipStreamSynchronize(ctx->stream));
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
