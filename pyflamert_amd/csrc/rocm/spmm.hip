// CSR SpMM / SpMV for gfx950 and the Gemm-orientation wrapper.
//
// Strict mode reproduces the reference CPU kernels bit-for-bit: every output
// is the ascending-k sequence acc = RN(acc + RN(w * x)) from +0, with the
// bias added last as RN(acc + RN(beta * c)) (math.cpp:416-435,
// sparse_tensor.cpp:500-510 / :543-548).  The whole file is compiled with
// floating-point contraction off; fast mode asks for fmaf explicitly.
#include <algorithm>

#include "common.hpp"

#pragma clang fp contract(off)

namespace {

constexpr int kWaves = 4;  // waves per 256-thread workgroup
constexpr int kSpmvThreads = 512;  // threads of the vector kernel's workgroup
constexpr int kSpmvCap = 4096;     // products staged per workgroup chunk (16 KB)

template <bool FAST>
__device__ __forceinline__ float madd(float acc, float w, float x) {
    if constexpr (FAST) {
        return __builtin_fmaf(w, x, acc);
    } else {
        const float p = w * x;
        return acc + p;
    }
}

// Bias epilogue of cpu_gemm (math.cpp:431-433): out[f] += beta * c[f % c_size].
__device__ __forceinline__ float bias_add(float v, int64_t f, const float* __restrict__ bias,
                                          int64_t c_size, float beta) {
    if (bias == nullptr) return v;
    const float t = beta * bias[f % c_size];
    return v + t;
}

// One wave per CSR row, lanes across the N columns (4 per lane when VEC).
// Output element (row, c) goes to Y[row * ldy_r + c * ldy_c].
template <bool FAST, bool VEC>
__global__ __launch_bounds__(256) void k_spmm_rows(
    int M, int N, const int32_t* __restrict__ rowptr, const int32_t* __restrict__ col,
    const float* __restrict__ val, const float* __restrict__ X, int64_t ldx,
    float* __restrict__ Y, int64_t ldy_r, int64_t ldy_c, const float* __restrict__ bias,
    int64_t c_size, float beta) {
    const int lane = threadIdx.x & 63;
    const int row = __builtin_amdgcn_readfirstlane((int)blockIdx.x * kWaves + (int)(threadIdx.x >> 6));
    if (row >= M) return;
    const int beg = rowptr[row];
    const int end = rowptr[row + 1];
    if constexpr (VEC) {
        for (int c0 = lane * 4; c0 < N; c0 += 256) {
            float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
            const float* xc = X + c0;
            int j = beg;
            for (; j + 4 <= end; j += 4) {
                float4 x[4];
                float w[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    x[i] = *reinterpret_cast<const float4*>(xc + (int64_t)col[j + i] * ldx);
                    w[i] = val[j + i];
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    a0 = madd<FAST>(a0, w[i], x[i].x);
                    a1 = madd<FAST>(a1, w[i], x[i].y);
                    a2 = madd<FAST>(a2, w[i], x[i].z);
                    a3 = madd<FAST>(a3, w[i], x[i].w);
                }
            }
            for (; j < end; ++j) {
                const float w = val[j];
                const float4 x = *reinterpret_cast<const float4*>(xc + (int64_t)col[j] * ldx);
                a0 = madd<FAST>(a0, w, x.x);
                a1 = madd<FAST>(a1, w, x.y);
                a2 = madd<FAST>(a2, w, x.z);
                a3 = madd<FAST>(a3, w, x.w);
            }
            const int64_t f = (int64_t)row * ldy_r + c0;  // ldy_c == 1 here
            float4 o;
            o.x = bias_add(a0, f, bias, c_size, beta);
            o.y = bias_add(a1, f + 1, bias, c_size, beta);
            o.z = bias_add(a2, f + 2, bias, c_size, beta);
            o.w = bias_add(a3, f + 3, bias, c_size, beta);
            *reinterpret_cast<float4*>(Y + f) = o;
        }
    } else {
        for (int c = lane; c < N; c += 64) {
            float a = 0.0f;
#pragma unroll 4
            for (int j = beg; j < end; ++j) a = madd<FAST>(a, val[j], X[(int64_t)col[j] * ldx + c]);
            const int64_t f = (int64_t)row * ldy_r + (int64_t)c * ldy_c;
            Y[f] = bias_add(a, f, bias, c_size, beta);
        }
    }
}

// NP lanes per row (NP = next power of two >= N, N < 64), 64 / NP rows per wave.
template <int NP, bool FAST>
__global__ __launch_bounds__(256) void k_spmm_small(
    int M, int N, const int32_t* __restrict__ rowptr, const int32_t* __restrict__ col,
    const float* __restrict__ val, const float* __restrict__ X, int64_t ldx,
    float* __restrict__ Y, int64_t ldy_r, int64_t ldy_c, const float* __restrict__ bias,
    int64_t c_size, float beta) {
    constexpr int RPW = 64 / NP;
    const int lane = threadIdx.x & 63;
    const int g = lane / NP, c = lane % NP;
    const int row = ((int)blockIdx.x * kWaves + (int)(threadIdx.x >> 6)) * RPW + g;
    if (row >= M || c >= N) return;
    const int beg = rowptr[row];
    const int end = rowptr[row + 1];
    float a = 0.0f;
#pragma unroll 4
    for (int j = beg; j < end; ++j) a = madd<FAST>(a, val[j], X[(int64_t)col[j] * ldx + c]);
    const int64_t f = (int64_t)row * ldy_r + (int64_t)c * ldy_c;
    Y[f] = bias_add(a, f, bias, c_size, beta);
}

// SpMV.  One workgroup per row block (<= 64 rows, <= kSpmvCap nnz unless a
// single longer row).  All kSpmvThreads threads form the products
// RN(w * x[col]) over the block's contiguous nnz range with all loads in
// flight at once, staging them in LDS; then lane g of wave 0 folds the
// products of row r0 + g in storage order.  Longer blocks go in chunks.
__global__ __launch_bounds__(kSpmvThreads) void k_spmv_wg(
    const int32_t* __restrict__ blocks, const int32_t* __restrict__ rowptr,
    const int32_t* __restrict__ col, const float* __restrict__ val, const float* __restrict__ x,
    int64_t ldx, float* __restrict__ y, int64_t ldy_r, const float* __restrict__ bias,
    int64_t c_size, float beta) {
    __shared__ float P[kSpmvCap];
    constexpr int kPer = kSpmvCap / kSpmvThreads;
    const int tid = threadIdx.x;
    const int r0 = blocks[blockIdx.x];
    const int r1 = blocks[blockIdx.x + 1];
    const int nb = rowptr[r0];
    const int ne = rowptr[r1];
    const int my_row = r0 + tid;
    const bool folder = tid < 64 && my_row < r1;
    const int my_beg = folder ? rowptr[my_row] : 0;
    const int my_end = folder ? rowptr[my_row + 1] : 0;
    float acc = 0.0f;
    for (int base = nb; base < ne; base += kSpmvCap) {
        const int cend = min(base + kSpmvCap, ne);
        int cl[kPer];
        float w[kPer];
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int j = base + tid + i * kSpmvThreads;
            cl[i] = j < cend ? col[j] : 0;
            w[i] = j < cend ? val[j] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int j = base + tid + i * kSpmvThreads;
            if (j < cend) {
                const float xv = x[(int64_t)cl[i] * ldx];
                P[j - base] = w[i] * xv;
            }
        }
        __syncthreads();
        if (folder) {
            int p = max(my_beg, base) - base;
            const int e = min(my_end, cend) - base;
            for (; p + 8 <= e; p += 8) {
                float t[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) t[i] = P[p + i];
#pragma unroll
                for (int i = 0; i < 8; ++i) acc = acc + t[i];
            }
            for (; p < e; ++p) acc = acc + P[p];
        }
        __syncthreads();
    }
    if (folder) {
        const int64_t f = (int64_t)my_row * ldy_r;
        y[f] = bias_add(acc, f, bias, c_size, beta);
    }
}

// At[k, i] = RN(alpha * A[i, k]) for A rows x cols (At cols x rows).
__global__ __launch_bounds__(256) void k_transpose_scale(const float* __restrict__ A, int64_t rows,
                                                         int64_t cols, float alpha, int scale,
                                                         float* __restrict__ At) {
    __shared__ float tile[64][65];
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const int64_t c0 = (int64_t)blockIdx.x * 64, r0 = (int64_t)blockIdx.y * 64;
    for (int i = ty; i < 64; i += 4) {
        const int64_t r = r0 + i, c = c0 + tx;
        if (r < rows && c < cols) {
            const float v = A[r * cols + c];
            tile[i][tx] = scale ? alpha * v : v;
        }
    }
    __syncthreads();
    for (int i = ty; i < 64; i += 4) {
        const int64_t c = c0 + i, r = r0 + tx;
        if (c < cols && r < rows) At[c * rows + r] = tile[tx][i];
    }
}

__global__ __launch_bounds__(256) void k_scale(const float* __restrict__ A, int64_t n, float alpha,
                                               float* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = alpha * A[i];
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int next_pow2(int n) {
    int p = 1;
    while (p < n) p <<= 1;
    return p;
}


// Launch the kernel that fits N.  Output (row, c) -> Y[row*ldy_r + c*ldy_c].
void launch_spmm(pfr_ctx* ctx, const pfr_csr* W, const float* X, int64_t N, int64_t ldx, float* Y,
                 int64_t ldy_r, int64_t ldy_c, const float* bias, int64_t c_size, float beta,
                 bool fast) {
    const int M = (int)W->M;
    if (M == 0 || N == 0) return;
    const float* val = static_cast<const float*>(W->val);
    hipStream_t s = ctx->stream;
    if (N == 1) {
        hipLaunchKernelGGL(k_spmv_wg, dim3((unsigned)W->n_spmv_blocks), dim3(kSpmvThreads), 0, s,
                           W->spmv_blocks, W->rowptr, W->col, val, X, ldx, Y, ldy_r, bias, c_size,
                           beta);
    } else if (N < 64) {
        const int np = next_pow2((int)N);
        const int rows_per_block = kWaves * (64 / np);
        const unsigned grid = (unsigned)((M + rows_per_block - 1) / rows_per_block);
#define PFR_SMALL(NPV)                                                                          \
    case NPV:                                                                                   \
        if (fast)                                                                               \
            hipLaunchKernelGGL((k_spmm_small<NPV, true>), dim3(grid), dim3(256), 0, s, M, (int)N, \
                               W->rowptr, W->col, val, X, ldx, Y, ldy_r, ldy_c, bias, c_size, beta); \
        else                                                                                    \
            hipLaunchKernelGGL((k_spmm_small<NPV, false>), dim3(grid), dim3(256), 0, s, M, (int)N,\
                               W->rowptr, W->col, val, X, ldx, Y, ldy_r, ldy_c, bias, c_size, beta); \
        break;
        switch (np) {
            PFR_SMALL(2)
            PFR_SMALL(4)
            PFR_SMALL(8)
            PFR_SMALL(16)
            PFR_SMALL(32)
            PFR_SMALL(64)
            default:
                throw pfr::Error(PFR_ERR_UNSUPPORTED, "unexpected column count");
        }
#undef PFR_SMALL
    } else {
        const unsigned grid = (unsigned)((M + kWaves - 1) / kWaves);
        const bool vec = (N % 4 == 0) && (ldx % 4 == 0) && ldy_c == 1 && (ldy_r % 4 == 0) &&
                         aligned16(X) && aligned16(Y);
        if (vec) {
            if (fast)
                hipLaunchKernelGGL((k_spmm_rows<true, true>), dim3(grid), dim3(256), 0, s, M, (int)N,
                                   W->rowptr, W->col, val, X, ldx, Y, ldy_r, ldy_c, bias, c_size, beta);
            else
                hipLaunchKernelGGL((k_spmm_rows<false, true>), dim3(grid), dim3(256), 0, s, M, (int)N,
                                   W->rowptr, W->col, val, X, ldx, Y, ldy_r, ldy_c, bias, c_size, beta);
        } else {
            if (fast)
                hipLaunchKernelGGL((k_spmm_rows<true, false>), dim3(grid), dim3(256), 0, s, M, (int)N,
                                   W->rowptr, W->col, val, X, ldx, Y, ldy_r, ldy_c, bias, c_size, beta);
            else
                hipLaunchKernelGGL((k_spmm_rows<false, false>), dim3(grid), dim3(256), 0, s, M, (int)N,
                                   W->rowptr, W->col, val, X, ldx, Y, ldy_r, ldy_c, bias, c_size, beta);
        }
    }
    PFR_HIP(hipGetLastError());
}

void check_csr(const pfr_csr* W) {
    pfr::require(W != nullptr, "null CSR handle");
    if (W->vdt != PFR_F32)
        throw pfr::Error(PFR_ERR_UNSUPPORTED, "this entry point takes float32 CSR values");
}

void spmm_dev(pfr_ctx* ctx, const pfr_csr* W, const float* X, int64_t N, int64_t ldx, float* Y,
              int64_t ldy, int mode) {
    check_csr(W);
    pfr::require(N >= 0 && N < INT32_MAX, "bad column count");
    pfr::require(ldx >= N && ldy >= N, "leading dimension smaller than N");
    pfr::require(mode == PFR_MODE_STRICT || mode == PFR_MODE_FAST, "unknown mode");
    pfr::require((X && Y) || W->M * N == 0, "null X/Y");
    launch_spmm(ctx, W, X, N, ldx, Y, ldy, 1, nullptr, 0, 0.0f, mode == PFR_MODE_FAST);
}

void gemm_dev(pfr_ctx* ctx, const float* A, int64_t Mb, int64_t K, int transA, const pfr_csr* BT,
              float alpha, float beta, const float* C, int64_t c_size, float* Y, int mode) {
    check_csr(BT);
    pfr::require(Mb >= 0 && Mb < INT32_MAX, "bad row count");
    pfr::require(BT->K == K, "Gemm: incompatible dimensions - A has K=" + std::to_string(K) +
                                 ", B has K=" + std::to_string(BT->K));
    pfr::require(mode == PFR_MODE_STRICT || mode == PFR_MODE_FAST, "unknown mode");
    const int64_t Nf = BT->M;
    if (Mb == 0 || Nf == 0) return;
    pfr::require(A != nullptr && Y != nullptr, "null A/Y");
    if (C == nullptr || c_size <= 0) {
        C = nullptr;
        c_size = 0;
    }
    // At = op(A)^T scaled by alpha: K x Mb, so each k row is contiguous.
    const float* At = A;
    hipStream_t s = ctx->stream;
    if (K == 0) {
        // No terms: every output is +0 (+ bias); At is never read.
    } else if (!transA) {
        float* t = static_cast<float*>(ctx->scratch[3].ensure(sizeof(float) * (size_t)(K * Mb)));
        dim3 grid((unsigned)((K + 63) / 64), (unsigned)((Mb + 63) / 64));
        pfr::require(grid.y < 65536u, "activation too tall for the transpose grid");
        hipLaunchKernelGGL(k_transpose_scale, grid, dim3(256), 0, s, A, Mb, K, alpha,
                           alpha != 1.0f ? 1 : 0, t);
        PFR_HIP(hipGetLastError());
        At = t;
    } else if (alpha != 1.0f) {
        float* t = static_cast<float*>(ctx->scratch[3].ensure(sizeof(float) * (size_t)(K * Mb)));
        const int64_t n = K * Mb;
        hipLaunchKernelGGL(k_scale, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, A, n, alpha, t);
        PFR_HIP(hipGetLastError());
        At = t;
    }
    // Output (feature j, batch i) -> Y[i * Nf + j]: the flat index the bias
    // modulo uses in cpu_gemm.
    launch_spmm(ctx, BT, At, Mb, Mb, Y, 1, Nf, C, c_size, beta, mode == PFR_MODE_FAST);
}

}  // namespace

extern "C" {

int pfr_spmm_csr_dev(pfr_ctx* ctx, const pfr_csr* W, const float* X, int64_t N, int64_t ldx,
                     float* Y, int64_t ldy, int mode) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        spmm_dev(ctx, W, X, N, ldx, Y, ldy, mode);
    });
}

int pfr_spmm_csr(pfr_ctx* ctx, const pfr_csr* W, const float* X, int64_t N, float* Y, int mode) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        check_csr(W);
        pfr::require(N >= 0, "bad column count");
        const size_t xb = sizeof(float) * (size_t)(W->K * N), yb = sizeof(float) * (size_t)(W->M * N);
        if (yb == 0) return;
        pfr::require(Y != nullptr && (X != nullptr || xb == 0), "null X/Y");
        hipStream_t s = ctx->stream;
        float* dX = static_cast<float*>(ctx->scratch[0].ensure(xb));
        float* dY = static_cast<float*>(ctx->scratch[2].ensure(yb));
        if (xb) PFR_HIP(hipMemcpyAsync(dX, X, xb, hipMemcpyHostToDevice, s));
        spmm_dev(ctx, W, dX, N, N, dY, N, mode);
        PFR_HIP(hipMemcpyAsync(Y, dY, yb, hipMemcpyDeviceToHost, s));
        PFR_HIP(hipStreamSynchronize(s));
    });
}

int pfr_gemm_csr_dev(pfr_ctx* ctx, const float* A, int64_t Mb, int64_t K, int transA,
                     const pfr_csr* BT, float alpha, float beta, const float* C, int64_t c_size,
                     float* Y, int mode) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        gemm_dev(ctx, A, Mb, K, transA, BT, alpha, beta, C, c_size, Y, mode);
    });
}

int pfr_gemm_csr(pfr_ctx* ctx, const float* A, int64_t Mb, int64_t K, int transA,
                 const pfr_csr* BT, float alpha, float beta, const float* C, int64_t c_size,
                 float* Y, int mode) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        check_csr(BT);
        pfr::require(Mb >= 0 && K >= 0, "negative dimension");
        const size_t ab = sizeof(float) * (size_t)(Mb * K);
        const size_t yb = sizeof(float) * (size_t)(Mb * BT->M);
        if (yb == 0) return;
        pfr::require(Y != nullptr && (A != nullptr || ab == 0), "null A/Y");
        hipStream_t s = ctx->stream;
        float* dA = static_cast<float*>(ctx->scratch[0].ensure(ab ? ab : 4));
        float* dC = nullptr;
        if (C && c_size > 0) {
            dC = static_cast<float*>(ctx->scratch[1].ensure(sizeof(float) * (size_t)c_size));
            PFR_HIP(hipMemcpyAsync(dC, C, sizeof(float) * (size_t)c_size, hipMemcpyHostToDevice, s));
        }
        float* dY = static_cast<float*>(ctx->scratch[2].ensure(yb));
        if (ab) PFR_HIP(hipMemcpyAsync(dA, A, ab, hipMemcpyHostToDevice, s));
        gemm_dev(ctx, dA, Mb, K, transA, BT, alpha, beta, dC, dC ? c_size : 0, dY, mode);
        PFR_HIP(hipMemcpyAsync(Y, dY, yb, hipMemcpyDeviceToHost, s));
        PFR_HIP(hipStreamSynchronize(s));
    });
}

}  // extern "C"
