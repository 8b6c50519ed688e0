// Dense float32 products for weights above the sparse path's density gate:
// the arithmetic of the reference's dense kernels, cpu_gemm and cpu_matmul
// (src/backends/cpu/ops/math.cpp:268-438), bit for bit.  Each output is
// summed in ascending k from +0 with a separate multiply and add per term,
// the term being (alpha * a[i, k]) * b[k, j] as the reference evaluates it,
// then beta * c[(i * N + j) % c_size] is added; the fused activation is the
// same function of that value as the separate Relu / Gelu kernels.  So
// non-finite inputs propagate exactly as there: an inf or NaN activation
// meets every weight, zeros included.
#include <algorithm>

#include "common.hpp"

namespace {

constexpr int kTM = 64, kTN = 64, kTK = 16;  // workgroup tile: 64 x 64 outputs, k in steps of 16

// 256 threads, each a 4 x 4 block of outputs (rows 4 * (t / 16) .., columns
// 4 * (t % 16) ..).  Per k step the op(A) and B tiles are staged in LDS
// (op(A) scaled by alpha on the way: the reference's alpha * a), then every
// output adds its 16 terms in k order.  Past K both tiles hold +0, whose
// terms (+0 * +0) leave every sum unchanged: a sum of products that starts
// at +0 is never -0 in round-to-nearest, and inf or NaN plus +0 is itself.
template <bool TA>
__global__ __launch_bounds__(256) void k_gemm_dense(const float* __restrict__ A, int64_t lda,
                                                    const float* __restrict__ B, int64_t ldb, int64_t M, int64_t N,
                                                    int64_t K, float alpha, int scale, const float* __restrict__ C,
                                                    int64_t c_size, float beta, int act, float* __restrict__ Y,
                                                    int64_t ldy) {
    __shared__ __align__(16) float As[kTK][kTM + 4];  // As[k][i]
    __shared__ __align__(16) float Bs[kTK][kTN + 4];  // Bs[k][j]
    const int tid = threadIdx.x, tx = tid % 16, ty = tid / 16;
    const int64_t i0 = (int64_t)blockIdx.y * kTM, j0 = (int64_t)blockIdx.x * kTN;
    float acc[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[r][c] = 0.0f;
    for (int64_t k0 = 0; k0 < K; k0 += kTK) {
#pragma unroll
        for (int e = tid; e < kTM * kTK; e += 256) {
            // op(A) = A (M x K, lda) or A^T (A is K x M, lda): consecutive
            // threads read consecutive addresses either way
            const int ii = TA ? e % kTM : e / kTK, kk = TA ? e / kTM : e % kTK;
            const int64_t gi = i0 + ii, gk = k0 + kk;
            float v = 0.0f;
            if (gi < M && gk < K) {
                v = TA ? A[gk * lda + gi] : A[gi * lda + gk];
                if (scale) v = alpha * v;
            }
            As[kk][ii] = v;
        }
#pragma unroll
        for (int e = tid; e < kTK * kTN; e += 256) {
            const int jj = e % kTN, kk = e / kTN;
            const int64_t gj = j0 + jj, gk = k0 + kk;
            Bs[kk][jj] = (gj < N && gk < K) ? B[gk * ldb + gj] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kTK; ++kk) {
            const float4 a = *reinterpret_cast<const float4*>(&As[kk][4 * ty]);
            const float4 b = *reinterpret_cast<const float4*>(&Bs[kk][4 * tx]);
            const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const float t = av[r] * bv[c];
                    acc[r][c] = acc[r][c] + t;
                }
        }
        __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int64_t i = i0 + 4 * ty + r;
        if (i >= M) continue;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int64_t j = j0 + 4 * tx + c;
            if (j < N) Y[i * ldy + j] = pfr::bias_add(acc[r][c], i * N + j, C, c_size, beta, act);
        }
    }
}

void gemm_dense_dev(pfr_ctx* ctx, const float* A, int64_t M, int64_t K, int transA, const float* B, int64_t N,
                    int64_t ldb, float alpha, float beta, const float* C, int64_t c_size, float* Y, int64_t ldy,
                    int act) {
    pfr::require(M >= 0 && K >= 0 && N >= 0, "negative dimension");
    pfr::require(ldb >= N && ldy >= N, "leading dimension smaller than N");
    pfr::require(act == PFR_ACT_NONE || act == PFR_ACT_RELU || act == PFR_ACT_GELU, "unknown activation");
    if (M == 0 || N == 0) return;
    pfr::require(Y != nullptr && ((A != nullptr && B != nullptr) || K == 0), "null A/B/Y");
    pfr::require((M + kTM - 1) / kTM < 65536, "too many rows for the dense product's grid");
    pfr::require((N + kTN - 1) / kTN < (int64_t(1) << 31), "too many columns for the dense product's grid");
    if (C == nullptr || c_size <= 0) {
        C = nullptr;
        c_size = 0;
    }
    const dim3 grid((unsigned)((N + kTN - 1) / kTN), (unsigned)((M + kTM - 1) / kTM));
    const int64_t lda = transA ? M : K;
    const int scale = alpha != 1.0f ? 1 : 0;
    if (transA)
        hipLaunchKernelGGL(k_gemm_dense<true>, grid, dim3(256), 0, ctx->stream, A, lda, B, ldb, M, N, K, alpha,
                           scale, C, c_size, beta, act, Y, ldy);
    else
        hipLaunchKernelGGL(k_gemm_dense<false>, grid, dim3(256), 0, ctx->stream, A, lda, B, ldb, M, N, K, alpha,
                           scale, C, c_size, beta, act, Y, ldy);
    PFR_HIP(hipGetLastError());
}

}  // namespace

extern "C" {

int pfr_gemm_dense_dev(pfr_ctx* ctx, const float* A, int64_t M, int64_t K, int transA, const float* B, int64_t N,
                       int64_t ldb, float alpha, float beta, const float* C, int64_t c_size, float* Y, int64_t ldy,
                       int act) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        gemm_dense_dev(ctx, A, M, K, transA, B, N, ldb, alpha, beta, C, c_size, Y, ldy, act);
    });
}

}  // extern "C"
