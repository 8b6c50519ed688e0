// 2:4 structured-sparse GEMM on gfx950 sparse MFMA (smfmac).
//
// Operand layouts (per lane l of a wave, established on the device with
// exact-integer tests of the builtins):
//   v_smfmac_i32_16x16x128_i8   A: row l%16, dense K [32*(l/16), +32) as 8
//                               groups of 4, two kept bytes per group
//                               (16 B), 2-bit positions in bits [2e, 2e+2)
//                               of the index VGPR;  B: column l%16, bytes
//                               0..15 = k 16*(l/16)+b, bytes 16..31 =
//                               k 64+16*(l/16)+(b-16);  D: column l%16,
//                               rows 4*(l/16)+i.
//   v_smfmac_f32_16x16x64_bf16  A: row l%16, dense K [16*(l/16), +16) as 4
//                               groups (8 bf16), 16 index bits selected by
//                               abid;  B: column l%16, elements 0..7 =
//                               k 8*(l/16)+e, 8..15 = k 32+8*(l/16)+(e-8).
// The weight is packed once, on the host, into that register order, so each
// lane fetches its A operand with one 16-byte load.
#include <cmath>
#include <vector>

#include "common.hpp"

#pragma clang fp contract(off)

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v16bf __attribute__((ext_vector_type(16)));

struct pfr_sp24 {
    pfr_ctx* ctx = nullptr;
    int64_t M = 0, K = 0;
    int64_t Mp = 0, Kp = 0;  // padded: Mp % 128 == 0, Kp % 128 == 0
    pfr_dtype dtype = PFR_I8;
    void* a = nullptr;        // compressed values, [Mp/16][Kp/KT][64][16 B]
    uint32_t* idx = nullptr;  // [Mp/16][Kp/KT (int8) | Kp/128 (bf16)][64]
    float* w_scale = nullptr; // [M] (per-tensor scales expanded)
};

namespace {

constexpr int kTileM = 128;  // rows per workgroup (4 waves x 32)
constexpr int kTileN = 64;   // columns per workgroup

int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

void free_sp24(pfr_sp24* w) {
    if (!w) return;
    for (void* p : {w->a, (void*)w->idx, (void*)w->w_scale})
        if (p) (void)hipFree(p);
    delete w;
}

// Choose the two kept positions of a 4-group (ascending, as the index
// encoding expects), or report more than two nonzeros.
template <class IsNz>
bool pick2(IsNz nz, int* p0, int* p1) {
    int pos[4], n = 0;
    for (int i = 0; i < 4; ++i)
        if (nz(i)) pos[n++] = i;
    if (n > 2) return false;
    if (n == 2) { *p0 = pos[0]; *p1 = pos[1]; return true; }
    if (n == 1) {
        const int p = pos[0];
        const int q = (p == 0) ? 1 : 0;
        *p0 = p < q ? p : q;
        *p1 = p < q ? q : p;
        return true;
    }
    *p0 = 0;
    *p1 = 1;
    return true;
}

// ---- kernels ----------------------------------------------------------------

// XT[n][k] (Np x Kp, zero padded) = X[k][n] (K x N, row stride ldx).
template <class T>
__global__ __launch_bounds__(256) void k_transpose_pad(const T* __restrict__ X, int64_t K, int64_t N,
                                                       int64_t ldx, T* __restrict__ XT, int64_t Kp) {
    __shared__ T tile[64][65];
    const int t = threadIdx.x;
    const int64_t k0 = (int64_t)blockIdx.x * 64, n0 = (int64_t)blockIdx.y * 64;
    for (int i = 0; i < 16; ++i) {
        const int kk = (t >> 6) + 4 * i, nn = t & 63;
        const int64_t k = k0 + kk, n = n0 + nn;
        tile[kk][nn] = (k < K && n < N) ? X[k * ldx + n] : T(0);
    }
    __syncthreads();
    for (int i = 0; i < 16; ++i) {
        const int nn = (t >> 6) + 4 * i, kk = t & 63;
        XT[(n0 + nn) * Kp + k0 + kk] = tile[kk][nn];
    }
}

// x86 static_cast<int32_t>(float): truncation, 0x80000000 for NaN / out of
// range (what the reference's requant does on its build target).
__device__ __forceinline__ int32_t f2i_trunc_x86(float r) {
    return (r >= -2147483648.0f && r < 2147483648.0f) ? (int32_t)r : INT32_MIN;
}

// One wave computes 32 rows x 64 columns (2 x 4 tiles of 16x16); four waves
// stack along M.  Operands come straight from global memory (A packed, B from
// the transposed activation).
template <int OUT>
__global__ __launch_bounds__(256) void k_sp24_i8(
    int nkt, const v4i* __restrict__ A, const uint32_t* __restrict__ I,
    const int8_t* __restrict__ XT, int64_t Kp, int M, int N, const float* __restrict__ sab,
    float inv_out, int32_t out_zp, void* __restrict__ Y, int64_t ldy) {
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int mt0 = (int)blockIdx.x * (kTileM / 16) + 2 * w;
    const int nt0 = (int)blockIdx.y * (kTileN / 16);
    const int kb = l >> 4, c = l & 15;
    v4i acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = v4i{0, 0, 0, 0};
    const v4i* a0p = A + ((int64_t)mt0 * nkt) * 64 + l;
    const v4i* a1p = A + ((int64_t)(mt0 + 1) * nkt) * 64 + l;
    const uint32_t* i0p = I + ((int64_t)mt0 * nkt) * 64 + l;
    const uint32_t* i1p = I + ((int64_t)(mt0 + 1) * nkt) * 64 + l;
    const int8_t* xb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) xb[j] = XT + (int64_t)((nt0 + j) * 16 + c) * Kp + 16 * kb;
    for (int kt = 0; kt < nkt; ++kt) {
        const v4i a0 = a0p[(int64_t)kt * 64], a1 = a1p[(int64_t)kt * 64];
        const int ix0 = (int)i0p[(int64_t)kt * 64], ix1 = (int)i1p[(int64_t)kt * 64];
        v8i b[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const v4i lo = *reinterpret_cast<const v4i*>(xb[j] + (int64_t)kt * 128);
            const v4i hi = *reinterpret_cast<const v4i*>(xb[j] + (int64_t)kt * 128 + 64);
            b[j] = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc[0][j] = __builtin_amdgcn_smfmac_i32_16x16x128_i8(a0, b[j], acc[0][j], ix0, 0, 0);
            acc[1][j] = __builtin_amdgcn_smfmac_i32_16x16x128_i8(a1, b[j], acc[1][j], ix1, 0, 0);
        }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = (nt0 + j) * 16 + c;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = (mt0 + i) * 16 + 4 * kb + r;
                if (m >= M || n >= N) continue;
                const int32_t v = acc[i][j][r];
                const int64_t o = (int64_t)m * ldy + n;
                if constexpr (OUT == PFR_SP24_OUT_I32) {
                    static_cast<int32_t*>(Y)[o] = v;
                } else {
                    const float f = (float)v * sab[m];
                    if constexpr (OUT == PFR_SP24_OUT_F32) {
                        static_cast<float*>(Y)[o] = f;
                    } else {
                        const float prod = f * inv_out;
                        int32_t q = (int32_t)((uint32_t)f2i_trunc_x86(roundf(prod)) + (uint32_t)out_zp);
                        q = q < -128 ? -128 : (q > 127 ? 127 : q);
                        static_cast<int8_t*>(Y)[o] = (int8_t)q;
                    }
                }
            }
        }
    }
}

// bf16: 16x16x64 tiles, index words hold two k-tiles (abid 0 / 1).
__global__ __launch_bounds__(256) void k_sp24_bf16(
    int nkt, const v4i* __restrict__ A, const uint32_t* __restrict__ I,
    const uint16_t* __restrict__ XT, int64_t Kp, int M, int N, float* __restrict__ Y, int64_t ldy) {
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int mt0 = (int)blockIdx.x * (kTileM / 16) + 2 * w;
    const int nt0 = (int)blockIdx.y * (kTileN / 16);
    const int kb = l >> 4, c = l & 15;
    v4f acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
    const int nkp = nkt / 2;  // index words per row tile
    const v4i* a0p = A + ((int64_t)mt0 * nkt) * 64 + l;
    const v4i* a1p = A + ((int64_t)(mt0 + 1) * nkt) * 64 + l;
    const uint32_t* i0p = I + ((int64_t)mt0 * nkp) * 64 + l;
    const uint32_t* i1p = I + ((int64_t)(mt0 + 1) * nkp) * 64 + l;
    const uint16_t* xb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) xb[j] = XT + (int64_t)((nt0 + j) * 16 + c) * Kp + 8 * kb;
    for (int kp = 0; kp < nkp; ++kp) {
        const int ix0 = (int)i0p[(int64_t)kp * 64], ix1 = (int)i1p[(int64_t)kp * 64];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int kt = 2 * kp + h;
            const v8bf a0 = __builtin_bit_cast(v8bf, a0p[(int64_t)kt * 64]);
            const v8bf a1 = __builtin_bit_cast(v8bf, a1p[(int64_t)kt * 64]);
            v16bf b[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const v4i lo = *reinterpret_cast<const v4i*>(xb[j] + (int64_t)kt * 64);
                const v4i hi = *reinterpret_cast<const v4i*>(xb[j] + (int64_t)kt * 64 + 32);
                b[j] = __builtin_bit_cast(v16bf, v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w});
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (h == 0) {
                    acc[0][j] = __builtin_amdgcn_smfmac_f32_16x16x64_bf16(a0, b[j], acc[0][j], ix0, 0, 0);
                    acc[1][j] = __builtin_amdgcn_smfmac_f32_16x16x64_bf16(a1, b[j], acc[1][j], ix1, 0, 0);
                } else {
                    acc[0][j] = __builtin_amdgcn_smfmac_f32_16x16x64_bf16(a0, b[j], acc[0][j], ix0, 0, 1);
                    acc[1][j] = __builtin_amdgcn_smfmac_f32_16x16x64_bf16(a1, b[j], acc[1][j], ix1, 0, 1);
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = (nt0 + j) * 16 + c;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = (mt0 + i) * 16 + 4 * kb + r;
                if (m < M && n < N) Y[(int64_t)m * ldy + n] = acc[i][j][r];
            }
        }
}

// s_ab[m] = w_scale[m] * x_scale, one rounding as on the host (quant_ops.cpp:435).
__global__ __launch_bounds__(256) void k_scale_rows(const float* __restrict__ ws, float xs, int64_t M,
                                                    float* __restrict__ out) {
    const int64_t m = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (m < M) out[m] = ws[m] * xs;
}

// ---- host -----------------------------------------------------------------

pfr_sp24* pack_i8(pfr_ctx* ctx, int64_t M, int64_t K, const int8_t* W) {
    const int64_t Mp = round_up(M, kTileM), Kp = round_up(K, 128), nkt = Kp / 128;
    std::vector<int8_t> a((size_t)(Mp / 16 * nkt * 64 * 16), 0);
    std::vector<uint32_t> ix((size_t)(Mp / 16 * nkt * 64), 0);
    auto wat = [&](int64_t r, int64_t k) -> int8_t { return (r < M && k < K) ? W[r * K + k] : 0; };
    for (int64_t r = 0; r < M; ++r)
        for (int64_t g = 0; g < Kp / 4; ++g) {
            int p0, p1;
            if (!pick2([&](int i) { return wat(r, 4 * g + i) != 0; }, &p0, &p1))
                throw pfr::Error(PFR_ERR_INVALID_ARG,
                                 "weight is not 2:4 sparse: row " + std::to_string(r) + ", k " +
                                     std::to_string(4 * g) + ".." + std::to_string(4 * g + 3) +
                                     " has more than two nonzeros");
            (void)p0;
            (void)p1;
        }
    for (int64_t mt = 0; mt < Mp / 16; ++mt)
        for (int64_t kt = 0; kt < nkt; ++kt)
            for (int l = 0; l < 64; ++l) {
                const int64_t r = mt * 16 + (l & 15);
                const int kb = l >> 4;
                const size_t base = (size_t)(((mt * nkt + kt) * 64 + l));
                uint32_t word = 0;
                for (int g = 0; g < 8; ++g) {
                    const int64_t ks = kt * 128 + 32 * kb + 4 * g;
                    int p0 = 0, p1 = 1;
                    pick2([&](int i) { return wat(r, ks + i) != 0; }, &p0, &p1);
                    a[base * 16 + 2 * g] = wat(r, ks + p0);
                    a[base * 16 + 2 * g + 1] = wat(r, ks + p1);
                    word |= (uint32_t)(p0 | (p1 << 2)) << (4 * g);
                }
                ix[base] = word;
            }
    auto* w = new pfr_sp24();
    try {
        w->ctx = ctx;
        w->M = M;
        w->K = K;
        w->Mp = Mp;
        w->Kp = Kp;
        w->dtype = PFR_I8;
        PFR_HIP(hipMalloc(&w->a, a.size()));
        PFR_HIP(hipMalloc(&w->idx, ix.size() * 4));
        PFR_HIP(hipMemcpy(w->a, a.data(), a.size(), hipMemcpyHostToDevice));
        PFR_HIP(hipMemcpy(w->idx, ix.data(), ix.size() * 4, hipMemcpyHostToDevice));
        return w;
    } catch (...) {
        free_sp24(w);
        throw;
    }
}

bool bf16_nz(uint16_t b) { return (b & 0x7FFF) != 0; }

pfr_sp24* pack_bf16(pfr_ctx* ctx, int64_t M, int64_t K, const uint16_t* W) {
    const int64_t Mp = round_up(M, kTileM), Kp = round_up(K, 128), nkt = Kp / 64, nkp = nkt / 2;
    std::vector<uint16_t> a((size_t)(Mp / 16 * nkt * 64 * 8), 0);
    std::vector<uint32_t> ix((size_t)(Mp / 16 * nkp * 64), 0);
    auto wat = [&](int64_t r, int64_t k) -> uint16_t { return (r < M && k < K) ? W[r * K + k] : 0; };
    for (int64_t r = 0; r < M; ++r)
        for (int64_t g = 0; g < Kp / 4; ++g) {
            int p0, p1;
            if (!pick2([&](int i) { return bf16_nz(wat(r, 4 * g + i)); }, &p0, &p1))
                throw pfr::Error(PFR_ERR_INVALID_ARG,
                                 "weight is not 2:4 sparse: row " + std::to_string(r) + ", k " +
                                     std::to_string(4 * g) + ".." + std::to_string(4 * g + 3) +
                                     " has more than two nonzeros");
        }
    for (int64_t mt = 0; mt < Mp / 16; ++mt)
        for (int64_t kt = 0; kt < nkt; ++kt)
            for (int l = 0; l < 64; ++l) {
                const int64_t r = mt * 16 + (l & 15);
                const int kb = l >> 4;
                const size_t base = (size_t)((mt * nkt + kt) * 64 + l);
                uint32_t half = 0;
                for (int g = 0; g < 4; ++g) {
                    const int64_t ks = kt * 64 + 16 * kb + 4 * g;
                    int p0 = 0, p1 = 1;
                    pick2([&](int i) { return bf16_nz(wat(r, ks + i)); }, &p0, &p1);
                    a[base * 8 + 2 * g] = wat(r, ks + p0);
                    a[base * 8 + 2 * g + 1] = wat(r, ks + p1);
                    half |= (uint32_t)(p0 | (p1 << 2)) << (4 * g);
                }
                ix[(size_t)((mt * nkp + kt / 2) * 64 + l)] |= half << (16 * (kt & 1));
            }
    auto* w = new pfr_sp24();
    try {
        w->ctx = ctx;
        w->M = M;
        w->K = K;
        w->Mp = Mp;
        w->Kp = Kp;
        w->dtype = PFR_BF16;
        PFR_HIP(hipMalloc(&w->a, a.size() * 2));
        PFR_HIP(hipMalloc(&w->idx, ix.size() * 4));
        PFR_HIP(hipMemcpy(w->a, a.data(), a.size() * 2, hipMemcpyHostToDevice));
        PFR_HIP(hipMemcpy(w->idx, ix.data(), ix.size() * 4, hipMemcpyHostToDevice));
        return w;
    } catch (...) {
        free_sp24(w);
        throw;
    }
}

void check_i8(const pfr_sp24* W) {
    pfr::require(W != nullptr, "null 2:4 weight handle");
    if (W->dtype != PFR_I8) throw pfr::Error(PFR_ERR_UNSUPPORTED, "weight is not int8");
}

// XT for the activation: int8 or bf16 bits, Np x Kp.
template <class T>
T* stage_xt(pfr_ctx* ctx, const T* X, int64_t K, int64_t N, int64_t ldx, int64_t Kp, int64_t Np) {
    T* xt = static_cast<T*>(ctx->scratch[3].ensure(sizeof(T) * (size_t)(Np * Kp)));
    dim3 grid((unsigned)(Kp / 64), (unsigned)(Np / 64));
    hipLaunchKernelGGL(k_transpose_pad<T>, grid, dim3(256), 0, ctx->stream, X, K, N, ldx, xt, Kp);
    PFR_HIP(hipGetLastError());
    return xt;
}

void gemm_i8_dev(pfr_ctx* ctx, const pfr_sp24* W, const int8_t* X, int64_t N, int64_t ldx, float x_scale,
                 int out_kind, float out_scale, int32_t out_zp, void* Y, int64_t ldy) {
    check_i8(W);
    pfr::require(N >= 0 && N < INT32_MAX, "bad column count");
    pfr::require(ldx >= N && ldy >= N, "leading dimension smaller than N");
    pfr::require(out_kind >= PFR_SP24_OUT_I32 && out_kind <= PFR_SP24_OUT_I8, "unknown output kind");
    if (W->M == 0 || N == 0) return;
    pfr::require(X != nullptr && Y != nullptr, "null X/Y");
    float inv_out = 1.0f;
    const float* sab = nullptr;
    if (out_kind != PFR_SP24_OUT_I32) {
        pfr::require(x_scale > 0.0f && std::isfinite(x_scale), "x_scale must be positive and finite");
        // s_ab[m] = a_scale * b_scale with a = the weight (quant_ops.cpp:435).
        float* d = static_cast<float*>(ctx->scratch[1].ensure(sizeof(float) * (size_t)W->M));
        hipLaunchKernelGGL(k_scale_rows, dim3((unsigned)((W->M + 255) / 256)), dim3(256), 0, ctx->stream,
                           W->w_scale, x_scale, W->M, d);
        PFR_HIP(hipGetLastError());
        sab = d;
    }
    if (out_kind == PFR_SP24_OUT_I8) {
        pfr::require(out_scale > 0.0f && std::isfinite(out_scale), "output scale must be positive and finite");
        inv_out = 1.0f / out_scale;  // quant_ops.cpp:41
    }
    const int64_t Np = round_up(N, kTileN);
    const int8_t* xt = stage_xt(ctx, X, W->K, N, ldx, W->Kp, Np);
    dim3 grid((unsigned)(W->Mp / kTileM), (unsigned)(Np / kTileN));
    const int nkt = (int)(W->Kp / 128);
    const v4i* A = static_cast<const v4i*>(W->a);
    switch (out_kind) {
        case PFR_SP24_OUT_I32:
            hipLaunchKernelGGL(k_sp24_i8<PFR_SP24_OUT_I32>, grid, dim3(256), 0, ctx->stream, nkt, A, W->idx, xt,
                               W->Kp, (int)W->M, (int)N, sab, inv_out, out_zp, Y, ldy);
            break;
        case PFR_SP24_OUT_F32:
            hipLaunchKernelGGL(k_sp24_i8<PFR_SP24_OUT_F32>, grid, dim3(256), 0, ctx->stream, nkt, A, W->idx, xt,
                               W->Kp, (int)W->M, (int)N, sab, inv_out, out_zp, Y, ldy);
            break;
        default:
            hipLaunchKernelGGL(k_sp24_i8<PFR_SP24_OUT_I8>, grid, dim3(256), 0, ctx->stream, nkt, A, W->idx, xt,
                               W->Kp, (int)W->M, (int)N, sab, inv_out, out_zp, Y, ldy);
    }
    PFR_HIP(hipGetLastError());
}

void gemm_bf16_dev(pfr_ctx* ctx, const pfr_sp24* W, const uint16_t* X, int64_t N, int64_t ldx, float* Y,
                   int64_t ldy) {
    pfr::require(W != nullptr, "null 2:4 weight handle");
    if (W->dtype != PFR_BF16) throw pfr::Error(PFR_ERR_UNSUPPORTED, "weight is not bf16");
    pfr::require(N >= 0 && N < INT32_MAX, "bad column count");
    pfr::require(ldx >= N && ldy >= N, "leading dimension smaller than N");
    if (W->M == 0 || N == 0) return;
    pfr::require(X != nullptr && Y != nullptr, "null X/Y");
    const int64_t Np = round_up(N, kTileN);
    const uint16_t* xt = stage_xt(ctx, X, W->K, N, ldx, W->Kp, Np);
    dim3 grid((unsigned)(W->Mp / kTileM), (unsigned)(Np / kTileN));
    hipLaunchKernelGGL(k_sp24_bf16, grid, dim3(256), 0, ctx->stream, (int)(W->Kp / 64),
                       static_cast<const v4i*>(W->a), W->idx, xt, W->Kp, (int)W->M, (int)N, Y, ldy);
    PFR_HIP(hipGetLastError());
}

}  // namespace

extern "C" {

int pfr_sp24_pack(pfr_ctx* ctx, int64_t M, int64_t K, const void* W, pfr_dtype dtype, const float* w_scales,
                  int64_t n_scales, pfr_sp24** out) {
    return pfr::guarded([&] {
        pfr::require(out != nullptr, "null output handle");
        *out = nullptr;
        pfr::bind(ctx);
        pfr::require(M >= 0 && K >= 0 && M < INT32_MAX && K < INT32_MAX, "bad weight dimensions");
        pfr::require(W != nullptr || M * K == 0, "null weight");
        pfr::require(dtype == PFR_I8 || dtype == PFR_BF16, "2:4 weights are int8 or bf16");
        std::vector<float> scales((size_t)M, 1.0f);
        if (dtype == PFR_I8) {
            pfr::require(w_scales != nullptr && (n_scales == 1 || n_scales == M),
                         "int8 weights need 1 or M scales");
            for (int64_t m = 0; m < M; ++m) {
                const float s = w_scales[n_scales == 1 ? 0 : m];
                pfr::require(s > 0.0f && std::isfinite(s), "weight scale must be positive and finite");
                scales[(size_t)m] = s;
            }
        }
        pfr_sp24* w = dtype == PFR_I8 ? pack_i8(ctx, M, K, static_cast<const int8_t*>(W))
                                      : pack_bf16(ctx, M, K, static_cast<const uint16_t*>(W));
        try {
            PFR_HIP(hipMalloc(&w->w_scale, sizeof(float) * (size_t)(M > 0 ? M : 1)));
            if (M) PFR_HIP(hipMemcpy(w->w_scale, scales.data(), sizeof(float) * (size_t)M, hipMemcpyHostToDevice));
        } catch (...) {
            free_sp24(w);
            throw;
        }
        *out = w;
    });
}

int pfr_sp24_info(const pfr_sp24* w, int64_t* M, int64_t* K, pfr_dtype* dtype) {
    return pfr::guarded([&] {
        pfr::require(w != nullptr, "null 2:4 weight handle");
        if (M) *M = w->M;
        if (K) *K = w->K;
        if (dtype) *dtype = w->dtype;
    });
}

int pfr_sp24_free(pfr_sp24* w) {
    return pfr::guarded([&] {
        if (!w) return;
        pfr::bind(w->ctx);
        (void)hipStreamSynchronize(w->ctx->stream);
        free_sp24(w);
    });
}

int pfr_sp24_gemm_i8_dev(pfr_ctx* ctx, const pfr_sp24* W, const int8_t* X, int64_t N, int64_t ldx, float x_scale,
                         int out_kind, float out_scale, int32_t out_zp, void* Y, int64_t ldy) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        gemm_i8_dev(ctx, W, X, N, ldx, x_scale, out_kind, out_scale, out_zp, Y, ldy);
    });
}

int pfr_sp24_gemm_i8(pfr_ctx* ctx, const pfr_sp24* W, const int8_t* X, int64_t N, float x_scale, int out_kind,
                     float out_scale, int32_t out_zp, void* Y) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        check_i8(W);
        pfr::require(N >= 0, "bad column count");
        const size_t esz = out_kind == PFR_SP24_OUT_I8 ? 1 : 4;
        const size_t xb = (size_t)(W->K * N), yb = esz * (size_t)(W->M * N);
        if (yb == 0) return;
        pfr::require(Y != nullptr && (X != nullptr || xb == 0), "null X/Y");
        hipStream_t s = ctx->stream;
        int8_t* dX = static_cast<int8_t*>(ctx->scratch[0].ensure(xb ? xb : 4));
        void* dY = ctx->scratch[2].ensure(yb);
        if (xb) PFR_HIP(hipMemcpyAsync(dX, X, xb, hipMemcpyHostToDevice, s));
        gemm_i8_dev(ctx, W, dX, N, N, x_scale, out_kind, out_scale, out_zp, dY, N);
        PFR_HIP(hipMemcpyAsync(Y, dY, yb, hipMemcpyDeviceToHost, s));
        PFR_HIP(hipStreamSynchronize(s));
    });
}

int pfr_sp24_gemm_bf16_dev(pfr_ctx* ctx, const pfr_sp24* W, const uint16_t* X, int64_t N, int64_t ldx, float* Y,
                           int64_t ldy) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        gemm_bf16_dev(ctx, W, X, N, ldx, Y, ldy);
    });
}

int pfr_sp24_gemm_bf16(pfr_ctx* ctx, const pfr_sp24* W, const uint16_t* X, int64_t N, float* Y) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        pfr::require(W != nullptr, "null 2:4 weight handle");
        pfr::require(N >= 0, "bad column count");
        const size_t xb = 2 * (size_t)(W->K * N), yb = 4 * (size_t)(W->M * N);
        if (yb == 0) return;
        pfr::require(Y != nullptr && (X != nullptr || xb == 0), "null X/Y");
        hipStream_t s = ctx->stream;
        uint16_t* dX = static_cast<uint16_t*>(ctx->scratch[0].ensure(xb ? xb : 4));
        float* dY = static_cast<float*>(ctx->scratch[2].ensure(yb));
        if (xb) PFR_HIP(hipMemcpyAsync(dX, X, xb, hipMemcpyHostToDevice, s));
        gemm_bf16_dev(ctx, W, dX, N, N, dY, N);
        PFR_HIP(hipMemcpyAsync(Y, dY, yb, hipMemcpyDeviceToHost, s));
        PFR_HIP(hipStreamSynchronize(s));
    });
}

}  // extern "C"
