// CSR SpMM / SpMV for gfx950 and the Gemm-orientation wrapper.
//
// Strict mode reproduces the reference CPU kernels bit-for-bit: every output
// is the ascending-k sequence acc = RN(acc + RN(w * x)) from +0, with the
// bias added last as RN(acc + RN(beta * c)) (math.cpp:416-435,
// sparse_tensor.cpp:500-510 / :543-548).  The whole file is compiled with
// floating-point contraction off; fast mode asks for fmaf explicitly.
#include <algorithm>
#include <climits>
#include <cstdint>
#include <mutex>
#include <type_traits>
#include <vector>

#include "common.hpp"

#pragma clang fp contract(off)

// Workspace of the allocation-free Gemm entry (pfr_gemm_csr_act_noalloc_dev):
// the transposed, alpha-scaled activation op(A)^T.  Every device the library
// runs on holds one copy until the process ends.  In host code `scratch` is a
// host-side stand-in, not a device address: host code uses only the per-device
// address that init_noalloc_workspace records.
constexpr int64_t kNoAllocFloats = int64_t(1) << 22;  // 16 MiB: K * Mb <= 4,194,304
static __device__ __align__(256) float scratch[kNoAllocFloats];

namespace {

using pfr::bias_add;

constexpr int kWaves = 4;  // waves per 256-thread workgroup
constexpr int kSpmvThreads = 512;  // threads of the vector kernel's workgroup
constexpr int kSpmvCap = 4096;     // products staged per workgroup chunk (16 KB)
constexpr int64_t kSellMinN = 16;  // column-slice kernel from this many columns on

// One 4-byte word per lane from base + off into LDS at dst + 4 lane, as a
// buffer load (bytes: the buffer's size; a lane past it reads zero).  A
// buffer load, not a global one: the compiler counts a global
// direct-to-LDS load as a flat access that may finish out of order and then
// turns every later wait on the memory counters into a wait for all loads.
__device__ __forceinline__ void lds_copy_dword(const void* base, int bytes, int off,
                                               __attribute__((address_space(3))) void* dst) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, dst, 4, off, 0, 0, 0);
}

template <bool FAST>
__device__ __forceinline__ float madd(float acc, float w, float x) {
    if constexpr (FAST) {
        return __builtin_fmaf(w, x, acc);
    } else {
        const float p = w * x;
        return acc + p;
    }
}

// Weight of nonzero j of `row`: the float32 value, or for int8 values the
// dequantised RN((float)q * scale[row]) of dequantize_tensor with zero point
// 0 (quant_ops.cpp:182-196: ((float)q - 0.0f) * scale rounds once).
template <bool I8>
__device__ __forceinline__ float wval(const void* __restrict__ val, const float* __restrict__ rs, int j, int row) {
    if constexpr (I8) {
        return (float)static_cast<const int8_t*>(val)[j] * rs[row];
    } else {
        return static_cast<const float*>(val)[j];
    }
}


// One wave per CSR row, lanes across the N columns (4 per lane when VEC).
// Output element (row, c) goes to Y[row * ldy_r + c * ldy_c].
template <bool FAST, bool VEC, bool I8, class C>
__global__ __launch_bounds__(256) void k_spmm_rows(
    int M, int N, const int32_t* __restrict__ rowptr, const C* __restrict__ col,
    const void* __restrict__ val, const float* __restrict__ rs, const float* __restrict__ X, int64_t ldx,
    float* __restrict__ Y, int64_t ldy_r, int64_t ldy_c, const float* __restrict__ bias,
    int64_t c_size, float beta, int act) {
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
                    w[i] = wval<I8>(val, rs, j + i, row);
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
                const float w = wval<I8>(val, rs, j, row);
                const float4 x = *reinterpret_cast<const float4*>(xc + (int64_t)col[j] * ldx);
                a0 = madd<FAST>(a0, w, x.x);
                a1 = madd<FAST>(a1, w, x.y);
                a2 = madd<FAST>(a2, w, x.z);
                a3 = madd<FAST>(a3, w, x.w);
            }
            const int64_t f = (int64_t)row * ldy_r + c0;  // ldy_c == 1 here
            float4 o;
            o.x = bias_add(a0, f, bias, c_size, beta, act);
            o.y = bias_add(a1, f + 1, bias, c_size, beta, act);
            o.z = bias_add(a2, f + 2, bias, c_size, beta, act);
            o.w = bias_add(a3, f + 3, bias, c_size, beta, act);
            *reinterpret_cast<float4*>(Y + f) = o;
        }
    } else {
        for (int c = lane; c < N; c += 64) {
            float a = 0.0f;
#pragma unroll 4
            for (int j = beg; j < end; ++j) a = madd<FAST>(a, wval<I8>(val, rs, j, row), X[(int64_t)col[j] * ldx + c]);
            const int64_t f = (int64_t)row * ldy_r + (int64_t)c * ldy_c;
            Y[f] = bias_add(a, f, bias, c_size, beta, act);
        }
    }
}

// NP lanes per row (NP = next power of two >= N, N < 64), 64 / NP rows per wave.
template <int NP, bool FAST, bool I8, class C>
__global__ __launch_bounds__(256) void k_spmm_small(
    int M, int N, const int32_t* __restrict__ rowptr, const C* __restrict__ col,
    const void* __restrict__ val, const float* __restrict__ rs, const float* __restrict__ X, int64_t ldx,
    float* __restrict__ Y, int64_t ldy_r, int64_t ldy_c, const float* __restrict__ bias,
    int64_t c_size, float beta, int act) {
    constexpr int RPW = 64 / NP;
    const int lane = threadIdx.x & 63;
    const int g = lane / NP, c = lane % NP;
    const int row = ((int)blockIdx.x * kWaves + (int)(threadIdx.x >> 6)) * RPW + g;
    if (row >= M || c >= N) return;
    const int beg = rowptr[row];
    const int end = rowptr[row + 1];
    float a = 0.0f;
#pragma unroll 4
    for (int j = beg; j < end; ++j) a = madd<FAST>(a, wval<I8>(val, rs, j, row), X[(int64_t)col[j] * ldx + c]);
    const int64_t f = (int64_t)row * ldy_r + (int64_t)c * ldy_c;
    Y[f] = bias_add(a, f, bias, c_size, beta, act);
}

// SpMV.  One workgroup per row block (<= 64 rows, <= kSpmvCap nnz unless a
// single longer row).  All kSpmvThreads threads gather over the block's
// contiguous nnz range with all loads in flight at once, staging in LDS
// either the products RN(w * x[col]) (float values) or x[col] and the int8
// value (int8 values: the product needs the row's scale); then lane g of
// wave 0 folds row r0 + g in storage order.  Longer blocks go in chunks.
template <bool I8, class C>
__global__ __launch_bounds__(kSpmvThreads) void k_spmv_wg(
    const int32_t* __restrict__ blocks, const int32_t* __restrict__ rowptr,
    const C* __restrict__ col, const void* __restrict__ val, const float* __restrict__ rs,
    const float* __restrict__ x, int64_t ldx, float* __restrict__ y, int64_t ldy_r,
    const float* __restrict__ bias, int64_t c_size, float beta, int act) {
    __shared__ float P[kSpmvCap];
    __shared__ int8_t Q[I8 ? kSpmvCap : 1];
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
    const float my_scale = (I8 && folder) ? rs[my_row] : 1.0f;
    float acc = 0.0f;
    for (int base = nb; base < ne; base += kSpmvCap) {
        const int cend = min(base + kSpmvCap, ne);
        int cl[kPer];
        float w[kPer];
        int8_t q[kPer];
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int j = base + tid + i * kSpmvThreads;
            cl[i] = j < cend ? (int)col[j] : 0;
            if constexpr (I8) q[i] = j < cend ? static_cast<const int8_t*>(val)[j] : 0;
            else w[i] = j < cend ? static_cast<const float*>(val)[j] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int j = base + tid + i * kSpmvThreads;
            if (j < cend) {
                const float xv = x[(int64_t)cl[i] * ldx];
                if constexpr (I8) {
                    P[j - base] = xv;
                    Q[j - base] = q[i];
                } else {
                    P[j - base] = w[i] * xv;
                }
            }
        }
        __syncthreads();
        if (folder) {
            int p = max(my_beg, base) - base;
            const int e = min(my_end, cend) - base;
            for (; p + 8 <= e; p += 8) {
                float t[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    if constexpr (I8) {
                        const float wv = (float)Q[p + i] * my_scale;
                        t[i] = wv * P[p + i];
                    } else {
                        t[i] = P[p + i];
                    }
                }
#pragma unroll
                for (int i = 0; i < 8; ++i) acc = acc + t[i];
            }
            for (; p < e; ++p) {
                if constexpr (I8) {
                    const float wv = (float)Q[p] * my_scale;
                    const float t = wv * P[p];
                    acc = acc + t;
                } else {
                    acc = acc + P[p];
                }
            }
        }
        __syncthreads();
    }
    if (folder) {
        const int64_t f = (int64_t)my_row * ldy_r;
        y[f] = bias_add(acc, f, bias, c_size, beta, act);
    }
}

// Strict SpMV over the row-chain copy (pfr_csr::chain_q0): one workgroup per
// slab of 64 rows.  Eight producer waves compute the products RN(w * x[col])
// (int8: w = RN(q * row scale)) of a 256-step chunk of all 64 rows into LDS,
// with the next chunk's values and columns already in flight, while wave 0
// folds the previous chunk: lane r adds row r's products in storage order,
// one 16-byte LDS read per four steps.  Steps past a row's count give +0,
// which leaves the sum unchanged (a sum that starts at +0 is never -0 under
// round-to-nearest).  Two LDS buffers of 64 KiB alternate between producers
// and folder, one barrier per chunk.
constexpr int kChainCH = 64;                 // quad rows per chunk
constexpr int kChainP = 8;                   // producer waves
constexpr int kChainT = kChainCH / kChainP;  // quad rows per producer lane per chunk

template <bool I8, bool C16>
__global__ __launch_bounds__(64 * (kChainP + 1)) void k_spmv_chain(
    const int32_t* __restrict__ q0, const int32_t* __restrict__ lens, const int32_t* __restrict__ perm,
    const void* __restrict__ vals, const void* __restrict__ cols, const float* __restrict__ rs,
    const float* __restrict__ x, int ldx, float* __restrict__ y, int64_t ldy_r,
    const float* __restrict__ bias, int64_t c_size, float beta, int act) {
    __shared__ float4 buf[2][kChainCH * 64];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int s = blockIdx.x;
    const int qb = q0[s], nq = q0[s + 1] - qb;
    const int nch = (nq + kChainCH - 1) / kChainCH;
    const int row = perm[s * 64 + lane];
    if (wave == 0) {
        float acc = 0.0f;
        for (int i = 0; i <= nch; ++i) {
            if (i > 0) {
                const float4* b = buf[(i - 1) & 1] + lane;
                const int gq = min(kChainCH, nq - (i - 1) * kChainCH);
#pragma unroll 8
                for (int g = 0; g < gq; ++g) {
                    const float4 v = b[g * 64];
                    acc = acc + v.x;
                    acc = acc + v.y;
                    acc = acc + v.z;
                    acc = acc + v.w;
                }
            }
            __syncthreads();
        }
        if (row >= 0) {
            const int64_t f = (int64_t)row * ldy_r;
            y[f] = bias_add(acc, f, bias, c_size, beta, act);
        }
        return;
    }
    using ValT = typename std::conditional<I8, uint32_t, float4>::type;  // four steps' values
    using ColT = typename std::conditional<C16, uint2, int4>::type;      // four steps' columns
    const ValT* V = static_cast<const ValT*>(vals);
    const ColT* Cl = static_cast<const ColT*>(cols);
    const int len = lens[s * 64 + lane];
    const float scale = (I8 && row >= 0) ? rs[row] : 1.0f;
    const int pw = wave - 1;
    ValT va[kChainT], vb[kChainT];
    ColT ca[kChainT], cb[kChainT];
    // Task t of chunk i is quad row i * kChainCH + pw + kChainP * t; the
    // address is clamped into the slab so every load is issued.
    auto load = [&](int i, ValT* v, ColT* c) {
#pragma unroll
        for (int t = 0; t < kChainT; ++t) {
            const int g = min(i * kChainCH + pw + kChainP * t, nq - 1);
            const int64_t at = (int64_t)(qb + g) * 64 + lane;
            v[t] = V[at];
            c[t] = Cl[at];
        }
    };
    auto colk = [&](const ColT& c, int e) -> int {
        if constexpr (C16) {
            const uint32_t d = e < 2 ? c.x : c.y;
            return (int)((e & 1) ? (d >> 16) : (d & 0xffffu));
        } else {
            return e == 0 ? c.x : (e == 1 ? c.y : (e == 2 ? c.z : c.w));
        }
    };
    auto valk = [&](const ValT& v, int e) -> float {
        if constexpr (I8) {
            const float w = (float)(int8_t)((v >> (8 * e)) & 0xffu);
            return w * scale;
        } else {
            return e == 0 ? v.x : (e == 1 ? v.y : (e == 2 ? v.z : v.w));
        }
    };
    // Chunk i from (vc, cc) into buffer i & 1, loading chunk i + 1 into
    // (vn, cn); the loop alternates the two register sets, so no copy waits
    // for the loads in flight.
    auto chunk = [&](int i, const ValT* vc, const ColT* cc, ValT* vn, ColT* cn) {
        if (i < nch) {
            float xg[kChainT][4];
#pragma unroll
            for (int t = 0; t < kChainT; ++t)
#pragma unroll
                for (int e = 0; e < 4; ++e) xg[t][e] = x[colk(cc[t], e) * ldx];
            load(i + 1 < nch ? i + 1 : i, vn, cn);
            float4* b = buf[i & 1] + lane;
#pragma unroll
            for (int t = 0; t < kChainT; ++t) {
                const int gl = pw + kChainP * t;         // quad row within the chunk
                const int j0 = 4 * (i * kChainCH + gl);  // first step of the quad
                float p[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float prod = valk(vc[t], e) * xg[t][e];
                    p[e] = j0 + e < len ? prod : 0.0f;
                }
                b[gl * 64] = make_float4(p[0], p[1], p[2], p[3]);
            }
        }
        __syncthreads();
    };
    if (nq > 0) load(0, va, ca);
    for (int i = 0; i <= nch; i += 2) {
        chunk(i, va, ca, vb, cb);
        if (i + 1 <= nch) chunk(i + 1, vb, cb, va, ca);
    }
}

// The same with x staged in LDS (K < kChainXMax) and slabs of R = 16, 32 or
// 64 rows (pfr_csr::chain_rows): one folding wave (lanes 0 .. R-1) and R / 8
// producer waves, each producer instruction covering 64 / R quad rows of the
// slab.  Columns are byte offsets into the LDS copy of x and padding steps
// read its zero slot at K, so their products are RN(+0 * +0) = +0 with no
// select.  A chunk is 64 steps (3 % faster than 128 on the 4096² SpMV: the
// fold trails the products by a smaller chunk); the values and offsets are
// loaded two chunks ahead (three register sets in turn).  The loads are
// never skipped (chunk indices past the slab are clamped, the spare padding
// row after the last slab covers an empty slab) and the iteration count is
// a multiple of six, so the loop body is straight-line code and the
// compiler waits only for the oldest loads.  Dynamic LDS: 2 x CH quad rows x R x 16 B of products,
// then K + 1 floats of x.
template <int R>
constexpr int chain_ch() { return 16; }  // quad rows per chunk (a multiple of 16: the fold's batches)
constexpr int kChainXUnroll = 6;

// x[0 .. K) (stride ldx) into LDS as xs[0 .. K) plus a zero at xs[K], by NT
// threads: eight loads per thread in flight (clamped addresses), then the
// stores, instead of one load latency per element a thread stages.
template <int NT>
__device__ __forceinline__ void stage_x(float* xs, const float* __restrict__ x, int K, int64_t ldx, int tid) {
    for (int k0 = 0; k0 <= K; k0 += 8 * NT) {
        float t[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) t[i] = x[(int64_t)min(k0 + tid + NT * i, K - 1) * ldx];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int k = k0 + tid + NT * i;
            if (k <= K) xs[k] = k < K ? t[i] : 0.0f;
        }
    }
}

template <bool I8, int R>
__global__ __launch_bounds__(64 * (1 + R / 8)) void k_spmv_chain_x(
    int K, const int32_t* __restrict__ q0, const int32_t* __restrict__ perm, const void* __restrict__ vals,
    const uint32_t* __restrict__ cols, const float* __restrict__ rs, const float* __restrict__ x, int ldx,
    float* __restrict__ y, int64_t ldy_r, const float* __restrict__ bias, int64_t c_size, float beta, int act) {
    constexpr int P = R / 8;    // producer waves
    constexpr int QW = 64 / R;  // quad rows per producer instruction
    constexpr int kChainXCH = chain_ch<R>();
    constexpr int kChainXT = kChainXCH * R / (64 * P);  // quad-row groups per producer lane per chunk
    static_assert(kChainXCH * R == 64 * P * kChainXT, "chunk split");
    extern __shared__ float4 dyn[];
    float4* const buf0 = dyn;
    float4* const buf1 = dyn + kChainXCH * R;
    float* const xs = reinterpret_cast<float*>(dyn + 2 * kChainXCH * R);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int s = blockIdx.x;
    const int qb = q0[s], nq = q0[s + 1] - qb;
    const int nch = (nq + kChainXCH - 1) / kChainXCH;
    // >= nch + 1 (the last fold needs one more barrier), a multiple of the unroll
    const int iters = (nch + kChainXUnroll) / kChainXUnroll * kChainXUnroll;
    if (wave == 0) {
        stage_x<64 * (1 + P)>(xs, x, K, ldx, tid);
        __syncthreads();
        // The fold is bound by the latency of its dependent adds; the LDS
        // reads of the next eight quad rows are issued before the adds of the
        // current eight.  Whole chunks are folded: quad rows past the slab
        // hold +0.
        const int row = lane < R ? perm[s * R + lane] : -1;
        float acc = 0.0f;
        auto rd = [&](const float4* b, float4* r, int batch) {
#pragma unroll
            for (int k = 0; k < 8; ++k) r[k] = b[(batch * 8 + k) * R];
        };
        auto add = [&](const float4* r) {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                acc = acc + r[k].x;
                acc = acc + r[k].y;
                acc = acc + r[k].z;
                acc = acc + r[k].w;
            }
        };
        for (int i = 0; i < iters; ++i) {
            if (lane < R && i > 0 && i - 1 < nch) {
                const float4* b = ((i - 1) & 1 ? buf1 : buf0) + lane;
                float4 ra[8], rb[8];
                rd(b, ra, 0);
#pragma unroll
                for (int h = 0; h < kChainXCH / 8; h += 2) {
                    if (h + 1 < kChainXCH / 8) rd(b, rb, h + 1);
                    add(ra);
                    if (h + 2 < kChainXCH / 8) rd(b, ra, h + 2);
                    if (h + 1 < kChainXCH / 8) add(rb);
                }
            }
            __syncthreads();
        }
        if (row >= 0) {
            const int64_t f = (int64_t)row * ldy_r;
            y[f] = bias_add(acc, f, bias, c_size, beta, act);
        }
        return;
    }
    using ValT = typename std::conditional<I8, uint32_t, float4>::type;
    const ValT* V = static_cast<const ValT*>(vals);
    const uint2* Cl = reinterpret_cast<const uint2*>(cols);
    const int prow = perm[s * R + lane % R];
    const float scale = (I8 && prow >= 0) ? rs[prow] : 1.0f;
    const int pw = wave - 1;
    const int sub = lane / R;  // quad row within the instruction's group
    const char* xb = reinterpret_cast<const char*>(xs);
    ValT v0[kChainXT], v1[kChainXT], v2[kChainXT];
    uint2 c0[kChainXT], c1[kChainXT], c2[kChainXT];
    // group t of chunk i: quad rows i * CH + (pw + P * t) * QW + sub
    auto load = [&](int i, ValT* v, uint2* c) {
#pragma unroll
        for (int t = 0; t < kChainXT; ++t) {
            const int g = max(min(i * kChainXCH + (pw + P * t) * QW + sub, nq - 1), 0);
            const int64_t at = (int64_t)(qb + g) * R + lane % R;
            v[t] = V[at];
            c[t] = Cl[at];
        }
    };
    auto valk = [&](const ValT& v, int e) -> float {
        if constexpr (I8) {
            const float w = (float)(int8_t)((v >> (8 * e)) & 0xffu);
            return w * scale;
        } else {
            return e == 0 ? v.x : (e == 1 ? v.y : (e == 2 ? v.z : v.w));
        }
    };
    // chunk i (its products land in buffer i & 1; past the slab they are
    // never folded), loading chunk i + 2
    auto chunk = [&](int i, const ValT* vc, const uint2* cc, ValT* vn, uint2* cn) {
        load(min(i + 2, nch - 1), vn, cn);
        float4* b = ((i & 1) ? buf1 : buf0) + lane;
#pragma unroll
        for (int t = 0; t < kChainXT; ++t) {
            const uint32_t o[4] = {cc[t].x & 0xffffu, cc[t].x >> 16, cc[t].y & 0xffffu, cc[t].y >> 16};
            const bool in = i * kChainXCH + (pw + P * t) * QW + sub < nq;  // else a clamped copy: fold +0
            float p[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float prod = valk(vc[t], e) * *reinterpret_cast<const float*>(xb + o[e]);
                p[e] = in ? prod : 0.0f;
            }
            b[(pw + P * t) * 64] = make_float4(p[0], p[1], p[2], p[3]);
        }
        __syncthreads();
    };
    // the first two chunks' loads go out before x is staged, so the two
    // latencies overlap
    load(0, v0, c0);
    load(min(1, nch - 1), v1, c1);
    stage_x<64 * (1 + P)>(xs, x, K, ldx, tid);
    __syncthreads();
    for (int i = 0; i < iters; i += 6) {
        chunk(i, v0, c0, v2, c2);
        chunk(i + 1, v1, c1, v0, c0);
        chunk(i + 2, v2, c2, v1, c1);
        chunk(i + 3, v0, c0, v2, c2);
        chunk(i + 4, v1, c1, v0, c0);
        chunk(i + 5, v2, c2, v1, c1);
    }
}

template <bool I8, int R>
void launch_chain_x(pfr_ctx* ctx, const pfr_csr* W, const float* X, int64_t ldx, float* Y, int64_t ldy_r,
                    const float* bias, int64_t c_size, float beta, int act) {
    auto kern = k_spmv_chain_x<I8, R>;
    constexpr int kChainXCH = chain_ch<R>();
    const size_t lds = (size_t)(2 * kChainXCH * R) * 16 + (size_t)(W->K + 1) * 4;
    // more than 64 KiB of dynamic LDS has to be allowed per kernel and device
    static uint64_t allowed = 0;  // bit d: done on device d (< 64)
    const uint64_t bit = ctx->device < 64 ? (uint64_t(1) << ctx->device) : 0;
    if (lds > 65536 && (!bit || !(__atomic_load_n(&allowed, __ATOMIC_ACQUIRE) & bit))) {
        const int most = 2 * kChainXCH * R * 16 + pfr::kChainXMax * 4;
        PFR_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                    most));
        if (bit) __atomic_fetch_or(&allowed, bit, __ATOMIC_RELEASE);
    }
    hipLaunchKernelGGL(kern, dim3((unsigned)W->chain_nslab), dim3(64 * (1 + R / 8)), lds, ctx->stream, (int)W->K,
                       W->chain_q0, W->chain_perm, W->chain_val, static_cast<const uint32_t*>(W->chain_col),
                       W->row_scale, X, (int)ldx, Y, ldy_r, bias, c_size, beta, act);
}

// Strict product for 2 <= N <= 8 columns over the row-chain copy, 16 rows
// per workgroup (a copy with 32- or 64-row slabs, which the N = 1 kernel
// prefers for tall weights, is taken 16 rows of a slab at a time): every
// (row, column) pair is its own in-order chain, one lane each,
// so NC / 4 waves fold (NC = 2, 4 or 8, N <= NC) while four producer waves
// load the values and offsets two chunks ahead, gather the x rows from global
// memory one chunk ahead (16-byte loads when x rows are aligned and N == NC
// >= 4) and write RN(w * x[col, n]) for every column.  The gathers are what
// bounds it: on the 4096 x 4096 int8 decode weight at batch 8 a timing-only
// copy without them takes 27.9 us, against 59.9 us when each chunk gathered
// its own x rows and 52.0 us gathering them a chunk ahead.  (x staged in LDS
// instead, 128 KiB at K = 4096, leaves room for 8-quad-row product chunks
// only, and the per-chunk barriers made that 68 us.)  Steps past a row's count (and quad
// rows past the slab) give +0; their gather addresses are clamped into x.
// LDS: 2 x 32 quad rows x NC x 16 rows x 16 B of products.
constexpr int kChainNR = 16;  // rows per workgroup of this kernel
constexpr int kChainNP = 4;   // producer waves

template <int NC>
constexpr int chain_n_folders() { return NC >= 4 ? NC / 4 : 1; }

template <bool I8, int NC, bool XV>
__global__ __launch_bounds__(64 * (chain_n_folders<NC>() + kChainNP)) void k_spmm_chain(
    int K, int N, int cshift, int rstride, const int32_t* __restrict__ q0, const int32_t* __restrict__ lens,
    const int32_t* __restrict__ perm, const void* __restrict__ vals, const uint32_t* __restrict__ cols,
    const float* __restrict__ rs, const float* __restrict__ X, int64_t ldx, float* __restrict__ Y, int64_t ldy_r,
    int64_t ldy_c, const float* __restrict__ bias, int64_t c_size, float beta, int act) {
    constexpr int R = kChainNR, CH = 32, P = kChainNP, F = chain_n_folders<NC>(), QW = 64 / R;
    constexpr int T = CH * R / (64 * P);  // quad-row groups per producer lane per chunk
    static_assert(CH * R == 64 * P * T, "chunk split");
    extern __shared__ float4 dyn[];
    float4* const buf0 = dyn;
    float4* const buf1 = dyn + CH * NC * R;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // a copy with slabs of rstride = 16, 32 or 64 rows: workgroup b takes
    // rows 16 * (b % (rstride / 16)) .. + 15 of slab b / (rstride / 16) (the
    // slab's quad rows and record stride are the copy's)
    const int nsub = rstride / R;
    const int s = blockIdx.x / nsub, ro = (blockIdx.x % nsub) * R;
    const int qb = q0[s], nq = q0[s + 1] - qb;
    const int nch = (nq + CH - 1) / CH;
    const int iters = (nch + kChainXUnroll) / kChainXUnroll * kChainXUnroll;
    if (wave < F) {
        const int c = wave * 64 + lane;  // chain: column c / R of slab row c % R
        const int n = c / R, r = c % R;
        const bool act_lane = c < NC * R && n < N;
        const int row = act_lane ? perm[s * rstride + ro + r] : -1;
        float acc = 0.0f;
        auto rd = [&](const float4* b, float4* v, int batch) {
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = b[(batch * 8 + k) * NC * R];
        };
        auto add = [&](const float4* v) {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                acc = acc + v[k].x;
                acc = acc + v[k].y;
                acc = acc + v[k].z;
                acc = acc + v[k].w;
            }
        };
        for (int i = 0; i < iters; ++i) {
            if (act_lane && i > 0 && i - 1 < nch) {
                const float4* b = ((i - 1) & 1 ? buf1 : buf0) + n * R + r;
                float4 ra[8], rb[8];
                rd(b, ra, 0);
#pragma unroll
                for (int h = 0; h < CH / 8; h += 2) {
                    rd(b, rb, h + 1);
                    add(ra);
                    if (h + 2 < CH / 8) rd(b, ra, h + 2);
                    add(rb);
                }
            }
            __syncthreads();
        }
        if (row >= 0) {
            const int64_t f = (int64_t)row * ldy_r + (int64_t)n * ldy_c;
            Y[f] = bias_add(acc, f, bias, c_size, beta, act);
        }
        return;
    }
    using ValT = typename std::conditional<I8, uint32_t, float4>::type;
    const ValT* V = static_cast<const ValT*>(vals);
    const uint2* Cl = reinterpret_cast<const uint2*>(cols);
    const int r = lane % R, sub = lane / R;
    const int prow = perm[s * rstride + ro + r];
    const int len = lens[s * rstride + ro + r];
    const float scale = (I8 && prow >= 0) ? rs[prow] : 1.0f;
    const int pw = wave - F;
    ValT v0[T], v1[T], v2[T];
    uint2 c0[T], c1[T], c2[T];
    auto load = [&](int i, ValT* v, uint2* cc) {
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int g = max(min(i * CH + (pw + P * t) * QW + sub, nq - 1), 0);
            const int64_t at = (int64_t)(qb + g) * rstride + ro + r;
            v[t] = V[at];
            cc[t] = Cl[at];
        }
    };
    auto valk = [&](const ValT& v, int e) -> float {
        if constexpr (I8) {
            const float w = (float)(int8_t)((v >> (8 * e)) & 0xffu);
            return w * scale;
        } else {
            return e == 0 ? v.x : (e == 1 ? v.y : (e == 2 ? v.z : v.w));
        }
    };
    // the x rows of a chunk's records, gathered one chunk ahead of their use
    // (their latency then overlaps a chunk's products instead of adding to it)
    using XG = float[T][4][NC];
    auto gather = [&](const uint2* cc, XG& xg) {
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t o = (e < 2 ? cc[t].x : cc[t].y) >> (16 * (e & 1)) & 0xffffu;
                const int col = min((int)(o >> cshift), K - 1);
                const float* xr = X + (int64_t)col * ldx;
                if constexpr (XV) {
#pragma unroll
                    for (int q = 0; q < NC / 4; ++q) {
                        const float4 v = *reinterpret_cast<const float4*>(xr + 4 * q);
                        xg[t][e][4 * q] = v.x;
                        xg[t][e][4 * q + 1] = v.y;
                        xg[t][e][4 * q + 2] = v.z;
                        xg[t][e][4 * q + 3] = v.w;
                    }
                } else {
#pragma unroll
                    for (int q = 0; q < NC; ++q) xg[t][e][q] = xr[min(q, N - 1)];
                }
            }
    };
    // chunk i: values and columns two chunks ahead, x one chunk ahead, then
    // chunk i's products from its values (vc) and the x gathered last chunk
    auto chunk = [&](int i, const ValT* vc, ValT* vn, uint2* cn, const uint2* cnext, XG& xg, XG& xnext) {
        load(min(i + 2, nch - 1), vn, cn);
        gather(cnext, xnext);
        float4* b = ((i & 1) ? buf1 : buf0);
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int gl = (pw + P * t) * QW + sub;  // quad row within the chunk
            const int j0 = 4 * (i * CH + gl);         // its first step
            float w[4];
            bool ok[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                w[e] = valk(vc[t], e);
                ok[e] = j0 + e < len;  // also false past the slab (len <= 4 * nq)
            }
#pragma unroll
            for (int q = 0; q < NC; ++q) {
                float p[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float prod = w[e] * xg[t][e][q];
                    p[e] = ok[e] ? prod : 0.0f;
                }
                b[(gl * NC + q) * R + r] = make_float4(p[0], p[1], p[2], p[3]);
            }
        }
        __syncthreads();
    };
    XG xa, xb;
    load(0, v0, c0);
    load(min(1, nch - 1), v1, c1);
    gather(c0, xa);
    for (int i = 0; i < iters; i += 6) {
        chunk(i, v0, v2, c2, c1, xa, xb);
        chunk(i + 1, v1, v0, c0, c2, xb, xa);
        chunk(i + 2, v2, v1, c1, c0, xa, xb);
        chunk(i + 3, v0, v2, c2, c1, xb, xa);
        chunk(i + 4, v1, v0, c0, c2, xa, xb);
        chunk(i + 5, v2, v1, c1, c0, xb, xa);
    }
}

template <bool I8, int NC, bool XV>
void launch_chain_n(pfr_ctx* ctx, const pfr_csr* W, const float* X, int N, int64_t ldx, float* Y, int64_t ldy_r,
                    int64_t ldy_c, const float* bias, int64_t c_size, float beta, int act) {
    auto kern = k_spmm_chain<I8, NC, XV>;
    const size_t lds = (size_t)2 * 32 * NC * kChainNR * 16;
    static uint64_t allowed = 0;  // bit d: more than 64 KiB of dynamic LDS allowed on device d (< 64)
    const uint64_t bit = ctx->device < 64 ? (uint64_t(1) << ctx->device) : 0;
    if (lds > 65536 && (!bit || !(__atomic_load_n(&allowed, __ATOMIC_ACQUIRE) & bit))) {
        PFR_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)lds));
        if (bit) __atomic_fetch_or(&allowed, bit, __ATOMIC_RELEASE);
    }
    const unsigned grid = (unsigned)(W->chain_nslab * (W->chain_rows / kChainNR));
    hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * (chain_n_folders<NC>() + kChainNP)), lds, ctx->stream,
                       (int)W->K, N, W->chain_xlds ? 2 : 0, (int)W->chain_rows, W->chain_q0, W->chain_len, W->chain_perm,
                       W->chain_val, static_cast<const uint32_t*>(W->chain_col), W->row_scale, X, ldx, Y, ldy_r,
                       ldy_c, bias, c_size, beta, act);
}

template <bool I8>
void launch_chain_cols(pfr_ctx* ctx, const pfr_csr* W, const float* X, int N, int64_t ldx, float* Y,
                       int64_t ldy_r, int64_t ldy_c, const float* bias, int64_t c_size, float beta, int act) {
    const bool xv = ldx % 4 == 0 && (reinterpret_cast<uintptr_t>(X) & 15) == 0;
    if (N <= 2) launch_chain_n<I8, 2, false>(ctx, W, X, N, ldx, Y, ldy_r, ldy_c, bias, c_size, beta, act);
    else if (N <= 4 && N == 4 && xv) launch_chain_n<I8, 4, true>(ctx, W, X, N, ldx, Y, ldy_r, ldy_c, bias, c_size, beta, act);
    else if (N <= 4) launch_chain_n<I8, 4, false>(ctx, W, X, N, ldx, Y, ldy_r, ldy_c, bias, c_size, beta, act);
    else if (N == 8 && xv) launch_chain_n<I8, 8, true>(ctx, W, X, N, ldx, Y, ldy_r, ldy_c, bias, c_size, beta, act);
    else launch_chain_n<I8, 8, false>(ctx, W, X, N, ldx, Y, ldy_r, ldy_c, bias, c_size, beta, act);
}

// Fast mode, N <= 8: one wave per row, lane l takes the row's nonzeros
// l, l + 64, ... (coalesced index and value streams).  Each lane issues the
// loads of U nonzeros at once (indices clamped into the row, so every load
// is unconditional and in flight together), then their X rows (two float4
// per nonzero for NB = 8 when X rows are 16-byte aligned), then fused
// multiply-adds into per-column partial sums, reduced across the wave at
// the end.  The sum is reassociated, so this kernel serves the fast mode
// only.  Columns are read as uint16 when the weight has that copy (K <=
// 65536: 3 bytes per int8 nonzero instead of 5).
//
// WG = true: the whole 256-thread workgroup takes one row (thread t takes
// the row's nonzeros t, t + 256, ...; the wave sums meet in LDS), so a row of
// a few thousand nonzeros has all its loads in flight at once instead of
// waiting for several rounds of one wave.
template <int NB, bool I8, bool XV, class CT, bool WG = false>
__global__ __launch_bounds__(256) void k_spmv_fast(
    int M, int N, const int32_t* __restrict__ rowptr, const CT* __restrict__ col,
    const void* __restrict__ val, const float* __restrict__ rs, const float* __restrict__ X, int64_t ldx,
    float* __restrict__ Y, int64_t ldy_r, int64_t ldy_c, const float* __restrict__ bias, int64_t c_size,
    float beta, int act) {
    constexpr int U = NB == 1 ? 16 : (NB <= 4 ? 8 : 4);
    constexpr int S = WG ? 256 : 64;  // threads sharing a row
    const int lane = WG ? (int)threadIdx.x : (int)(threadIdx.x & 63);
    const int row = WG ? (int)blockIdx.x
                       : __builtin_amdgcn_readfirstlane((int)blockIdx.x * kWaves + (int)(threadIdx.x >> 6));
    if (row >= M) return;
    const int beg = rowptr[row], end = rowptr[row + 1];
    float acc[NB];
#pragma unroll
    for (int c = 0; c < NB; ++c) acc[c] = 0.0f;
    for (int base = beg; base < end; base += S * U) {
        int cl[U];
        float w[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int jj = max(min(base + lane + S * u, end - 1), 0);
            cl[u] = (int)col[jj];
            w[u] = wval<I8>(val, rs, jj, row);
        }
        float xv[U][NB];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const float* xr = X + (int64_t)cl[u] * ldx;
            if constexpr (XV && NB % 4 == 0) {
#pragma unroll
                for (int c = 0; c < NB; c += 4) {
                    const float4 v = *reinterpret_cast<const float4*>(xr + c);
                    xv[u][c] = v.x; xv[u][c + 1] = v.y; xv[u][c + 2] = v.z; xv[u][c + 3] = v.w;
                }
            } else {
#pragma unroll
                for (int c = 0; c < NB; ++c) xv[u][c] = c < N ? xr[c] : 0.0f;
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (base + lane + S * u < end) {
#pragma unroll
                for (int c = 0; c < NB; ++c) acc[c] = __builtin_fmaf(w[u], xv[u][c], acc[c]);
            }
        }
    }
#pragma unroll
    for (int c = 0; c < NB; ++c) {
        float v = acc[c];
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
        acc[c] = v;
    }
    if constexpr (WG) {
        __shared__ float part[4][NB];
        const int wv = threadIdx.x >> 6, l = threadIdx.x & 63;
        if (l == 0) {
#pragma unroll
            for (int c = 0; c < NB; ++c) part[wv][c] = acc[c];
        }
        __syncthreads();
        if (wv != 0) return;
#pragma unroll
        for (int c = 0; c < NB; ++c) acc[c] = (part[0][c] + part[1][c]) + (part[2][c] + part[3][c]);
    }
    if (lane < N && lane < NB) {
        float v = acc[0];
#pragma unroll
        for (int c = 1; c < NB; ++c)
            if (lane == c) v = acc[c];
        const int64_t f = (int64_t)row * ldy_r + (int64_t)lane * ldy_c;
        Y[f] = bias_add(v, f, bias, c_size, beta, act);
    }
}

// x staged for the balanced copy's N = 1 kernel: chunk c of x (columns
// c * kcw .. c * kcw + kcw - 1) at xs[c * (kcw + 1) ..], each chunk followed
// by a zero (the slot its padding entries index), eight loads per thread in
// flight.
template <int NT>
__device__ __forceinline__ void stage_x_chunks(float* xs, const float* __restrict__ x, int K, int64_t ldx, int nch,
                                               int kcw, int tid) {
    if (nch == 1) {  // kcw == K: x with its zero at K
        stage_x<NT>(xs, x, K, ldx, tid);
        return;
    }
    const int n = nch * (kcw + 1);
    // e / (kcw + 1) as a multiply-high by a rounded-up reciprocal: exact for
    // e < 2^16 and a divisor below 2^13
    const uint32_t inv = 0xFFFFFFFFu / (uint32_t)(kcw + 1) + 1u;
    for (int e0 = 0; e0 < n; e0 += 8 * NT) {
        float t[8];
        int k[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int e = e0 + tid + NT * i;
            const int c = (int)__umulhi((uint32_t)e, inv);
            const int o = e - c * (kcw + 1);
            k[i] = o < kcw ? c * kcw + o : K;  // K: a zero slot (or past the end)
            t[i] = x[(int64_t)min(k[i], K - 1) * ldx];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int e = e0 + tid + NT * i;
            if (e < n) xs[e] = k[i] < K ? t[i] : 0.0f;
        }
    }
}

// Fast N = 1 SpMV over the nnz-balanced copy (layout at pfr_csr::bal_meta):
// every group holds about the same number of nonzeros however skewed the
// row lengths are (fixed 16-row slabs of rows sorted by length measured
// 1.45x slower on 4096 x 11008 at 30 % with lognormal rows, whose slab of
// the 16 longest rows holds 3.7x the mean slab's nonzeros).  A workgroup
// stages x once and takes H groups, W / H waves each (the copy holds about
// two groups per CU).  Within a group, R (the group's row count) is a power
// of two up to 64 and G = 64 / R: one wave instruction covers G consecutive
// quad rows (64 consecutive records: coalesced 4-byte int8 or 16-byte float
// values and 8-byte offset loads); lane (r, sub) takes row r of quad rows
// sub, sub + G, ... .  Each lane loads U records per batch, two batches in
// flight (quad rows clamped into the group, so every load is unconditional;
// a clamped record is folded as value 0 at a zero slot of x, as its own x
// may be inf or NaN), gathers their x values from LDS and accumulates with
// fused multiply-adds into four partial sums, reduced across the lanes of a
// row (shuffles) and then across the group's waves (LDS); an int8 row's sum
// is scaled once at the end.  The sum is reassociated, so this kernel serves
// the fast mode only.  Measured on the int8 decode shapes at 30 % (4096²,
// 11008 x 4096, 4096 x 11008): 6.1 / 11.0 / 12.8 us with U = 2 and two
// batches in flight, 6.7 / 11.8 / 13.3 us with U = 4 and one.
template <bool I8, int W, int H, int U>
__global__ __launch_bounds__(64 * W) void k_spmv_bal_fast(
    int K, int ngroup, int nch, int kcw, const int4* __restrict__ meta, const int32_t* __restrict__ perm,
    const void* __restrict__ vals, const uint16_t* __restrict__ cols, const float* __restrict__ rs,
    const float* __restrict__ x, int ldx, float* __restrict__ y, int64_t ldy_r, const float* __restrict__ bias,
    int64_t c_size, float beta, int act) {
    static_assert(W % H == 0, "waves split evenly over the groups");
    constexpr int WG = W / H;  // waves per group
    extern __shared__ float4 dyn[];
    float* const xs = reinterpret_cast<float*>(dyn);  // [nch * (kcw + 1)]
    __shared__ float part[W][64];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int gw = wave % WG;                                   // the wave's index within its group
    const int grp = (int)blockIdx.x * H + wave / WG;            // uniform
    const bool live = grp < ngroup;                             // the last workgroup's second group may not exist
    const int4 m = meta[min(grp, ngroup - 1)];
    const int lgR = __builtin_amdgcn_readfirstlane(m.x), p0 = __builtin_amdgcn_readfirstlane(m.y);
    const int rec0 = __builtin_amdgcn_readfirstlane(m.z), nq = live ? __builtin_amdgcn_readfirstlane(m.w) : 0;
    const int R = 1 << lgR, G = 64 >> lgR;
    using ValT = typename std::conditional<I8, uint32_t, float4>::type;
    const ValT* V = static_cast<const ValT*>(vals);
    const uint2* Cl = reinterpret_cast<const uint2*>(cols);
    const char* xb = reinterpret_cast<const char*>(xs);
    const int r = lane & (R - 1), sub = lane >> lgR;
    ValT va[U], vb[U];
    uint2 ca[U], cb[U];
    auto load = [&](ValT* v, uint2* cc, int b) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t at = rec0 + (int64_t)min(b + sub + G * WG * u, nq - 1) * R + r;
            v[u] = V[at];
            cc[u] = Cl[at];
        }
    };
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    // records past the group (clamped loads repeat its last one) are folded
    // as value 0 at the chunk-0 zero slot, with selects rather than branches
    const uint32_t z2 = (uint32_t)(4 * kcw) * 0x10001u;
    auto fold = [&](const ValT* v, const uint2* cc, int b) {
        const int g0 = b + sub;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const bool in = g0 + G * WG * u < nq;
            const uint32_t cx = in ? cc[u].x : z2, cy = in ? cc[u].y : z2;
            const float x0 = *reinterpret_cast<const float*>(xb + (cx & 0xFFFF));
            const float x1 = *reinterpret_cast<const float*>(xb + (cx >> 16));
            const float x2 = *reinterpret_cast<const float*>(xb + (cy & 0xFFFF));
            const float x3 = *reinterpret_cast<const float*>(xb + (cy >> 16));
            float w0, w1, w2, w3;
            if constexpr (I8) {
                const uint32_t q = in ? v[u] : 0u;
                w0 = (float)(int8_t)(q & 0xFF);
                w1 = (float)(int8_t)((q >> 8) & 0xFF);
                w2 = (float)(int8_t)((q >> 16) & 0xFF);
                w3 = (float)(int8_t)(q >> 24);
            } else {
                w0 = in ? v[u].x : 0.0f; w1 = in ? v[u].y : 0.0f;
                w2 = in ? v[u].z : 0.0f; w3 = in ? v[u].w : 0.0f;
            }
            a0 = __builtin_fmaf(w0, x0, a0);
            a1 = __builtin_fmaf(w1, x1, a1);
            a2 = __builtin_fmaf(w2, x2, a2);
            a3 = __builtin_fmaf(w3, x3, a3);
        }
    };
    const int step = G * WG * U;
    const int b0 = G * gw;
    const int nit = b0 < nq ? (nq - b0 + step - 1) / step : 0;  // the wave's batches (uniform)
    if (nit > 0) load(va, ca, b0);
    stage_x_chunks<64 * W>(xs, x, K, ldx, nch, kcw, tid);
    __syncthreads();
    // two batches in flight: batch i + 1's loads are issued before batch i is
    // folded (past the last batch they are clamped repeats, never folded)
    int i = 0;
    for (; i + 2 <= nit; i += 2) {
        load(vb, cb, b0 + (i + 1) * step);
        fold(va, ca, b0 + i * step);
        load(va, ca, b0 + (i + 2) * step);
        fold(vb, cb, b0 + (i + 1) * step);
    }
    if (i < nit) fold(va, ca, b0 + i * step);
    float acc = (a0 + a1) + (a2 + a3);
    for (int o = R; o < 64; o <<= 1) acc += __shfl_xor(acc, o, 64);
    if (lane < R) part[wave][lane] = acc;
    __syncthreads();
    if (gw != 0 || lane >= R || !live) return;
    float sum = 0.0f;
#pragma unroll
    for (int w = 0; w < WG; ++w) sum += part[wave + w][lane];
    const int row = perm[p0 + lane];
    if constexpr (I8) sum *= rs[row];
    const int64_t f = (int64_t)row * ldy_r;
    y[f] = bias_add(sum, f, bias, c_size, beta, act);
}

constexpr int kBalFastH = 2, kBalFastU = 2;  // groups per workgroup, records per lane and batch

template <bool I8>
void launch_bal_fast(pfr_ctx* ctx, const pfr_csr* W, const float* X, int64_t ldx, float* Y, int64_t ldy_r,
                     const float* bias, int64_t c_size, float beta, int act) {
    const size_t lds = (size_t)W->bal_nchunk * (W->bal_kcw + 1) * 4;  // at most 64 KiB (checked at upload)
    const unsigned grid = (unsigned)((W->bal_ngroup + kBalFastH - 1) / kBalFastH);
    hipLaunchKernelGGL((k_spmv_bal_fast<I8, 16, kBalFastH, kBalFastU>), dim3(grid), dim3(64 * 16), lds, ctx->stream,
                       (int)W->K, W->bal_ngroup, W->bal_nchunk, W->bal_kcw, W->bal_meta, W->bal_perm, W->bal_val,
                       W->bal_col, W->row_scale, X, (int)ldx, Y, ldy_r, bias, c_size, beta, act);
}

// The sum of v over the wave's 64 lanes, uniform (returned in an SGPR): DPP
// adds within quads, half rows and rows, then the row broadcasts carry the
// row sums into lane 63, which is read out.  One fixed order, so the same
// bits every time.
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_f(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROWS, 0xF, false));
}
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<0xB1, 0xF>(v);   // quad_perm [1, 0, 3, 2]
    v += dpp_f<0x4E, 0xF>(v);   // quad_perm [2, 3, 0, 1]
    v += dpp_f<0x141, 0xF>(v);  // row_half_mirror
    v += dpp_f<0x140, 0xF>(v);  // row_mirror: every lane holds its row's sum
    v += dpp_f<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
    v += dpp_f<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Entry k (0..3) of a four-entry record: value (int8 or float) and column.
template <bool I8>
__device__ __forceinline__ float rec_val(const typename std::conditional<I8, uint32_t, float4>::type& v, int k) {
    if constexpr (I8) return (float)(int8_t)((v >> (8 * k)) & 0xFF);
    else return k == 0 ? v.x : k == 1 ? v.y : k == 2 ? v.z : v.w;
}
__device__ __forceinline__ uint32_t rec_col(const uint2& c, int k) {
    const uint32_t h = k < 2 ? c.x : c.y;
    return (k & 1) ? (h >> 16) : (h & 0xFFFFu);
}

// A row cut by workgroup boundaries, finished by whichever of its
// contributors arrives last, so no workgroup waits for another (A: the
// workgroup where the row starts, Bw: the one that takes its end; `give`:
// the caller is not Bw).  Everything goes through device-scope (agent)
// atomics, which the hardware keeps coherent across the XCDs' L2 caches; an
// acquire/release fence would instead write back and invalidate the whole L2
// of the XCD, once per workgroup.
// - Two contributors (Bw == A + 1, the usual cut): each swaps its tagged
//   partial into xchg[Bw]; whoever finds the other's there holds both, adds
//   them in order (A's first) and clears the word.  One round trip.
// - More: each stores its partial (carry[2p] for A .. Bw - 1, carry[2Bw + 1]
//   for Bw), waits until the store is complete and counts itself in cnt[Bw];
//   the last arrival sums carry[2A] + ... + carry[2Bw + 1] in workgroup order
//   and clears the counter.
// The sum is the same whatever the arrival order.
template <bool I8>
__device__ __forceinline__ void merge_arrive(unsigned long long* __restrict__ xchg, float* __restrict__ carry,
                                             uint32_t* __restrict__ cnt, int p, bool give, float v, int A, int Bw,
                                             int row, float scale, float* __restrict__ y, int64_t ldy_r,
                                             const float* __restrict__ bias, int64_t c_size, float beta, int act) {
    float s;
    if (Bw == A + 1) {
        const unsigned long long mine = (give ? 1ull : 2ull) << 32 | (uint32_t)__float_as_int(v);
        const unsigned long long old =
            __hip_atomic_exchange(xchg + Bw, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if ((old >> 32) == 0) return;  // the other contributor finishes the row
        const float other = __int_as_float((int)(uint32_t)old);
        s = give ? v + other : other + v;
        __hip_atomic_store(xchg + Bw, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
        __hip_atomic_store(carry + (give ? 2 * p : 2 * p + 1), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);  // every counter zero: the partial has reached its coherent home
        const uint32_t old = __hip_atomic_fetch_add(cnt + Bw, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old != (uint32_t)(Bw - A)) return;
        s = __hip_atomic_load(carry + 2 * A, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (int t = A + 1; t < Bw; ++t)
            s += __hip_atomic_load(carry + 2 * t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s += __hip_atomic_load(carry + 2 * Bw + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(cnt + Bw, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if constexpr (I8) s *= scale;
    const int64_t f = (int64_t)row * ldy_r;
    y[f] = bias_add(s, f, bias, c_size, beta, act);
}

// Fast N = 1 SpMV with merge-path work partitioning (pfr_csr::mp_wave),
// reading the CSR's own uint16 columns and values, so it needs no copy of
// the weight.  Every wave takes an equal share of its workgroup's row ends
// and nonzeros, and workgroups end at row ends wherever a row is shorter
// than a share, so the launch is balanced however skewed the rows are.  A
// wave streams the records (four consecutive entries) that hold its share
// (lane l takes records l, l + 64, ...: coalesced 4-byte int8 or 16-byte
// float values and 8-byte column loads), U records per lane and batch, two
// batches in flight; loads past the share read the spare record after the
// last one, whose entries (like the last record's padding) are value 0 at
// x's zero slot.  x is staged in LDS once per workgroup.  Per lane, fused multiply-adds into four partial sums of the
// current segment; where a segment ends inside a batch (a uniform test
// against the next boundary), the batch's products are split with selects
// and the wave reduces the finished segment.  The segments are: the entries
// of the share's first record before the share (dropped; only a share that
// starts a workgroup, at a row end, begins inside a record), the rows whose
// ends the share takes, the row that continues past the share, and, when
// the share ends inside a record, that record's rest (dropped).
// Lane (e % 64) keeps the e-th finished row's sum, written out 64 rows at a
// time, so the walk stores nothing to memory.  A row that started in an
// earlier wave, and the continuing one, are left in LDS, and each wave, when
// it is done, counts itself in those rows' arrival counters (LDS atomics;
// the planner gives every shared row its first wave, the wave that takes its
// end and how many waves add to it): the last to arrive sums the row's
// partials in wave order and writes it, so no wave waits for another, and a
// row cut by a workgroup boundary goes on to merge_arrive.  The row scales
// those writes need are loaded at the start.  An int8 row's sum is scaled
// once at the end.  The sum is reassociated, so this kernel serves the fast
// mode only.
template <bool I8, int U, int XL>
__global__ __launch_bounds__(64 * pfr::kMergeWaves) void k_spmv_merge(
    int M, int K, int spare, const int2* __restrict__ wpart, const int4* __restrict__ wmeta,
    const int4* __restrict__ gpart,
    const int32_t* __restrict__ rowptr, const void* __restrict__ vals, const uint16_t* __restrict__ cols,
    const float* __restrict__ rs, const float* __restrict__ x, int ldx, float* __restrict__ y, int64_t ldy_r,
    const float* __restrict__ bias, int64_t c_size, float beta, int act, float* __restrict__ carry,
    unsigned long long* __restrict__ xchg, uint32_t* __restrict__ cnt) {
    constexpr int W = pfr::kMergeWaves, NT = 64 * W, B = 64 * U;  // B: records per wave and batch
    extern __shared__ float4 dyn[];
    float* const xs = reinterpret_cast<float*>(dyn);  // x[0 .. K) and zeros to XL * NT (K < XL * NT)
    __shared__ float hv[W], gv[W];  // each wave's partial of its first row (hv) and of its last (gv)
    // each wave's first row and that row's scale (entry W: the workgroup's
    // end), and the arrival counters of the rows the waves share (entry t:
    // the row wave t ends, W: the one continuing past the workgroup)
    __shared__ int wi[W + 1];
    __shared__ float wsc[W + 1];
    __shared__ uint32_t lcnt[W + 1];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int p = (int)blockIdx.x, q = p * W + wave;
    const int is = __builtin_amdgcn_readfirstlane(wpart[q].x), js = __builtin_amdgcn_readfirstlane(wpart[q].y);
    const int ie = __builtin_amdgcn_readfirstlane(wpart[q + 1].x);
    const int je = __builtin_amdgcn_readfirstlane(wpart[q + 1].y);
    using ValT = typename std::conditional<I8, uint32_t, float4>::type;
    const ValT* V = static_cast<const ValT*>(vals);
    const uint2* Cl = reinterpret_cast<const uint2*>(cols);
    const int ra = js >> 2, rb = (je + 3) >> 2;  // the records holding entries js .. je - 1
    const int nb = (rb - ra + B - 1) / B;
    ValT va[U], vb[U];
    uint2 ca[U], cb[U];
    auto load = [&](ValT* v, uint2* c, int b) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int rec = ra + b * B + 64 * u + lane;
            const int at = rec < rb ? rec : spare;
            v[u] = V[at];
            c[u] = Cl[at];
        }
        // keep the next batch's loads ahead of the fold of the one before:
        // scheduled after them, that fold's first use would wait for every
        // load in flight
        __builtin_amdgcn_sched_barrier(0);
    };
    // x's loads first (XL per thread), then the first batch's, so the wait
    // before x goes to LDS leaves the batch in flight
    // (x contiguous: copied straight into LDS, the slots from K on reading
    // zero; else through registers)
    const bool xdma = ldx == 1;
    float xt[XL];
    if (xdma) {
#pragma unroll
        for (int i = 0; i < XL; ++i) {
            const int sb = NT * i + wave * 64;
            lds_copy_dword(x, 4 * K, 4 * (sb + lane), (__attribute__((address_space(3))) void*)(xs + sb));
        }
        __builtin_amdgcn_sched_barrier(0);
    } else {
#pragma unroll
        for (int i = 0; i < XL; ++i) xt[i] = x[(int64_t)min(tid + NT * i, K - 1) * ldx];
    }
    // lane l: rowptr[is + l] (up to ie + 1), so the walk reads its row ends
    // from registers instead of waiting on memory at each one
    const int my_rp = rowptr[min(is + lane, ie < M ? ie + 1 : M)];
    __builtin_amdgcn_sched_barrier(0);
    load(va, ca, 0);  // unconditional (an empty share reads the spare record): waits after it stay exact
    const int4 g = gpart[p], wm = wmeta[q];
    const int rp_is = __builtin_amdgcn_readfirstlane(my_rp);
    // the scales the write-out needs, loaded now and used after the walk:
    // lane l's for row is + l, and those of the share's first and last rows
    float my_sc = 1.0f, sc_is = 1.0f, sc_ie = 1.0f;
    if constexpr (I8) {
        my_sc = is + lane < ie ? rs[is + lane] : 1.0f;
        sc_is = rs[min(is, M - 1)];
        sc_ie = rs[min(ie, M - 1)];
    }
    if (xdma) {
        // this wave's copies have landed: at most the first batch's 2 U
        // loads (issued after them) are still in flight
        constexpr int n = 2 * U;
        __builtin_amdgcn_s_waitcnt((n & 0xF) | ((n >> 4) << 14) | (7 << 4) | (0xF << 8));
    } else {
#pragma unroll
        for (int i = 0; i < XL; ++i) xs[tid + NT * i] = tid + NT * i < K ? xt[i] : 0.0f;
    }
    if (lane == 0) {
        gv[wave] = 0.0f;  // a share holding no entry of its last row adds nothing to it
        hv[wave] = 0.0f;
        wi[wave] = is;
        wsc[wave] = sc_is;
        lcnt[wave] = 0u;
        if (wave == W - 1) {
            wi[W] = ie;
            wsc[W] = sc_ie;
            lcnt[W] = 0u;
        }
    }
    __syncthreads();
    const bool head_cut = rp_is < js;  // the first row started in an earlier wave
    // segment k ends at: js for k < is (the first record's entries before
    // the share), rowptr[k + 1] for the rows whose ends the share takes, je
    // for the row that continues (k == ie) when the share ends inside a
    // record (past a whole record only padding follows, which adds +0), and
    // never after that
    auto row_end = [&](int k) {  // rowptr[k + 1], is <= k < ie
        return k + 1 - is < 64 ? __builtin_amdgcn_readlane(my_rp, k + 1 - is) : rowptr[k + 1];
    };
    auto seg_end = [&](int k) { return k < is ? js : k < ie ? row_end(k) : k == ie && (je & 3) ? je : INT_MAX; };
    int r = (js & 3) ? is - 1 : is;  // the current segment
    int bnd = seg_end(r), bnd2 = seg_end(r + 1);
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float outv = 0.0f;  // lane e % 64: the sum of finished row is + e
    auto flush = [&](int base, int n) {  // rows base .. base + n - 1 from lanes 0 .. n - 1
        const int row = base + lane;
        if (lane < n && !(row == is && head_cut)) {
            float v = outv;
            if constexpr (I8) v *= base == is ? my_sc : rs[row];
            const int64_t f = (int64_t)row * ldy_r;
            y[f] = bias_add(v, f, bias, c_size, beta, act);
        }
    };
    // segment r ends: reduce its partials (a) and keep the sum
    auto emit = [&]() {
        const float v = wave_sum((a[0] + a[1]) + (a[2] + a[3]));
        a[0] = a[1] = a[2] = a[3] = 0.0f;
        if (r >= is && r < ie) {
            const int e = r - is;
            if (r == is && head_cut && lane == 0) hv[wave] = v;
            outv = lane == (e & 63) ? v : outv;
            if ((e & 63) == 63) flush(r - 63, 64);
        } else if (r == ie && lane == 0) {
            gv[wave] = v;
        }
        ++r;
        bnd = bnd2;
        bnd2 = seg_end(r + 1);
    };
    auto fold = [&](const ValT* v, const uint2* c, int b) {
        const int n0 = 4 * (ra + b * B), n1 = n0 + 4 * B;  // the batch's entries n0 .. n1 - 1
        if (bnd >= n1) {  // no segment ends in this batch
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int k = 0; k < 4; ++k) a[k] = __builtin_fmaf(rec_val<I8>(v[u], k), xs[rec_col(c[u], k)], a[k]);
            return;
        }
        // products once, then each segment ending in the batch takes those
        // before its end
        float pr[U][4];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int k = 0; k < 4; ++k) pr[u][k] = rec_val<I8>(v[u], k) * xs[rec_col(c[u], k)];
        do {
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const bool pre = n0 + 4 * (64 * u + lane) + k < bnd;
                    a[k] += pre ? pr[u][k] : 0.0f;
                    pr[u][k] = pre ? 0.0f : pr[u][k];
                }
            emit();
        } while (bnd < n1);
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int k = 0; k < 4; ++k) a[k] += pr[u][k];
    };
    // batch b + 1's loads are issued before batch b is folded (past the last
    // batch they read the spare record and are never folded)
    int b = 0;
    for (; b + 2 <= nb; b += 2) {
        load(vb, cb, b + 1);
        fold(va, ca, b);
        load(va, ca, b + 2);
        fold(vb, cb, b + 1);
    }
    if (b < nb) fold(va, ca, b);
    while (r <= ie) emit();  // segments ending where the last batch ends (or a share of row ends only)
    flush(ie - ((ie - is) & 63), (ie - is) & 63);
    if (lane != 0) return;
    // count this wave in the rows it shares; the last arrival of a row (from
    // wave a0, or the workgroup's start when a0 < 0, to the one that takes
    // its end, b, or past the workgroup when b == W) finishes it
    auto arrive = [&](int a0, int b, int n) {
        const uint32_t old = __hip_atomic_fetch_add(lcnt + b, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (old != (uint32_t)(n - 1)) return;
        const int u1 = a0 < 0 ? 0 : a0;
        float s = u1 < b ? gv[u1] : hv[b];
        for (int u = u1 + 1; u < b; ++u) s += gv[u];
        if (u1 < b && b < W) s += hv[b];
        const int row = wi[b];
        if (a0 >= 0 && b < W) {
            if constexpr (I8) s *= wsc[b];
            const int64_t f = (int64_t)row * ldy_r;
            y[f] = bias_add(s, f, bias, c_size, beta, act);
        } else if (b < W) {  // the row started in an earlier workgroup (g.x)
            merge_arrive<I8>(xchg, carry, cnt, p, false, s, g.x, p, row, wsc[b], y, ldy_r, bias, c_size, beta, act);
        } else {  // the row continues past the workgroup, to g.y (it started in g.z)
            merge_arrive<I8>(xchg, carry, cnt, p, true, s, g.z, g.y, row, wsc[W], y, ldy_r, bias, c_size, beta, act);
        }
    };
    if (wm.x != -2) arrive(wm.x, wave, wm.w & 0xFFFF);
    if (wm.z != -1) arrive(wm.y, wm.z, wm.w >> 16);
}

constexpr int kMergeU = 2;  // records per lane and batch

template <bool I8>
void launch_merge(pfr_ctx* ctx, const pfr_csr* W, const float* X, int64_t ldx, float* Y, int64_t ldy_r,
                  const float* bias, int64_t c_size, float beta, int act) {
    constexpr int NT = 64 * pfr::kMergeWaves;
    const int xl = (int)(W->K / NT + 1);  // x loads per thread, K + 1 <= xl * NT (K <= kMergeMaxK, checked at upload)
    const int XLs = xl <= 5 ? 5 : xl <= 8 ? 8 : xl <= 12 ? 12 : 16;
    const size_t lds = (size_t)XLs * NT * 4;
#define PFR_MERGE(XLV)                                                                                          \
    hipLaunchKernelGGL((k_spmv_merge<I8, kMergeU, XLV>), dim3((unsigned)W->mp_groups), dim3(NT), lds, ctx->stream, \
                       (int)W->M, (int)W->K, (int)((W->nnz + 3) / 4), W->mp_wave, W->mp_wmeta, W->mp_grp,       \
                       W->rowptr, W->val,                                                                         \
                       W->col16, W->row_scale, X, (int)ldx, Y, ldy_r, bias, c_size, beta, act, W->mp_carry,       \
                       W->mp_xchg, W->mp_cnt)
    if (XLs == 5) PFR_MERGE(5);
    else if (XLs == 8) PFR_MERGE(8);
    else if (XLs == 12) PFR_MERGE(12);
    else PFR_MERGE(16);
#undef PFR_MERGE
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Fast 2 <= N <= 8 over the nnz-balanced copy: workgroup i takes the two
// groups of bal_pair[i] (the copy holds at most two per CU, paired largest
// with smallest), waves 0 .. na - 1 the first and the rest the second, na in
// proportion to their records, and walks K chunk by chunk: the chunk's X
// rows are staged in LDS as rows of eight floats (kcw + 1 rows with the zero
// row, 32 B each), then each group's waves fold its records of that chunk
// into per-lane sums (the two groups' record streams, and the
// latencies of their starts, overlap; walked one after the other with all
// sixteen waves, the second group's start measured as a bubble).  Lanes work
// in pairs: each lane loads its own record (four nonzeros of one row), takes
// its partner's by DPP, and reads one 16-byte half of the X row of all eight
// nonzeros (columns 4h .. 4h + 3 for lane parity h), so a pair reads a whole
// 32-byte row.  Records are loaded a batch ahead of the one folded, and each
// group's first batch of a chunk before the chunk is staged.  The sums of a
// row's lanes meet by shuffles, then across the group's waves in LDS (added
// in wave order, so the order is fixed).
template <bool I8, int W, int U, bool XV>
__global__ __launch_bounds__(64 * W) void k_spmm_bal_fast8(
    int K, int N, int kcw, int nch, const int4* __restrict__ pair, const int4* __restrict__ meta,
    const int2* __restrict__ cmeta, const int32_t* __restrict__ perm, const void* __restrict__ vals,
    const uint16_t* __restrict__ cols, const float* __restrict__ rs, const float* __restrict__ X, int64_t ldx,
    float* __restrict__ Y, int64_t ldy_r, int64_t ldy_c, const float* __restrict__ bias, int64_t c_size, float beta,
    int act) {
    static_assert(W == 16, "the pair table splits sixteen waves");
    constexpr int NT = 64 * W;
    // [(kcw + 1) * 2]: row k at xs[2k], xs[2k + 1]; after the walk, each
    // wave's row sums ([W][64][8] floats)
    extern __shared__ float4 xs[];
    const int tid = threadIdx.x, lane = tid & 63, h = lane & 1;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // the workgroup's pair: waves 0 .. na - 1 walk the first group, the rest
    // the second (wb: the group's first wave, nw its waves, gw and gt the
    // wave and thread in them)
    const int4 pq = pair[blockIdx.x];
    const int na = __builtin_amdgcn_readfirstlane(pq.z), second = wave >= na ? 1 : 0;
    const int wb = second ? na : 0, nw = second ? W - na : na, gw = wave - wb, gt = tid - 64 * wb;
    using ValT = typename std::conditional<I8, uint32_t, float4>::type;
    const ValT* V = static_cast<const ValT*>(vals);
    const uint2* Cl = reinterpret_cast<const uint2*>(cols);
    const char* xbh = reinterpret_cast<const char*>(xs) + 16 * h;  // this lane's half of every X row
    const int grp = __builtin_amdgcn_readfirstlane(second ? pq.y : pq.x);
    const bool live = grp >= 0;
    const int lgR = live ? __builtin_amdgcn_readfirstlane(meta[grp].x) : 0;
    const int R = 1 << lgR, G = 64 >> lgR;
    const int r = lane & (R - 1), sub = lane >> lgR, psub = (lane ^ 1) >> lgR;
    // own[e]: the lane's row, column 4h + e; par[e]: the partner lane's row,
    // same columns
    float own[4] = {0.0f, 0.0f, 0.0f, 0.0f}, par[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    ValT va[U], vb[U];
    uint2 ca[U], cb[U];
    auto load = [&](ValT* v, uint2* cc, int rec0, int nq, int b) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t at = rec0 + (int64_t)min(b + sub + G * nw * u, nq - 1) * R + r;
            v[u] = V[at];
            cc[u] = Cl[at];
        }
    };
    // the group's output row and scale (group thread t < 8R writes row t / 8,
    // column t % 8), loaded now rather than as dependent loads at the end
    int orow = 0;
    float oscale = 1.0f;
    if (live && gt < (8 << lgR)) {
        orow = perm[meta[grp].y + (gt >> 3)];
        if constexpr (I8) oscale = rs[orow];
    }
    // DPP quad_perm [1, 0, 3, 2]: the partner lane's value
    auto swap = [](auto v) { return __builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false); };
    const int step = G * nw * U, b0 = G * gw;
    int2 cm = live ? cmeta[grp * nch] : make_int2(0, 0);
    for (int ch = 0; ch < nch; ++ch) {
        const int rec0 = __builtin_amdgcn_readfirstlane(cm.x), nq = __builtin_amdgcn_readfirstlane(cm.y);
        const int nit = b0 < nq ? (nq - b0 + step - 1) / step : 0;  // the wave's batches (uniform)
        // the chunk's first batch is requested before X is staged, so their
        // latencies overlap
        if (nit > 0) load(va, ca, rec0, nq, b0);
        if (live && ch + 1 < nch) cm = cmeta[grp * nch + ch + 1];
        // stage the chunk's X rows: eight 16-byte (XV) or 4-byte loads per
        // thread in flight, clamped; rows past the chunk or K are zero
        const int k0 = ch * kcw, nq4 = (kcw + 1) * 2;  // float4 slots
        const uint32_t cbase = (uint32_t)(ch * (kcw + 1) * 4);  // byte offset of the chunk's first float
        bool copied = false;
        if constexpr (XV) {
            if (kcw >= 32) {
                // 16-byte rows straight from X into LDS: slot e (row e / 2,
                // half e % 2) from lane e - base of a wave instruction at
                // base, the last instruction moved back to end at the last
                // row (it rewrites slots with the same bytes); rows are
                // clamped to X's last one (rows past K in the last chunk are
                // never read: every stored column is below K), and the zero
                // row kcw is written once the copies have landed.  (Through
                // registers this took about a quarter of the kernel's
                // vector instructions: the 64-bit address of every piece.)
                const int nslot = 2 * kcw;
                for (int e0 = wave * 64; e0 < nslot; e0 += NT) {
                    const int base = min(e0, nslot - 64), e = base + lane;
                    const int k = min(k0 + (e >> 1), K - 1);
                    __builtin_amdgcn_global_load_lds(X + (int64_t)k * ldx + (e & 1) * 4,
                                                     (__attribute__((address_space(3))) void*)((__attribute__((address_space(3))) char*)xs + base * 16),
                                                     16, 0, 0);
                }
                __builtin_amdgcn_s_waitcnt(0);  // every counter: this wave's copies have landed
                if (tid < 2) xs[nslot + tid] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                copied = true;
            }
        }
        for (int e0 = 0; !copied && e0 < nq4; e0 += 8 * NT) {
            float4 t[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int e = min(e0 + tid + NT * i, nq4 - 1);
                const int k = min(k0 + (e >> 1), K - 1), c0 = (e & 1) * 4;
                const float* xr = X + (int64_t)k * ldx;
                if constexpr (XV) {
                    t[i] = *reinterpret_cast<const float4*>(xr + c0);
                } else {
                    t[i].x = xr[min(c0, N - 1)];
                    t[i].y = xr[min(c0 + 1, N - 1)];
                    t[i].z = xr[min(c0 + 2, N - 1)];
                    t[i].w = xr[min(c0 + 3, N - 1)];
                }
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int e = e0 + tid + NT * i;
                if (e < nq4) {
                    const int kk = e >> 1, c0 = (e & 1) * 4;
                    float4 v = t[i];
                    if (kk >= kcw || k0 + kk >= K) v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    if (c0 >= N) v.x = 0.0f;
                    if (c0 + 1 >= N) v.y = 0.0f;
                    if (c0 + 2 >= N) v.z = 0.0f;
                    if (c0 + 3 >= N) v.w = 0.0f;
                    xs[e] = v;
                }
            }
        }
        __syncthreads();
        // one batch: U records of this lane and U of its partner; a record
        // past the chunk's quad rows (a clamped repeat) adds nothing
        auto fold = [&](const ValT* v, const uint2* cc, int b) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const bool in_own = b + sub + G * nw * u < nq, in_par = b + psub + G * nw * u < nq;
                float wo[4], wp[4];
                if constexpr (I8) {
                    const uint32_t qo = v[u], qp = (uint32_t)swap(v[u]);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        wo[j] = (float)(int8_t)((qo >> (8 * j)) & 0xFF);
                        wp[j] = (float)(int8_t)((qp >> (8 * j)) & 0xFF);
                    }
                } else {
                    wo[0] = v[u].x; wo[1] = v[u].y; wo[2] = v[u].z; wo[3] = v[u].w;
                    wp[0] = __int_as_float(swap(__float_as_int(v[u].x)));
                    wp[1] = __int_as_float(swap(__float_as_int(v[u].y)));
                    wp[2] = __int_as_float(swap(__float_as_int(v[u].z)));
                    wp[3] = __int_as_float(swap(__float_as_int(v[u].w)));
                }
                const uint32_t px = (uint32_t)swap(cc[u].x), py = (uint32_t)swap(cc[u].y);
                // offsets count x's floats from the start of chunk 0 (with
                // the zeros after earlier chunks); a staged X row is 32
                // bytes, eight times a float
                const uint32_t oo[4] = {(cc[u].x & 0xFFFF) - cbase, (cc[u].x >> 16) - cbase,
                                        (cc[u].y & 0xFFFF) - cbase, (cc[u].y >> 16) - cbase};
                const uint32_t op[4] = {(px & 0xFFFF) - cbase, (px >> 16) - cbase, (py & 0xFFFF) - cbase,
                                        (py >> 16) - cbase};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float4 xo = *reinterpret_cast<const float4*>(xbh + (oo[j] << 3));
                    const float4 xp = *reinterpret_cast<const float4*>(xbh + (op[j] << 3));
                    if (in_own) {
                        own[0] = __builtin_fmaf(wo[j], xo.x, own[0]);
                        own[1] = __builtin_fmaf(wo[j], xo.y, own[1]);
                        own[2] = __builtin_fmaf(wo[j], xo.z, own[2]);
                        own[3] = __builtin_fmaf(wo[j], xo.w, own[3]);
                    }
                    if (in_par) {
                        par[0] = __builtin_fmaf(wp[j], xp.x, par[0]);
                        par[1] = __builtin_fmaf(wp[j], xp.y, par[1]);
                        par[2] = __builtin_fmaf(wp[j], xp.z, par[2]);
                        par[3] = __builtin_fmaf(wp[j], xp.w, par[3]);
                    }
                }
            }
        };
        // batch i + 1's loads are issued before batch i is folded (past the
        // last batch they are clamped repeats, never folded)
        int i = 0;
        for (; i + 2 <= nit; i += 2) {
            load(vb, cb, rec0, nq, b0 + (i + 1) * step);
            fold(va, ca, b0 + i * step);
            load(va, ca, rec0, nq, b0 + (i + 2) * step);
            fold(vb, cb, b0 + (i + 1) * step);
        }
        if (i < nit) fold(va, ca, b0 + i * step);
        __syncthreads();  // the next chunk overwrites X
    }
    // R = 1: every lane's record and its partner's are of row 0
    if (R == 1) {
#pragma unroll
        for (int e = 0; e < 4; ++e) own[e] += par[e];
    }
    // lanes of one row and half: lane ^ s for s = max(R, 2) .. 32
#pragma unroll
    for (int e = 0; e < 4; ++e)
        for (int s = R < 2 ? 2 : R; s < 64; s <<= 1) {
            own[e] += __shfl_xor(own[e], s, 64);
            if (R > 1) par[e] += __shfl_xor(par[e], s, 64);
        }
    // lane r < max(R, 2) holds row r's half h (own) and, for R > 1, row r ^
    // 1's half h (par): every (row, column) once per wave, stored to the
    // wave's slot (X is no longer read: the last chunk's barrier is behind)
    float(*const ws)[64][8] = reinterpret_cast<float(*)[64][8]>(xs);
    if (lane < (R < 2 ? 2 : R)) {
        const int ro = R < 2 ? 0 : lane, rp = lane ^ 1;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            ws[wave][ro][4 * h + e] = own[e];
            if (R > 1) ws[wave][rp][4 * h + e] = par[e];
        }
    }
    __syncthreads();
    // the group's threads write its R x 8 outputs (row o / 8, column o % 8),
    // each the sum of the group's waves in wave order
    for (int o = gt; live && o < R * 8; o += 64 * nw) {
        const int rr = o >> 3, c = o & 7;
        float sum = ws[wb][rr][c];
        for (int w2 = 1; w2 < nw; ++w2) sum += ws[wb + w2][rr][c];
        if (c < N) {
            const int row = o == gt ? orow : perm[meta[grp].y + rr];
            if constexpr (I8) sum *= o == gt ? oscale : rs[row];
            const int64_t f = (int64_t)row * ldy_r + (int64_t)c * ldy_c;
            Y[f] = bias_add(sum, f, bias, c_size, beta, act);
        }
    }
}

// Records per lane and batch of the batch kernel.  With the waves balanced
// by the pair table, one record per batch measured fastest: the first
// batch, which all 4096 waves ask for together, is a quarter of the size
// at U = 4 (stacked batch-8 step 2.42-2.49 ms against 2.50-2.61 at U = 2
// and 2.67-2.84 at U = 4).
constexpr int kBalFast8U = 1;

template <bool I8, bool XV>
void launch_bal_fast8(pfr_ctx* ctx, const pfr_csr* W, const float* X, int N, int64_t ldx, float* Y,
                      int64_t ldy_r, int64_t ldy_c, const float* bias, int64_t c_size, float beta, int act) {
    auto kern = k_spmm_bal_fast8<I8, 16, kBalFast8U, XV>;
    // the X chunk, and after the walk the waves' sums (16 x 64 x 8 floats):
    // <= (4096 + 1) * 32 B = 128 KiB
    const size_t lds = std::max<size_t>((size_t)(W->bal_kcw + 1) * 32, 16 * 64 * 8 * sizeof(float));
    static uint64_t allowed = 0;  // bit d: the dynamic LDS limit raised on device d (< 64)
    const uint64_t bit = ctx->device < 64 ? (uint64_t(1) << ctx->device) : 0;
    if (lds > 65536 && (!bit || !(__atomic_load_n(&allowed, __ATOMIC_ACQUIRE) & bit))) {
        PFR_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)((pfr::kBalChunk + 1) * 32)));
        if (bit) __atomic_fetch_or(&allowed, bit, __ATOMIC_RELEASE);
    }
    hipLaunchKernelGGL(kern, dim3((unsigned)W->bal_npair), dim3(64 * 16), lds, ctx->stream, (int)W->K, N,
                       W->bal_kcw, W->bal_nchunk, W->bal_pair, W->bal_meta, W->bal_cmeta, W->bal_perm, W->bal_val, W->bal_col,
                       W->row_scale, X, ldx, Y, ldy_r, ldy_c, bias, c_size, beta, act);
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

// The same transpose for rows and cols multiples of 4 and a 16-byte aligned
// A: 16-byte loads and stores, every load issued before the first LDS
// write (addresses clamped into the matrix, out-of-range values dropped).
// Both LDS passes are free of bank conflicts (row pitch 65).
__global__ __launch_bounds__(256) void k_transpose_scale4(const float* __restrict__ A, int64_t rows,
                                                          int64_t cols, float alpha, int scale,
                                                          float* __restrict__ At) {
    __shared__ float tile[64][65];
    const int t = threadIdx.x;
    const int64_t c0 = (int64_t)blockIdx.x * 64, r0 = (int64_t)blockIdx.y * 64;
    const int lc = (t & 15) * 4;
    float4 v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t r = r0 + (t >> 4) + 16 * i, c = c0 + lc;
        const int64_t rc = r < rows ? r : rows - 1, cc = c < cols ? c : cols - 4;
        v[i] = *reinterpret_cast<const float4*>(A + rc * cols + cc);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int lr = (t >> 4) + 16 * i;
        float4 w = v[i];
        if (scale) {
            w.x = alpha * w.x;
            w.y = alpha * w.y;
            w.z = alpha * w.z;
            w.w = alpha * w.w;
        }
        tile[lr][lc] = w.x;
        tile[lr][lc + 1] = w.y;
        tile[lr][lc + 2] = w.z;
        tile[lr][lc + 3] = w.w;
    }
    __syncthreads();
    const int lr4 = (t & 15) * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int lcol = (t >> 4) + 16 * i;
        const int64_t c = c0 + lcol, r = r0 + lr4;
        if (c < cols && r < rows)
            *reinterpret_cast<float4*>(At + c * rows + r) =
                make_float4(tile[lr4][lcol], tile[lr4 + 1][lcol], tile[lr4 + 2][lcol], tile[lr4 + 3][lcol]);
    }
}

__global__ __launch_bounds__(256) void k_scale(const float* __restrict__ A, int64_t n, float alpha,
                                               float* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = alpha * A[i];
}

template <int I, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < E) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, E>(f);
    }
}

template <int W>
constexpr int sell_loads_per_iter() {
    // a chunk's 16-row loads per wave, spread over about three iterations of
    // the walk (four groups each); the rest are issued after the walk
    return (pfr::kSellMaxKC / 16 / W + 2) / 3;
}

using lds_char = __attribute__((address_space(3))) char;

// One (slab, chunk) run of the column-slice kernel: T groups of 8 steps.
// The groups' int4 sit in a ring of four registers: four groups per
// iteration, each reloaded with the group four ahead as soon as it is used
// (so loads run three groups ahead), past the run's end into the next run or
// the tail, and never used there; a last partial iteration uses what is
// already loaded.  xb is the lane's view of the chunk's X rows.  With MORE,
// the walk also copies DPI 16-row blocks of the next chunk per iteration
// into nxt, through registers: loaded in one iteration, written to LDS in the
// next, so each wait is for loads one iteration old.  Block i is rows 16j ..
// 16j+15, j = min(j0 + jstep * i, jmax); lane 4r+q copies row min(16j + r,
// last) of src (which points at the lane's four columns) to nxt + 1024 j +
// 16 lane.  The loads are unconditional (clamped), so no branch splits the
// load queue; d counts the blocks issued.
template <bool FAST, bool MORE, int DPI>
__device__ __forceinline__ void sell_walk(const int4* __restrict__ blk, int p, int T, const char* __restrict__ xb,
                                          float4* __restrict__ nxt, const float* __restrict__ src, int64_t ldx,
                                          int lane, int j0, int jstep, int jmax, int last, int& d, float& a0,
                                          float& a1, float& a2, float& a3) {
    auto comp = [&](const int4 w) {
        float4 xv[8];
        static_for<0, 8>([&](auto tc) {
            constexpr int t = decltype(tc)::value, ctrl = (t / 2) * 0x55;  // quad_perm [j,j,j,j]
            const int o = __builtin_amdgcn_mov_dpp((t & 1) ? w.z : w.x, ctrl, 0xF, 0xF, true);
            xv[t] = *reinterpret_cast<const float4*>(xb + o);
        });
        if constexpr (FAST) {
        static_for<0, 8>([&](auto tc) {
            constexpr int t = decltype(tc)::value, ctrl = (t / 2) * 0x55;
            const float wv = __int_as_float(__builtin_amdgcn_mov_dpp((t & 1) ? w.w : w.y, ctrl, 0xF, 0xF, true));
            a0 = madd<FAST>(a0, wv, xv[t].x);
            a1 = madd<FAST>(a1, wv, xv[t].y);
            a2 = madd<FAST>(a2, wv, xv[t].z);
            a3 = madd<FAST>(a3, wv, xv[t].w);
        });
        } else {
            // the group's 32 products first, then the adds in storage order
            // behind a scheduling barrier, so no add waits on the multiply
            // just before it (N = 256: 44.8 -> 43.2 us, same bits)
            float pr[8][4];
            static_for<0, 8>([&](auto tc) {
                constexpr int t = decltype(tc)::value, ctrl = (t / 2) * 0x55;
                const float wv = __int_as_float(__builtin_amdgcn_mov_dpp((t & 1) ? w.w : w.y, ctrl, 0xF, 0xF, true));
                pr[t][0] = wv * xv[t].x;
                pr[t][1] = wv * xv[t].y;
                pr[t][2] = wv * xv[t].z;
                pr[t][3] = wv * xv[t].w;
            });
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                a0 = a0 + pr[t][0];
                a1 = a1 + pr[t][1];
                a2 = a2 + pr[t][2];
                a3 = a3 + pr[t][3];
            }
        }
    };
    const int r = lane >> 2;
    constexpr int ND = MORE ? DPI : 1;
    using f4 = float __attribute__((ext_vector_type(4)));  // a plain vector: stays in registers
    f4 st[ND];
    int js[ND];
    auto load_next = [&]() {
#pragma unroll
        for (int i = 0; i < ND; ++i) {
            js[i] = min(j0 + jstep * (d + i), jmax);
            st[i] = *reinterpret_cast<const f4*>(src + (int64_t)min(js[i] * 16 + r, last) * ldx);
        }
        d += ND;
    };
    auto store_next = [&]() {
#pragma unroll
        for (int i = 0; i < ND; ++i) *reinterpret_cast<f4*>(nxt + js[i] * 64 + lane) = st[i];
    };
    int4 w0 = blk[p], w1 = blk[p + 64], w2 = blk[p + 128], w3 = blk[p + 192];
    if constexpr (MORE) load_next();
    int t = 0;
    for (; t + 4 <= T; t += 4) {
        comp(w0);
        w0 = blk[p + 256];
        asm volatile("" ::: "memory");  // keep each reload ahead of the next group's LDS reads
        comp(w1);
        w1 = blk[p + 320];
        asm volatile("" ::: "memory");
        if constexpr (MORE) {
            store_next();
            load_next();
        }
        comp(w2);
        w2 = blk[p + 384];
        asm volatile("" ::: "memory");
        comp(w3);
        w3 = blk[p + 448];
        asm volatile("" ::: "memory");
        p += 256;
    }
    if (t < T) comp(w0);
    if (t + 1 < T) comp(w1);
    if (t + 2 < T) comp(w2);
    if constexpr (MORE) store_next();
}

// The walk of one run for the 4-wave launch's walking waves (one wave per
// SIMD, nothing else to hide their latencies): a ring of eight groups' int4
// (loads seven groups ahead), the X rows of group g + 1 read from LDS before
// the products of group g, kept apart by a scheduling barrier so the reads
// are issued a whole group before their use, and in strict mode the group's
// 32 products computed before its adds (in storage order), so no add waits
// on the multiply just before it.  Measured against the plain walk on the
// 4096 x 4096, 10 % weight: N = 16 19.6 -> 17.3 us, N = 64 20.4 -> 19.0 us
// strict and 19.1 -> 15.8 us fast; with two waves per SIMD (the 8-wave
// launch) it did not help.
template <bool FAST>
__device__ __forceinline__ void sell_walk_pipe(const int4* __restrict__ blk, int p, int T, const char* __restrict__ xb,
                                               float& a0, float& a1, float& a2, float& a3) {
    constexpr int R = 8;
    auto fetch = [&](const int4 w, float4 (&xv)[8]) {
        static_for<0, 8>([&](auto tc) {
            constexpr int t = decltype(tc)::value, ctrl = (t / 2) * 0x55;
            const int o = __builtin_amdgcn_mov_dpp((t & 1) ? w.z : w.x, ctrl, 0xF, 0xF, true);
            xv[t] = *reinterpret_cast<const float4*>(xb + o);
        });
    };
    auto accum = [&](const int4 w, const float4 (&xv)[8]) {
        if constexpr (FAST) {
            static_for<0, 8>([&](auto tc) {
                constexpr int t = decltype(tc)::value, ctrl = (t / 2) * 0x55;
                const float wv = __int_as_float(__builtin_amdgcn_mov_dpp((t & 1) ? w.w : w.y, ctrl, 0xF, 0xF, true));
                a0 = __builtin_fmaf(wv, xv[t].x, a0);
                a1 = __builtin_fmaf(wv, xv[t].y, a1);
                a2 = __builtin_fmaf(wv, xv[t].z, a2);
                a3 = __builtin_fmaf(wv, xv[t].w, a3);
            });
        } else {
            // the group's 32 products first, then the adds in storage order
            float pr[8][4];
            static_for<0, 8>([&](auto tc) {
                constexpr int t = decltype(tc)::value, ctrl = (t / 2) * 0x55;
                const float wv = __int_as_float(__builtin_amdgcn_mov_dpp((t & 1) ? w.w : w.y, ctrl, 0xF, 0xF, true));
                pr[t][0] = wv * xv[t].x;
                pr[t][1] = wv * xv[t].y;
                pr[t][2] = wv * xv[t].z;
                pr[t][3] = wv * xv[t].w;
            });
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                a0 = a0 + pr[t][0];
                a1 = a1 + pr[t][1];
                a2 = a2 + pr[t][2];
                a3 = a3 + pr[t][3];
            }
        }
    };
    int4 wr[R];
    static_for<0, R>([&](auto ic) { wr[decltype(ic)::value] = blk[p + 64 * decltype(ic)::value]; });
    float4 xa[8], xc[8];
    fetch(wr[0], xa);  // in bounds and unused when T = 0
    auto group = [&](auto ic, bool has_next) {
        constexpr int i = decltype(ic)::value;
        if constexpr (i & 1) {
            if (has_next) fetch(wr[(i + 1) % R], xa);
            __builtin_amdgcn_sched_barrier(0);
            accum(wr[i], xc);
        } else {
            if (has_next) fetch(wr[(i + 1) % R], xc);
            __builtin_amdgcn_sched_barrier(0);
            accum(wr[i], xa);
        }
    };
    int t = 0;
    for (; t + R <= T; t += R) {
        static_for<0, R>([&](auto ic) {
            constexpr int i = decltype(ic)::value;
            group(ic, true);  // past the run's end the next group's reads are in bounds and unused
            wr[i] = blk[p + 64 * (R + i)];
            asm volatile("" ::: "memory");
        });
        p += 64 * R;
    }
    static_for<0, R - 1>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        if (t + i < T) group(ic, t + i + 1 < T);
    });
}

// Column-slice kernel over the sliced-ELL copy (layout at pfr_csr::sell_blk).
// A workgroup of W waves owns W slabs (16 rows each) and one 16-column slice
// of X.  X is staged chunk by chunk (kc rows of 64 B) into two LDS buffers:
// while the waves walk chunk c in one buffer, the 16-row loads of chunk c + 1
// go straight from global memory into the other (global_load_lds, one 1 KiB
// load per wave instruction), interleaved with the walk.  Each wave walks its
// slab: lane 4r+q accumulates columns 4q..4q+3 of slab row r.  The pairs of a
// step come from one int4 per lane per eight steps, broadcast to the row's
// four lanes with quad_perm DPP (which the compiler folds into the address
// add and the multiply).  Products are added in the row's storage order, so
// strict mode matches the row kernels bit for bit; padding steps add
// RN(+0 * +0) = +0, which leaves any sum unchanged (an accumulator that
// starts at +0 never becomes -0 under RN addition).
// With one or two waves per SIMD (W = 4, 8) and 16-byte X rows, the
// workgroup has one more wave that only stages X: while the W waves walk
// chunk c, it copies chunk c + 1 into the other buffer with direct-to-LDS
// loads and waits for them, then meets the others at the chunk's barrier.
// (Staged by the walking waves themselves, through registers, a chunk cost
// about 35 clocks per step of the walk, measured with s_memtime: 10.6k
// against 6.6k clocks for the last chunk, which stages nothing; with a DMA
// in flight the compiler makes every later LDS read of that wave wait for
// all its loads.)
template <bool XVEC, int W, bool XT>
constexpr bool sell_stager() { return (XVEC || XT) && W <= 8; }
template <bool XVEC, int W, bool XT>
constexpr int sell_threads() { return 64 * (W + (sell_stager<XVEC, W, XT>() ? 1 : 0)); }

// XT: X is given transposed, as the Gemm form's activation A (N x K,
// row-major, rows ldx floats apart, 16-byte aligned, K % 4 == 0): each
// chunk is staged from A's rows through registers into the same LDS layout,
// scaled by alpha when `scale` (RN(alpha * a), the operand the reference's
// Gemm multiplies), so no transposed copy is written first.  The 16-wave
// launch stages every chunk with all its waves; the 4- and 8-wave launches
// take it only for one chunk, staged by all their waves.
template <bool FAST, bool XVEC, int W, bool XT>
__global__ __launch_bounds__((sell_threads<XVEC, W, XT>())) void k_spmm_sell(
    int N, int K, int kc, int nch, int nslab, const int32_t* __restrict__ perm,
    const int32_t* __restrict__ soff, const int4* __restrict__ blk, const float* __restrict__ X,
    int64_t ldx, float* __restrict__ Y, int64_t ldy_r, int64_t ldy_c, int yvec,
    const float* __restrict__ bias, int64_t c_size, float beta, int act, float alpha, int scale) {
    // two buffers of kc + 1 rows of 16 floats; row kc of each is zero
    extern __shared__ float4 xs[];
    constexpr int NT = 64 * W;  // the walking waves' threads
    constexpr bool STAGER = sell_stager<XVEC, W, XT>();
    constexpr int DPI = sell_loads_per_iter<W>();
    const int tid = threadIdx.x, lane = tid & 63, r = lane >> 2, q = lane & 3;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int slab = __builtin_amdgcn_readfirstlane((int)blockIdx.x * W + wave);
    const int n0 = (int)blockIdx.y * pfr::kSellCols;
    const int bufq = (kc + 1) * 4;  // float4 per buffer
    if (tid < 8) xs[(tid >> 2) * bufq + kc * 4 + (tid & 3)] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;

    // Load i of this wave for chunk c: rows 16j .. 16j+15 of the chunk, lane
    // 4r+q copying row 16j+r, columns n0+4q .. n0+4q+3, to LDS bytes
    // j*1024 + 16*lane of the chunk's buffer.  Loads past the wave's share
    // repeat its last one, rows past K repeat the chunk's last row and
    // columns past N repeat the last four; nothing reads those copies.
    const int nld = kc / 16;
    const int nd = (nld + W - 1) / W;
    const float* xcol = X + min(n0 + q * 4, N - 4);
    auto dma = [&](int c, int i) {
        const int j = min(wave + W * i, nld - 1);
        const int k0 = c * kc, last = min(kc, K - k0) - 1;
        const float* src = xcol + (int64_t)(k0 + min(j * 16 + r, last)) * ldx;
        lds_char* dst = (lds_char*)(xs + (c & 1) * bufq) + j * 1024;
        __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
    };
    // Register staging (any N and alignment) of chunk c into its buffer.
    auto stage_regs = [&](int c) {
        const int k0 = c * kc, rows = min(kc, K - k0);
        float4* xb = xs + (c & 1) * bufq;
        for (int e = tid; e < kc * 4; e += NT) {
            const int kr = e >> 2, n = n0 + (e & 3) * 4;
            float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (kr < rows) {
                const float* xr = X + (int64_t)(k0 + kr) * ldx;
                if (n < N) v.x = xr[n];
                if (n + 1 < N) v.y = xr[n + 1];
                if (n + 2 < N) v.z = xr[n + 2];
                if (n + 3 < N) v.w = xr[n + 3];
            }
            xb[e] = v;
        }
    };
    // XT staging of chunk c by threads t, t + nthr, ..: piece e is the float4
    // of A's row n0 + e % 16 at k = 4 (e / 16) (eight loads in flight,
    // clamped addresses), written as four floats of four LDS rows; piece e
    // writes its floats in the order j = (i + e / 16) % 4 (i = 0..3), so the
    // four groups of 16 lanes in one write instruction hit four different
    // 16-bank quarters (rows 64 B apart would otherwise all meet in one).
    // Rows past N or K are zero.
    auto stage_xt = [&](int c, int t, int nthr) {
        const int k0 = c * kc, total = 4 * kc;  // 16 rows x kc / 4 pieces
        float* xb = reinterpret_cast<float*>(xs + (c & 1) * bufq);
        for (int e0 = 0; e0 < total; e0 += 8 * nthr) {
            float4 v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int e = min(e0 + t + nthr * i, total - 1), n = e & 15, k = k0 + 4 * (e >> 4);
                v[i] = *reinterpret_cast<const float4*>(X + (int64_t)min(n0 + n, N - 1) * ldx + min(k, K - 4));
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int e = e0 + t + nthr * i;
                if (e < total) {
                    const int n = e & 15, kq = e >> 4, kl = 4 * kq;
                    const bool ok = n0 + n < N && k0 + kl < K;
                    const float a[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
                    for (int ii = 0; ii < 4; ++ii) {
                        const int j = (ii + kq) & 3;
                        const float x = j == 0 ? a[0] : (j == 1 ? a[1] : (j == 2 ? a[2] : a[3]));
                        const float y = scale ? alpha * x : x;
                        xb[(kl + j) * 16 + n] = ok ? y : 0.0f;
                    }
                }
            }
        }
    };
    auto sync_chunk = [&]() {
        if constexpr (XVEC && !XT) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's loads have landed
        __syncthreads();
    };

    if constexpr (STAGER) {
        if (wave == W) {
            // the staging wave: every 16-row load of each chunk, one chunk
            // ahead of the walk, then the same barriers as the walking waves
            auto stage = [&](int c) {
                if constexpr (XT) {
                    stage_xt(c, lane, 64);
                } else {
                    const int k0 = c * kc, last = min(kc, K - k0) - 1;
                    lds_char* dst = (lds_char*)(xs + (c & 1) * bufq);
                    for (int j = 0; j < nld; ++j) {
                        const float* src = xcol + (int64_t)(k0 + min(j * 16 + r, last)) * ldx;
                        __builtin_amdgcn_global_load_lds(src, dst + j * 1024, 16, 0, 0);
                    }
                    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the chunk has landed
                }
            };
            // XT: every thread stages chunk 0 (launched only with one chunk)
            if constexpr (XT) stage_xt(0, tid, NT + 64);
            else stage(0);
            __syncthreads();
            for (int c = 0; c + 1 < nch; ++c) {
                stage(c + 1);  // the other buffer: last read in chunk c - 1
                __syncthreads();
            }
            return;
        }
        if constexpr (XT) stage_xt(0, tid, NT + 64);
        __syncthreads();
        for (int c = 0; c < nch; ++c) {
            const char* xb = reinterpret_cast<const char*>(xs + (c & 1) * bufq) + q * 16;
            int d = 0;
            if (slab < nslab) {
                const int s0 = soff[slab * (nch + 1) + c], s1 = soff[slab * (nch + 1) + c + 1];
                const int T = __builtin_amdgcn_readfirstlane((s1 - s0) / 64);
                if constexpr (W == 4)
                    sell_walk_pipe<FAST>(blk, s0 + lane, T, xb, a0, a1, a2, a3);
                else
                    sell_walk<FAST, false, DPI>(blk, s0 + lane, T, xb, xs, xcol, ldx, lane, wave, W, nld - 1, 0, d,
                                                a0, a1, a2, a3);
            }
            if (c + 1 < nch) __syncthreads();
        }
    } else {
    if constexpr (XT) {
        stage_xt(0, tid, NT);
    } else if constexpr (XVEC) {
        for (int i = 0; i < nd; ++i) dma(0, i);
    } else {
        stage_regs(0);
    }
    sync_chunk();
    for (int c = 0; c < nch; ++c) {
        const char* xb = reinterpret_cast<const char*>(xs + (c & 1) * bufq) + q * 16;
        int d = 0;  // loads of chunk c + 1 issued by this wave
        const bool more = c + 1 < nch;
        if (slab < nslab) {
            const int s0 = soff[slab * (nch + 1) + c], s1 = soff[slab * (nch + 1) + c + 1];
            const int T = __builtin_amdgcn_readfirstlane((s1 - s0) / 64);
            const int k1 = (c + 1) * kc;
            float4* nxt = xs + ((c + 1) & 1) * bufq;
            // the 16-wave launch (four waves per SIMD hide each other's
            // latencies) stages whole chunks between walks instead
            if (XVEC && !XT && W <= 8 && more)
                sell_walk<FAST, true, DPI>(blk, s0 + lane, T, xb, nxt, xcol + (int64_t)k1 * ldx, ldx, lane, wave, W,
                                           nld - 1, min(kc, K - k1) - 1, d, a0, a1, a2, a3);
            else
                sell_walk<FAST, false, DPI>(blk, s0 + lane, T, xb, nxt, xcol, ldx, lane, wave, W, nld - 1, 0, d, a0,
                                            a1, a2, a3);
        }
        if (more) {
            if constexpr (XT) {
                stage_xt(c + 1, tid, NT);  // the other buffer: last read in chunk c - 1
            } else if constexpr (XVEC) {
                for (; d < nd; ++d) dma(c + 1, d);
            } else {
                stage_regs(c + 1);  // the other buffer: last read in chunk c - 1
            }
            sync_chunk();
        }
    }
    }
    if (slab < nslab) {
        const int row = perm[slab * pfr::kSellRows + r];
        const int cn = n0 + q * 4;
        if (row >= 0 && cn < N) {
            float* yr = Y + (int64_t)row * ldy_r;
            if (yvec && cn + 3 < N) {
                if (act == PFR_ACT_RELU) {
                    a0 = (0.0f < a0) ? a0 : 0.0f;
                    a1 = (0.0f < a1) ? a1 : 0.0f;
                    a2 = (0.0f < a2) ? a2 : 0.0f;
                    a3 = (0.0f < a3) ? a3 : 0.0f;
                } else if (act == PFR_ACT_GELU) {
                    a0 = pfr::gelu(a0);
                    a1 = pfr::gelu(a1);
                    a2 = pfr::gelu(a2);
                    a3 = pfr::gelu(a3);
                }
                *reinterpret_cast<float4*>(yr + cn) = make_float4(a0, a1, a2, a3);
            } else {
                const float a[4] = {a0, a1, a2, a3};
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (cn + i < N) {
                        const int64_t f = (int64_t)row * ldy_r + (int64_t)(cn + i) * ldy_c;
                        Y[f] = bias_add(a[i], f, bias, c_size, beta, act);
                    }
            }
        }
    }
}


int next_pow2(int n) {
    int p = 1;
    while (p < n) p <<= 1;
    return p;
}


// The sliced-ELL runs a product in this mode reads (null: neither copy).
const int4* sell_runs(const pfr_csr* W, bool fast) {
    return fast && W->sell_blk_fast != nullptr ? W->sell_blk_fast : W->sell_blk;
}

// Column-slice kernel launch with W waves per workgroup.
template <bool FAST, bool XVEC, int W, bool XT>
void launch_sell_w(pfr_ctx* ctx, const pfr_csr* Wt, const float* X, int N, int64_t ldx, float* Y,
                   int64_t ldy_r, int64_t ldy_c, int yvec, const float* bias, int64_t c_size, float beta, int act,
                   float alpha) {
    auto kern = k_spmm_sell<FAST, XVEC, W, XT>;
    const size_t lds = (size_t)(Wt->sell_kc + 1) * 64 * 2;
    // more than 64 KiB of dynamic LDS has to be allowed per kernel and device
    static uint64_t allowed = 0;  // bit d: done on device d (< 64)
    const uint64_t bit = ctx->device < 64 ? (uint64_t(1) << ctx->device) : 0;
    if (!bit || !(__atomic_load_n(&allowed, __ATOMIC_ACQUIRE) & bit)) {
        PFR_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        if (bit && lds == (size_t)(pfr::kSellMaxKC + 1) * 64 * 2) __atomic_fetch_or(&allowed, bit, __ATOMIC_RELEASE);
    }
    dim3 grid((unsigned)((Wt->sell_nslab + W - 1) / W), (unsigned)((N + pfr::kSellCols - 1) / pfr::kSellCols));
    hipLaunchKernelGGL(kern, grid, dim3(sell_threads<XVEC, W, XT>()), lds, ctx->stream, N, (int)Wt->K,
                       Wt->sell_kc, Wt->sell_nch, Wt->sell_nslab, Wt->sell_perm, Wt->sell_soff, sell_runs(Wt, FAST), X, ldx,
                       Y, ldy_r, ldy_c, yvec, bias, c_size, beta, act, alpha, alpha != 1.0f ? 1 : 0);
}

// Waves per workgroup of the column-slice launch for N columns, and its
// rounds.  One workgroup runs per CU (its LDS takes most of the CU), so the
// launch takes ceil(workgroups / CUs) rounds.  A round of 4-, 8- and 16-wave
// workgroups takes about 1 : 1.30 : 2.14 (measured on the 4096 x 4096, 10 %
// weight at N = 64, 128 and 256, one round each); the wave count with the
// fewest estimated clocks runs, the larger on a tie.  Fewer than four waves
// lose: each wave then stages more of X than it walks.
int sell_waves(const pfr_ctx* ctx, const pfr_csr* Wt, int64_t N, int64_t* rounds_out = nullptr) {
    const int64_t slices = (N + pfr::kSellCols - 1) / pfr::kSellCols;
    auto rounds = [&](int64_t w) { return ((Wt->sell_nslab + w - 1) / w * slices + ctx->num_cu - 1) / ctx->num_cu; };
    const int64_t c16 = rounds(16) * 214, c8 = rounds(8) * 130, c4 = rounds(4) * 100;
    const int w = (c16 <= c8 && c16 <= c4) ? 16 : (c8 <= c4 ? 8 : 4);
    if (rounds_out) *rounds_out = rounds(w);
    return w;
}

template <bool FAST, bool XVEC, bool XT>
void launch_sell_x(pfr_ctx* ctx, const pfr_csr* Wt, const float* X, int N, int64_t ldx, float* Y,
                   int64_t ldy_r, int64_t ldy_c, int yvec, const float* bias, int64_t c_size, float beta, int act,
                   float alpha) {
#define PFR_SELLW(WV) \
    launch_sell_w<FAST, XVEC, WV, XT>(ctx, Wt, X, N, ldx, Y, ldy_r, ldy_c, yvec, bias, c_size, beta, act, alpha)
    const int w = sell_waves(ctx, Wt, N);
    if (w == 16) PFR_SELLW(16);
    else if (w == 8) PFR_SELLW(8);
    else PFR_SELLW(4);
#undef PFR_SELLW
}

// xt: X is the transposed activation (see k_spmm_sell), alpha its scale.
void launch_sell(pfr_ctx* ctx, const pfr_csr* Wt, const float* X, int N, int64_t ldx, float* Y,
                 int64_t ldy_r, int64_t ldy_c, const float* bias, int64_t c_size, float beta, bool fast, int act,
                 bool xt = false, float alpha = 1.0f) {
    const bool xvec = (ldx % 4 == 0) && (N % 4 == 0) && aligned16(X);
    const int yvec = (ldy_c == 1 && ldy_r % 4 == 0 && aligned16(Y) && bias == nullptr) ? 1 : 0;
#define PFR_SELLX(F, XV, T) \
    launch_sell_x<F, XV, T>(ctx, Wt, X, N, ldx, Y, ldy_r, ldy_c, yvec, bias, c_size, beta, act, alpha)
    if (xt) {
        if (fast) PFR_SELLX(true, false, true);
        else PFR_SELLX(false, false, true);
    } else if (fast) {
        if (xvec) PFR_SELLX(true, true, false);
        else PFR_SELLX(true, false, false);
    } else {
        if (xvec) PFR_SELLX(false, true, false);
        else PFR_SELLX(false, false, false);
    }
#undef PFR_SELLX
}

// The kernels that read the CSR in place, columns of type C: the block
// SpMV, the small-N kernel and the row kernel.
template <bool FAST, bool I8, class C>
void launch_inplace(pfr_ctx* ctx, const pfr_csr* W, const C* col, const float* X, int64_t N, int64_t ldx, float* Y,
                    int64_t ldy_r, int64_t ldy_c, const float* bias, int64_t c_size, float beta, int act) {
    const int M = (int)W->M;
    hipStream_t s = ctx->stream;
    const void* val = W->val;
    const float* rs = W->row_scale;
    if (N == 1) {
        hipLaunchKernelGGL((k_spmv_wg<I8, C>), dim3((unsigned)W->n_spmv_blocks), dim3(kSpmvThreads), 0, s,
                           W->spmv_blocks, W->rowptr, col, val, rs, X, ldx, Y, ldy_r, bias, c_size, beta, act);
    } else if (N < 64) {
        const int np = next_pow2((int)N);
        const int rows_per_block = kWaves * (64 / np);
        const unsigned grid = (unsigned)((M + rows_per_block - 1) / rows_per_block);
#define PFR_SMALL(NPV)                                                                                \
    case NPV:                                                                                         \
        hipLaunchKernelGGL((k_spmm_small<NPV, FAST, I8, C>), dim3(grid), dim3(256), 0, s, M, (int)N,  \
                           W->rowptr, col, val, rs, X, ldx, Y, ldy_r, ldy_c, bias, c_size, beta, act);  \
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
        if (vec)
            hipLaunchKernelGGL((k_spmm_rows<FAST, true, I8, C>), dim3(grid), dim3(256), 0, s, M, (int)N, W->rowptr,
                               col, val, rs, X, ldx, Y, ldy_r, ldy_c, bias, c_size, beta, act);
        else
            hipLaunchKernelGGL((k_spmm_rows<FAST, false, I8, C>), dim3(grid), dim3(256), 0, s, M, (int)N, W->rowptr,
                               col, val, rs, X, ldx, Y, ldy_r, ldy_c, bias, c_size, beta, act);
    }
}

// Row, small-N and vector kernels for one value type.
template <bool FAST, bool I8>
void launch_csr_kernels(pfr_ctx* ctx, const pfr_csr* W, const float* X, int64_t N, int64_t ldx, float* Y,
                        int64_t ldy_r, int64_t ldy_c, const float* bias, int64_t c_size, float beta, int act) {
    const int M = (int)W->M;
    hipStream_t s = ctx->stream;
    const void* val = W->val;
    const float* rs = W->row_scale;
    if (FAST && N == 1 && ctx->merge && W->mp_wave != nullptr && ldx < INT32_MAX) {
        launch_merge<I8>(ctx, W, X, ldx, Y, ldy_r, bias, c_size, beta, act);
    } else if (FAST && N == 1 && W->bal_meta != nullptr && ldx < INT32_MAX) {
        launch_bal_fast<I8>(ctx, W, X, ldx, Y, ldy_r, bias, c_size, beta, act);
    } else if (FAST && N >= 2 && N <= 8 && W->bal_meta != nullptr) {
        if (N == 8 && ldx % 4 == 0 && aligned16(X))
            launch_bal_fast8<I8, true>(ctx, W, X, (int)N, ldx, Y, ldy_r, ldy_c, bias, c_size, beta, act);
        else
            launch_bal_fast8<I8, false>(ctx, W, X, (int)N, ldx, Y, ldy_r, ldy_c, bias, c_size, beta, act);
    } else if (FAST && N <= 8) {
        const unsigned grid = (unsigned)((M + kWaves - 1) / kWaves);
        const bool xv = N == 8 && ldx % 4 == 0 && aligned16(X);
        // a workgroup per row when rows are long (mean of at least 2048
        // nonzeros: measured faster on 4096 x 11008 at 30 %, slower on
        // 4096 x 4096 and 11008 x 4096 at 30 %)
        const bool wg = W->nnz >= 2048 * (int64_t)M;
#define PFR_FASTV(NBV, XVV, COL)                                                                               \
    do {                                                                                                       \
        using CTy = std::remove_const_t<std::remove_pointer_t<decltype(COL)>>;                                 \
        if (wg)                                                                                                \
            hipLaunchKernelGGL((k_spmv_fast<NBV, I8, XVV, CTy, true>), dim3((unsigned)M), dim3(256), 0, s, M, \
                               (int)N, W->rowptr, COL, val, rs, X, ldx, Y, ldy_r, ldy_c, bias, c_size, beta, act); \
        else                                                                                                   \
            hipLaunchKernelGGL((k_spmv_fast<NBV, I8, XVV, CTy>), dim3(grid), dim3(256), 0, s, M, (int)N,       \
                               W->rowptr, COL, val, rs, X, ldx, Y, ldy_r, ldy_c, bias, c_size, beta, act);     \
    } while (0)
#define PFR_FASTC(COL)                               \
    if (N == 1) PFR_FASTV(1, false, COL);            \
    else if (N <= 4) PFR_FASTV(4, false, COL);       \
    else if (xv) PFR_FASTV(8, true, COL);            \
    else PFR_FASTV(8, false, COL);
        if (W->col16) {
            const uint16_t* c16 = W->col16;
            PFR_FASTC(c16)
        } else {
            const int32_t* c32 = W->col;
            PFR_FASTC(c32)
        }
#undef PFR_FASTC
#undef PFR_FASTV
    } else if (N == 1 && W->chain_q0 != nullptr && W->chain_xlds && ldx < INT32_MAX) {
        if (W->chain_rows == 16) launch_chain_x<I8, 16>(ctx, W, X, ldx, Y, ldy_r, bias, c_size, beta, act);
        else if (W->chain_rows == 32) launch_chain_x<I8, 32>(ctx, W, X, ldx, Y, ldy_r, bias, c_size, beta, act);
        else launch_chain_x<I8, 64>(ctx, W, X, ldx, Y, ldy_r, bias, c_size, beta, act);
    } else if (N >= 2 && N <= 8 && W->chain_q0 != nullptr && W->chain_rows % kChainNR == 0 && W->chain_c16) {
        launch_chain_cols<I8>(ctx, W, X, (int)N, ldx, Y, ldy_r, ldy_c, bias, c_size, beta, act);
    } else if (N == 1 && W->chain_q0 != nullptr && W->K * ldx < INT32_MAX) {
        const dim3 grid((unsigned)W->chain_nslab), block(64 * (kChainP + 1));
        if (W->chain_c16)
            hipLaunchKernelGGL((k_spmv_chain<I8, true>), grid, block, 0, s, W->chain_q0, W->chain_len,
                               W->chain_perm, W->chain_val, W->chain_col, rs, X, (int)ldx, Y, ldy_r, bias, c_size,
                               beta, act);
        else
            hipLaunchKernelGGL((k_spmv_chain<I8, false>), grid, block, 0, s, W->chain_q0, W->chain_len,
                               W->chain_perm, W->chain_val, W->chain_col, rs, X, (int)ldx, Y, ldy_r, bias, c_size,
                               beta, act);
    } else if (W->col16 != nullptr) {
        launch_inplace<FAST, I8>(ctx, W, W->col16, X, N, ldx, Y, ldy_r, ldy_c, bias, c_size, beta, act);
    } else {
        launch_inplace<FAST, I8>(ctx, W, W->col, X, N, ldx, Y, ldy_r, ldy_c, bias, c_size, beta, act);
    }
}

// Non-finite fix-up for a handle with the stored-entry bitmap: the dense
// kernels (math.cpp:268-438) multiply every activation by every weight, so
// x[k, c] = NaN makes output column c NaN in every row, and x[k, c] = +-inf
// makes (row, c) NaN wherever row does not store k (inf * 0); the sparse
// kernels skip those terms.  One workgroup per 64 x 64 tile of X (k x c),
// read coalesced into LDS; a wave per column reduces its 64 k to a NaN flag
// and an inf mask (ballots), and only a column with either walks the rows,
// writing the epilogue of NaN (bias and activation as the product kernels
// apply them) where the rule says so.  Columns without non-finite values --
// the normal case -- cost one read of X.  x[k, c] is X[k * sk + c * sn]
// (sn = 1: X as the products read it; sk = 1: the Gemm form's activation
// read in place), times alpha when `scale`.
__global__ __launch_bounds__(256) void k_nonfinite_fix(const float* __restrict__ X, int64_t sk, int64_t sn,
                                                       float alpha, int scale, int64_t K, int64_t N, int64_t M,
                                                       const uint64_t* __restrict__ bm, int64_t nw,
                                                       float* __restrict__ Y, int64_t ldy_r, int64_t ldy_c,
                                                       const float* __restrict__ bias, int64_t c_size, float beta,
                                                       int act) {
    __shared__ float t[64][65];  // t[c][k]
    const int64_t kt = blockIdx.x, k0 = kt * 64, c0 = (int64_t)blockIdx.y * 64;
    for (int e = threadIdx.x; e < 64 * 64; e += 256) {
        // consecutive threads along whichever index X's rows run
        const int cc = sn == 1 ? e % 64 : e / 64, kk = sn == 1 ? e / 64 : e % 64;
        const int64_t k = k0 + kk, c = c0 + cc;
        const float v = (k < K && c < N) ? X[k * sk + c * sn] : 0.0f;
        t[cc][kk] = scale ? alpha * v : v;
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float qnan = __builtin_nanf("");
    for (int cc = wave; cc < 64 && c0 + cc < N; cc += 4) {
        const float v = t[cc][lane];
        const bool nan = __ballot(v != v) != 0;
        const uint64_t inf = __ballot(__builtin_isinf(v));
        if (!nan && inf == 0) continue;
        const int64_t c = c0 + cc;
        for (int64_t r = lane; r < M; r += 64) {
            if (nan || (inf & ~bm[r * nw + kt]) != 0) {
                const int64_t f = r * ldy_r + c * ldy_c;
                Y[f] = bias_add(qnan, f, bias, c_size, beta, act);
            }
        }
    }
}

// The column-slice kernel serves this product (float32 weight, N >= 16):
// the fast mode runs on either sliced-ELL copy (its own when built), the
// strict mode on the storage-order one.
bool sell_serves(const pfr_csr* W, int64_t N, bool fast) {
    return W->vdt != PFR_I8 && N >= kSellMinN && sell_runs(W, fast) != nullptr &&
           N < (int64_t)pfr::kSellCols * 65535;
}

// Its launch for N columns runs in one round, with 16-wave workgroups or,
// for a single chunk, 4 or 8 (their chunk 0 is staged by every wave; later
// chunks would fall to the staging wave alone).
bool sell_one_round(const pfr_ctx* ctx, const pfr_csr* W, int64_t N) {
    int64_t rounds = 0;
    const int w = sell_waves(ctx, W, N, &rounds);
    return rounds == 1 && (w == 16 || W->sell_nch == 1);
}

// Launch the kernel that fits N.  Output (row, c) -> Y[row*ldy_r + c*ldy_c].
// xt: X is the Gemm form's activation A (N x K, rows ldx apart) read in
// place, scaled by alpha; only where sell_serves.
void launch_spmm(pfr_ctx* ctx, const pfr_csr* W, const float* X, int64_t N, int64_t ldx, float* Y,
                 int64_t ldy_r, int64_t ldy_c, const float* bias, int64_t c_size, float beta,
                 bool fast, int act, bool xt = false, float alpha = 1.0f) {
    if (W->M == 0 || N == 0) return;
    const bool i8 = W->vdt == PFR_I8;
    pfr::require(!xt || sell_serves(W, N, fast), "transposed activation without the column-slice copy");
    if (sell_serves(W, N, fast)) {
        launch_sell(ctx, W, X, (int)N, ldx, Y, ldy_r, ldy_c, bias, c_size, beta, fast, act, xt, alpha);
    } else if (i8) {
        if (fast) launch_csr_kernels<true, true>(ctx, W, X, N, ldx, Y, ldy_r, ldy_c, bias, c_size, beta, act);
        else launch_csr_kernels<false, true>(ctx, W, X, N, ldx, Y, ldy_r, ldy_c, bias, c_size, beta, act);
    } else {
        if (fast) launch_csr_kernels<true, false>(ctx, W, X, N, ldx, Y, ldy_r, ldy_c, bias, c_size, beta, act);
        else launch_csr_kernels<false, false>(ctx, W, X, N, ldx, Y, ldy_r, ldy_c, bias, c_size, beta, act);
    }
    PFR_HIP(hipGetLastError());
    if (W->pattern != nullptr && W->K > 0) {
        pfr::require((N + 63) / 64 < 65536, "too many columns for the non-finite fix-up's grid");
        const dim3 grid((unsigned)((W->K + 63) / 64), (unsigned)((N + 63) / 64));
        hipLaunchKernelGGL(k_nonfinite_fix, grid, dim3(256), 0, ctx->stream, X, xt ? (int64_t)1 : ldx,
                           xt ? ldx : (int64_t)1, alpha, xt && alpha != 1.0f ? 1 : 0, W->K, N, W->M, W->pattern,
                           W->pattern_nw, Y, ldy_r, ldy_c, bias, c_size, beta, act);
        PFR_HIP(hipGetLastError());
    }
}

void check_csr(const pfr_csr* W) {
    pfr::require(W != nullptr, "null CSR handle");
    if (W->vdt != PFR_F32 && W->vdt != PFR_I8)
        throw pfr::Error(PFR_ERR_UNSUPPORTED, "CSR values must be float32 or int8");
}

void check_act(int act) {
    pfr::require(act == PFR_ACT_NONE || act == PFR_ACT_RELU || act == PFR_ACT_GELU, "unknown activation");
}

// Builds the derived copy that a product of N columns in this mode runs on,
// when the handle still has it pending (its first such product).
void ensure_copies(const pfr_ctx* ctx, const pfr_csr* W, int64_t N, bool fast) {
    uint32_t need = 0;
    if (W->vdt == PFR_F32 && N >= kSellMinN) need |= fast ? pfr::kCopySellFast : pfr::kCopySell;
    if (fast && ((N >= 2 && N <= 8) || (N == 1 && !(ctx->merge && W->mp_wave != nullptr)))) need |= pfr::kCopyBal;
    if (!fast && N <= 8) need |= pfr::kCopyChain;
    if ((W->pending.load(std::memory_order_acquire) & need) != 0) pfr::csr_build_copies(const_cast<pfr_csr*>(W), need);
}

void spmm_dev(pfr_ctx* ctx, const pfr_csr* W, const float* X, int64_t N, int64_t ldx, float* Y,
              int64_t ldy, int mode, int act = PFR_ACT_NONE) {
    check_csr(W);
    pfr::require(N >= 0 && N < INT32_MAX, "bad column count");
    pfr::require(ldx >= N && ldy >= N, "leading dimension smaller than N");
    pfr::require(mode == PFR_MODE_STRICT || mode == PFR_MODE_FAST, "unknown mode");
    pfr::require((X && Y) || W->M * N == 0, "null X/Y");
    check_act(act);
    if (W->M > 0 && N > 0) ensure_copies(ctx, W, N, mode == PFR_MODE_FAST);
    launch_spmm(ctx, W, X, N, ldx, Y, ldy, 1, nullptr, 0, 0.0f, mode == PFR_MODE_FAST, act);
}

// ws / ws_floats: a caller-provided workspace for op(A)^T (the
// allocation-free entry); null uses the context's grow-only buffer.
void gemm_dev(pfr_ctx* ctx, const float* A, int64_t Mb, int64_t K, int transA, const pfr_csr* BT,
              float alpha, float beta, const float* C, int64_t c_size, float* Y, int mode,
              int act = PFR_ACT_NONE, float* ws = nullptr, int64_t ws_floats = 0) {
    check_csr(BT);
    check_act(act);
    pfr::require(Mb >= 0 && Mb < INT32_MAX, "bad row count");
    pfr::require(BT->K == K, "Gemm: incompatible dimensions - A has K=" + std::to_string(K) +
                                 ", B has K=" + std::to_string(BT->K));
    pfr::require(mode == PFR_MODE_STRICT || mode == PFR_MODE_FAST, "unknown mode");
    const int64_t Nf = BT->M;
    if (Mb == 0 || Nf == 0) return;
    pfr::require(A != nullptr && Y != nullptr, "null A/Y");
    if (ws == nullptr) ensure_copies(ctx, BT, Mb, mode == PFR_MODE_FAST);  // the allocation-free entry builds none
    if (C == nullptr || c_size <= 0) {
        C = nullptr;
        c_size = 0;
    }
    // At = op(A)^T scaled by alpha: K x Mb, so each k row is contiguous.
    const float* At = A;
    hipStream_t s = ctx->stream;
    auto tbuf = [&]() -> float* {
        if (ws == nullptr) return static_cast<float*>(ctx->scratch[3].ensure(sizeof(float) * (size_t)(K * Mb)));
        pfr::require(K * Mb <= ws_floats,
                     "allocation-free Gemm: op(A) has K * Mb = " + std::to_string(K * Mb) +
                         " elements, more than its workspace of " + std::to_string(ws_floats) + " floats");
        return ws;
    };
    if (K == 0) {
        // No terms: every output is +0 (+ bias); At is never read.
    } else if (!transA && ws == nullptr && sell_serves(BT, Mb, mode == PFR_MODE_FAST) && K % 4 == 0 && aligned16(A) &&
               sell_one_round(ctx, BT, Mb)) {
        // the column-slice kernel stages A's rows itself, transposed and
        // scaled on the way into LDS (the allocation-free entry keeps its
        // workspace copy and the size limit it states).  Its workgroups
        // stage through registers, more slowly than the direct-to-LDS copy of
        // a transposed A, so this pays off when the launch runs in one round
        // (every workgroup stages once, side by side): 768 x 768 at 1024
        // tokens 26.0 -> 21.7 us; 3072 x 768 (three rounds) 66.1 -> 67.8 us.
        launch_spmm(ctx, BT, A, Mb, K, Y, 1, Nf, C, c_size, beta, mode == PFR_MODE_FAST, act, true, alpha);
        return;
    } else if (!transA) {
        float* t = tbuf();
        dim3 grid((unsigned)((K + 63) / 64), (unsigned)((Mb + 63) / 64));
        pfr::require(grid.y < 65536u, "activation too tall for the transpose grid");
        if (Mb % 4 == 0 && K % 4 == 0 && (reinterpret_cast<uintptr_t>(A) & 15) == 0)
            hipLaunchKernelGGL(k_transpose_scale4, grid, dim3(256), 0, s, A, Mb, K, alpha,
                               alpha != 1.0f ? 1 : 0, t);
        else
            hipLaunchKernelGGL(k_transpose_scale, grid, dim3(256), 0, s, A, Mb, K, alpha,
                               alpha != 1.0f ? 1 : 0, t);
        PFR_HIP(hipGetLastError());
        At = t;
    } else if (alpha != 1.0f) {
        float* t = tbuf();
        const int64_t n = K * Mb;
        hipLaunchKernelGGL(k_scale, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, A, n, alpha, t);
        PFR_HIP(hipGetLastError());
        At = t;
    }
    // Output (feature j, batch i) -> Y[i * Nf + j]: the flat index the bias
    // modulo uses in cpu_gemm.
    launch_spmm(ctx, BT, At, Mb, Mb, Y, 1, Nf, C, c_size, beta, mode == PFR_MODE_FAST, act);
}

std::mutex g_ws_mu;
std::vector<float*> g_ws_ptr;  // device address of `scratch`, per device

float* noalloc_workspace(int device) {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    return device >= 0 && device < (int)g_ws_ptr.size() ? g_ws_ptr[(size_t)device] : nullptr;
}

}  // namespace

namespace pfr {

// Records the device address of `scratch` on `device`, which must be current;
// once per device (the context's init calls it).
void init_noalloc_workspace(int device) {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    if (device < (int)g_ws_ptr.size() && g_ws_ptr[(size_t)device] != nullptr) return;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
        throw Error(PFR_ERR_HIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    if (device >= (int)g_ws_ptr.size()) g_ws_ptr.resize((size_t)device + 1, nullptr);
    g_ws_ptr[(size_t)device] = static_cast<float*>(p);
}

}  // namespace pfr

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

int pfr_spmm_csr_act_dev(pfr_ctx* ctx, const pfr_csr* W, const float* X, int64_t N, int64_t ldx,
                         float* Y, int64_t ldy, int mode, int act) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        spmm_dev(ctx, W, X, N, ldx, Y, ldy, mode, act);
    });
}

int pfr_gemm_csr_act_dev(pfr_ctx* ctx, const float* A, int64_t Mb, int64_t K, int transA,
                         const pfr_csr* BT, float alpha, float beta, const float* C, int64_t c_size,
                         float* Y, int mode, int act) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        gemm_dev(ctx, A, Mb, K, transA, BT, alpha, beta, C, c_size, Y, mode, act);
    });
}

int pfr_gemm_csr_act_noalloc_dev(pfr_ctx* ctx, const float* A, int64_t Mb, int64_t K, int transA,
                                 const pfr_csr* BT, float alpha, float beta, const float* C,
                                 int64_t c_size, float* Y, int mode, int act) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        float* ws = noalloc_workspace(ctx->device);
        pfr::require(ws != nullptr, "allocation-free Gemm: no workspace address recorded for this device");
        gemm_dev(ctx, A, Mb, K, transA, BT, alpha, beta, C, c_size, Y, mode, act, ws, kNoAllocFloats);
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
