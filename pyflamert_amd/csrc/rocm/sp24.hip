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
#include <algorithm>
#include <cmath>
#include <type_traits>
#include <vector>

#include "common.hpp"

#pragma clang fp contract(off)

typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v16bf __attribute__((ext_vector_type(16)));

struct pfr_sp24 {
    pfr_ctx* ctx = nullptr;
    int64_t M = 0, K = 0;
    int64_t Mp = 0, Kp = 0;  // padded: Mp % 256 == 0; Kp % 512 == 0 (int8) or % 256 (bf16), at least one tile
    pfr_dtype dtype = PFR_I8;
    void* a = nullptr;        // compressed values, [Mp/16][Kp/KT][64][16 B]
    uint32_t* idx = nullptr;  // [Mp/16][Kp/KT (int8) | Kp/128 (bf16)][64]
    float* w_scale = nullptr; // [M] (per-tensor scales expanded)
    float w_scale_max = 0.0f; // the largest of them
    int32_t* row_sum = nullptr;  // int8: [Mp] sum over k of W[m, k] (the zero-point correction)
    // int8: idx regrouped by kRB row blocks, [ceil(Mp/16/kRB)][Kp/128][64][4]:
    // element r < kRB of lane l is idx[kRB g + r][step][l] (other elements
    // and row blocks past Mp/16 are 0), so a wave owning row blocks kRB g ..
    // kRB g + kRB - 1 loads a step's positions with one load per lane
    uint32_t* idxw = nullptr;
};

namespace {

constexpr int kPadM = 256;   // packed weights pad M to this (the int8 tile height)

int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

void free_sp24(pfr_sp24* w) {
    if (!w) return;
    for (void* p : {w->a, (void*)w->idx, (void*)w->w_scale, (void*)w->row_sum, (void*)w->idxw})
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

template <int I, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < E) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, E>(f);
    }
}

// ---- kernels ----------------------------------------------------------------

// XT[n][k] (Np x Kp) = X[k][n] for 16-bit elements (bf16 bits), zero
// outside K x N: a 64 x 64 block per workgroup, read as 8-byte runs of four
// columns along X rows and written as 8-byte runs of four k along XT rows
// (the element-wise form spent 10.5 us on 4096 x 512, about 4x this).
__global__ __launch_bounds__(256) void k_transpose_b16(const uint16_t* __restrict__ X, int64_t K, int64_t N,
                                                       int64_t ldx, int vec, uint16_t* __restrict__ XT, int64_t Kp) {
    __shared__ uint16_t tile[64][68];  // tile[k][n], rows 136 B apart (8-byte aligned)
    const int t = threadIdx.x;
    const int64_t k0 = (int64_t)blockIdx.x * 64, n0 = (int64_t)blockIdx.y * 64;
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // X row k0 + kk, columns n0 + 4q .. +3
        const int e = t + 256 * i, kk = e >> 4, q = e & 15;
        const int64_t k = k0 + kk, n = n0 + 4 * q;
        uint16_t v[4] = {0, 0, 0, 0};
        if (k < K) {
            if (vec && n + 4 <= N) {
                const uint2 u = *reinterpret_cast<const uint2*>(X + k * ldx + n);
                v[0] = (uint16_t)u.x; v[1] = (uint16_t)(u.x >> 16); v[2] = (uint16_t)u.y; v[3] = (uint16_t)(u.y >> 16);
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) v[j] = n + j < N ? X[k * ldx + n + j] : (uint16_t)0;
            }
        }
        *reinterpret_cast<uint2*>(&tile[kk][4 * q]) = make_uint2(v[0] | ((uint32_t)v[1] << 16), v[2] | ((uint32_t)v[3] << 16));
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // XT row n0 + nn, k0 + 4q .. +3
        const int e = t + 256 * i, nn = e >> 4, q = e & 15;
        const uint32_t lo = tile[4 * q][nn] | ((uint32_t)tile[4 * q + 1][nn] << 16);
        const uint32_t hi = tile[4 * q + 2][nn] | ((uint32_t)tile[4 * q + 3][nn] << 16);
        *reinterpret_cast<uint2*>(XT + (n0 + nn) * Kp + k0 + 4 * q) = make_uint2(lo, hi);
    }
}

// XT[n][k] (Np x Kp) = X[k][n] for int8, zero outside K x N.  A wave owns a
// 64 x 64 block: lane (rg = l / 4, cg = l % 4) loads rows 4rg .. 4rg+3,
// columns 16cg .. 16cg+15 (each load instruction covers 16 rows x 64
// contiguous bytes), transposes each 4 x 4 byte square with v_perm_b32 and
// stores dwords (each store instruction covers 4 XT rows x 64 bytes).
__global__ __launch_bounds__(256) void k_transpose_i8(const int8_t* __restrict__ X, int64_t K, int64_t N,
                                                      int64_t ldx, int vec, int8_t* __restrict__ XT,
                                                      int64_t Kp, int64_t Np) {
    const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int rg = l >> 2, cg = l & 3;
    const int64_t k = (int64_t)blockIdx.x * 64 + 4 * rg;
    const int64_t n0 = ((int64_t)blockIdx.y * 4 + w) * 64 + 16 * cg;
    if (n0 >= Np) return;
    uint32_t r[4][4];
#pragma unroll
    for (int row = 0; row < 4; ++row) {
        const int64_t kk = k + row;
        if (vec && kk < K && n0 + 16 <= N) {
            const v4i v = *reinterpret_cast<const v4i*>(X + kk * ldx + n0);
            r[row][0] = (uint32_t)v.x; r[row][1] = (uint32_t)v.y; r[row][2] = (uint32_t)v.z; r[row][3] = (uint32_t)v.w;
        } else {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                uint32_t d = 0;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const int64_t n = n0 + 4 * g + b;
                    if (kk < K && n < N) d |= (uint32_t)(uint8_t)X[kk * ldx + n] << (8 * b);
                }
                r[row][g] = d;
            }
        }
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        // byte j of r[row][g] is X[k + row][n0 + 4g + j]; o[j] gathers it over row
        const uint32_t lo01 = __builtin_amdgcn_perm(r[1][g], r[0][g], 0x05010400u);
        const uint32_t hi01 = __builtin_amdgcn_perm(r[1][g], r[0][g], 0x07030602u);
        const uint32_t lo23 = __builtin_amdgcn_perm(r[3][g], r[2][g], 0x05010400u);
        const uint32_t hi23 = __builtin_amdgcn_perm(r[3][g], r[2][g], 0x07030602u);
        const uint32_t o[4] = {__builtin_amdgcn_perm(lo23, lo01, 0x05040100u),
                               __builtin_amdgcn_perm(lo23, lo01, 0x07060302u),
                               __builtin_amdgcn_perm(hi23, hi01, 0x05040100u),
                               __builtin_amdgcn_perm(hi23, hi01, 0x07060302u)};
#pragma unroll
        for (int j = 0; j < 4; ++j)
            *reinterpret_cast<uint32_t*>(XT + (n0 + 4 * g + j) * Kp + k) = o[j];
    }
}

// int8 2:4 GEMM, 256 x 128 outputs per workgroup of four waves, one per
// SIMD, each owning 64 rows x all 128 columns (4 x 8 tiles of 16 x 16: 128
// accumulator registers, so the wave runs alone on its SIMD with room for
// two fragment sets).  A k step is 128 wide; its operands live in one of
// four LDS stages:
//   A values  [16 row blocks][64 lanes][16 B]   (the packed register order)
//   A indices [16 row blocks][64 lanes] u32
//   B         [128 columns][128 B]: the k bytes of one XT row, its 16-byte
//             chunk c stored at position c ^ ((column >> 1) & 7), so the 16
//             lanes of a ds_read_b128 group (16 consecutive columns, one
//             chunk) hit 16 distinct 4-bank groups.
// Per k step a workgroup fetches 36 KiB from global memory (16 KiB of A
// values, 4 KiB of positions, 16 KiB of X), which at the ~56 B per clock a
// CU's vector memory path delivers (measured with direct-to-LDS loads of
// L2-resident data) is ~660 clocks against 512 clocks of MFMA work per SIMD;
// each B fragment is read from LDS by the four waves and each A fragment by
// one.  Measured per step (s_memtime inside the kernel, 11008 x 4096 x 512):
// 1163 clocks with the weight streamed from HBM, 898 with it cache-resident;
// the loads alone take 1229 (HBM) and 659 (L2), the MFMAs and fragment reads
// alone 711: the step is bound by the operand loads, and with the weight in
// HBM by their latency (four stages of 36 KiB are all the LDS holds).  Stages are filled by direct-to-LDS loads
// (global_load_lds_dword[x4]: each wave instruction writes its lanes' data
// contiguously) four steps ahead of the MFMAs; each wave reads the next
// step's fragments into a second register set while the current step's
// MFMAs run; one barrier per step.  nkt is a multiple of 4 (packed K is
// padded to 512), so the loop unrolls over the four stages with each stage's
// address static, which lets the compiler wait for only the oldest loads
// (vmcnt) instead of all of them.  The last four steps, peeled from the
// loop, have no stage left to load; they issue the same loads with every
// lane pointed at one address (one 64-byte request per instruction) into the
// stage just consumed, so the count of loads per step stays fixed for the
// vmcnt waits.  (Any branch or select around the loop's loads makes the
// compiler wait for all of them before every LDS read.)
constexpr int kI8TileM = 256, kI8TileN = 128;
constexpr int kI8Waves = 4, kI8Threads = 64 * kI8Waves;
constexpr int kLdsA = 16 * 64 * 16, kLdsI = 16 * 64 * 4, kLdsB = 128 * 128;
constexpr int kStage = kLdsA + kLdsI + kLdsB;  // 36 KiB

#define PFR_LDS(p) ((__attribute__((address_space(3))) void*)(p))
// word 3 of a raw buffer resource on CDNA (32-bit data format, no swizzle)
constexpr int kBufWord3 = 0x00020000;

// 16 bytes per lane from base + off (base wave-uniform) to LDS dst + 16 lane,
// as a buffer load: the compiler counts a global direct-to-LDS load as a
// flat access that may finish out of order and then turns every later wait
// on the LDS counter into a wait for all LDS reads while one is in flight.
__device__ __forceinline__ void lds_copy16(const void* base, int off, __attribute__((address_space(3))) void* dst) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, -1, kBufWord3);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, dst, 16, off, 0, 0, 0);
}

// B source: XROW = false reads XT (Np x Kp, the transposed activation),
// XROW = true reads the row-major activation X itself (K % 512 == 0,
// N % 128 == 0, rows 16-byte aligned).  In the XROW form LDS holds the step's
// 128 X rows (128 bytes each, 16-byte chunk c of row k at position
// c ^ xrow_swizzle(k)) and the B fragments are assembled with
// ds_read_b64_tr_b8: within each 16-lane group the sixteen 8-byte reads form
// a 16 x 8 byte matrix S and lane t receives S[2i + t/8][t % 8], i = 0..7;
// so source lane s pointing at row k0 + s/2, bytes 8(s % 2) of the column
// chunk gives lane t the eight k values k0 .. k0+7 of column chunk + t.
__device__ __forceinline__ int xrow_swizzle(int k) { return ((k >> 1) & 3) | (((k >> 4) & 1) << 2); }

// quantize_tensor's rounding and cast for an output zero point of 0
// (quant_ops.cpp:42-47): q = clamp((int32_t)std::round(p), -128, 127) with
// the x86 conversion (NaN and |p| >= 2^31 give INT32_MIN, so -128).
// std::round(p) = trunc(p + copysign(0.5 - 2^-25, p)) for every float p:
// the addend is the largest float below one half, so a fraction of exactly
// one half still carries (the sum rounds up to the next integer) while the
// largest fraction below one half does not; from 2^23 up every float is an
// integer and the addend is below half an ulp.  The clamp runs in float
// (exact on integers), and one select supplies the x86 value.
// INRANGE: p is known finite with |p| < 2^31 (the host bounds |acc| * scale
// * (1 / out_scale) for the whole launch), so the select is not needed, and
// the clamp can come first: rounding is monotone and the bounds are
// integers, so clamping p to [-128, 127] and then rounding gives the same
// value, and the conversion to int (which truncates) does the trunc.
template <bool INRANGE>
__device__ __forceinline__ int32_t round_clamp_i8(float p) {
    if constexpr (INRANGE) {
        const float c = __builtin_amdgcn_fmed3f(p, -128.0f, 127.0f);
        return (int32_t)(c + __builtin_copysignf(0.49999997f, c));
    }
    const float r = __builtin_truncf(p + __builtin_copysignf(0.49999997f, p));
    const float c = __builtin_amdgcn_fmed3f(r, -128.0f, 127.0f);
    return (int32_t)(__builtin_fabsf(r) < 2147483648.0f ? c : -128.0f);
}

// The per-row weight scales of this lane's 16 output rows of the int8 2:4
// GEMM's tile (wave w: row blocks mb0 + 4w + i, rows 4kb + r of each), from
// clamped rows, loaded together so they cost one load latency.
__device__ __forceinline__ void sp24_i8_row_scales(float (&wsv)[4][4], const float* __restrict__ ws, int64_t mb0,
                                                   int M) {
    const int t = threadIdx.x, w = __builtin_amdgcn_readfirstlane(t >> 6), kb = (t & 63) >> 4;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) wsv[i][r] = ws[min((int)(mb0 + w * 4 + i) * 16 + 4 * kb + r, M - 1)];
}

// The epilogue of the int8 2:4 GEMM: wave w of the workgroup holds the
// accumulators of the RB row blocks RB w + i of the tile (rows 16 RB w ..
// 16 RB w + 16 RB - 1) x columns 16j + c; tile + 128 ml (ml in those rows)
// is LDS no longer in use, which only wave w touches: each wave requantises
// its rows there and stores them itself, so the waves need no barrier
// between the two.  The
// 16-byte chunk j of row ml sits at chunk j ^ ((ml >> 2) & 3): a byte write
// covers rows 4kb + r of a row block (kb = 0..3), whose 128-byte rows would
// otherwise all start in the same bank, and the 16-byte reads of two
// neighbouring rows stay on distinct banks.
template <int OUT, int RB>
__device__ __forceinline__ void sp24_i8_epilogue(
    const v4i (&acc)[RB][8], char* tile, int64_t mb0, int64_t n0, int M, int N, const float (&wsv)[RB][4],
    float xs, float inv_out, int32_t out_zp, int inrange, void* __restrict__ Y, int64_t ldy, int yvec,
    int32_t x_zp, int32_t zp_shift, const float* __restrict__ xs_dev, const uint8_t* __restrict__ zp_dev,
    const int32_t* __restrict__ row_sum) {
    const int t = threadIdx.x, w = __builtin_amdgcn_readfirstlane(t >> 6), l = t & 63;
    const int kb = l >> 4, c = l & 15;
    const float xs_eff = xs_dev ? *xs_dev : xs;
    const int32_t zpv = zp_dev ? (int32_t)*zp_dev : x_zp;
    const uint32_t zcorr = (uint32_t)(zpv - zp_shift);
    // the row sums of this lane's 4 RB rows, for a zero-point correction
    // (loaded together, from clamped rows)
    uint32_t rsv[RB][4];
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = min((int)(mb0 + w * RB + i) * 16 + 4 * kb + r, M - 1);
            rsv[i][r] = zcorr ? (uint32_t)row_sum[m] : 0u;
        }
    // the exact accumulator of a row (int32 wrap-around arithmetic; the true
    // value is within int32 for K < 2^17)
    auto exact = [&](int32_t a, uint32_t rs) { return (int32_t)((uint32_t)a - zcorr * rs); };
    if constexpr (OUT == PFR_SP24_OUT_I8) {
        // requantise into the LDS tile (128-byte rows), then store 16-byte row
        // pieces
        // ZERO: no zero-point correction and output zero point 0 (the usual
        // symmetric case; the terms it drops are exact identities), chosen
        // once per workgroup so the per-output work shrinks
        auto requant = [&](auto zero, auto inr) {
            constexpr bool ZERO = decltype(zero)::value, INRANGE = decltype(inr)::value;
#pragma unroll
            for (int i = 0; i < RB; ++i) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int ml = (w * RB + i) * 16 + 4 * kb + r;
                    const int m = (int)(mb0 * 16) + ml;
                    const float sab = m < M ? wsv[i][r] * xs_eff : 0.0f;  // a_scale * b_scale (quant_ops.cpp:435)
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        int32_t q;
                        if constexpr (ZERO) {
                            q = round_clamp_i8<INRANGE>(((float)acc[i][j][r] * sab) * inv_out);
                        } else {
                            const float prod = ((float)exact(acc[i][j][r], rsv[i][r]) * sab) * inv_out;
                            q = (int32_t)((uint32_t)pfr::f2i_trunc_x86(roundf(prod)) + (uint32_t)out_zp);
                            q = q < -128 ? -128 : (q > 127 ? 127 : q);
                        }
                        tile[ml * 128 + 16 * (j ^ ((ml >> 2) & 3)) + c] = (char)q;
                    }
                }
            }
        };
        if (zcorr == 0 && out_zp == 0) {
            if (inrange) requant(std::true_type{}, std::true_type{});
            else requant(std::true_type{}, std::false_type{});
        } else {
            requant(std::false_type{}, std::false_type{});
        }
        __builtin_amdgcn_s_waitcnt(0xF | (7 << 4) | (0 << 8) | (0x3 << 14));  // lgkmcnt(0) only
        // the wave's 16 RB rows x 8 pieces, 2 RB per lane: all read from LDS
        // first, then stored
        v4i piece[2 * RB];
#pragma unroll
        for (int i = 0; i < 2 * RB; ++i) {
            const int q16 = l + 64 * i, ml = 16 * RB * w + (q16 >> 3), cc = q16 & 7;
            piece[i] = *reinterpret_cast<const v4i*>(tile + ml * 128 + 16 * (cc ^ ((ml >> 2) & 3)));
        }
#pragma unroll
        for (int i = 0; i < 2 * RB; ++i) {
            const int q16 = l + 64 * i, ml = 16 * RB * w + (q16 >> 3), cc = q16 & 7;
            const int64_t m = mb0 * 16 + ml, n = n0 + 16 * cc;
            if (m >= M) continue;
            int8_t* yr = static_cast<int8_t*>(Y) + m * ldy;
            if (yvec && n + 16 <= N) {
                *reinterpret_cast<v4i*>(yr + n) = piece[i];
            } else {
#pragma unroll
                for (int b = 0; b < 16; ++b)
                    if (n + b < N) yr[n + b] = (int8_t)(piece[i][b / 4] >> (8 * (b % 4)));
            }
        }
    } else {
        // 4-byte outputs, one row block at a time through the wave's first
        // 8 KiB of LDS (16 rows x 512 B; the 64-byte chunk j of row 4kb + r
        // at chunk j ^ kb, so a write's four rows hit four bank groups),
        // then 16-byte row pieces from distinct registers: stored one element
        // at a time from one register, each store waited for the one before
        char* wt = tile + 2048 * RB * w;
        const bool vec = yvec && (ldy % 4 == 0) && n0 + 128 <= N;
#pragma unroll
        for (int i = 0; i < RB; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = (int)(mb0 + w * RB + i) * 16 + 4 * kb + r;
                float sab = 1.0f;
                if constexpr (OUT == PFR_SP24_OUT_F32) sab = m < M ? wsv[i][r] * xs_eff : 0.0f;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int32_t v = exact(acc[i][j][r], rsv[i][r]);
                    uint32_t bits;
                    if constexpr (OUT == PFR_SP24_OUT_I32) bits = (uint32_t)v;
                    else bits = __float_as_uint((float)v * sab);
                    *reinterpret_cast<uint32_t*>(wt + (4 * kb + r) * 512 + 64 * (j ^ kb) + 4 * c) = bits;
                }
            }
            __builtin_amdgcn_s_waitcnt(0xF | (7 << 4) | (0 << 8) | (0x3 << 14));  // lgkmcnt(0) only
            // 16 rows x 32 pieces of 16 B, 8 per lane
            v4i piece[8];
#pragma unroll
            for (int h = 0; h < 8; ++h) {
                const int q16 = l + 64 * h, row = q16 >> 5, pc = q16 & 31;
                piece[h] = *reinterpret_cast<const v4i*>(wt + row * 512 + 64 * ((pc >> 2) ^ (row >> 2)) + 16 * (pc & 3));
            }
#pragma unroll
            for (int h = 0; h < 8; ++h) {
                const int q16 = l + 64 * h, row = q16 >> 5, pc = q16 & 31;
                const int64_t m = (mb0 + w * RB + i) * 16 + row, n = n0 + 4 * pc;
                if (m >= M) continue;
                uint32_t* yr = static_cast<uint32_t*>(Y) + m * ldy;
                if (vec) {
                    *reinterpret_cast<v4i*>(yr + n) = piece[h];
                } else {
#pragma unroll
                    for (int b = 0; b < 4; ++b)
                        if (n + b < N) yr[n + b] = (uint32_t)piece[h][b];
                }
            }
            // this block's reads have completed before the next block's writes
            __builtin_amdgcn_s_waitcnt(0xF | (7 << 4) | (0 << 8) | (0x3 << 14));
        }
    }
}

// Activation zero point: acc = sum_k w[m, k] (x[k, n] - zp) =
// sum_k w x - zp * row_sum[m], exact in int32.  A uint8 activation arrives
// as x - 128 (sign bit flipped by k_flip_sign), so its correction uses
// zp - 128 (zp_shift = 128).  The activation's scale and zero point come
// from xs / x_zp or, when xs_dev / zp_dev are set, from device scalars (the
// outputs of a DynamicQuantizeLinear on the same stream).
template <int OUT, bool XROW>
__global__ __launch_bounds__(kI8Threads, 1) void k_sp24_i8(
    int nkt, const v4i* __restrict__ A, const uint32_t* __restrict__ I,
    const int8_t* __restrict__ B, int64_t ldb, int M, int N, const float* __restrict__ ws, float xs,
    float inv_out, int32_t out_zp, int inrange, void* __restrict__ Y, int64_t ldy, int yvec, int ntn,
    int32_t x_zp, int32_t zp_shift, const float* __restrict__ xs_dev, const uint8_t* __restrict__ zp_dev,
    const int32_t* __restrict__ row_sum) {
    __shared__ __attribute__((aligned(1024))) char st0[kStage];
    __shared__ __attribute__((aligned(1024))) char st1[kStage];
    __shared__ __attribute__((aligned(1024))) char st2[kStage];
    __shared__ __attribute__((aligned(1024))) char st3[kStage];
    const int t = threadIdx.x, w = __builtin_amdgcn_readfirstlane(t >> 6), l = t & 63;
    const int kb = l >> 4, c = l & 15;
    int mt, nt;
    {
        const int G = (int)gridDim.x, L = (int)blockIdx.x, xcd = L & 7, slot = L >> 3;
        const int q = G >> 3, rem = G & 7;
        const int T = xcd * q + min(xcd, rem) + slot;
        mt = T / ntn;
        nt = T % ntn;
    }
    const int64_t mb0 = (int64_t)mt * (kI8TileM / 16);
    const int64_t n0 = (int64_t)nt * kI8TileN;
    // per k step every wave issues twelve direct-to-LDS loads: A row blocks
    // w + 4i (1 KiB each), their index rows (256 B each), and B runs w + 4i
    // (8 rows of 128 B each, rows 8j .. 8j + 7 of run j), i = 0..3
    constexpr int kLoads = 12;
    const v4i* asrc = A + ((mb0 + w) * nkt) * 64 + l;
    const uint32_t* isrc = I + ((mb0 + w) * nkt) * 64 + l;
    const int64_t rb4 = (int64_t)4 * nkt * 64;  // elements between row blocks w + 4i and w + 4i + 4
    const v4i* bsrc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int n = 8 * (w + 4 * i) + (l >> 3);
        if constexpr (XROW) {
            const int chunk = (l & 7) ^ xrow_swizzle(n);
            bsrc[i] = reinterpret_cast<const v4i*>(B + (int64_t)n * ldb + n0 + 16 * chunk);
        } else {
            const int chunk = (l & 7) ^ ((n >> 1) & 7);
            bsrc[i] = reinterpret_cast<const v4i*>(B + (n0 + n) * ldb + 16 * chunk);
        }
    }
    const int64_t b_step = XROW ? 128 * ldb / 16 : 8;  // v4i per k step
    auto issue = [&](char* st, int s) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __builtin_amdgcn_global_load_lds(asrc + i * rb4 + (int64_t)s * 64, PFR_LDS(st + (w + 4 * i) * 1024), 16,
                                             0, 0);
            __builtin_amdgcn_global_load_lds(isrc + i * rb4 + (int64_t)s * 64, PFR_LDS(st + kLdsA + (w + 4 * i) * 256),
                                             4, 0, 0);
            __builtin_amdgcn_global_load_lds(bsrc[i] + (int64_t)s * b_step,
                                             PFR_LDS(st + kLdsA + kLdsI + 8 * (w + 4 * i) * 128), 16, 0, 0);
        }
    };
    // the tail's loads: the same instructions, every lane reading A[0]
    auto issue_tail = [&](char* st) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __builtin_amdgcn_global_load_lds(A, PFR_LDS(st + (w + 4 * i) * 1024), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(A, PFR_LDS(st + kLdsA + (w + 4 * i) * 256), 4, 0, 0);
            __builtin_amdgcn_global_load_lds(A, PFR_LDS(st + kLdsA + kLdsI + 8 * (w + 4 * i) * 128), 16, 0, 0);
        }
    };
    // X-row form: transpose read r of this lane starts at row
    // k_r = 16kb + 8(r & 1) + 64(r >> 1) + c/2, bytes 8(c % 2) of the chunk.
    // xrow_swizzle(k_r) is the same for all four reads (bits 1-2 of k_r come
    // from c/2, bit 4 from kb), and the rows differ by constants, so one base
    // and one swizzle serve them all.
    const int trk = kLdsA + kLdsI + (16 * kb + (c >> 1)) * 128 + 8 * (c & 1);
    const int trf = xrow_swizzle(16 * kb + (c >> 1));
    // XT form: the two 16-byte pieces of column n = 16j + c sit at chunks
    // kb and 4 + kb of its row, swizzled by (n >> 1) & 7 = (c >> 1) for
    // every j
    const int xsw = (c >> 1) & 7;
    const int bxt = kLdsA + kLdsI + c * 128;
    v4i acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = v4i{0, 0, 0, 0};
    struct Frag {
        v4i a[4];
        int ix[4];
        v8i b[8];
    };
    auto fetch = [&](Frag& f, const char* st) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if constexpr (XROW) {
                v2i q[4];
                const char* bp = st + trk + 16 * (j ^ trf);
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    q[r] = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                        (__attribute__((address_space(3))) v2i*)(bp + 1024 * (r & 1) + 8192 * (r >> 1)));
                f.b[j] = v8i{q[0].x, q[0].y, q[1].x, q[1].y, q[2].x, q[2].y, q[3].x, q[3].y};
            } else {
                const char* bp = st + bxt + j * 16 * 128;
                const v4i lo = *reinterpret_cast<const v4i*>(bp + 16 * (kb ^ xsw));
                const v4i hi = *reinterpret_cast<const v4i*>(bp + 16 * ((4 + kb) ^ xsw));
                f.b[j] = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f.a[i] = *reinterpret_cast<const v4i*>(st + ((w * 4 + i) * 64 + l) * 16);
            f.ix[i] = *reinterpret_cast<const int*>(st + kLdsA + ((w * 4 + i) * 64 + l) * 4);
        }
    };
    auto mma = [&](const Frag& f) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                acc[i][j] = __builtin_amdgcn_smfmac_i32_16x16x128_i8(f.a[i], f.b[j], acc[i][j], f.ix[i], 0, 0);
    };
    // Step s: fragments of stage s are in registers (cur).  Wait for stage
    // s+1's loads (vmcnt(24): stages s+2 and s+3 may still be in flight),
    // barrier (every wave's stage s+1 loads have landed, and every wave has
    // read stage s's fragments, so its LDS buffer is free), start the loads
    // of stage s+4 into that buffer, read stage s+1's fragments into `nxt`
    // while the MFMAs run on `cur`.
    // vmcnt(24) and lgkmcnt(0): this wave's fragment reads of the previous
    // step have completed before the barrier lets other waves refill a stage
    // (vmcnt holds 6 bits: low 4 in [3:0], high 2 in [15:14])
    auto vm_wait = [](int n) { return (n & 0xF) | ((n >> 4) << 14) | (7 << 4) | (0 << 8); };
    Frag fa, fb;
    // (sched_barrier keeps each step's loads, reads and MFMAs between its
    // own barriers: otherwise the scheduler hoists the next step's wait and
    // barrier above most of this step's MFMAs, exposing the fragment reads'
    // latency)
    auto step = [&](Frag& cur, Frag& nxt, char* st_cur, char* st_next, int s) {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(vm_wait(2 * kLoads));
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        if (s >= 0) issue(st_cur, s + 4);  // s is a literal -1 in the peeled tail
        else issue_tail(st_cur);
        fetch(nxt, st_next);
        mma(cur);
        // the step's 32 MFMAs each followed by one or two of its 40 fragment
        // reads, and its 12 stage loads spread evenly among them: the LDS and
        // vector-memory pipes stay busy while the MFMA pipe runs (a wave
        // whose loads or reads are issued in a block stalls on their queues
        // before the MFMAs behind them)
        static_for<0, 32>([&](auto gc) {
            constexpr int g = decltype(gc)::value;
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);               // MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, g < 8 ? 2 : 1, 0);   // DS read
            if constexpr ((g + 1) * 12 / 32 > g * 12 / 32)
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);           // VMEM read (stage load)
        });
    };
    issue(st0, 0);
    issue(st1, 1);
    issue(st2, 2);
    issue(st3, 3);
    __builtin_amdgcn_s_waitcnt(vm_wait(3 * kLoads) | (0xF << 8));  // stage 0 landed (lgkmcnt left alone)
    __builtin_amdgcn_s_barrier();
    fetch(fa, st0);
    for (int s = 0; s < nkt - 4; s += 4) {
        step(fa, fb, st0, st1, s);
        step(fb, fa, st1, st2, s + 1);
        step(fa, fb, st2, st3, s + 2);
        step(fb, fa, st3, st0, s + 3);
    }
    step(fa, fb, st0, st1, -1);
    step(fb, fa, st1, st2, -1);
    step(fa, fb, st2, st3, -1);
    step(fb, fa, st3, st0, -1);
    __builtin_amdgcn_s_waitcnt(0);  // the tail's loads have landed
    __builtin_amdgcn_s_barrier();
    float wsv[4][4];
    if constexpr (OUT != PFR_SP24_OUT_I32) sp24_i8_row_scales(wsv, ws, mb0, M);
    sp24_i8_epilogue<OUT, 4>(acc, st0, mb0, n0, M, N, wsv, xs, inv_out, out_zp, inrange, Y, ldy, yvec, x_zp, zp_shift,
                          xs_dev, zp_dev, row_sum);
}

// int8 2:4 GEMM with the weight streamed into registers.  Tiles of 256 x
// 128 outputs, 16 / RB waves, wave w owning RB row blocks (rows 16 RB w ..
// 16 RB w + 16 RB - 1) and all 128 columns, with
// k_sp24_i8's MFMA order; each wave loads its own row blocks' packed values
// and positions straight from global memory into a ring of register slots
// (one per k step: eight at RB = 4, six at RB = 2; the packed order is the
// MFMA's lane order, so one 16-byte load per row block and step, and one for
// the row blocks' positions from the regrouped idxw), and only X goes
// through LDS, in 16 KiB stages filled by direct-to-LDS loads (RB loads per
// wave and step).  Against k_sp24_i8 this takes the weight out of LDS (40
// KiB of writes and reads per step) and keeps SLOTS - 1 steps of loads in
// flight per wave instead of three, which the weight, streamed from HBM,
// needs to cover its latency: 2 RB + 1 loads per step, within the 63
// vector-memory instructions a wave can have outstanding.  RB = 2 (eight
// waves, two per SIMD: one wave's memory stalls leave the SIMD's MFMA unit
// to the other) is launched: 26.8 against 27.4 us for RB = 4 (four waves of
// 64 rows), bit-identical.  192-row tiles (RB = 3, 232 tiles for 11008 x 512
// instead of 172) measured slower, 29.4 against 28.2 us, as every tile also
// streams all of X.
// Per step s (slot and stage u = s % SLOTS) each wave runs the 8 RB MFMAs of
// column blocks j = 0..7, reading the B fragment of column block j + 3
// (the next step's blocks 0..2 for j >= 5) from LDS while block j's MFMAs
// run, in a ring of four fragment registers.  On even steps, before
// reading the next step's first block, it waits for its own loads of steps
// s + 1 and s + 2 (vmcnt: the loads of the steps issued after them may
// still be in flight) and for its LDS reads, and meets the other waves at
// the barrier: stages s + 1 and s + 2 are then complete, and every wave has
// read all of stage s.  Every step then loads step s + SLOTS - 1 into stage
// and register slot (s - 1) % SLOTS, the previous step's: after an even step's
// barrier that stage has been read by every wave, and an odd step reuses
// the stage of the even step before it, read before that step's barrier.
// (A barrier every step cost about a fifth of a streaming step.)  X is the row-major activation (XROW form of
// k_sp24_i8).  The NKT steps are fully unrolled, so every wait count is a
// compile-time constant (as a loop the compiler's wait counting loses track
// of the ring at the back edge and drains all loads there).  The eight
// stages are separate arrays so the compiler's wait counting sees that a
// stage load never writes the stages being read.
constexpr int kRSlots = 8, kRStage = 128 * 128, kRB = 4;
// the launched form: RB = 2, eight waves (two per SIMD, each with half the
// registers, so a ring of six slots)
constexpr int kRB8 = 2, kRSlots8 = 6;
// the last step issued before step s's loads (sr_last<LEAD>(0): the
// prologue's), LEAD steps ahead
template <int LEAD>
constexpr int sr_last(int s) { return s + LEAD - 1; }

template <int OUT, int NKT, int RB>
__global__ __launch_bounds__(64 * (16 / RB), 1) void k_sp24_i8r(
    int nkt_arg, const v4i* __restrict__ A, const uint32_t* __restrict__ I,
    const int8_t* __restrict__ B, int64_t ldb, int M, int N, const float* __restrict__ ws, float xs,
    float inv_out, int32_t out_zp, int inrange, void* __restrict__ Y, int64_t ldy, int yvec, int ntn,
    int32_t x_zp, int32_t zp_shift, const float* __restrict__ xs_dev, const uint8_t* __restrict__ zp_dev,
    const int32_t* __restrict__ row_sum) {
    __shared__ __attribute__((aligned(1024))) char b0[kRStage];
    __shared__ __attribute__((aligned(1024))) char b1[kRStage];
    __shared__ __attribute__((aligned(1024))) char b2[kRStage];
    __shared__ __attribute__((aligned(1024))) char b3[kRStage];
    __shared__ __attribute__((aligned(1024))) char b4[kRStage];
    __shared__ __attribute__((aligned(1024))) char b5[kRStage];
    __shared__ __attribute__((aligned(1024))) char b6[kRStage];
    __shared__ __attribute__((aligned(1024))) char b7[kRStage];
    // NW waves of RB row blocks each: 16 row blocks (256 rows) per tile
    constexpr int NW = 16 / RB;
    __shared__ __attribute__((aligned(16))) float scl[64 * NW];  // the tile's row scales (and the next rows)
    constexpr int nkt = NKT, kRLoads = 2 * RB + 1;
    constexpr int SLOTS = RB == 4 ? kRSlots : kRSlots8, LEAD = SLOTS - 1;
    static_assert((RB == 2 || RB == 4) && kRLoads * LEAD <= 63, "loads in flight exceed the wave's counter");
    (void)nkt_arg;
    const int t = threadIdx.x, w = __builtin_amdgcn_readfirstlane(t >> 6), l = t & 63;
    const int kb = l >> 4, c = l & 15;
    int mt, nt;
    {
        const int G = (int)gridDim.x, L = (int)blockIdx.x, xcd = L & 7, slot = L >> 3;
        const int q = G >> 3, rem = G & 7;
        const int T = xcd * q + min(xcd, rem) + slot;
        mt = T / ntn;
        nt = T % ntn;
    }
    const int64_t mb0 = (int64_t)mt * (NW * RB);  // the tile's first row block
    const int64_t n0 = (int64_t)nt * kI8TileN;
    auto stage = [&](auto uc) -> char* {
        constexpr int u = decltype(uc)::value;
        if constexpr (u == 0) return b0;
        else if constexpr (u == 1) return b1;
        else if constexpr (u == 2) return b2;
        else if constexpr (u == 3) return b3;
        else if constexpr (u == 4) return b4;
        else if constexpr (u == 5) return b5;
        else if constexpr (u == 6) return b6;
        else return b7;
    };
    // Every load address is a wave-uniform base (scalar registers) plus a
    // per-lane offset fixed for the whole kernel, so the loads take the
    // scalar-base form and the loop needs no per-load address arithmetic.
    // This wave's row blocks mb0 + RB w + i: element (row block, step) at
    // (rb * nkt + step) * 64 + lane; their positions are elements
    // (RB w) % 4 .. of group (mb0 + RB w) / 4 of idxw (four row blocks per
    // group).
    // (the positions are loaded as exactly RB dwords of the lane's 16 bytes:
    // a dead fourth register of a pending load would be handed to other
    // values, and writing it makes the compiler drain every load first)
    typedef int vrb __attribute__((ext_vector_type(RB)));
    const v4i* aw = A + (mb0 + RB * w) * nkt * 64;
    const uint32_t* iw = I + ((mb0 + RB * w) / 4 * nkt * 64) * 4 + (RB * w) % 4;
    // B: the step's 128 X rows, row n = 8 (w + NW i) + l / 8 loaded by this
    // lane (16-byte chunk (l % 8) ^ xrow_swizzle(n) of the tile's 128
    // columns), RB loads per wave: base bw + 128 ldb per step, lane offset
    // boff[i]
    const int8_t* bw = B + n0 + (int64_t)8 * w * ldb;
    int boff[RB];
#pragma unroll
    for (int i = 0; i < RB; ++i) {
        const int n = 8 * (w + NW * i) + (l >> 3);
        const int chunk = (l & 7) ^ xrow_swizzle(n);
        boff[i] = (int)((int64_t)(8 * NW * i + (l >> 3)) * ldb) + 16 * chunk;
    }
    v4i ar[SLOTS][RB];
    vrb ir[SLOTS];
    // the nine loads of step TS (a compile-time step, below nkt) into slot
    // and stage TS % 8
    auto issue = [&](auto tc) {
        constexpr int ts = decltype(tc)::value, u = ts % SLOTS;
        char* st = stage(std::integral_constant<int, u>{});
#pragma unroll
        for (int i = 0; i < RB; ++i) ar[u][i] = aw[(i * nkt + ts) * 64 + l];
        ir[u] = *reinterpret_cast<const vrb*>(iw + (ts * 64 + l) * 4);
        const int8_t* bs = bw + (int64_t)ts * 128 * ldb;
#pragma unroll
        for (int i = 0; i < RB; ++i) lds_copy16(bs, boff[i], PFR_LDS(st + 8 * (w + NW * i) * 128));
    };
    // B fragment of column block j from a stage (see k_sp24_i8, XROW form)
    const int trk = (16 * kb + (c >> 1)) * 128 + 8 * (c & 1);
    const int trf = xrow_swizzle(16 * kb + (c >> 1));
    auto fetch_b = [&](v8i& f, const char* st, int j) {
        v2i q[4];
        const char* bp = st + trk + 16 * (j ^ trf);
#pragma unroll
        for (int r = 0; r < 4; ++r)
            q[r] = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                (__attribute__((address_space(3))) v2i*)(bp + 1024 * (r & 1) + 8192 * (r >> 1)));
        f = v8i{q[0].x, q[0].y, q[1].x, q[1].y, q[2].x, q[2].y, q[3].x, q[3].y};
    };
    v4i acc[RB][8];
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = v4i{0, 0, 0, 0};
    v8i bq[4];
    auto vm_wait = [](int n) { return (n & 0xF) | ((n >> 4) << 14) | (7 << 4) | (0 << 8); };
    // the epilogue's row scales go to LDS ahead of everything (their latency
    // is then hidden by the whole product): row 64w + l by lane l of wave w,
    // clamped to the last row
    if constexpr (OUT != PFR_SP24_OUT_I32)
        __builtin_amdgcn_global_load_lds(ws + min((int)(mb0 * 16) + t, M - 1), PFR_LDS(scl + 64 * w), 4, 0, 0);
    // Load schedule: the prologue issues steps 0 .. 6 and waits for step 0;
    // then step s issues, after its barrier, step s + 7 (none past the end).
    // The wait of step s is for step s + 1: the steps issued after it, nine
    // loads each, may still be in flight (all counts are compile-time).
    // (Issuing fewer steps up front and catching up two per step starts the
    // MFMAs ~3k clocks earlier but costs more than that in the first steps:
    // the CU's address unit, not the latency, paces the loads there.)  Every wave issues step 0
    // before any wave issues step 1 (a barrier): the address unit takes
    // loads in arrival order, and the first MFMAs wait for every wave's step
    // 0.  Each step's loads are kept apart by scheduling barriers: the waits
    // count them in step order, and the LDS stages are filled by loads the
    // compiler does not wait for itself.
    auto prologue_issue = [&](auto tc) {
        __builtin_amdgcn_sched_barrier(0);
        issue(tc);
        __builtin_amdgcn_sched_barrier(0);
    };
    static_assert(nkt > sr_last<LEAD>(0), "the prologue issues seven steps");
    prologue_issue(std::integral_constant<int, 0>{});
    __builtin_amdgcn_s_barrier();
    static_for<1, sr_last<LEAD>(0) + 1>([&](auto tc) { prologue_issue(tc); });
    __builtin_amdgcn_s_waitcnt(vm_wait(kRLoads * sr_last<LEAD>(0)));
    __builtin_amdgcn_s_barrier();
    fetch_b(bq[0], b0, 0);
    fetch_b(bq[1], b0, 1);
    fetch_b(bq[2], b0, 2);
    // step S (compile-time)
    auto step = [&](auto sc) {
        constexpr int S = decltype(sc)::value, u = S % SLOTS, un = (u + 1) % SLOTS;
        constexpr int first = sr_last<LEAD>(S) + 1, last = std::min(sr_last<LEAD>(S + 1), nkt - 1);
        // even steps wait for steps S + 1 and S + 2 (the loads issued after
        // them may still be in flight) and meet at the barrier; odd steps
        // read stage S + 1, already waited for, and load without a barrier
        constexpr bool SYNC = S % 2 == 0;
        constexpr int later = std::max(0, std::min(sr_last<LEAD>(S), nkt - 1) - S - 2);  // issued after step S + 2
        const char* cur = stage(std::integral_constant<int, u>{});
        const char* nxt = stage(std::integral_constant<int, un>{});
        __builtin_amdgcn_sched_barrier(0);
        static_for<0, 5>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            fetch_b(bq[(j + 3) % 4], cur, j + 3);
#pragma unroll
            for (int i = 0; i < RB; ++i)
                acc[i][j] = __builtin_amdgcn_smfmac_i32_16x16x128_i8(ar[u][i], bq[j % 4], acc[i][j], ir[u][i], 0, 0);
        });
        static_for<0, 20>([&](auto gc) {
            if constexpr (decltype(gc)::value < 5 * RB) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
        });
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (SYNC) {
            // vmcnt only: the stage reuse needs this wave's loads and every
            // wave at the barrier, not its fragment reads of stage s, which
            // keep flowing through the barrier (lgkmcnt left alone)
            __builtin_amdgcn_s_waitcnt(vm_wait(kRLoads * later) | (0xF << 8));
            __builtin_amdgcn_s_barrier();
        }
        __builtin_amdgcn_sched_barrier(0);
        static_for<first, last + 1>([&](auto tc) { issue(tc); });
        static_for<5, 8>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            fetch_b(bq[(j + 3) % 4], nxt, j - 5);
#pragma unroll
            for (int i = 0; i < RB; ++i)
                acc[i][j] = __builtin_amdgcn_smfmac_i32_16x16x128_i8(ar[u][i], bq[j % 4], acc[i][j], ir[u][i], 0, 0);
        });
        static_for<0, 12>([&](auto gc) {
            constexpr int g = decltype(gc)::value;
            if constexpr (g < 3 * RB) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
            if constexpr (g < kRLoads * std::max(0, last - first + 1))
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read (next loads)
        });
    };
    static_for<0, nkt>([&](auto sc) { step(sc); });
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0);  // the repeated loads have landed
    __builtin_amdgcn_s_barrier();
    // wave w's epilogue rows go to a stage of its own (every second one for
    // four waves)
    char* own;
    if constexpr (NW == 4) {
        own = w == 0 ? b0 : (w == 1 ? b2 : (w == 2 ? b4 : b6));
    } else {
        own = w == 0 ? b0 : w == 1 ? b1 : w == 2 ? b2 : w == 3 ? b3 : w == 4 ? b4 : w == 5 ? b5 : w == 6 ? b6 : b7;
    }
    char* tile = own - w * 16 * RB * 128;
    float wsv[RB][4];
    if constexpr (OUT != PFR_SP24_OUT_I32) {
#pragma unroll
        for (int i = 0; i < RB; ++i) {
            const v4f v = *reinterpret_cast<const v4f*>(scl + (w * RB + i) * 16 + 4 * kb);
#pragma unroll
            for (int r = 0; r < 4; ++r) wsv[i][r] = v[r];
        }
    }
    sp24_i8_epilogue<OUT, RB>(acc, tile, mb0, n0, M, N, wsv, xs, inv_out, out_zp, inrange, Y, ldy, yvec, x_zp, zp_shift,
                          xs_dev, zp_dev, row_sum);
}

// bf16 2:4 GEMM with the int8 kernel's pipeline: 256 x 128 outputs per
// workgroup of four waves (one per SIMD, 64 rows x 128 columns each: 4 x 8
// tiles of 16 x 16, 128 fp32 accumulators), a k step of 64 (one
// v_smfmac_f32_16x16x64_bf16 per tile), operands in four 36 KiB LDS stages
// filled by direct-to-LDS loads four steps ahead:
//   A values  [16 row blocks][64 lanes][16 B]  (8 kept bf16 per lane)
//   A indices [16 row blocks][64 lanes] u32    (the word of the step's k
//             pair; the step uses half abid = step % 2)
//   B         [128 columns][128 B]: the 64 bf16 of one XT row, 16-byte chunk
//             c stored at c ^ ((column >> 1) & 7) (16 distinct bank groups
//             per ds_read_b128)
// The per-lane B fragment of the bf16 instruction (k 8 kb + e, then 32 +
// 8 kb + e) occupies the same bytes of the 128-byte row as the int8 one (k
// 16 kb + b, then 64 + 16 kb + b), so the B reads are the int8 kernel's.
// Per step a workgroup loads 36 KiB for 4 x 32 smfmac (16 clocks each per
// SIMD: 512), the int8 kernel's balance, so it is bound the same way: by
// the operand loads.  nkt (steps) is a multiple of 4 (K padded to 256).
// XROW = true reads the row-major activation X itself (K % 256 == 0, N %
// 128 == 0, rows 16-byte aligned) instead of a transposed copy: LDS then
// holds the step's 64 X rows (256 B each; 16-byte piece q of row k at q ^
// 2 bf16_swizzle(k), pairs kept together) and the B fragments come from
// ds_read_b64_tr_b16, which (measured on the device) gives lane t of each
// 16-lane group element t % 4 of the 8-byte reads of source lanes t / 4 +
// 4i, i = 0..3; so source lane s pointing at row k0 + s / 4, columns
// 4 (s % 4) .. + 3 of a 16-column chunk gives lane t the four k values k0 ..
// k0 + 3 of column chunk + t.
__device__ __forceinline__ int bf16_swizzle(int k) { return (k & 3) | (((k >> 3) & 1) << 2); }

template <bool XROW>
__global__ __launch_bounds__(kI8Threads, 1) void k_sp24_bf16p(int nkt, const v4i* __restrict__ A,
                                                              const uint32_t* __restrict__ I,
                                                              const uint16_t* __restrict__ XT, int64_t ldb_bytes,
                                                              int M, int N, float* __restrict__ Y, int64_t ldy,
                                                              int ntn) {
    __shared__ __attribute__((aligned(1024))) char st0[kStage];
    __shared__ __attribute__((aligned(1024))) char st1[kStage];
    __shared__ __attribute__((aligned(1024))) char st2[kStage];
    __shared__ __attribute__((aligned(1024))) char st3[kStage];
    const int t = threadIdx.x, w = __builtin_amdgcn_readfirstlane(t >> 6), l = t & 63;
    const int kb = l >> 4, c = l & 15;
    int mt, nt;
    {  // consecutive tiles of the m-major order go to one XCD
        const int G = (int)gridDim.x, L = (int)blockIdx.x, xcd = L & 7, slot = L >> 3;
        const int q = G >> 3, rem = G & 7;
        const int T = xcd * q + min(xcd, rem) + slot;
        mt = T / ntn;
        nt = T % ntn;
    }
    const int64_t mb0 = (int64_t)mt * (kI8TileM / 16);
    const int64_t n0 = (int64_t)nt * kI8TileN;
    constexpr int kLoads = 12;
    const int nkp = nkt / 2;
    const v4i* asrc = A + ((mb0 + w) * nkt) * 64 + l;
    const uint32_t* isrc = I + ((mb0 + w) * nkp) * 64 + l;
    const int64_t arb4 = (int64_t)4 * nkt * 64, irb4 = (int64_t)4 * nkp * 64;
    // B: per k step, XT form: 128 XT rows (columns n0 ..) of 128 B, 8 per
    // wave instruction; X-row form: 64 X rows (k) of 256 B, 4 per instruction
    const v4i* bsrc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (XROW) {
            const int k = 4 * (w + 4 * i) + (l >> 4);
            const int piece = (l & 15) ^ (2 * bf16_swizzle(k));
            bsrc[i] = reinterpret_cast<const v4i*>(reinterpret_cast<const char*>(XT) + k * ldb_bytes + 2 * n0 +
                                                   16 * piece);
        } else {
            const int n = 8 * (w + 4 * i) + (l >> 3);
            const int chunk = (l & 7) ^ ((n >> 1) & 7);
            bsrc[i] = reinterpret_cast<const v4i*>(reinterpret_cast<const char*>(XT) + (n0 + n) * ldb_bytes +
                                                   16 * chunk);
        }
    }
    const int64_t b_step = XROW ? 64 * ldb_bytes / 16 : 8;  // v4i per k step
    auto issue = [&](char* st, int s) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __builtin_amdgcn_global_load_lds(asrc + i * arb4 + (int64_t)s * 64, PFR_LDS(st + (w + 4 * i) * 1024), 16,
                                             0, 0);
            __builtin_amdgcn_global_load_lds(isrc + i * irb4 + (int64_t)(s >> 1) * 64,
                                             PFR_LDS(st + kLdsA + (w + 4 * i) * 256), 4, 0, 0);
            __builtin_amdgcn_global_load_lds(bsrc[i] + (int64_t)s * b_step,
                                             PFR_LDS(st + kLdsA + kLdsI + 8 * (w + 4 * i) * 128), 16, 0, 0);
        }
    };
    auto issue_tail = [&](char* st) {  // same instructions, every lane reading A[0]
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __builtin_amdgcn_global_load_lds(A, PFR_LDS(st + (w + 4 * i) * 1024), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(A, PFR_LDS(st + kLdsA + (w + 4 * i) * 256), 4, 0, 0);
            __builtin_amdgcn_global_load_lds(A, PFR_LDS(st + kLdsA + kLdsI + 8 * (w + 4 * i) * 128), 16, 0, 0);
        }
    };
    const int xsw = (c >> 1) & 7;
    const int bxt = kLdsA + kLdsI + c * 128;
    // X-row form: read r (k0 = 8 kb + 4 (r & 1) + 32 (r >> 1)) of this lane
    // starts at row k0 + c / 4, bytes 8 ((c % 4) & 1) of logical piece 2j +
    // (c % 4) / 2; bf16_swizzle of that row is the same for all four reads
    const int trg = 2 * ((c >> 2) | ((kb & 1) << 2));
    const int trb = kLdsA + kLdsI + (8 * kb + (c >> 2)) * 256 + 8 * (c & 1);
    v4f acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
    struct Frag {
        v4i a[4];
        int ix[4];
        v8i b[8];
    };
    auto fetch = [&](Frag& f, const char* st) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if constexpr (XROW) {
                typedef short v4s __attribute__((ext_vector_type(4)));
                v2i q[4];
                const char* bp = st + trb + 16 * ((2 * j + ((c >> 1) & 1)) ^ trg);
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    q[r] = __builtin_bit_cast(
                        v2i, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                 (__attribute__((address_space(3))) v4s*)(bp + 1024 * (r & 1) + 8192 * (r >> 1))));
                f.b[j] = v8i{q[0].x, q[0].y, q[1].x, q[1].y, q[2].x, q[2].y, q[3].x, q[3].y};
            } else {
                const char* bp = st + bxt + j * 16 * 128;
                const v4i lo = *reinterpret_cast<const v4i*>(bp + 16 * (kb ^ xsw));
                const v4i hi = *reinterpret_cast<const v4i*>(bp + 16 * ((4 + kb) ^ xsw));
                f.b[j] = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f.a[i] = *reinterpret_cast<const v4i*>(st + ((w * 4 + i) * 64 + l) * 16);
            f.ix[i] = *reinterpret_cast<const int*>(st + kLdsA + ((w * 4 + i) * 64 + l) * 4);
        }
    };
    auto mma = [&](const Frag& f, auto abid) {
        constexpr int H = decltype(abid)::value;
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                acc[i][j] = __builtin_amdgcn_smfmac_f32_16x16x64_bf16(__builtin_bit_cast(v8bf, f.a[i]),
                                                                      __builtin_bit_cast(v16bf, f.b[j]), acc[i][j],
                                                                      f.ix[i], 0, H);
    };
    auto vm_wait = [](int n) { return (n & 0xF) | ((n >> 4) << 14) | (7 << 4) | (0 << 8); };
    Frag fa, fb;
    auto step = [&](Frag& cur, Frag& nxt, char* st_cur, char* st_next, int s, auto abid) {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(vm_wait(2 * kLoads));
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        if (s >= 0) issue(st_cur, s + 4);
        else issue_tail(st_cur);
        fetch(nxt, st_next);
        mma(cur, abid);
        static_for<0, 32>([&](auto gc) {
            constexpr int g = decltype(gc)::value;
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);               // MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, g < 8 ? 2 : 1, 0);   // DS read
            if constexpr ((g + 1) * 12 / 32 > g * 12 / 32)
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);           // VMEM read (stage load)
        });
    };
    const std::integral_constant<int, 0> h0{};
    const std::integral_constant<int, 1> h1{};
    issue(st0, 0);
    issue(st1, 1);
    issue(st2, 2);
    issue(st3, 3);
    __builtin_amdgcn_s_waitcnt(vm_wait(3 * kLoads) | (0xF << 8));
    __builtin_amdgcn_s_barrier();
    fetch(fa, st0);
    for (int s = 0; s < nkt - 4; s += 4) {
        step(fa, fb, st0, st1, s, h0);
        step(fb, fa, st1, st2, s + 1, h1);
        step(fa, fb, st2, st3, s + 2, h0);
        step(fb, fa, st3, st0, s + 3, h1);
    }
    step(fa, fb, st0, st1, -1, h0);
    step(fb, fa, st1, st2, -1, h1);
    step(fa, fb, st2, st3, -1, h0);
    step(fb, fa, st3, st0, -1, h1);
    __builtin_amdgcn_s_waitcnt(0);  // the tail's loads have landed
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t m = (mb0 + 4 * w + i) * 16 + 4 * kb + r;
            if (m >= M) continue;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int64_t n = n0 + 16 * j + c;
                if (n < N) Y[m * ldy + n] = acc[i][j][r];
            }
        }
}

// x - 128 as int8 for uint8 x (K rows of N bytes, ldx apart, to a compact
// copy): VEC (N and ldx multiples of 16, X 16-byte aligned) flips 16 bytes
// per thread, otherwise one byte per thread, blockIdx.y striding the rows.
template <bool VEC>
__global__ __launch_bounds__(256) void k_flip_sign(const uint8_t* __restrict__ X, int64_t K, int64_t N,
                                                   int64_t ldx, uint8_t* __restrict__ Y) {
    if constexpr (VEC) {
        const int64_t cpr = N / 16, total = K * cpr;
        for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
            const int64_t r = i / cpr, c = i - r * cpr;
            uint4 v = *reinterpret_cast<const uint4*>(X + r * ldx + 16 * c);
            v.x ^= 0x80808080u;
            v.y ^= 0x80808080u;
            v.z ^= 0x80808080u;
            v.w ^= 0x80808080u;
            *reinterpret_cast<uint4*>(Y + r * N + 16 * c) = v;
        }
    } else {
        const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
        if (n >= N) return;
        for (int64_t r = blockIdx.y; r < K; r += gridDim.y) Y[r * N + n] = X[r * ldx + n] ^ 0x80u;
    }
}

// ---- host -----------------------------------------------------------------

pfr_sp24* pack_i8(pfr_ctx* ctx, int64_t M, int64_t K, const int8_t* W) {
    const int64_t Mp = round_up(M, kPadM), Kp = round_up(std::max<int64_t>(K, 1), 512), nkt = Kp / 128;
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
        std::vector<int32_t> rs((size_t)Mp, 0);
        for (int64_t r = 0; r < M; ++r) {
            int64_t sum = 0;
            for (int64_t k = 0; k < K; ++k) sum += W[r * K + k];
            rs[(size_t)r] = (int32_t)sum;  // |sum| <= 128 K < 2^31
        }
        PFR_HIP(hipMalloc(&w->a, a.size()));
        PFR_HIP(hipMalloc(&w->idx, ix.size() * 4));
        PFR_HIP(hipMalloc(&w->row_sum, rs.size() * 4));
        PFR_HIP(hipMemcpy(w->a, a.data(), a.size(), hipMemcpyHostToDevice));
        PFR_HIP(hipMemcpy(w->idx, ix.data(), ix.size() * 4, hipMemcpyHostToDevice));
        PFR_HIP(hipMemcpy(w->row_sum, rs.data(), rs.size() * 4, hipMemcpyHostToDevice));
        return w;
    } catch (...) {
        free_sp24(w);
        throw;
    }
}

bool bf16_nz(uint16_t b) { return (b & 0x7FFF) != 0; }

pfr_sp24* pack_bf16(pfr_ctx* ctx, int64_t M, int64_t K, const uint16_t* W) {
    const int64_t Mp = round_up(M, kPadM), Kp = round_up(std::max<int64_t>(K, 1), 256), nkt = Kp / 64, nkp = nkt / 2;
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

// ---- Packing a weight already on the device -------------------------------
// The same layouts as pack_i8 / pack_bf16, written by one thread per
// (16-row tile, k tile, lane) from a device weight; the 2:4 check reports
// the first offending group (row-major order) through an atomic minimum.

template <class T>
__device__ __forceinline__ bool sp24_nz(T v) {
    if constexpr (sizeof(T) == 1) return v != 0;
    else return (v & 0x7FFF) != 0;  // bf16: +0 and -0 are zeros
}

// The two kept positions of a 4-group (ascending), as pick2 chooses them.
__device__ __forceinline__ void pick2_dev(unsigned nzmask, int* p0, int* p1) {
    const int n = __popc(nzmask);
    if (n >= 2) {
        *p0 = __ffs(nzmask) - 1;
        *p1 = __ffs(nzmask & (nzmask - 1)) - 1;
    } else if (n == 1) {
        const int p = __ffs(nzmask) - 1;
        *p0 = 0;
        *p1 = p == 0 ? 1 : p;
    } else {
        *p0 = 0;
        *p1 = 1;
    }
}

template <class T>
__device__ __forceinline__ T sp24_at(const T* __restrict__ W, int64_t M, int64_t K, int64_t r, int64_t k) {
    return (r < M && k < K) ? W[r * K + k] : T(0);
}

template <class T>
__global__ __launch_bounds__(256) void k_sp24_check(const T* __restrict__ W, int64_t M, int64_t K, int64_t ng,
                                                    unsigned long long* __restrict__ first_bad) {
    const int64_t n = M * ng;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const int64_t r = i / ng, k = (i % ng) * 4;
        int c = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t) c += sp24_nz(sp24_at(W, M, K, r, k + t)) ? 1 : 0;
        if (c > 2) atomicMin(first_bad, (unsigned long long)i);
    }
}

// int8: thread (mt, kt, l) writes the 16 kept bytes and the index word of
// lane l's fragment: groups g = 0..7 at k = kt * 128 + 32 * (l >> 4) + 4 g of
// row mt * 16 + (l & 15).
__global__ __launch_bounds__(256) void k_sp24_pack_i8(const int8_t* __restrict__ W, int64_t M, int64_t K,
                                                      int64_t nmt, int64_t nkt, int4* __restrict__ a,
                                                      uint32_t* __restrict__ ix) {
    const int64_t n = nmt * nkt * 64;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const int l = (int)(i & 63);
        const int64_t kt = (i >> 6) % nkt, mt = (i >> 6) / nkt;
        const int64_t r = mt * 16 + (l & 15);
        uint32_t word = 0, b[4] = {0, 0, 0, 0};
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const int64_t ks = kt * 128 + 32 * (l >> 4) + 4 * g;
            int8_t v[4];
            unsigned nz = 0;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                v[t] = sp24_at(W, M, K, r, ks + t);
                nz |= (v[t] != 0 ? 1u : 0u) << t;
            }
            int p0, p1;
            pick2_dev(nz, &p0, &p1);
            const uint32_t pair = (uint32_t)(uint8_t)v[p0] | ((uint32_t)(uint8_t)v[p1] << 8);
            b[g / 2] |= pair << (16 * (g % 2));
            word |= (uint32_t)(p0 | (p1 << 2)) << (4 * g);
        }
        a[i] = make_int4((int)b[0], (int)b[1], (int)b[2], (int)b[3]);
        ix[i] = word;
    }
}

// bf16: thread (mt, kp, l) writes lane l's two fragments of k tiles 2 kp and
// 2 kp + 1 (8 kept values each) and their shared index word (low half: the
// even tile).
__global__ __launch_bounds__(256) void k_sp24_pack_bf16(const uint16_t* __restrict__ W, int64_t M, int64_t K,
                                                        int64_t nmt, int64_t nkp, int4* __restrict__ a,
                                                        uint32_t* __restrict__ ix) {
    const int64_t n = nmt * nkp * 64, nkt = 2 * nkp;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const int l = (int)(i & 63);
        const int64_t kp = (i >> 6) % nkp, mt = (i >> 6) / nkp;
        const int64_t r = mt * 16 + (l & 15);
        uint32_t word = 0;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int64_t kt = 2 * kp + h;
            uint32_t b[4] = {0, 0, 0, 0}, half = 0;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int64_t ks = kt * 64 + 16 * (l >> 4) + 4 * g;
                uint16_t v[4];
                unsigned nz = 0;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    v[t] = sp24_at(W, M, K, r, ks + t);
                    nz |= (sp24_nz(v[t]) ? 1u : 0u) << t;
                }
                int p0, p1;
                pick2_dev(nz, &p0, &p1);
                b[g] = (uint32_t)v[p0] | ((uint32_t)v[p1] << 16);
                half |= (uint32_t)(p0 | (p1 << 2)) << (4 * g);
            }
            a[(mt * nkt + kt) * 64 + l] = make_int4((int)b[0], (int)b[1], (int)b[2], (int)b[3]);
            word |= half << (16 * h);
        }
        ix[i] = word;
    }
}

// Row sums of an int8 weight (the zero-point correction), one workgroup per
// row.
// idxw[((g * nkt + s) * 64 + l) * 4 + r] = idx[((kRB g + r) * nkt + s) * 64 + l]
// for r < kRB and row blocks below nrb, else 0
__global__ __launch_bounds__(256) void k_sp24_idxw(const uint32_t* __restrict__ idx, int64_t nrb, int64_t ngrp,
                                                   int64_t nkt, v4i* __restrict__ idxw) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (g, s, l)
    if (e >= ngrp * nkt * 64) return;
    const int64_t g = e / (nkt * 64), sl = e % (nkt * 64);
    v4i v = v4i{0, 0, 0, 0};
#pragma unroll
    for (int r = 0; r < kRB; ++r)
        if (kRB * g + r < nrb) v[r] = (int)idx[(kRB * g + r) * nkt * 64 + sl];
    idxw[e] = v;
}

__global__ __launch_bounds__(256) void k_sp24_row_sum(const int8_t* __restrict__ W, int64_t K,
                                                      int32_t* __restrict__ rs) {
    __shared__ int part[4];
    const int64_t r = blockIdx.x;
    int sum = 0;
    for (int64_t k = threadIdx.x; k < K; k += 256) sum += W[r * K + k];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o, 64);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = sum;
    __syncthreads();
    if (threadIdx.x == 0) rs[r] = (part[0] + part[1]) + (part[2] + part[3]);
}

unsigned grid_for(int64_t n) { return (unsigned)std::min<int64_t>((n + 255) / 256, 8192); }

pfr_sp24* pack_dev(pfr_ctx* ctx, int64_t M, int64_t K, const void* Wv, pfr_dtype dtype) {
    hipStream_t s = ctx->stream;
    const bool i8 = dtype == PFR_I8;
    const int64_t Mp = round_up(M, kPadM), Kp = round_up(std::max<int64_t>(K, 1), i8 ? 512 : 256);
    // the 2:4 check over every 4-group of the padded rows (the padding is zero)
    {
        unsigned long long* bad = nullptr;
        PFR_HIP(hipMalloc(&bad, sizeof(unsigned long long)));
        const unsigned long long none = ~0ull;
        unsigned long long first = none;
        hipError_t e = hipMemcpyAsync(bad, &none, sizeof(none), hipMemcpyHostToDevice, s);
        const int64_t ng = Kp / 4;
        if (e == hipSuccess && M > 0) {
            if (i8)
                hipLaunchKernelGGL(k_sp24_check<int8_t>, dim3(grid_for(M * ng)), dim3(256), 0, s,
                                   static_cast<const int8_t*>(Wv), M, K, ng, bad);
            else
                hipLaunchKernelGGL(k_sp24_check<uint16_t>, dim3(grid_for(M * ng)), dim3(256), 0, s,
                                   static_cast<const uint16_t*>(Wv), M, K, ng, bad);
            e = hipGetLastError();
        }
        if (e == hipSuccess) e = hipMemcpyAsync(&first, bad, sizeof(first), hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        (void)hipFree(bad);
        if (e != hipSuccess) throw pfr::Error(PFR_ERR_HIP, std::string("2:4 check: ") + hipGetErrorString(e));
        if (first != none) {
            const int64_t r = (int64_t)(first / (unsigned long long)ng), k = (int64_t)(first % (unsigned long long)ng) * 4;
            throw pfr::Error(PFR_ERR_INVALID_ARG, "weight is not 2:4 sparse: row " + std::to_string(r) + ", k " +
                                                      std::to_string(k) + ".." + std::to_string(k + 3) +
                                                      " has more than two nonzeros");
        }
    }
    auto* w = new pfr_sp24();
    try {
        w->ctx = ctx;
        w->M = M;
        w->K = K;
        w->Mp = Mp;
        w->Kp = Kp;
        w->dtype = dtype;
        const int64_t nmt = Mp / 16;
        if (i8) {
            const int64_t nkt = Kp / 128;
            PFR_HIP(hipMalloc(&w->a, (size_t)(nmt * nkt * 64 * 16)));
            PFR_HIP(hipMalloc(&w->idx, (size_t)(nmt * nkt * 64 * 4)));
            PFR_HIP(hipMalloc(&w->row_sum, (size_t)Mp * 4));
            hipLaunchKernelGGL(k_sp24_pack_i8, dim3(grid_for(nmt * nkt * 64)), dim3(256), 0, s,
                               static_cast<const int8_t*>(Wv), M, K, nmt, nkt, static_cast<int4*>(w->a), w->idx);
            PFR_HIP(hipMemcpyAsync(w->row_sum, std::vector<int32_t>((size_t)Mp, 0).data(), (size_t)Mp * 4,
                                   hipMemcpyHostToDevice, s));
            PFR_HIP(hipStreamSynchronize(s));  // the zero vector is a temporary
            if (M > 0 && K > 0)
                hipLaunchKernelGGL(k_sp24_row_sum, dim3((unsigned)M), dim3(256), 0, s,
                                   static_cast<const int8_t*>(Wv), K, w->row_sum);
        } else {
            const int64_t nkp = Kp / 128;
            PFR_HIP(hipMalloc(&w->a, (size_t)(nmt * 2 * nkp * 64 * 16)));
            PFR_HIP(hipMalloc(&w->idx, (size_t)(nmt * nkp * 64 * 4)));
            hipLaunchKernelGGL(k_sp24_pack_bf16, dim3(grid_for(nmt * nkp * 64)), dim3(256), 0, s,
                               static_cast<const uint16_t*>(Wv), M, K, nmt, nkp, static_cast<int4*>(w->a), w->idx);
        }
        PFR_HIP(hipGetLastError());
        PFR_HIP(hipStreamSynchronize(s));
        return w;
    } catch (...) {
        (void)hipStreamSynchronize(s);
        free_sp24(w);
        throw;
    }
}

void check_i8(const pfr_sp24* W) {
    pfr::require(W != nullptr, "null 2:4 weight handle");
    if (W->dtype != PFR_I8) throw pfr::Error(PFR_ERR_UNSUPPORTED, "weight is not int8");
}

// XT for the activation: int8 or bf16 bits, Np x Kp.
// x_u8: X holds uint8 values.  x_zp: the activation zero point, or
// (zp_dev set) a device uint8 holding it; x_scale likewise with xs_dev.
void gemm_i8_dev(pfr_ctx* ctx, const pfr_sp24* W, const int8_t* X, int64_t N, int64_t ldx, float x_scale,
                 int out_kind, float out_scale, int32_t out_zp, void* Y, int64_t ldy, bool x_u8 = false,
                 int32_t x_zp = 0, const float* xs_dev = nullptr, const uint8_t* zp_dev = nullptr) {
    check_i8(W);
    pfr::require(W->K < (1 << 17), "K must be below 2^17 for exact int32 accumulation");
    pfr::require(x_u8 ? (x_zp >= 0 && x_zp <= 255) : (x_zp >= -128 && x_zp <= 127),
                 "activation zero point outside the activation type's range");
    pfr::require(N >= 0 && N < INT32_MAX, "bad column count");
    pfr::require(ldx >= N && ldy >= N, "leading dimension smaller than N");
    pfr::require(out_kind >= PFR_SP24_OUT_I32 && out_kind <= PFR_SP24_OUT_I8, "unknown output kind");
    if (W->M == 0 || N == 0) return;
    pfr::require(X != nullptr && Y != nullptr, "null X/Y");
    float inv_out = 1.0f;
    if (out_kind != PFR_SP24_OUT_I32 && !xs_dev)
        pfr::require(x_scale > 0.0f && std::isfinite(x_scale), "x_scale must be positive and finite");
    int inrange = 0;
    if (out_kind == PFR_SP24_OUT_I8) {
        pfr::require(out_scale > 0.0f && std::isfinite(out_scale), "output scale must be positive and finite");
        inv_out = 1.0f / out_scale;  // quant_ops.cpp:41
        // |acc| <= (K / 2 kept terms) * 128 * 128 per output; with that times
        // the largest scale product below 2^30 every requantised value is
        // finite and below 2^31 in magnitude (two float roundings add far
        // less than the factor of two), so the kernel may clamp directly
        if (!xs_dev && !x_u8 && x_zp == 0)
            inrange = (double)W->Kp * 8192.0 * (double)W->w_scale_max * (double)x_scale * (double)inv_out <
                      1073741824.0;
    }
    if (x_u8) {
        // the signed MFMA takes x - 128; the zero-point correction adds the 128 back
        uint8_t* xs8 = static_cast<uint8_t*>(ctx->scratch[1].ensure((size_t)(W->K * N) + 16));
        if (N % 16 == 0 && ldx % 16 == 0 && (reinterpret_cast<uintptr_t>(X) & 15) == 0)
            hipLaunchKernelGGL(k_flip_sign<true>,
                               dim3((unsigned)std::min<int64_t>(4096, (W->K * (N / 16) + 255) / 256)), dim3(256), 0,
                               ctx->stream, reinterpret_cast<const uint8_t*>(X), W->K, N, ldx, xs8);
        else
            hipLaunchKernelGGL(k_flip_sign<false>, dim3((unsigned)((N + 255) / 256), (unsigned)std::min<int64_t>(W->K, 1024)),
                               dim3(256), 0, ctx->stream, reinterpret_cast<const uint8_t*>(X), W->K, N, ldx, xs8);
        PFR_HIP(hipGetLastError());
        X = reinterpret_cast<const int8_t*>(xs8);
        ldx = N;
    }
    const int64_t Kp = W->Kp;
    const int nkt = (int)(Kp / 128);
    const int yvec = (ldy % 16 == 0 && (reinterpret_cast<uintptr_t>(Y) & 15) == 0) ? 1 : 0;
    const v4i* A = static_cast<const v4i*>(W->a);
    // The kernel reads whole 128-column, 128-row B tiles.  X itself serves
    // when those stay inside it and its rows are 16-byte aligned; otherwise
    // it is transposed into a zero-padded XT (Np x Kp) first.
    const bool xrow = W->K == Kp && N % kI8TileN == 0 && ldx % 16 == 0 &&
                      (reinterpret_cast<uintptr_t>(X) & 15) == 0;
    int64_t Np = N;
    const int8_t* B = X;
    int64_t ldb = ldx;
    if (!xrow) {
        Np = round_up(N, kI8TileN);
        int8_t* xt = static_cast<int8_t*>(ctx->scratch[3].ensure((size_t)(Np * Kp)));
        const int vec = (ldx % 16 == 0 && (reinterpret_cast<uintptr_t>(X) & 15) == 0) ? 1 : 0;
        hipLaunchKernelGGL(k_transpose_i8, dim3((unsigned)(Kp / 64), (unsigned)((Np + 255) / 256)), dim3(256), 0,
                           ctx->stream, X, W->K, N, ldx, vec, xt, Kp, Np);
        PFR_HIP(hipGetLastError());
        B = xt;
        ldb = Kp;
    }
    const int ntn = (int)(Np / kI8TileN);
    dim3 grid((unsigned)(W->Mp / kI8TileM * ntn));
#define PFR_SP24_LAUNCH_X(OUTK, XR)                                                                             \
    hipLaunchKernelGGL((k_sp24_i8<OUTK, XR>), grid, dim3(kI8Threads), 0, ctx->stream, nkt, A, W->idx, B, ldb,    \
                       (int)W->M, (int)N, W->w_scale, x_scale, inv_out, out_zp, inrange, Y, ldy, yvec, ntn, x_zp,   \
                       x_u8 ? 128 : 0, xs_dev, zp_dev, W->row_sum)
    const int64_t rtiles = (W->M + 64 * kRB - 1) / (64 * kRB);  // 256-row tiles (64 * kRB rows)
    const dim3 rgrid((unsigned)(rtiles * ntn));
#define PFR_SP24_LAUNCH_R(OUTK)                                                                                 \
    hipLaunchKernelGGL((k_sp24_i8r<OUTK, 32, kRB8>), rgrid, dim3(64 * 16 / kRB8), 0, ctx->stream, nkt, A, W->idxw, \
                       B, ldb, (int)W->M, (int)N, W->w_scale, x_scale, inv_out, out_zp, inrange, Y, ldy, yvec, ntn, \
                       x_zp, x_u8 ? 128 : 0, xs_dev, zp_dev, W->row_sum)
    // the register-streamed kernel for the X-row form at 32 k steps, when
    // its tiles stay inside the packed rows and its per-lane B offsets (up to
    // 128 rows of X) fit in 32 bits
    const bool rring = xrow && nkt == 32 && rtiles * 64 * kRB <= W->Mp && ldb * 128 < INT32_MAX;
#define PFR_SP24_LAUNCH(OUTK)                      \
    do {                                           \
        if (rring) PFR_SP24_LAUNCH_R(OUTK);        \
        else if (xrow) PFR_SP24_LAUNCH_X(OUTK, true);   \
        else PFR_SP24_LAUNCH_X(OUTK, false);       \
    } while (0)
    switch (out_kind) {
        case PFR_SP24_OUT_I32: PFR_SP24_LAUNCH(PFR_SP24_OUT_I32); break;
        case PFR_SP24_OUT_F32: PFR_SP24_LAUNCH(PFR_SP24_OUT_F32); break;
        default: PFR_SP24_LAUNCH(PFR_SP24_OUT_I8);
    }
#undef PFR_SP24_LAUNCH
#undef PFR_SP24_LAUNCH_R
#undef PFR_SP24_LAUNCH_X
    PFR_HIP(hipGetLastError());
}

// The activation of the x . W form, act[T, K] row-major, as the kernel's
// K-contiguous B operand XT (Np x Kp): XT[n][k] = act[n][k] (with the sign
// bit flipped for uint8: the signed MFMA takes x - 128), zero outside T x K.
template <bool FLIP>
__global__ __launch_bounds__(256) void k_pad_act(const uint8_t* __restrict__ X, int64_t T, int64_t K, int64_t ldx,
                                                 uint8_t* __restrict__ xt, int64_t Kp, int64_t Np) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= Np * Kp) return;
    const int64_t n = i / Kp, k = i % Kp;
    uint8_t v = 0;
    if (n < T && k < K) v = FLIP ? (uint8_t)(X[n * ldx + k] ^ 0x80u) : X[n * ldx + k];
    xt[i] = v;
}

// Y[t, m] = Yp[m, t] for m < M, t < T (the x . W product's transpose).
__global__ __launch_bounds__(256) void k_transpose_out(const float* __restrict__ Yp, int64_t M, int64_t T,
                                                       int64_t ldyp, float* __restrict__ Y, int64_t ldy) {
    __shared__ float tile[64][65];
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const int64_t t0 = (int64_t)blockIdx.x * 64, m0 = (int64_t)blockIdx.y * 64;
    for (int i = ty; i < 64; i += 4) {
        const int64_t m = m0 + i, t = t0 + tx;
        if (m < M && t < T) tile[i][tx] = Yp[m * ldyp + t];
    }
    __syncthreads();
    for (int i = ty; i < 64; i += 4) {
        const int64_t t = t0 + i, m = m0 + tx;
        if (m < M && t < T) Y[t * ldy + m] = tile[tx][i];
    }
}

// Y[T, M] (float) = act[T, K] . W^T with the 2:4 weight W[M, K] as the
// second operand (the x . W form of a Linear layer), act int8 or uint8 with
// a zero point: the W . X product on XT = act, then its transpose.
void gemm_qt_dev(pfr_ctx* ctx, const pfr_sp24* W, const uint8_t* X, bool x_u8, int64_t T, int64_t ldx,
                 float x_scale, int32_t x_zp, const float* xs_dev, const uint8_t* zp_dev, float* Y, int64_t ldy) {
    check_i8(W);
    pfr::require(W->K < (1 << 17), "K must be below 2^17 for exact int32 accumulation");
    pfr::require(x_u8 ? (x_zp >= 0 && x_zp <= 255) : (x_zp >= -128 && x_zp <= 127),
                 "activation zero point outside the activation type's range");
    pfr::require(T >= 0 && T < INT32_MAX, "bad row count");
    pfr::require(ldx >= W->K && ldy >= W->M, "leading dimension smaller than the row");
    if (W->M == 0 || T == 0) return;
    pfr::require(X != nullptr && Y != nullptr, "null X/Y");
    if (!xs_dev) pfr::require(x_scale > 0.0f && std::isfinite(x_scale), "x_scale must be positive and finite");
    const int64_t Kp = W->Kp, Np = round_up(T, kI8TileN), ldyp = round_up(T, 16);
    uint8_t* xt = static_cast<uint8_t*>(ctx->scratch[3].ensure((size_t)(Np * Kp)));
    float* yp = static_cast<float*>(ctx->scratch[5].ensure((size_t)(W->M * ldyp) * 4));
    const unsigned pb = (unsigned)((Np * Kp + 255) / 256);
    if (x_u8) hipLaunchKernelGGL(k_pad_act<true>, dim3(pb), dim3(256), 0, ctx->stream, X, T, W->K, ldx, xt, Kp, Np);
    else hipLaunchKernelGGL(k_pad_act<false>, dim3(pb), dim3(256), 0, ctx->stream, X, T, W->K, ldx, xt, Kp, Np);
    PFR_HIP(hipGetLastError());
    const int ntn = (int)(Np / kI8TileN);
    const int nkt = (int)(Kp / 128);
    hipLaunchKernelGGL((k_sp24_i8<PFR_SP24_OUT_F32, false>), dim3((unsigned)(W->Mp / kI8TileM * ntn)),
                       dim3(kI8Threads), 0, ctx->stream, nkt, static_cast<const v4i*>(W->a), W->idx,
                       reinterpret_cast<const int8_t*>(xt), Kp, (int)W->M, (int)T, W->w_scale, x_scale, 1.0f, 0, 0,
                       static_cast<void*>(yp), ldyp, 1, ntn, x_zp, x_u8 ? 128 : 0, xs_dev, zp_dev, W->row_sum);
    PFR_HIP(hipGetLastError());
    hipLaunchKernelGGL(k_transpose_out, dim3((unsigned)((T + 63) / 64), (unsigned)((W->M + 63) / 64)), dim3(256), 0,
                       ctx->stream, yp, W->M, T, ldyp, Y, ldy);
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
    // The kernel reads whole 128-column, 64-row B tiles.  X itself serves
    // when those stay inside it and its rows are 16-byte aligned; otherwise
    // it is transposed into a zero-padded XT (Np x Kp) first.
    const bool xrow = W->K == W->Kp && N % kI8TileN == 0 && ldx % 8 == 0 &&
                      (reinterpret_cast<uintptr_t>(X) & 15) == 0;
    const int64_t Np = round_up(N, kI8TileN);
    const int ntn = (int)(Np / kI8TileN);
    const dim3 grid((unsigned)(W->Mp / kI8TileM * ntn));
    if (xrow) {
        hipLaunchKernelGGL(k_sp24_bf16p<true>, grid, dim3(kI8Threads), 0, ctx->stream, (int)(W->Kp / 64),
                           static_cast<const v4i*>(W->a), W->idx, X, ldx * 2, (int)W->M, (int)N, Y, ldy, ntn);
    } else {
        uint16_t* xt = static_cast<uint16_t*>(ctx->scratch[3].ensure(sizeof(uint16_t) * (size_t)(Np * W->Kp)));
        const int vec = (ldx % 4 == 0 && (reinterpret_cast<uintptr_t>(X) & 7) == 0) ? 1 : 0;
        hipLaunchKernelGGL(k_transpose_b16, dim3((unsigned)(W->Kp / 64), (unsigned)(Np / 64)), dim3(256), 0,
                           ctx->stream, X, W->K, N, ldx, vec, xt, W->Kp);
        PFR_HIP(hipGetLastError());
        hipLaunchKernelGGL(k_sp24_bf16p<false>, grid, dim3(kI8Threads), 0, ctx->stream, (int)(W->Kp / 64),
                           static_cast<const v4i*>(W->a), W->idx, xt, W->Kp * 2, (int)W->M, (int)N, Y, ldy, ntn);
    }
    PFR_HIP(hipGetLastError());
}

}  // namespace

namespace {
// Shared by both pack entry points: argument checks, the packing itself
// (host or device weight) and the per-row scales.
template <class Pack>
int sp24_pack_any(pfr_ctx* ctx, int64_t M, int64_t K, const void* W, pfr_dtype dtype, const float* w_scales,
                  int64_t n_scales, pfr_sp24** out, Pack&& pack) {
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
        pfr_sp24* w = pack();
        for (float v : scales) w->w_scale_max = std::max(w->w_scale_max, v);
        try {
            PFR_HIP(hipMalloc(&w->w_scale, sizeof(float) * (size_t)(M > 0 ? M : 1)));
            if (M) PFR_HIP(hipMemcpy(w->w_scale, scales.data(), sizeof(float) * (size_t)M, hipMemcpyHostToDevice));
            if (dtype == PFR_I8) {
                const int64_t nrb = w->Mp / 16, ngrp = (nrb + kRB - 1) / kRB, nkt = w->Kp / 128,
                              n = ngrp * nkt * 64;
                PFR_HIP(hipMalloc(&w->idxw, (size_t)n * 16));
                hipLaunchKernelGGL(k_sp24_idxw, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, ctx->stream, w->idx,
                                   nrb, ngrp, nkt, reinterpret_cast<v4i*>(w->idxw));
                PFR_HIP(hipGetLastError());
                PFR_HIP(hipStreamSynchronize(ctx->stream));
            }
        } catch (...) {
            free_sp24(w);
            throw;
        }
        *out = w;
    });
}
}  // namespace

extern "C" {

int pfr_sp24_pack(pfr_ctx* ctx, int64_t M, int64_t K, const void* W, pfr_dtype dtype, const float* w_scales,
                  int64_t n_scales, pfr_sp24** out) {
    return sp24_pack_any(ctx, M, K, W, dtype, w_scales, n_scales, out, [&] {
        return dtype == PFR_I8 ? pack_i8(ctx, M, K, static_cast<const int8_t*>(W))
                               : pack_bf16(ctx, M, K, static_cast<const uint16_t*>(W));
    });
}

int pfr_sp24_pack_dev(pfr_ctx* ctx, int64_t M, int64_t K, const void* W, pfr_dtype dtype, const float* w_scales,
                      int64_t n_scales, pfr_sp24** out) {
    return sp24_pack_any(ctx, M, K, W, dtype, w_scales, n_scales, out,
                         [&] { return pack_dev(ctx, M, K, W, dtype); });
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

int pfr_sp24_gemm_q_dev(pfr_ctx* ctx, const pfr_sp24* W, const void* X, pfr_dtype x_dtype, int64_t N,
                        int64_t ldx, float x_scale, int32_t x_zero_point, const float* x_scale_dev,
                        const uint8_t* x_zero_point_dev, int out_kind, float out_scale, int32_t out_zp, void* Y,
                        int64_t ldy) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        pfr::require(x_dtype == PFR_I8 || x_dtype == PFR_U8, "activation must be int8 or uint8");
        gemm_i8_dev(ctx, W, static_cast<const int8_t*>(X), N, ldx, x_scale, out_kind, out_scale, out_zp, Y, ldy,
                    x_dtype == PFR_U8, x_zero_point, x_scale_dev, x_zero_point_dev);
    });
}

int pfr_sp24_gemm_q(pfr_ctx* ctx, const pfr_sp24* W, const void* X, pfr_dtype x_dtype, int64_t N, float x_scale,
                    int32_t x_zero_point, int out_kind, float out_scale, int32_t out_zp, void* Y) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        check_i8(W);
        pfr::require(x_dtype == PFR_I8 || x_dtype == PFR_U8, "activation must be int8 or uint8");
        pfr::require(N >= 0, "bad column count");
        const size_t esz = out_kind == PFR_SP24_OUT_I8 ? 1 : 4;
        const size_t xb = (size_t)(W->K * N), yb = esz * (size_t)(W->M * N);
        if (yb == 0) return;
        pfr::require(Y != nullptr && (X != nullptr || xb == 0), "null X/Y");
        hipStream_t s = ctx->stream;
        int8_t* dX = static_cast<int8_t*>(ctx->scratch[0].ensure(xb ? xb : 4));
        void* dY = ctx->scratch[2].ensure(yb);
        if (xb) PFR_HIP(hipMemcpyAsync(dX, X, xb, hipMemcpyHostToDevice, s));
        gemm_i8_dev(ctx, W, dX, N, N, x_scale, out_kind, out_scale, out_zp, dY, N, x_dtype == PFR_U8, x_zero_point);
        PFR_HIP(hipMemcpyAsync(Y, dY, yb, hipMemcpyDeviceToHost, s));
        PFR_HIP(hipStreamSynchronize(s));
    });
}

int pfr_sp24_gemm_qt_dev(pfr_ctx* ctx, const pfr_sp24* W, const void* X, pfr_dtype x_dtype, int64_t T,
                         int64_t ldx, float x_scale, int32_t x_zero_point, const float* x_scale_dev,
                         const uint8_t* x_zero_point_dev, float* Y, int64_t ldy) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        pfr::require(x_dtype == PFR_I8 || x_dtype == PFR_U8, "activation must be int8 or uint8");
        gemm_qt_dev(ctx, W, static_cast<const uint8_t*>(X), x_dtype == PFR_U8, T, ldx, x_scale, x_zero_point,
                    x_scale_dev, x_zero_point_dev, Y, ldy);
    });
}

int pfr_sp24_gemm_qt(pfr_ctx* ctx, const pfr_sp24* W, const void* X, pfr_dtype x_dtype, int64_t T, float x_scale,
                     int32_t x_zero_point, float* Y) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        check_i8(W);
        pfr::require(x_dtype == PFR_I8 || x_dtype == PFR_U8, "activation must be int8 or uint8");
        pfr::require(T >= 0, "bad row count");
        const size_t xb = (size_t)(W->K * T), yb = 4 * (size_t)(W->M * T);
        if (yb == 0) return;
        pfr::require(Y != nullptr && (X != nullptr || xb == 0), "null X/Y");
        hipStream_t s = ctx->stream;
        uint8_t* dX = static_cast<uint8_t*>(ctx->scratch[0].ensure(xb ? xb : 4));
        float* dY = static_cast<float*>(ctx->scratch[2].ensure(yb));
        if (xb) PFR_HIP(hipMemcpyAsync(dX, X, xb, hipMemcpyHostToDevice, s));
        gemm_qt_dev(ctx, W, dX, x_dtype == PFR_U8, T, W->K, x_scale, x_zero_point, nullptr, nullptr, dY, W->M);
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
