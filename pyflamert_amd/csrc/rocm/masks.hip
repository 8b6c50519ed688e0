// Pruning masks on the GPU, bit-identical to the reference's CPU producers.
//
// Magnitude (MagnitudePruning::compute_mask, magnitude_pruning.cpp:22-102):
//   importance |w| (:8-20); threshold = the element at index
//   min(floor((double)n * s), n - 1) of the ascending sort (:65-73); keep
//   |w| > threshold (:79-81); then, while more than (size_t)((float)n * s)
//   zeros remain (:84), restore elements equal to the threshold in flat
//   order (:91-99).  Here the order statistic is a radix select over the
//   |w| bit patterns (non-negative floats order as their uint32 bits; NaN,
//   whose position the reference's std::sort leaves unspecified, sorts above
//   +inf, and, as in the reference's comparisons, is never kept and counts
//   among the zeros), four 8-bit passes, each a histogram kernel and a one-block bucket
//   choice, all on the stream; the tie restore is a flat-order rank of the
//   elements equal to the threshold (per-block counts, a one-block scan,
//   then per-element ranks).
//
// N:M (NMSparsityPruning::compute_mask, nm_sparsity.cpp:45-120): in every
//   group of m consecutive elements keep the n of largest |w| (a last,
//   partial group of g elements keeps ceil((float)(g n) / m)).  Which of
//   equal magnitudes win is decided by std::partial_sort with the comparator
//   |w[a]| > |w[b]|; libstdc++ implements partial_sort as a heap select
//   (bits/stl_algo.h __heap_select: make a heap of the first `keep`
//   positions, then every later position that compares ahead of the heap
//   top replaces it) followed by a sort of the heap, which does not change
//   the kept set.  One thread runs that heap select on its group's indices.
#include <algorithm>
#include <cmath>
#include <vector>

#include <type_traits>

#include "common.hpp"

namespace {

constexpr int kMaskThreads = 256;
constexpr int kMaskPerThread = 16;
constexpr int kMaskPerBlock = kMaskThreads * kMaskPerThread;  // 4096 elements
constexpr int kMaxM = 16;

__device__ __forceinline__ uint32_t mag_bits(float v) { return __float_as_uint(v) & 0x7FFFFFFFu; }

// ---- N:M --------------------------------------------------------------------

// libstdc++'s heap primitives on an index array, with comp(a, b) = "a is
// kept before b" = |w[a]| > |w[b]| (the heap top is the weakest kept index).
struct NmHeap {
    const float* mag;  // |w| of the group
    int* idx;
    __device__ bool comp(int a, int b) const { return mag[a] > mag[b]; }
    __device__ void push(int hole, int top, int value) {
        int parent = (hole - 1) / 2;
        while (hole > top && comp(idx[parent], value)) {
            idx[hole] = idx[parent];
            hole = parent;
            parent = (hole - 1) / 2;
        }
        idx[hole] = value;
    }
    __device__ void adjust(int hole, int len, int value) {
        const int top = hole;
        int child = hole;
        while (child < (len - 1) / 2) {
            child = 2 * (child + 1);
            if (comp(idx[child], idx[child - 1])) child--;
            idx[hole] = idx[child];
            hole = child;
        }
        if ((len & 1) == 0 && child == (len - 2) / 2) {
            child = 2 * (child + 1);
            idx[hole] = idx[child - 1];
            hole = child - 1;
        }
        push(hole, top, value);
    }
    __device__ void make(int len) {
        if (len < 2) return;
        for (int parent = (len - 2) / 2;; --parent) {
            adjust(parent, len, idx[parent]);
            if (parent == 0) return;
        }
    }
    // The first `keep` slots of idx end holding the kept indices.
    __device__ void select(int keep, int len) {
        make(keep);
        for (int i = keep; i < len; ++i)
            if (comp(idx[i], idx[0])) {
                const int value = idx[i];
                idx[i] = idx[0];
                adjust(0, keep, value);
            }
    }
};

__global__ __launch_bounds__(256) void k_nm_mask(const float* __restrict__ w, int64_t total, int n, int m,
                                                 int64_t groups, float* __restrict__ mask) {
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (g >= groups) return;
    const int64_t base = g * m;
    const int len = (int)min<int64_t>(m, total - base);
    int keep = n;
    if (len < m) {
        // nm_sparsity.cpp:84-86: ceil in float, capped at the group size
        keep = (int)ceilf((float)(len * n) / (float)m);
        keep = keep < len ? keep : len;
    }
    float mag[kMaxM];
    int idx[kMaxM];
    for (int i = 0; i < len; ++i) {
        mag[i] = fabsf(w[base + i]);
        idx[i] = i;
    }
    NmHeap h{mag, idx};
    h.select(keep, len);
    uint32_t kept = 0;
    for (int j = 0; j < keep; ++j) kept |= 1u << idx[j];
    for (int i = 0; i < len; ++i) mask[base + i] = (kept >> i) & 1u ? 1.0f : 0.0f;
}

// 2:4 over whole groups of 16-byte aligned data: the heap select above
// worked out for keep = 2 of 4, with the same comparator (|a| > |b|, false
// for NaN), so every tie goes the same way.  Making the two-element heap
// leaves the smaller of elements 0 and 1 at the root (element 1 when
// neither is greater); each later element greater than the root replaces it,
// and the new root is that element when the other kept one is greater than
// it, else the other kept one.  One float4 in and one out per thread.
__global__ __launch_bounds__(256) void k_nm24(const float4* __restrict__ w, int64_t groups,
                                              float4* __restrict__ mask) {
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (g >= groups) return;
    const float4 v = w[g];
    const float mg[4] = {fabsf(v.x), fabsf(v.y), fabsf(v.z), fabsf(v.w)};
    const bool first = mg[1] > mg[0];
    int root = first ? 0 : 1, other = first ? 1 : 0;
    float mr = first ? mg[0] : mg[1], mo = first ? mg[1] : mg[0];
#pragma unroll
    for (int i = 2; i < 4; ++i) {
        if (mg[i] > mr) {
            if (mo > mg[i]) {
                root = i;
                mr = mg[i];
            } else {
                root = other;
                mr = mo;
                other = i;
                mo = mg[i];
            }
        }
    }
    const uint32_t kept = (1u << root) | (1u << other);
    mask[g] = make_float4(kept & 1u ? 1.0f : 0.0f, kept & 2u ? 1.0f : 0.0f, kept & 4u ? 1.0f : 0.0f,
                          kept & 8u ? 1.0f : 0.0f);
}

// ---- magnitude --------------------------------------------------------------

// Selection state, in scratch, followed by the per-block tie counts (then
// their exclusive prefix), the per-block counts of keys at or below the
// threshold, and the histogram blocks' rows of 256 counts.
struct MagState {
    uint32_t prefix;   // high bits of the threshold found so far
    uint32_t pad;
    uint64_t k;        // rank still to find among keys matching the prefix
    uint64_t zeros;    // keys <= threshold
    uint64_t target;   // (size_t)((float)n * s)
};

__global__ __launch_bounds__(256) void k_mag_init(MagState* st, uint64_t k, uint64_t target) {
    if (threadIdx.x == 0) {
        st->prefix = 0;
        st->k = k;
        st->zeros = 0;
        st->target = target;
    }
}

// The 16 keys a thread owns from `start` (consecutive elements): four
// 16-byte loads when VEC (w 16-byte aligned) and all 16 lie below n, else
// one element at a time; keys past n are 0 (and `valid` says how many).
template <bool VEC>
__device__ __forceinline__ int load_keys16(const float* __restrict__ w, int64_t n, int64_t start, uint32_t* keys) {
    if (VEC && start + kMaskPerThread <= n) {
        const float4* w4 = reinterpret_cast<const float4*>(w + start);
#pragma unroll
        for (int j = 0; j < kMaskPerThread / 4; ++j) {
            const float4 v = w4[j];
            keys[4 * j] = mag_bits(v.x);
            keys[4 * j + 1] = mag_bits(v.y);
            keys[4 * j + 2] = mag_bits(v.z);
            keys[4 * j + 3] = mag_bits(v.w);
        }
        return kMaskPerThread;
    }
    int valid = 0;
#pragma unroll
    for (int i = 0; i < kMaskPerThread; ++i) {
        const int64_t e = start + i;
        keys[i] = e < n ? mag_bits(w[e]) : 0u;
        valid += e < n;
    }
    return valid;
}

// Histogram of digit `pass` (bits 31-8*pass .. 24-8*pass) over keys whose
// higher bits equal the prefix.
template <bool VEC>
__global__ __launch_bounds__(kMaskThreads) void k_mag_hist(const float* __restrict__ w, int64_t n, int pass,
                                                            const MagState* __restrict__ st, int64_t nchunks,
                                                            uint32_t* __restrict__ part) {
    // 32 sub-histograms, lane l counting into copy l % 32, rows 257 words
    // apart: the first pass bins by exponent, where a wave's keys share a
    // few bins, and with one copy per half-wave lane those atomics neither
    // collide nor share a bank
    constexpr int kCopies = 32, kPitch = 257;
    __shared__ uint32_t h[kCopies * kPitch];
#pragma unroll
    for (int c = 0; c < kCopies; ++c) h[c * kPitch + threadIdx.x] = 0;
    __syncthreads();
    const int shift = 24 - 8 * pass;
    const uint32_t prefix = st->prefix;
    uint32_t* hc = h + (threadIdx.x & (kCopies - 1)) * kPitch;
    for (int64_t chunk = blockIdx.x; chunk < nchunks; chunk += gridDim.x) {
        const int64_t start = chunk * kMaskPerBlock + (int64_t)threadIdx.x * kMaskPerThread;
        uint32_t keys[kMaskPerThread];
        const int valid = load_keys16<VEC>(w, n, start, keys);
#pragma unroll
        for (int i = 0; i < kMaskPerThread; ++i) {
            const bool match = i < valid && (pass == 0 || (keys[i] >> (shift + 8)) == prefix);
            if (match) atomicAdd(&hc[(keys[i] >> shift) & 255u], 1u);
        }
    }
    __syncthreads();
    uint32_t tot = 0;
#pragma unroll
    for (int c = 0; c < kCopies; ++c) tot += h[c * kPitch + threadIdx.x];
    // the block's row of counts (plain stores: global atomics on 256
    // addresses from every block serialise)
    part[(int64_t)blockIdx.x * 256 + threadIdx.x] = tot;
}

// One block of 1024 threads: the histogram (the sum of the hist blocks'
// rows: thread q * 256 + t adds rows q, q + 4, ... of bin t, sixteen loads
// in flight), then, in the first 256 threads, the bucket holding rank k.
__global__ __launch_bounds__(1024) void k_mag_pick(MagState* st, const uint32_t* __restrict__ part, int64_t nrows) {
    __shared__ uint64_t cum[256];
    __shared__ uint64_t quarter[4][256];
    const int t = threadIdx.x & 255, qd = threadIdx.x >> 8;
    uint64_t sum = 0;
    for (int64_t r0 = qd; r0 < nrows; r0 += 4 * 16) {
        uint32_t v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int64_t r = r0 + 4 * i;
            v[i] = r < nrows ? part[r * 256 + t] : 0u;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) sum += v[i];
    }
    quarter[qd][t] = sum;
    __syncthreads();
    // every thread stays for the barriers; the first 256 do the scan
    const bool lead = qd == 0;
    if (lead) cum[t] = quarter[0][t] + quarter[1][t] + quarter[2][t] + quarter[3][t];
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {  // inclusive scan
        const uint64_t v = lead && t >= off ? cum[t - off] : 0;
        __syncthreads();
        if (lead) cum[t] += v;
        __syncthreads();
    }
    const uint64_t k = st->k;
    const uint64_t before = lead && t ? cum[t - 1] : 0;
    const bool here = lead && before <= k && k < cum[t];
    __syncthreads();
    if (here) {
        st->prefix = (st->prefix << 8) | (uint32_t)t;
        st->k = k - before;
    }
}

// The reference's float comparisons on |w| keys: a NaN key (bits above
// +inf's) is never greater than or equal to the threshold, and nothing is
// greater than or equal to a NaN threshold; for other keys the uint32 order
// is the float order.
__device__ __forceinline__ bool key_nan(uint32_t k) { return k > 0x7F800000u; }
__device__ __forceinline__ bool key_gt(uint32_t k, uint32_t thr) { return !key_nan(k) && !key_nan(thr) && k > thr; }
__device__ __forceinline__ bool key_eq(uint32_t k, uint32_t thr) { return !key_nan(k) && k == thr; }

// Per block: keys equal to the threshold (in the block's flat range) and,
// across blocks, keys not above it (the mask's zeros before the restore,
// NaN keys included, as the reference counts them).
template <bool VEC>
__global__ __launch_bounds__(kMaskThreads) void k_mag_count(const float* __restrict__ w, int64_t n,
                                                             const MagState* __restrict__ st,
                                                             uint32_t* __restrict__ ties, uint32_t* __restrict__ les) {
    __shared__ uint32_t s_tie, s_le;
    if (threadIdx.x == 0) s_tie = s_le = 0;
    __syncthreads();
    const uint32_t thr = st->prefix;
    const int64_t start = (int64_t)blockIdx.x * kMaskPerBlock + (int64_t)threadIdx.x * kMaskPerThread;
    uint32_t keys[kMaskPerThread];
    const int valid = load_keys16<VEC>(w, n, start, keys);
    uint32_t tie = 0, le = 0;
#pragma unroll
    for (int i = 0; i < kMaskPerThread; ++i) {
        tie += i < valid && key_eq(keys[i], thr);
        le += i < valid && !key_gt(keys[i], thr);
    }
    // one LDS atomic per wave, not per thread
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        tie += __shfl_xor(tie, o, 64);
        le += __shfl_xor(le, o, 64);
    }
    if ((threadIdx.x & 63) == 0) {
        if (tie) atomicAdd(&s_tie, tie);
        if (le) atomicAdd(&s_le, le);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        ties[blockIdx.x] = s_tie;
        les[blockIdx.x] = s_le;  // summed by k_mag_scan (one global atomic per block would serialise)
    }
}

// One block: exclusive prefix of the per-block tie counts, in place, and
// the count of keys at or below the threshold (the sum of les).  Thread t
// owns a contiguous run of the counts: its run's sum, one scan of the 1024
// run sums, then the run's prefixes written back.
__global__ __launch_bounds__(1024) void k_mag_scan(uint32_t* ties, int64_t nblocks, const uint32_t* __restrict__ les,
                                                   MagState* __restrict__ st) {
    __shared__ uint64_t part[1024];
    __shared__ unsigned long long le_sum;
    const int t = threadIdx.x;
    if (t == 0) le_sum = 0;
    const int64_t per = (nblocks + 1023) / 1024;
    const int64_t b0 = min<int64_t>(nblocks, t * per), b1 = min<int64_t>(nblocks, b0 + per);
    uint64_t run = 0, le = 0;
    for (int64_t b = b0; b < b1; ++b) {
        run += ties[b];
        le += les[b];
    }
    part[t] = run;
    __syncthreads();
    atomicAdd(&le_sum, (unsigned long long)le);
    for (int off = 1; off < 1024; off <<= 1) {  // inclusive scan of the run sums
        const uint64_t u = t >= off ? part[t - off] : 0;
        __syncthreads();
        part[t] += u;
        __syncthreads();
    }
    uint64_t excl = part[t] - run;
    for (int64_t b = b0; b < b1; ++b) {
        const uint32_t v = ties[b];
        ties[b] = (uint32_t)excl;  // ranks stay below 2^32 (n < 2^32)
        excl += v;
    }
    if (t == 0) st->zeros = le_sum;
}

// mask = key > threshold, plus the first (zeros - target) threshold ties in
// flat order.  Each thread owns 16 consecutive elements, so flat order is
// (block, thread, element) order.
template <bool VEC>
__global__ __launch_bounds__(kMaskThreads) void k_mag_write(const float* __restrict__ w, int64_t n,
                                                             const MagState* __restrict__ st,
                                                             const uint32_t* __restrict__ tie_off,
                                                             float* __restrict__ mask) {
    __shared__ uint32_t scan[kMaskThreads];
    const int t = threadIdx.x;
    const uint32_t thr = st->prefix;
    const uint64_t zeros = st->zeros, target = st->target;
    const uint64_t restore = zeros > target ? zeros - target : 0;
    const int64_t start = (int64_t)blockIdx.x * kMaskPerBlock + (int64_t)t * kMaskPerThread;
    uint32_t keys[kMaskPerThread];
    const int valid = load_keys16<VEC>(w, n, start, keys);
    uint32_t mine = 0;
#pragma unroll
    for (int i = 0; i < kMaskPerThread; ++i) mine += i < valid && key_eq(keys[i], thr);
    scan[t] = mine;
    __syncthreads();
    for (int off = 1; off < kMaskThreads; off <<= 1) {
        const uint32_t u = t >= off ? scan[t - off] : 0;
        __syncthreads();
        scan[t] += u;
        __syncthreads();
    }
    uint64_t rank = (uint64_t)tie_off[blockIdx.x] + scan[t] - mine;
    float v[kMaskPerThread];
#pragma unroll
    for (int i = 0; i < kMaskPerThread; ++i) {
        v[i] = key_gt(keys[i], thr) ? 1.0f : 0.0f;
        if (key_eq(keys[i], thr) && i < valid) {
            if (rank < restore) v[i] = 1.0f;
            ++rank;
        }
    }
    if (VEC && valid == kMaskPerThread) {
        float4* m4 = reinterpret_cast<float4*>(mask + start);
#pragma unroll
        for (int j = 0; j < kMaskPerThread / 4; ++j) m4[j] = make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
    } else {
        for (int i = 0; i < valid; ++i) mask[start + i] = v[i];
    }
}

__global__ __launch_bounds__(256) void k_fill(float* __restrict__ y, int64_t n, float v) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) y[i] = v;
}

void fill_dev(pfr_ctx* ctx, float* y, int64_t n, float v) {
    if (n == 0) return;
    hipLaunchKernelGGL(k_fill, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, ctx->stream, y, n, v);
    PFR_HIP(hipGetLastError());
}

void magnitude_mask_dev(pfr_ctx* ctx, const float* w, int64_t n, float s, float* mask) {
    pfr::require(n >= 0, "negative element count");
    pfr::require(!std::isnan(s), "sparsity is NaN");
    pfr::require(n == 0 || mask != nullptr, "null mask");
    if (s <= 0.0f) return fill_dev(ctx, mask, n, 1.0f);  // magnitude_pruning.cpp:31-37
    if (s >= 1.0f) return fill_dev(ctx, mask, n, 0.0f);  // :39-45
    if (n == 0) throw pfr::Error(PFR_ERR_INVALID_ARG, "Cannot prune empty weight tensor");  // :52-54
    pfr::require(w != nullptr, "null weights");
    pfr::require(n < ((int64_t)1 << 32), "more than 2^32 - 1 elements");
    // :69-72 index in double, clamped; :84 target in float
    uint64_t k = (uint64_t)std::floor((double)n * (double)s);
    if (k > (uint64_t)(n - 1)) k = (uint64_t)(n - 1);
    const uint64_t target = (uint64_t)((float)n * s);
    const int64_t nblocks = (n + kMaskPerBlock - 1) / kMaskPerBlock;
    // histogram blocks: at most two per CU, each looping over chunks
    const int64_t hblocks = std::min<int64_t>(nblocks, 2 * (int64_t)(ctx->num_cu > 0 ? ctx->num_cu : 256));
    char* scr = static_cast<char*>(
        ctx->scratch[4].ensure(sizeof(MagState) + 8 * (size_t)nblocks + 1024 * (size_t)hblocks));
    MagState* st = reinterpret_cast<MagState*>(scr);
    uint32_t* ties = reinterpret_cast<uint32_t*>(scr + sizeof(MagState));
    uint32_t* les = ties + nblocks;
    uint32_t* part = les + nblocks;  // [hblocks][256]
    hipStream_t q = ctx->stream;
    const bool vec = ((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(mask)) & 15) == 0;
    hipLaunchKernelGGL(k_mag_init, dim3(1), dim3(256), 0, q, st, k, target);
    auto passes = [&](auto v) {
        constexpr bool VEC = decltype(v)::value;
        for (int pass = 0; pass < 4; ++pass) {
            hipLaunchKernelGGL(k_mag_hist<VEC>, dim3((unsigned)hblocks), dim3(kMaskThreads), 0, q, w, n, pass, st,
                               nblocks, part);
            hipLaunchKernelGGL(k_mag_pick, dim3(1), dim3(1024), 0, q, st, part, hblocks);
        }
        hipLaunchKernelGGL(k_mag_count<VEC>, dim3((unsigned)nblocks), dim3(kMaskThreads), 0, q, w, n, st, ties, les);
        hipLaunchKernelGGL(k_mag_scan, dim3(1), dim3(1024), 0, q, ties, nblocks, les, st);
        hipLaunchKernelGGL(k_mag_write<VEC>, dim3((unsigned)nblocks), dim3(kMaskThreads), 0, q, w, n, st, ties,
                           mask);
    };
    if (vec) passes(std::true_type{});
    else passes(std::false_type{});
    PFR_HIP(hipGetLastError());
}

void nm_mask_dev(pfr_ctx* ctx, const float* w, int64_t total, int n, int m, float* mask) {
    pfr::require(total >= 0, "negative element count");
    // NMSparsityPruning's constructor (nm_sparsity.cpp:9-18) rejects n > m
    // and zeros; groups of more than 16 are outside this kernel
    pfr::require(n > 0 && m > 0 && n <= m, "N:M needs 0 < n <= m");
    pfr::require(m <= kMaxM, "N:M groups larger than 16 are not supported");
    if (total == 0) return;
    pfr::require(w && mask, "null w/mask");
    const int64_t groups = (total + m - 1) / m;
    const bool a16 = ((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(mask)) & 15) == 0;
    if (n == 2 && m == 4 && a16 && total >= 4) {
        // whole groups vectorised; a partial last group through the general kernel
        const int64_t full = total / 4;
        hipLaunchKernelGGL(k_nm24, dim3((unsigned)((full + 255) / 256)), dim3(256), 0, ctx->stream,
                           reinterpret_cast<const float4*>(w), full, reinterpret_cast<float4*>(mask));
        if (total > full * 4)
            hipLaunchKernelGGL(k_nm_mask, dim3(1), dim3(256), 0, ctx->stream, w + full * 4, total - full * 4, n, m,
                               (int64_t)1, mask + full * 4);
    } else {
        hipLaunchKernelGGL(k_nm_mask, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, ctx->stream, w, total,
                           n, m, groups, mask);
    }
    PFR_HIP(hipGetLastError());
}

// apply_mask (sparse_tensor.cpp:616-631): out[i] = w[i] * mask[i], one fp32
// multiply per element (so NaN or inf against a 0 mask gives NaN, and -w * 0
// gives -0, as there).  16-byte loads and stores when all three pointers
// allow them.
template <bool V4>
__global__ __launch_bounds__(256) void k_apply_mask(const float* w, const float* __restrict__ m, int64_t n,
                                                    float* out) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    if constexpr (V4) {
        const int64_t n4 = n / 4;
        for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride) {
            const float4 a = reinterpret_cast<const float4*>(w)[i], b = reinterpret_cast<const float4*>(m)[i];
            reinterpret_cast<float4*>(out)[i] = make_float4(a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w);
        }
        for (int64_t i = n4 * 4 + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) out[i] = w[i] * m[i];
    } else {
        for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) out[i] = w[i] * m[i];
    }
}

// Host-pointer form: stage, run, copy back, synchronise.
template <class F>
void host_mask_call(pfr_ctx* ctx, const float* w, int64_t n, float* mask, F&& f) {
    if (n == 0) return f(nullptr, nullptr);
    pfr::require(w && mask, "null w/mask");
    float* dw = static_cast<float*>(ctx->scratch[0].ensure((size_t)n * 4));
    float* dm = static_cast<float*>(ctx->scratch[2].ensure((size_t)n * 4));
    PFR_HIP(hipMemcpyAsync(dw, w, (size_t)n * 4, hipMemcpyHostToDevice, ctx->stream));
    f(dw, dm);
    PFR_HIP(hipMemcpyAsync(mask, dm, (size_t)n * 4, hipMemcpyDeviceToHost, ctx->stream));
    PFR_HIP(hipStreamSynchronize(ctx->stream));
}

}  // namespace

namespace pfr {
void apply_mask_dev(hipStream_t s, const float* w, const float* mask, int64_t n, float* out) {
    if (n == 0) return;
    require(w && mask && out, "null weight, mask or output");
    const int64_t blocks = std::min<int64_t>((n / 4 + 255) / 256 + 1, 8192);
    const auto a = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    if (a(w) && a(mask) && a(out))
        hipLaunchKernelGGL(k_apply_mask<true>, dim3((unsigned)blocks), dim3(256), 0, s, w, mask, n, out);
    else
        hipLaunchKernelGGL(k_apply_mask<false>, dim3((unsigned)blocks), dim3(256), 0, s, w, mask, n, out);
    PFR_HIP(hipGetLastError());
}
}  // namespace pfr

extern "C" {

int pfr_apply_mask_dev(pfr_ctx* ctx, const float* w, const float* mask, int64_t n, float* out) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        pfr::require(n >= 0, "negative element count");
        pfr::apply_mask_dev(ctx->stream, w, mask, n, out);
    });
}

int pfr_apply_mask(pfr_ctx* ctx, const float* w, const float* mask, int64_t n, float* out) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        pfr::require(n >= 0, "negative element count");
        if (n == 0) return;
        pfr::require(w && mask && out, "null weight, mask or output");
        float* dw = static_cast<float*>(ctx->scratch[0].ensure((size_t)n * 4));
        float* dm = static_cast<float*>(ctx->scratch[1].ensure((size_t)n * 4));
        float* dy = static_cast<float*>(ctx->scratch[2].ensure((size_t)n * 4));
        PFR_HIP(hipMemcpyAsync(dw, w, (size_t)n * 4, hipMemcpyHostToDevice, ctx->stream));
        PFR_HIP(hipMemcpyAsync(dm, mask, (size_t)n * 4, hipMemcpyHostToDevice, ctx->stream));
        pfr::apply_mask_dev(ctx->stream, dw, dm, n, dy);
        PFR_HIP(hipMemcpyAsync(out, dy, (size_t)n * 4, hipMemcpyDeviceToHost, ctx->stream));
        PFR_HIP(hipStreamSynchronize(ctx->stream));
    });
}

int pfr_magnitude_mask_dev(pfr_ctx* ctx, const float* w, int64_t n, float sparsity, float* mask) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        magnitude_mask_dev(ctx, w, n, sparsity, mask);
    });
}

int pfr_magnitude_mask(pfr_ctx* ctx, const float* w, int64_t n, float sparsity, float* mask) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        pfr::require(n >= 0, "negative element count");
        host_mask_call(ctx, w, n, mask, [&](float* dw, float* dm) { magnitude_mask_dev(ctx, dw, n, sparsity, dm); });
    });
}

int pfr_nm_mask_dev(pfr_ctx* ctx, const float* w, int64_t total, int n, int m, float* mask) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        nm_mask_dev(ctx, w, total, n, m, mask);
    });
}

int pfr_nm_mask(pfr_ctx* ctx, const float* w, int64_t total, int n, int m, float* mask) {
    return pfr::guarded([&] {
        pfr::bind(ctx);
        pfr::require(total >= 0, "negative element count");
        host_mask_call(ctx, w, total, mask, [&](float* dw, float* dm) { nm_mask_dev(ctx, dw, total, n, m, dm); });
    });
}

}  // extern "C"
