// Internal plumbing shared by the gfx950 kernel library: error capture for
// the C ABI, the context and weight handles, grow-only device scratch.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "pfr_rocm.h"

namespace pfr {

struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

void set_last_error(const std::string& msg);
void clear_last_error();

#define PFR_HIP(call)                                                          \
    do {                                                                       \
        hipError_t e_ = (call);                                                \
        if (e_ != hipSuccess)                                                  \
            throw ::pfr::Error(PFR_ERR_HIP, std::string(#call) + ": " +        \
                                                hipGetErrorString(e_));        \
    } while (0)

inline void require(bool ok, const std::string& msg) {
    if (!ok) throw Error(PFR_ERR_INVALID_ARG, msg);
}

// Runs f and converts exceptions into a C status + thread-local message.
template <class F>
int guarded(F&& f) {
    try {
        clear_last_error();
        f();
        return PFR_OK;
    } catch (const Error& e) {
        set_last_error(e.what());
        return e.code;
    } catch (const std::bad_alloc&) {
        set_last_error("host allocation failed");
        return PFR_ERR_INVALID_ARG;
    } catch (const std::exception& e) {
        set_last_error(e.what());
        return PFR_ERR_INVALID_ARG;
    }
}

// x86 static_cast<int32_t>(float): truncation, 0x80000000 for NaN or out of
// range (what the reference's quantize_tensor and requant do on its build
// target, quant_ops.cpp:42-47).
__device__ __forceinline__ int32_t f2i_trunc_x86(float r) {
    return (r >= -2147483648.0f && r < 2147483648.0f) ? (int32_t)r : INT32_MIN;
}

// cpu_gelu (activation.cpp:249-256), same operations in the same order;
// tanhf is the device's, so results are within a few ulp of the reference's
// glibc tanhf, not bit-identical.
__device__ __forceinline__ float gelu(float v) {
    const float inner = 0.7978845608028654f * (v + 0.044715f * v * v * v);
    return 0.5f * v * (1.0f + tanhf(inner));
}

// Bias epilogue of cpu_gemm (math.cpp:431-433): out[f] += beta * c[f % c_size],
// then optionally a fused Relu (activation.cpp:45-60: std::max(0.0f, v), which
// is (0 < v) ? v : +0, so -0 and NaN give +0) or Gelu (activation.cpp:239-259).
__device__ __forceinline__ float bias_add(float v, int64_t f, const float* __restrict__ bias,
                                          int64_t c_size, float beta, int act) {
    if (bias != nullptr) {
        const float t = beta * bias[f % c_size];
        v = v + t;
    }
    if (act == PFR_ACT_RELU) v = (0.0f < v) ? v : 0.0f;
    else if (act == PFR_ACT_GELU) v = pfr::gelu(v);
    return v;
}

// Grow-only device buffer owned by a context.
struct DevBuf {
    void* p = nullptr;
    size_t bytes = 0;
    void* ensure(size_t n) {
        if (p && n <= bytes) return p;
        if (p) PFR_HIP(hipFree(p));
        p = nullptr;
        bytes = 0;
        size_t want = n < 256 ? 256 : n;
        PFR_HIP(hipMalloc(&p, want));
        bytes = want;
        return p;
    }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        bytes = 0;
    }
};

}  // namespace pfr

struct pfr_ctx {
    int device = 0;
    int num_cu = 256;
    // Fast products with few columns use the merge-path kernels where the
    // weight has that partition (PFR_CSR_MERGE=0 at init selects the
    // nnz-balanced kernels instead, for comparison).
    bool merge = true;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    // scratch[0..1]: staged inputs, scratch[2]: staged output, scratch[3]:
    // transposed activations of the Gemm form, scratch[4]: the magnitude
    // mask's selection state (histogram, counters, per-block tie counts).
    // scratch[5]: the product before its transpose in the 2:4 x . W form.
    pfr::DevBuf scratch[6];
};

struct pfr_csr {
    pfr_ctx* ctx = nullptr;
    int64_t M = 0, K = 0, nnz = 0;
    int32_t* rowptr = nullptr;  // [M+1]
    // The columns in storage order, in one of two widths: col16 when K <=
    // 65536 (col is then null), else col.  col16 and val are padded to whole
    // records of four and one spare record (value 0, column K); see mp_wave.
    int32_t* col = nullptr;     // [nnz] when K > 65536
    uint16_t* col16 = nullptr;  // [nnz padded] when K <= 65536
    void* val = nullptr;        // [nnz padded] float or int8
    pfr_dtype vdt = PFR_F32;
    float* row_scale = nullptr;  // [M] for int8 values
    // Row blocks for the vector (N == 1) kernel: each block is a run of
    // consecutive rows holding at most a fixed nnz budget.
    int32_t* spmv_blocks = nullptr;  // [n_spmv_blocks + 1] first row of each
    int64_t n_spmv_blocks = 0;
    int32_t max_row_nnz = 0;
    // Columns ascend within every row (the order to_sparse produces).
    bool cols_sorted = false;
    // Sliced-ELL copy of a float32 weight for the column-slice kernel (null
    // when the shape does not qualify).  Rows are reordered into slabs of
    // kSellRows; K is cut into chunks of sell_kc rows (a multiple of 16, at
    // most kSellMaxKC; the last chunk may be partial).  For slab s and chunk
    // c, sell_soff[s * (sell_nch + 1) + c] is the first int4 of its run of
    // 8-step groups (the run ends at entry c + 1).  A group is 64 int4: entry
    // 4*r + j holds steps 2j and 2j+1 of the slab's row r as {byte offset of
    // the column's row in the chunk's LDS copy, value bits} twice.  Every
    // run is a multiple of kSellStepPad steps; padding steps point at the
    // zero row (offset sell_kc * 64, value +0).
    int32_t* sell_perm = nullptr;  // [sell_nslab * kSellRows] row of each slab lane, -1 none
    int32_t* sell_soff = nullptr;  // [sell_nslab * (sell_nch + 1)]
    int4* sell_blk = nullptr;      // [sell_len + kSellTail]
    // The same runs for the fast mode (reassociated sums), each row's steps
    // of a chunk reordered so that at every step the four slab rows whose
    // 16-byte X reads the LDS serves together ({0, 3, 5, 6}, {1, 2, 4, 7},
    // {8, 11, 13, 14}, {9, 10, 12, 15}) take X rows in different bank
    // quarters (column % 4) where their counts allow; null until a fast
    // product builds it.  Either copy may exist without the other; the
    // tables above serve both.
    int4* sell_blk_fast = nullptr;  // [sell_len + kSellTail]
    int32_t sell_nslab = 0, sell_nch = 0, sell_kc = 0;
    int64_t sell_len = 0;
    // Row-chain copy for the in-order vector kernels (few columns, strict):
    // rows sorted by count (descending) into slabs of chain_rows (16, 32 or
    // 64); slab s holds chain_q0[s + 1] - chain_q0[s] quad rows, quad row g
    // of slab s at index (chain_q0[s] + g) * chain_rows + lane, each holding steps
    // 4g .. 4g+3 of that lane's row in storage order: four values (int8 or
    // float, as val) and four columns.  When K < kChainXMax (chain_xlds) the
    // kernel stages x in LDS with a zero at index K and a column is stored as
    // the uint16 byte offset 4 * col; steps past a row's count hold value 0
    // and offset 4 * K.  Otherwise columns are indices (uint16 when K <=
    // 65536, else int32) and steps past a row's count hold value 0, column 0.
    int32_t* chain_q0 = nullptr;    // [chain_nslab + 1]
    int32_t* chain_len = nullptr;   // [chain_nslab * chain_rows] steps of each lane's row (0: none)
    int32_t* chain_perm = nullptr;  // [chain_nslab * chain_rows] row of each lane, -1 none
    void* chain_val = nullptr;
    void* chain_col = nullptr;
    int32_t chain_nslab = 0;
    int32_t chain_rows = 64;
    bool chain_c16 = false;
    bool chain_xlds = false;
    // nnz-balanced copy for the fast kernels with few columns (N <= 8): rows
    // sorted by count (descending) and cut into groups of a power-of-two
    // number of rows R <= 64, as many as keep the group's records under a
    // common budget, so every workgroup streams about the same number of
    // nonzeros.  K is cut into bal_nchunk chunks of bal_kcw columns (the
    // last may be shorter; a chunk's X rows of eight floats fit LDS).  Group
    // g is bal_meta[g] = {log2 R, first bal_perm entry, first record, quad
    // rows}; its records run chunk by chunk, chunk c's starting at
    // bal_cmeta[g * bal_nchunk + c].x and spanning .y quad rows: record
    // (start + q * R + lane) holds entries 4q .. 4q+3 of the group's row
    // `lane` among those with a column in chunk c, as values (as val) and
    // uint16 byte offsets into x staged chunk by chunk with a zero after
    // each chunk (at most 16384 floats): column k of chunk c at float
    // c * (bal_kcw + 1) + k - c * bal_kcw; padding is value 0 at the chunk's
    // zero, float c * (bal_kcw + 1) + bal_kcw.
    int4* bal_meta = nullptr;      // [bal_ngroup]
    int2* bal_cmeta = nullptr;     // [bal_ngroup * bal_nchunk]
    int32_t* bal_perm = nullptr;   // [M] row of each group lane
    // The batch kernel's workgroups: bal_pair[i] = {group, group or -1,
    // waves of the first}; groups are paired largest with smallest (by
    // records) and a workgroup's 16 waves split between its two in
    // proportion to their records, so every wave walks about as many.
    int4* bal_pair = nullptr;      // [bal_npair]
    int32_t bal_npair = 0;
    void* bal_val = nullptr;
    uint16_t* bal_col = nullptr;
    int32_t bal_ngroup = 0, bal_nchunk = 0, bal_kcw = 0;
    // Merge-path partition for the fast kernels that read col16 and val in
    // place: the M row ends and nnz nonzeros, taken as one sequence in which
    // row r's end follows its last nonzero, are cut into mp_groups *
    // kMergeWaves equal shares, one per wave.  mp_wave[q] = {row, nonzero}
    // is the merge coordinate where wave q starts (rows < row ended, nonzeros
    // < nonzero taken); mp_wave[Q] = {M, nnz}.  Workgroup p is waves
    // p * kMergeWaves ...; a row cut by a workgroup boundary is summed by its
    // contributors' partials: mp_grp[p] = {A, B, A', 0}, where A >= 0 when p
    // takes the end of a row that started in workgroup A < p, and B >= 0 when
    // p's last row continues to workgroup B (which takes its end; the row
    // started in A').  A row cut between two workgroups meets in
    // mp_xchg[B] (tag << 32 | partial's bits, zero between launches); one
    // cut by more: mp_carry[2p] holds p's partial of its continuing row,
    // mp_carry[2p + 1] of the row whose end it takes, and mp_cnt[p] counts
    // the arrivals of the row p ends (zero between launches).  col16 and val
    // hold whole records of four entries and then one spare record (padding
    // entries: value 0, column K).
    int2* mp_wave = nullptr;
    int4* mp_wmeta = nullptr;  // [Q] the rows each wave shares within its workgroup (set_merge)
    int4* mp_grp = nullptr;
    unsigned long long* mp_xchg = nullptr;
    float* mp_carry = nullptr;
    uint32_t* mp_cnt = nullptr;
    int32_t mp_groups = 0;
    // Stored-entry bitmap (set by pfr_csr_dense_semantics): bit k % 64 of
    // pattern[r * pattern_nw + k / 64] is set when row r stores column k.
    // While it is set, every product through the handle is followed by the
    // non-finite fix-up, which gives the dense kernels' results where an inf
    // or NaN activation meets a weight the CSR does not store (a zero).
    uint64_t* pattern = nullptr;
    int64_t pattern_nw = 0;
    // The sliced-ELL, row-chain and balanced copies are built on the first
    // product that would use them (pfr::csr_build_copies): `pending` holds
    // the pfr::kCopy* bits of those still to build, and the host keeps what
    // their plans need -- the row pointers and the per-row counts of each
    // copy's column chunks (M x a few integers; empty when that copy is not
    // wanted).  Freed when nothing is pending.
    std::atomic<uint32_t> pending{0};
    std::mutex lazy_mu;
    std::vector<int32_t> h_rowptr, h_sell_cnt, h_bal_cnt;
    // Device bytes the handle holds (every array above).
    int64_t dev_bytes = 0;
};

namespace pfr {
constexpr int kChainRows = 64;     // rows per row-chain slab of the global-gather form (one folding lane each)
constexpr int kChainXMax = 16384;  // x staged in LDS (with its zero slot) below this K
constexpr int kSellRows = 16;      // rows per slab (one wave: 4 lanes x 4 columns per row)
constexpr int kSellCols = 16;      // columns of X per workgroup slice
constexpr int kSellMaxKC = 1024;   // K rows per LDS chunk (1024 x 64 B = 64 KiB, two buffers)
constexpr int kSellStepPad = 8;    // steps per (slab, chunk) run are a multiple of this (one group)
constexpr int kSellTail = 512;     // int4 after the last run, read by the unconditional prefetch (8 groups)
constexpr int kBalChunk = 4096;    // most columns per chunk of the balanced copy
constexpr int kMergeWaves = 16;    // waves per merge-path workgroup
constexpr int kMergeMinItems = 256;  // fewest merge items (row ends + nonzeros) per wave
constexpr int kMergeMaxK = 16383;  // x staged in LDS with its zero slot: (K + 1) * 4 B <= 64 KiB
}

namespace pfr {
// Makes ctx's device current (cheap when it already is).
void bind(pfr_ctx* ctx);
// Derived copies of a CSR weight, built on first use.
constexpr uint32_t kCopySell = 1, kCopyChain = 2, kCopyBal = 4, kCopySellFast = 8;
// Builds the copies among `which` that w still has pending, on w's context
// stream (allocates, plans on the host and fills on the device, then
// synchronizes).  A copy whose plan does not fit is dropped from pending and
// its products keep the kernels that read the CSR in place.
void csr_build_copies(pfr_csr* w, uint32_t which);
// out[i] = w[i] * mask[i] on stream s (apply_mask); out may alias w.
void apply_mask_dev(hipStream_t s, const float* w, const float* mask, int64_t n, float* out);
// Records, once per device, the workspace address of the allocation-free
// Gemm entry; `device` must be current.
void init_noalloc_workspace(int device);
}  // namespace pfr
