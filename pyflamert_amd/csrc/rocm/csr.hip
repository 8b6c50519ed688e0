// Device-resident CSR weights: upload from the reference's SparseTensor
// arrays or from a dense zero-filled pruned weight, with the range checks the
// reference leaves out, the row-block table used by the vector kernel and the
// sliced-ELL copy used by the column-slice kernel.
#include <algorithm>
#include <climits>
#include <cstring>
#include <numeric>
#include <vector>

#include "common.hpp"

namespace {

constexpr int64_t kSpmvBudget = 4096;  // nnz per vector-kernel row block
constexpr int64_t kSpmvMaxRows = 64;   // rows per block (one fold lane each)

template <class T>
T* dev_alloc_copy(const T* host, int64_t count, hipStream_t s) {
    void* p = nullptr;
    size_t bytes = sizeof(T) * (size_t)(count > 0 ? count : 1);
    PFR_HIP(hipMalloc(&p, bytes));
    if (count > 0) {
        hipError_t e = hipMemcpyAsync(p, host, sizeof(T) * (size_t)count, hipMemcpyHostToDevice, s);
        if (e != hipSuccess) {
            (void)hipFree(p);
            throw pfr::Error(PFR_ERR_HIP, std::string("hipMemcpyAsync: ") + hipGetErrorString(e));
        }
    }
    return static_cast<T*>(p);
}

void free_csr(pfr_csr* w) {
    if (!w) return;
    for (void* p : {(void*)w->rowptr, (void*)w->col, w->val, (void*)w->row_scale, (void*)w->spmv_blocks,
                    (void*)w->sell_perm, (void*)w->sell_soff, (void*)w->sell_blk, (void*)w->chain_q0, (void*)w->col16,
                    (void*)w->chain_len, (void*)w->chain_perm, w->chain_val, w->chain_col, (void*)w->bal_meta,
                    (void*)w->bal_cmeta, (void*)w->bal_perm, w->bal_val, (void*)w->bal_col})
        if (p) (void)hipFree(p);
    delete w;
}

// Greedy row blocks of <= kSpmvBudget nnz and <= kSpmvMaxRows rows; a longer
// row is a block of its own (folded in several LDS chunks).
std::vector<int32_t> spmv_blocks(const std::vector<int32_t>& rowptr, int64_t M) {
    std::vector<int32_t> starts;
    int64_t r = 0;
    while (r < M) {
        starts.push_back((int32_t)r);
        int64_t nz = 0, rows = 0;
        while (r < M && rows < kSpmvMaxRows) {
            int64_t rn = rowptr[r + 1] - rowptr[r];
            if (rows > 0 && nz + rn > kSpmvBudget) break;
            nz += rn;
            ++rows;
            ++r;
            if (nz >= kSpmvBudget) break;
        }
    }
    starts.push_back((int32_t)M);
    return starts;
}

// Row order of the sliced-ELL copy over b[0, n): the rows of a slab should
// have similar counts in every chunk, which keeps the padding to the slab
// maximum small.  A k-d split: the range is sorted by one chunk's count
// (cycling through the chunks with the depth) and cut at a multiple of the
// slab height near its middle, down to single slabs.  On the 4096 x 4096,
// 10 % workload (four chunks) the stored steps are 1.079 x nnz, against 1.107
// for sorting by chunk 0, then by chunk 1 within 8 buckets, and so on.
void sell_order(const std::vector<int32_t>& cnt, int64_t nch, int32_t* b, int64_t n, int64_t depth) {
    const int64_t R = pfr::kSellRows;
    if (n <= R) return;
    const int64_t c = depth % nch;
    std::stable_sort(b, b + n, [&](int32_t x, int32_t y) {
        return cnt[(size_t)(x * nch + c)] > cnt[(size_t)(y * nch + c)];
    });
    const int64_t h = (n / 2 + R - 1) / R * R;  // R <= h < n for n > R
    sell_order(cnt, nch, b, h, depth + 1);
    sell_order(cnt, nch, b + h, n - h, depth + 1);
}

// Sliced-ELL copy (layout described at pfr_csr::sell_blk).  Each row keeps
// its storage order inside a chunk and chunks are visited in order, so the
// copy needs the chunk index to be non-decreasing along every row (always
// true for one chunk, and for ascending columns).  Rows are ordered by
// sell_order.
void build_sell(pfr_csr* w, const std::vector<int32_t>& rowptr, const std::vector<int32_t>& col,
                const float* vals, hipStream_t s) {
    const int64_t M = w->M, K = w->K;
    if (M == 0 || K == 0 || w->nnz == 0) return;
    // chunks of whole 16-row LDS loads: the staging of a chunk never reaches
    // the zero row that follows it
    const int64_t kc = std::min<int64_t>((K + 15) / 16 * 16, pfr::kSellMaxKC);
    const int64_t nch = (K + kc - 1) / kc;
    if (M * nch > (int64_t(1) << 26)) return;  // count table too large: keep the row kernels
    for (int64_t r = 0; r < M; ++r)
        for (int32_t j = rowptr[r] + 1; j < rowptr[r + 1]; ++j)
            if (col[j] / kc < col[j - 1] / kc) return;
    std::vector<int32_t> cnt((size_t)(M * nch), 0);
    for (int64_t r = 0; r < M; ++r)
        for (int32_t j = rowptr[r]; j < rowptr[r + 1]; ++j) ++cnt[(size_t)(r * nch + col[j] / kc)];
    const int64_t R = pfr::kSellRows;
    const int64_t nslab = (M + R - 1) / R;
    std::vector<int32_t> order((size_t)M);
    std::iota(order.begin(), order.end(), 0);
    sell_order(cnt, nch, order.data(), M, 0);
    std::vector<int64_t> off((size_t)(nslab * nch + 1), 0);
    for (int64_t sl = 0; sl < nslab; ++sl)
        for (int64_t c = 0; c < nch; ++c) {
            int32_t mx = 0;
            for (int64_t i = sl * R; i < std::min(M, sl * R + R); ++i)
                mx = std::max(mx, cnt[(size_t)(order[(size_t)i] * nch + c)]);
            const int64_t steps = (mx + pfr::kSellStepPad - 1) / pfr::kSellStepPad * pfr::kSellStepPad;
            off[(size_t)(sl * nch + c + 1)] = off[(size_t)(sl * nch + c)] + steps / 8 * 64;
        }
    const int64_t len = off.back();
    if (len + pfr::kSellTail > INT32_MAX) return;
    const int32_t pad_off = (int32_t)(kc * 64);
    std::vector<int4> blk((size_t)(len + pfr::kSellTail));
    for (auto& b : blk) b = make_int4(pad_off, 0, pad_off, 0);
    std::vector<int32_t> perm((size_t)(nslab * R), -1);
    std::vector<int32_t> t((size_t)nch);
    for (int64_t i = 0; i < M; ++i) {
        const int32_t row = order[(size_t)i];
        perm[(size_t)i] = row;
        const int64_t sl = i / R, r = i % R;
        std::fill(t.begin(), t.end(), 0);
        for (int32_t j = rowptr[row]; j < rowptr[row + 1]; ++j) {
            const int64_t c = col[j] / kc;
            const int32_t step = t[(size_t)c]++;
            int4& b = blk[(size_t)(off[(size_t)(sl * nch + c)] + (step / 8) * 64 + 4 * r + (step % 8) / 2)];
            int32_t bits;
            std::memcpy(&bits, &vals[j], 4);
            const int32_t o = (int32_t)((col[j] - c * kc) * 64);
            if (step % 2 == 0) { b.x = o; b.y = bits; } else { b.z = o; b.w = bits; }
        }
    }
    std::vector<int32_t> soff((size_t)(nslab * (nch + 1)));
    for (int64_t sl = 0; sl < nslab; ++sl)
        for (int64_t c = 0; c <= nch; ++c)  // c == nch: end of the slab's last run
            soff[(size_t)(sl * (nch + 1) + c)] = (int32_t)off[(size_t)(sl * nch + c)];
    w->sell_perm = dev_alloc_copy(perm.data(), (int64_t)perm.size(), s);
    w->sell_soff = dev_alloc_copy(soff.data(), (int64_t)soff.size(), s);
    w->sell_blk = dev_alloc_copy(blk.data(), (int64_t)blk.size(), s);
    w->sell_nslab = (int32_t)nslab;
    w->sell_nch = (int32_t)nch;
    w->sell_kc = (int32_t)kc;
    w->sell_len = len;
    // the host copies must outlive the asynchronous uploads
    PFR_HIP(hipStreamSynchronize(s));
}

// Row-chain copy (layout described at pfr_csr::chain_q0).  Rows are sorted
// by count, longest first (ties by row index), so each slab's rows have
// similar lengths and the padding to the slab maximum stays small.
template <class V, class C>
void fill_chain(pfr_csr* w, const std::vector<int32_t>& rowptr, const std::vector<int32_t>& col, const V* vals,
                const std::vector<int32_t>& order, const std::vector<int32_t>& q0, hipStream_t s) {
    const int64_t R = w->chain_rows, nslab = w->chain_nslab, nrec = (int64_t)q0.back() * R;
    // staged-x form: byte offsets into the LDS copy of x, padding at its zero
    // slot K; otherwise column indices, padding at column 0
    // one spare quad row of padding after the last slab: the kernels' clamped
    // loads may touch it
    const int64_t mul = w->chain_xlds ? 4 : 1;
    std::vector<V> v((size_t)((nrec + R) * 4), V(0));
    std::vector<C> c((size_t)((nrec + R) * 4), C(w->chain_xlds ? w->K * 4 : 0));
    std::vector<int32_t> len((size_t)(nslab * R), 0), perm((size_t)(nslab * R), -1);
    for (int64_t i = 0; i < (int64_t)order.size(); ++i) {
        const int32_t row = order[(size_t)i];
        const int64_t sl = i / R, lane = i % R;
        perm[(size_t)i] = row;
        len[(size_t)i] = rowptr[row + 1] - rowptr[row];
        for (int32_t j = rowptr[row]; j < rowptr[row + 1]; ++j) {
            const int64_t step = j - rowptr[row];
            const size_t at = (size_t)((((int64_t)q0[(size_t)sl] + step / 4) * R + lane) * 4 + step % 4);
            v[at] = vals[j];
            c[at] = (C)(col[j] * mul);
        }
    }
    w->chain_val = dev_alloc_copy(v.data(), (int64_t)v.size(), s);
    w->chain_col = dev_alloc_copy(c.data(), (int64_t)c.size(), s);
    w->chain_len = dev_alloc_copy(len.data(), (int64_t)len.size(), s);
    w->chain_perm = dev_alloc_copy(perm.data(), (int64_t)perm.size(), s);
    w->chain_q0 = dev_alloc_copy(q0.data(), (int64_t)q0.size(), s);
    PFR_HIP(hipStreamSynchronize(s));  // the host vectors go out of scope here
}

void build_chain(pfr_csr* w, const std::vector<int32_t>& rowptr, const std::vector<int32_t>& col,
                 const void* vals, hipStream_t s) {
    const int64_t M = w->M;
    if (M == 0 || w->nnz == 0) return;
    // Slab height: the staged-x kernels' per-CU traffic and producer work per
    // step grow with the rows a workgroup folds, so the slabs are as short as
    // keeps about four workgroups per CU: 16 rows (which also lets the strict
    // 2 <= N <= 8 kernel run), else 32, else 64.  Measured on 4096 x 4096 at
    // 10 %: strict N = 1 8.47 -> 7.52 us and strict N = 2 / 8 69 / 57 ->
    // 9.9 / 12.7 us against 64-row slabs (which this rule used to keep for
    // short rows while x was staged one load at a time).  The global-gather
    // kernel takes 64.
    w->chain_xlds = w->K < pfr::kChainXMax;
    const int64_t cu = w->ctx->num_cu > 0 ? w->ctx->num_cu : 256;
    const int64_t R = !w->chain_xlds ? pfr::kChainRows : (M < 16 * 4 * cu ? 16 : (M < 32 * 4 * cu ? 32 : 64));
    w->chain_rows = (int32_t)R;
    std::vector<int32_t> order((size_t)M);
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(), [&](int32_t a, int32_t b) {
        return rowptr[a + 1] - rowptr[a] > rowptr[b + 1] - rowptr[b];
    });
    const int64_t nslab = (M + R - 1) / R;
    std::vector<int32_t> q0((size_t)nslab + 1, 0);
    int64_t total = 0;
    for (int64_t sl = 0; sl < nslab; ++sl) {
        const int32_t first = order[(size_t)(sl * R)];  // the slab's longest row
        total += (rowptr[first + 1] - rowptr[first] + 3) / 4;
        if ((total + 1) * R * 4 > INT32_MAX) return;  // keep the block kernels
        q0[(size_t)sl + 1] = (int32_t)total;
    }
    w->chain_nslab = (int32_t)nslab;
    w->chain_c16 = w->chain_xlds || w->K <= 65536;
    if (w->vdt == PFR_F32) {
        if (w->chain_c16) fill_chain<float, uint16_t>(w, rowptr, col, static_cast<const float*>(vals), order, q0, s);
        else fill_chain<float, int32_t>(w, rowptr, col, static_cast<const float*>(vals), order, q0, s);
    } else {
        if (w->chain_c16) fill_chain<int8_t, uint16_t>(w, rowptr, col, static_cast<const int8_t*>(vals), order, q0, s);
        else fill_chain<int8_t, int32_t>(w, rowptr, col, static_cast<const int8_t*>(vals), order, q0, s);
    }
}

// nnz-balanced copy (layout described at pfr_csr::bal_meta).  Rows are taken
// longest first; each group takes as many rows as the largest power of two
// (at most 64 and at most the rows left) whose padded records -- R times the
// sum over chunks of its longest row there -- fit the budget, so a row
// longer than the budget makes a group of its own.  The budget is the
// smallest that keeps the group count at most two per CU.  Only for K whose
// chunks, each with its zero slot, fit 64 KiB of staged x (the N = 1
// kernel stages all of x at once).
template <class V>
void build_bal(pfr_csr* w, const std::vector<int32_t>& rowptr, const std::vector<int32_t>& col, const V* vals,
               hipStream_t s) {
    const int64_t M = w->M, K = w->K;
    if (M == 0 || w->nnz == 0 || K == 0) return;
    const int64_t C = (K + pfr::kBalChunk - 1) / pfr::kBalChunk, kcw = (K + C - 1) / C;
    if (C * (kcw + 1) * 4 > 65536) return;
    std::vector<int32_t> order((size_t)M);
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(), [&](int32_t a, int32_t b) {
        return rowptr[a + 1] - rowptr[a] > rowptr[b + 1] - rowptr[b];
    });
    // quad rows per (sorted position, chunk)
    std::vector<int32_t> qz((size_t)(M * C), 0);
    for (int64_t i = 0; i < M; ++i) {
        const int32_t r = order[(size_t)i];
        for (int32_t j = rowptr[r]; j < rowptr[r + 1]; ++j) ++qz[(size_t)(i * C + col[j] / kcw)];
        for (int64_t c = 0; c < C; ++c) qz[(size_t)(i * C + c)] = (qz[(size_t)(i * C + c)] + 3) / 4;
    }
    auto recs = [&](int64_t i, int64_t p) {  // padded records of rows i .. i+p-1 as one group
        int64_t t = 0;
        for (int64_t c = 0; c < C; ++c) {
            int32_t mx = 0;
            for (int64_t j = i; j < i + p; ++j) mx = std::max(mx, qz[(size_t)(j * C + c)]);
            t += mx;
        }
        return p * t;
    };
    auto cut = [&](int64_t budget, std::vector<int>* out) {
        int64_t n = 0;
        for (int64_t i = 0; i < M;) {
            int p = 64;
            while (p > 1 && (p > M - i || recs(i, p) > budget)) p >>= 1;
            if (out) out->push_back(p);
            i += p;
            ++n;
        }
        return n;
    };
    const int64_t cu = w->ctx->num_cu > 0 ? w->ctx->num_cu : 256;
    int64_t lo = 1, hi = 1;
    for (int64_t i = 0; i < M; ++i) lo = std::max(lo, recs(i, 1));
    hi = std::max<int64_t>(64 * lo, 1);
    while (lo < hi) {  // smallest budget with at most two groups per CU
        const int64_t mid = lo + (hi - lo) / 2;
        if (cut(mid, nullptr) <= 2 * cu) hi = mid;
        else lo = mid + 1;
    }
    std::vector<int> groups;
    cut(lo, &groups);
    const int64_t G = (int64_t)groups.size();
    std::vector<int4> meta((size_t)G);
    std::vector<int2> cmeta((size_t)(G * C));
    int64_t nrec = 0;
    {
        int64_t i = 0;
        for (int64_t g = 0; g < G; ++g) {
            const int R = groups[(size_t)g];
            for (int64_t c = 0; c < C; ++c) {
                int32_t mx = 0;
                for (int64_t j = i; j < i + R; ++j) mx = std::max(mx, qz[(size_t)(j * C + c)]);
                cmeta[(size_t)(g * C + c)] = make_int2((int)nrec, mx);
                nrec += (int64_t)R * mx;
            }
            i += R;
        }
    }
    if ((nrec + 64) * 4 > INT32_MAX || G > INT32_MAX) return;
    std::vector<int32_t> perm((size_t)M, -1);
    // one spare record per lane after the last group
    std::vector<V> v((size_t)((nrec + 64) * 4), V(0));
    std::vector<uint16_t> cidx((size_t)((nrec + 64) * 4), (uint16_t)(4 * kcw));  // chunk 0's zero
    std::vector<int32_t> k_in((size_t)C);
    int64_t i = 0;
    for (int64_t g = 0; g < G; ++g) {
        const int R = groups[(size_t)g];
        int lg = 0;
        while ((1 << lg) < R) ++lg;
        int nq = 0;
        for (int64_t c = 0; c < C; ++c) {
            const int2 cm = cmeta[(size_t)(g * C + c)];
            nq += cm.y;
            for (int64_t e = (int64_t)cm.x * 4; e < ((int64_t)cm.x + (int64_t)R * cm.y) * 4; ++e)
                cidx[(size_t)e] = (uint16_t)(4 * (c * (kcw + 1) + kcw));  // padding: this chunk's zero
        }
        meta[(size_t)g] = make_int4(lg, (int)i, cmeta[(size_t)(g * C)].x, nq);
        for (int lane = 0; lane < R; ++lane, ++i) {
            const int32_t row = order[(size_t)i];
            perm[(size_t)i] = row;
            std::fill(k_in.begin(), k_in.end(), 0);
            for (int32_t j = rowptr[row]; j < rowptr[row + 1]; ++j) {
                const int64_t c = col[j] / kcw, k = k_in[(size_t)c]++;
                const size_t at = (size_t)(((cmeta[(size_t)(g * C + c)].x + (k / 4) * R + lane) * 4) + k % 4);
                v[at] = vals[j];
                cidx[at] = (uint16_t)(4 * (c * (kcw + 1) + col[j] - c * kcw));
            }
        }
    }
    w->bal_meta = dev_alloc_copy(meta.data(), G, s);
    w->bal_cmeta = dev_alloc_copy(cmeta.data(), G * C, s);
    w->bal_perm = dev_alloc_copy(perm.data(), M, s);
    w->bal_val = dev_alloc_copy(v.data(), (int64_t)v.size(), s);
    w->bal_col = dev_alloc_copy(cidx.data(), (int64_t)cidx.size(), s);
    w->bal_ngroup = (int32_t)G;
    w->bal_nchunk = (int32_t)C;
    w->bal_kcw = (int32_t)kcw;
    PFR_HIP(hipStreamSynchronize(s));  // the host vectors go out of scope here
}

pfr_csr* build(pfr_ctx* ctx, int64_t M, int64_t K, const std::vector<int32_t>& rowptr,
               const std::vector<int32_t>& col, const void* vals, pfr_dtype vdt,
               const float* row_scales) {
    auto* w = new pfr_csr();
    try {
        w->ctx = ctx;
        w->M = M;
        w->K = K;
        w->nnz = rowptr[M];
        w->vdt = vdt;
        int32_t mx = 0;
        for (int64_t r = 0; r < M; ++r) mx = std::max(mx, rowptr[r + 1] - rowptr[r]);
        w->max_row_nnz = mx;
        hipStream_t s = ctx->stream;
        w->rowptr = dev_alloc_copy(rowptr.data(), M + 1, s);
        w->col = dev_alloc_copy(col.data(), w->nnz, s);
        if (K <= 65536 && w->nnz > 0) {
            std::vector<uint16_t> c16(col.begin(), col.end());
            w->col16 = dev_alloc_copy(c16.data(), w->nnz, s);
            PFR_HIP(hipStreamSynchronize(s));  // c16 goes out of scope
        }
        if (vdt == PFR_F32)
            w->val = dev_alloc_copy(static_cast<const float*>(vals), w->nnz, s);
        else
            w->val = dev_alloc_copy(static_cast<const int8_t*>(vals), w->nnz, s);
        if (row_scales) w->row_scale = dev_alloc_copy(row_scales, M, s);
        std::vector<int32_t> blocks = spmv_blocks(rowptr, M);
        w->n_spmv_blocks = (int64_t)blocks.size() - 1;
        w->spmv_blocks = dev_alloc_copy(blocks.data(), (int64_t)blocks.size(), s);
        bool sorted = true;
        for (int64_t r = 0; r < M && sorted; ++r)
            for (int32_t j = rowptr[r] + 1; j < rowptr[r + 1]; ++j)
                if (col[j] <= col[j - 1]) { sorted = false; break; }
        w->cols_sorted = sorted;
        if (vdt == PFR_F32) build_sell(w, rowptr, col, static_cast<const float*>(vals), s);
        build_chain(w, rowptr, col, vals, s);
        if (vdt == PFR_F32) build_bal(w, rowptr, col, static_cast<const float*>(vals), s);
        else build_bal(w, rowptr, col, static_cast<const int8_t*>(vals), s);
        PFR_HIP(hipStreamSynchronize(s));
        return w;
    } catch (...) {
        free_csr(w);
        throw;
    }
}

}  // namespace

extern "C" {

extern "C++" {
namespace {
template <class IDX>
int csr_upload_any(pfr_ctx* ctx, int64_t M, int64_t K, int64_t nnz, const int64_t* indptr, const IDX* indices,
                   const void* values, pfr_dtype values_dtype, const float* row_scales, pfr_csr** out) {
    return pfr::guarded([&] {
        pfr::require(out != nullptr, "null output handle");
        *out = nullptr;
        pfr::bind(ctx);
        pfr::require(M >= 0 && K >= 0 && nnz >= 0, "negative CSR dimension");
        pfr::require(M < INT32_MAX && K < INT32_MAX && nnz < INT32_MAX,
                     "CSR dimensions must fit 32-bit device indices");
        pfr::require(indptr != nullptr, "null indptr");
        pfr::require(nnz == 0 || (indices && values), "null indices/values");
        pfr::require(values_dtype == PFR_F32 || values_dtype == PFR_I8,
                     "CSR values must be float32 or int8");
        pfr::require(values_dtype != PFR_I8 || row_scales != nullptr,
                     "int8 CSR values need per-row scales");
        pfr::require(indptr[0] == 0, "CSR indptr[0] must be 0");
        pfr::require(indptr[M] == nnz, "CSR indptr[M] must equal nnz");
        std::vector<int32_t> rp((size_t)M + 1);
        for (int64_t r = 0; r <= M; ++r) {
            if (r > 0) pfr::require(indptr[r] >= indptr[r - 1], "CSR indptr must be non-decreasing");
            rp[(size_t)r] = (int32_t)indptr[r];
        }
        std::vector<int32_t> cl((size_t)nnz);
        for (int64_t j = 0; j < nnz; ++j) {
            const int64_t c = indices[j];
            pfr::require(c >= 0 && c < K, "CSR column index " + std::to_string(c) +
                                              " out of range [0, " + std::to_string(K) + ")");
            cl[(size_t)j] = (int32_t)c;
        }
        if (row_scales && values_dtype == PFR_I8)
            for (int64_t r = 0; r < M; ++r)
                pfr::require(row_scales[r] > 0.0f && std::isfinite(row_scales[r]),
                             "row scale must be positive and finite");
        *out = build(ctx, M, K, rp, cl, values, values_dtype,
                     values_dtype == PFR_I8 ? row_scales : nullptr);
    });
}
}  // namespace
}  // extern "C++"

int pfr_csr_upload(pfr_ctx* ctx, int64_t M, int64_t K, int64_t nnz, const int64_t* indptr,
                   const int64_t* indices, const void* values, pfr_dtype values_dtype,
                   const float* row_scales, pfr_csr** out) {
    return csr_upload_any(ctx, M, K, nnz, indptr, indices, values, values_dtype, row_scales, out);
}

int pfr_csr_upload_i32(pfr_ctx* ctx, int64_t M, int64_t K, int64_t nnz, const int64_t* indptr,
                       const int32_t* indices, const void* values, pfr_dtype values_dtype,
                       const float* row_scales, pfr_csr** out) {
    return csr_upload_any(ctx, M, K, nnz, indptr, indices, values, values_dtype, row_scales, out);
}

int pfr_csr_from_dense(pfr_ctx* ctx, const float* dense, int64_t rows, int64_t cols, int transpose,
                       float threshold, pfr_csr** out) {
    return pfr::guarded([&] {
        pfr::require(out != nullptr, "null output handle");
        *out = nullptr;
        pfr::bind(ctx);
        pfr::require(rows >= 0 && cols >= 0, "negative dimension");
        pfr::require(rows < INT32_MAX && cols < INT32_MAX, "dimension exceeds 32-bit indices");
        pfr::require(dense != nullptr || rows * cols == 0, "null dense weight");
        const int64_t M = transpose ? cols : rows, K = transpose ? rows : cols;
        auto at = [&](int64_t r, int64_t c) {
            return transpose ? dense[c * cols + r] : dense[r * cols + c];
        };
        std::vector<int32_t> rp((size_t)M + 1, 0);
        for (int64_t r = 0; r < M; ++r) {
            int64_t n = 0;
            for (int64_t c = 0; c < K; ++c) n += std::fabs(at(r, c)) > threshold;
            rp[(size_t)r + 1] = (int32_t)(rp[(size_t)r] + n);
            pfr::require((int64_t)rp[(size_t)r] + n < INT32_MAX, "nnz exceeds 32-bit indices");
        }
        std::vector<int32_t> cl((size_t)rp[(size_t)M]);
        std::vector<float> vv((size_t)rp[(size_t)M]);
        for (int64_t r = 0; r < M; ++r) {
            int64_t j = rp[(size_t)r];
            for (int64_t c = 0; c < K; ++c) {
                float v = at(r, c);
                if (std::fabs(v) > threshold) {
                    cl[(size_t)j] = (int32_t)c;
                    vv[(size_t)j] = v;
                    ++j;
                }
            }
        }
        *out = build(ctx, M, K, rp, cl, vv.data(), PFR_F32, nullptr);
    });
}

int pfr_csr_info(const pfr_csr* w, int64_t* M, int64_t* K, int64_t* nnz) {
    return pfr::guarded([&] {
        pfr::require(w != nullptr, "null CSR handle");
        if (M) *M = w->M;
        if (K) *K = w->K;
        if (nnz) *nnz = w->nnz;
    });
}

int pfr_csr_free(pfr_csr* w) {
    return pfr::guarded([&] {
        if (!w) return;
        pfr::bind(w->ctx);
        (void)hipStreamSynchronize(w->ctx->stream);
        free_csr(w);
    });
}

}  // extern "C"
