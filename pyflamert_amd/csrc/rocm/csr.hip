// Device-resident CSR weights: upload from the reference's SparseTensor
// arrays or from a dense zero-filled pruned weight, with the range checks the
// reference leaves out, and the derived copies the product kernels read (the
// row-block table and merge-path partition at build, the sliced-ELL,
// row-chain and balanced copies on first use).
#include <algorithm>
#include <climits>
#include <cstring>
#include <memory>
#include <numeric>
#include <set>
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

template <class T>
T* dev_alloc(int64_t count) {
    void* p = nullptr;
    PFR_HIP(hipMalloc(&p, sizeof(T) * (size_t)(count > 0 ? count : 1)));
    return static_cast<T*>(p);
}

template <class T>
__global__ __launch_bounds__(256) void k_fill(T* __restrict__ p, int64_t n, T v) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = v;
}

template <class T>
void fill_dev(T* p, int64_t n, T v, hipStream_t s) {
    if (n <= 0) return;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(k_fill<T>, dim3((unsigned)blocks), dim3(256), 0, s, p, n, v);
    PFR_HIP(hipGetLastError());
}

// Allocations a handle keeps, counted in its dev_bytes.
template <class T>
T* walloc(pfr_csr* w, int64_t count) {
    T* p = dev_alloc<T>(count);
    w->dev_bytes += (int64_t)sizeof(T) * (count > 0 ? count : 1);
    return p;
}

template <class T>
T* walloc_copy(pfr_csr* w, const T* host, int64_t count, hipStream_t s) {
    T* p = dev_alloc_copy(host, count, s);
    w->dev_bytes += (int64_t)sizeof(T) * (count > 0 ? count : 1);
    return p;
}

void free_csr(pfr_csr* w) {
    if (!w) return;
    for (void* p : {(void*)w->rowptr, (void*)w->col, w->val, (void*)w->row_scale, (void*)w->spmv_blocks,
                    (void*)w->sell_perm, (void*)w->sell_soff, (void*)w->sell_blk, (void*)w->sell_blk_fast,
                    (void*)w->chain_q0, (void*)w->col16,
                    (void*)w->chain_len, (void*)w->chain_perm, w->chain_val, w->chain_col, (void*)w->bal_meta,
                    (void*)w->bal_cmeta, (void*)w->bal_perm, (void*)w->bal_pair, w->bal_val, (void*)w->bal_col, (void*)w->pattern,
                    (void*)w->mp_wave, (void*)w->mp_wmeta, (void*)w->mp_grp, (void*)w->mp_xchg,
                    (void*)w->mp_carry, (void*)w->mp_cnt})
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

// Slab placement of the sliced-ELL copy.  Slab positions 16g .. 16g + 15 are
// one workgroup of the 16-wave column-slice launch (wave i on SIMD i % 4, four
// waves per SIMD), all workgroups of a slice run at once (one per CU), and
// the waves meet at a barrier after each chunk: a workgroup takes about the
// sum over chunks of its busiest SIMD's steps, and the launch its slowest
// workgroup.  The k-d order puts slabs with long runs next to each other, so
// the first workgroup got the longest ones (on the 4096 x 4096, 10 % weight:
// 2008 steps against a mean of 1831).  The placement deals them out: slabs,
// longest total first, go greedily into bins of four (one SIMD's waves), each
// to the bin among the 64 least loaded whose largest per-chunk load stays
// smallest; bins, heaviest first, are dealt out to workgroups in snake
// order; wave i of workgroup g gets slab i / 4 of its group's bin i % 4
// (1808 steps on that weight; the 8-wave launch's slowest workgroup goes from
// 1024 to 968 steps, the 4-wave launch's is unchanged).  Measured on that
// weight at N = 256, the launch went from 40.0-40.2 to 38.6-39.4 us: less
// than the step counts promise, so the imbalance was a small part of what
// the launch spends beyond its vector-ALU issue.  The slabs that do not fill
// a whole group of 16 are the lightest and go last, in k-d order.
// steps: [nslab * nch] padded steps of slab s in chunk c; returns the slab
// at each position.
std::vector<int64_t> sell_place(const std::vector<int64_t>& steps, int64_t nslab, int64_t nch) {
    std::vector<int64_t> pos((size_t)nslab);
    std::iota(pos.begin(), pos.end(), 0);
    if (nslab < 32 || nslab > 65536) return pos;  // one workgroup, or too many to place
    std::vector<int64_t> tot((size_t)nslab, 0);
    for (int64_t s = 0; s < nslab; ++s)
        for (int64_t c = 0; c < nch; ++c) tot[(size_t)s] += steps[(size_t)(s * nch + c)];
    std::vector<int64_t> by_len(pos);
    std::stable_sort(by_len.begin(), by_len.end(), [&](int64_t a, int64_t b) { return tot[(size_t)a] > tot[(size_t)b]; });
    const int64_t nfull = nslab / 16 * 16, nb = nfull / 4, ng = nfull / 16;
    std::vector<int64_t> load((size_t)(nb * nch), 0), btot((size_t)nb, 0);
    std::vector<std::vector<int64_t>> bins((size_t)nb);
    std::set<std::pair<int64_t, int64_t>> open;  // (total load, bin) of bins with room
    for (int64_t b = 0; b < nb; ++b) open.insert({0, b});
    for (int64_t k = 0; k < nfull; ++k) {
        const int64_t s = by_len[(size_t)k];
        int64_t best = -1, best_mx = 0;
        int seen = 0;
        for (auto it = open.begin(); it != open.end() && seen < 64; ++it, ++seen) {
            const int64_t b = it->second;
            int64_t mx = 0;
            for (int64_t c = 0; c < nch; ++c)
                mx = std::max(mx, load[(size_t)(b * nch + c)] + steps[(size_t)(s * nch + c)]);
            if (best < 0 || mx < best_mx) best = b, best_mx = mx;
        }
        open.erase({btot[(size_t)best], best});
        for (int64_t c = 0; c < nch; ++c) load[(size_t)(best * nch + c)] += steps[(size_t)(s * nch + c)];
        btot[(size_t)best] += tot[(size_t)s];
        bins[(size_t)best].push_back(s);
        if (bins[(size_t)best].size() < 4) open.insert({btot[(size_t)best], best});
    }
    std::vector<int64_t> border((size_t)nb);
    std::iota(border.begin(), border.end(), 0);
    std::stable_sort(border.begin(), border.end(), [&](int64_t a, int64_t b) { return btot[(size_t)a] > btot[(size_t)b]; });
    std::vector<std::vector<int64_t>> grp((size_t)ng);
    for (int64_t k = 0; k < nb; ++k) {
        const int64_t rnd = k / ng, p = k % ng;
        grp[(size_t)(rnd % 2 == 0 ? p : ng - 1 - p)].push_back(border[(size_t)k]);
    }
    for (int64_t g = 0; g < ng; ++g)
        for (int64_t i = 0; i < 16; ++i) pos[(size_t)(16 * g + i)] = bins[(size_t)grp[(size_t)g][(size_t)(i % 4)]][(size_t)(i / 4)];
    std::vector<int64_t> rest(by_len.begin() + nfull, by_len.end());
    std::sort(rest.begin(), rest.end());
    std::copy(rest.begin(), rest.end(), pos.begin() + nfull);
    return pos;
}

// ---- Derived copies ---------------------------------------------------------
// Each derived copy is planned from per-row (per-chunk) nonzero counts alone:
// row order, slab or group shapes and run offsets.  The upload path counts
// on the host, the build from a dense device weight on the device (copying
// back M x a few integers); either keeps the counts, and the first product
// that would use a copy plans it on the host and fills it on the device from
// the resident CSR, so both paths give the same layout and a weight holds
// only the copies its products use.

// Chunking of the sliced-ELL copy: chunks of whole 16-row LDS loads (the
// staging of a chunk never reaches the zero row that follows it).
void sell_geom(int64_t K, int64_t* kc, int64_t* nch) {
    *kc = std::min<int64_t>((K + 15) / 16 * 16, pfr::kSellMaxKC);
    *nch = K > 0 ? (K + *kc - 1) / *kc : 0;
}

constexpr int kMaxCountChunks = 4096;  // sliced-ELL chunks counted in LDS by the device build (K <= 4M)

// The sliced-ELL copy exists for float32 weights whose count table stays
// small and whose chunks the device build can count in LDS (else the row
// kernels serve), the same limit for the host and the device build, so
// every product through either handle runs the same kernel.
bool sell_wanted(int64_t M, int64_t K, int64_t nnz) {
    int64_t kc, nch;
    sell_geom(K, &kc, &nch);
    return M > 0 && K > 0 && nnz > 0 && M * nch <= (int64_t(1) << 26) && nch <= kMaxCountChunks;
}

struct SellPlan {
    int64_t kc = 0, nch = 0, nslab = 0, len = 0;
    std::vector<int32_t> perm;  // [nslab * kSellRows] row of each slab lane, -1 none
    std::vector<int64_t> off;   // [nslab * nch + 1] first int4 of each (slab, chunk) run
};

// cnt: [M * nch] nonzeros of row r in chunk c at r * nch + c.  False when
// the copy would outgrow 32-bit offsets.
bool plan_sell(int64_t M, int64_t K, const std::vector<int32_t>& cnt, SellPlan* p) {
    sell_geom(K, &p->kc, &p->nch);
    const int64_t nch = p->nch, R = pfr::kSellRows;
    p->nslab = (M + R - 1) / R;
    std::vector<int32_t> order((size_t)M);
    std::iota(order.begin(), order.end(), 0);
    sell_order(cnt, nch, order.data(), M, 0);
    // padded steps of each k-d slab in each chunk
    std::vector<int64_t> steps((size_t)(p->nslab * nch));
    for (int64_t sl = 0; sl < p->nslab; ++sl)
        for (int64_t c = 0; c < nch; ++c) {
            int32_t mx = 0;
            for (int64_t i = sl * R; i < std::min(M, sl * R + R); ++i)
                mx = std::max(mx, cnt[(size_t)(order[(size_t)i] * nch + c)]);
            steps[(size_t)(sl * nch + c)] = (mx + pfr::kSellStepPad - 1) / pfr::kSellStepPad * pfr::kSellStepPad;
        }
    const std::vector<int64_t> place = sell_place(steps, p->nslab, nch);
    p->off.assign((size_t)(p->nslab * nch + 1), 0);
    p->perm.assign((size_t)(p->nslab * R), -1);
    for (int64_t sl = 0; sl < p->nslab; ++sl) {
        const int64_t from = place[(size_t)sl];
        for (int64_t c = 0; c < nch; ++c)
            p->off[(size_t)(sl * nch + c + 1)] = p->off[(size_t)(sl * nch + c)] + steps[(size_t)(from * nch + c)] / 8 * 64;
        for (int64_t i = from * R; i < std::min(M, from * R + R); ++i) p->perm[(size_t)(sl * R + i - from * R)] = order[(size_t)i];
    }
    p->len = p->off.back();
    return p->len + pfr::kSellTail <= INT32_MAX;
}

// Uploads the plan's tables (sell_blk is set by the fill).
void set_sell(pfr_csr* w, const SellPlan& p, hipStream_t s) {
    std::vector<int32_t> soff((size_t)(p.nslab * (p.nch + 1)));
    for (int64_t sl = 0; sl < p.nslab; ++sl)
        for (int64_t c = 0; c <= p.nch; ++c)  // c == nch: end of the slab's last run
            soff[(size_t)(sl * (p.nch + 1) + c)] = (int32_t)p.off[(size_t)(sl * p.nch + c)];
    w->sell_perm = walloc_copy(w, p.perm.data(), (int64_t)p.perm.size(), s);
    w->sell_soff = walloc_copy(w, soff.data(), (int64_t)soff.size(), s);
    w->sell_nslab = (int32_t)p.nslab;
    w->sell_nch = (int32_t)p.nch;
    w->sell_kc = (int32_t)p.kc;
    w->sell_len = p.len;
    PFR_HIP(hipStreamSynchronize(s));  // soff goes out of scope
}

// Rows sorted by count, longest first, ties by row index (the row order of
// the row-chain and balanced copies).
std::vector<int32_t> order_by_length(const std::vector<int32_t>& len) {
    std::vector<int32_t> order(len.size());
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(), [&](int32_t a, int32_t b) { return len[a] > len[b]; });
    return order;
}

struct ChainPlan {
    int64_t R = 0, nslab = 0;
    bool xlds = false, c16 = false;
    std::vector<int32_t> perm, len;  // [nslab * R] row and count of each slab lane (-1 / 0: none)
    std::vector<int32_t> q0;         // [nslab + 1] first quad row of each slab
};

// Row-chain plan from the row counts.  Slab height: the staged-x kernels'
// per-CU traffic and producer work per step grow with the rows a workgroup
// folds, so the slabs are as short as keeps about four workgroups per CU: 16
// rows (which also lets the strict 2 <= N <= 8 kernel run), else 32, else
// 64.  Measured on 4096 x 4096 at 10 %: strict N = 1 8.47 -> 7.52 us and
// strict N = 2 / 8 69 / 57 -> 9.9 / 12.7 us against 64-row slabs (which this
// rule used to keep for short rows while x was staged one load at a time).
// The global-gather kernel takes 64.  False when the copy would outgrow
// 32-bit offsets.
bool plan_chain(const pfr_csr* w, const std::vector<int32_t>& len, ChainPlan* p) {
    const int64_t M = w->M;
    p->xlds = w->K < pfr::kChainXMax;
    const int64_t cu = w->ctx->num_cu > 0 ? w->ctx->num_cu : 256;
    p->R = !p->xlds ? pfr::kChainRows : (M < 16 * 4 * cu ? 16 : (M < 32 * 4 * cu ? 32 : 64));
    const int64_t R = p->R;
    const std::vector<int32_t> order = order_by_length(len);
    p->nslab = (M + R - 1) / R;
    p->q0.assign((size_t)p->nslab + 1, 0);
    int64_t total = 0;
    for (int64_t sl = 0; sl < p->nslab; ++sl) {
        total += (len[(size_t)order[(size_t)(sl * R)]] + 3) / 4;  // the slab's longest row
        if ((total + 1) * R * 4 > INT32_MAX) return false;
        p->q0[(size_t)sl + 1] = (int32_t)total;
    }
    p->c16 = p->xlds || w->K <= 65536;
    p->perm.assign((size_t)(p->nslab * R), -1);
    p->len.assign((size_t)(p->nslab * R), 0);
    for (int64_t i = 0; i < M; ++i) {
        p->perm[(size_t)i] = order[(size_t)i];
        p->len[(size_t)i] = len[(size_t)order[(size_t)i]];
    }
    return true;
}

// Uploads the plan's tables (chain_val / chain_col are set by the fill).
void set_chain(pfr_csr* w, const ChainPlan& p, hipStream_t s) {
    w->chain_len = walloc_copy(w, p.len.data(), (int64_t)p.len.size(), s);
    w->chain_perm = walloc_copy(w, p.perm.data(), (int64_t)p.perm.size(), s);
    w->chain_q0 = walloc_copy(w, p.q0.data(), (int64_t)p.q0.size(), s);
    w->chain_rows = (int32_t)p.R;
    w->chain_nslab = (int32_t)p.nslab;
    w->chain_xlds = p.xlds;
    w->chain_c16 = p.c16;
    PFR_HIP(hipStreamSynchronize(s));
}

// Chunking of the balanced copy: C chunks of kcw columns; false when the
// chunks, each with its zero slot, exceed 64 KiB of staged x (the N = 1
// kernel stages all of x at once).
bool bal_geom(int64_t K, int64_t* C, int64_t* kcw) {
    if (K <= 0) return false;
    *C = (K + pfr::kBalChunk - 1) / pfr::kBalChunk;
    *kcw = (K + *C - 1) / *C;
    return *C * (*kcw + 1) * 4 <= 65536;
}

struct BalPlan {
    int64_t C = 0, kcw = 0, G = 0, nrec = 0;
    std::vector<int4> meta;    // [G] {log2 R, first perm entry, first record, quad rows}
    std::vector<int2> cmeta;   // [G * C] {first record, quad rows} of each (group, chunk)
    std::vector<int32_t> perm; // [M] row of each sorted position
    std::vector<int32_t> gpos; // [M] group of each sorted position
    std::vector<int4> pair;    // [ceil(G / 2)] the batch kernel's workgroups (pfr_csr::bal_pair)
};

// nnz-balanced plan (layout described at pfr_csr::bal_meta) from the row
// counts and the per-chunk counts cntc[r * C + c].  Rows are taken longest
// first; each group takes as many rows as the largest power of two (at most
// 64 and at most the rows left) whose padded records -- R times the sum over
// chunks of its longest row there -- fit the budget, so a row longer than
// the budget makes a group of its own.  The budget is the smallest that
// keeps the group count at most two per CU.  Power-of-two heights leave the
// heaviest group about 1.45 times the mean, so the batch kernel's
// workgroups take the groups in pairs, largest with smallest, and split
// their 16 waves between the two in proportion to their records (the
// split with the least records per wave on the busier side).  False when
// the copy would outgrow 32-bit offsets.
bool plan_bal(const pfr_csr* w, const std::vector<int32_t>& len, const std::vector<int32_t>& cntc, BalPlan* p) {
    const int64_t M = w->M;
    if (!bal_geom(w->K, &p->C, &p->kcw)) return false;
    const int64_t C = p->C;
    const std::vector<int32_t> order = order_by_length(len);
    // quad rows per (sorted position, chunk)
    std::vector<int32_t> qz((size_t)(M * C));
    for (int64_t i = 0; i < M; ++i)
        for (int64_t c = 0; c < C; ++c)
            qz[(size_t)(i * C + c)] = (cntc[(size_t)(order[(size_t)i] * C + c)] + 3) / 4;
    auto recs = [&](int64_t i, int64_t n) {  // padded records of rows i .. i+n-1 as one group
        int64_t t = 0;
        for (int64_t c = 0; c < C; ++c) {
            int32_t mx = 0;
            for (int64_t j = i; j < i + n; ++j) mx = std::max(mx, qz[(size_t)(j * C + c)]);
            t += mx;
        }
        return n * t;
    };
    auto cut = [&](int64_t budget, std::vector<int>* out) {
        int64_t n = 0;
        for (int64_t i = 0; i < M;) {
            int q = 64;
            while (q > 1 && (q > M - i || recs(i, q) > budget)) q >>= 1;
            if (out) out->push_back(q);
            i += q;
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
    p->G = G;
    p->meta.resize((size_t)G);
    p->cmeta.resize((size_t)(G * C));
    p->perm.assign(order.begin(), order.end());
    p->gpos.resize((size_t)M);
    int64_t nrec = 0, i = 0;
    for (int64_t g = 0; g < G; ++g) {
        const int R = groups[(size_t)g];
        int lg = 0;
        while ((1 << lg) < R) ++lg;
        int64_t nq = 0;
        for (int64_t c = 0; c < C; ++c) {
            int32_t mx = 0;
            for (int64_t j = i; j < i + R; ++j) mx = std::max(mx, qz[(size_t)(j * C + c)]);
            if (nrec > INT32_MAX) return false;
            p->cmeta[(size_t)(g * C + c)] = make_int2((int)nrec, mx);
            nrec += (int64_t)R * mx;
            nq += mx;
        }
        p->meta[(size_t)g] = make_int4(lg, (int)i, p->cmeta[(size_t)(g * C)].x, (int)std::min<int64_t>(nq, INT32_MAX));
        for (int64_t j = i; j < i + R; ++j) p->gpos[(size_t)j] = (int32_t)g;
        i += R;
    }
    p->nrec = nrec;
    std::vector<int64_t> grec((size_t)G, 0);  // records per group
    for (int64_t g = 0; g < G; ++g)
        for (int64_t c = 0; c < C; ++c)
            grec[(size_t)g] += ((int64_t)1 << p->meta[(size_t)g].x) * p->cmeta[(size_t)(g * C + c)].y;
    std::vector<int32_t> by((size_t)G);
    for (int64_t g = 0; g < G; ++g) by[(size_t)g] = (int32_t)g;
    std::stable_sort(by.begin(), by.end(), [&](int32_t a, int32_t b) { return grec[(size_t)a] > grec[(size_t)b]; });
    const int64_t P = (G + 1) / 2, WW = 16;
    p->pair.resize((size_t)P);
    for (int64_t i = 0; i < P; ++i) {
        const int32_t a = by[(size_t)i], b = G - 1 - i > i ? by[(size_t)(G - 1 - i)] : -1;
        int64_t na = WW;
        if (b >= 0) {
            const int64_t ra = std::max<int64_t>(grec[(size_t)a], 1), rb = std::max<int64_t>(grec[(size_t)b], 1);
            double best = 0.0;
            for (int64_t n = 1; n < WW; ++n) {
                const double t = std::max((double)ra / (double)n, (double)rb / (double)(WW - n));
                if (n == 1 || t < best) best = t, na = n;
            }
        }
        p->pair[(size_t)i] = make_int4(a, b, (int)na, 0);
    }
    return (nrec + 64) * 4 <= INT32_MAX && G <= INT32_MAX;
}

// Uploads the plan's tables (bal_val / bal_col are set by the fill).
void set_bal(pfr_csr* w, const BalPlan& p, hipStream_t s) {
    w->bal_meta = walloc_copy(w, p.meta.data(), p.G, s);
    w->bal_cmeta = walloc_copy(w, p.cmeta.data(), p.G * p.C, s);
    w->bal_perm = walloc_copy(w, p.perm.data(), (int64_t)p.perm.size(), s);
    w->bal_pair = walloc_copy(w, p.pair.data(), (int64_t)p.pair.size(), s);
    w->bal_npair = (int32_t)p.pair.size();
    w->bal_ngroup = (int32_t)p.G;
    w->bal_nchunk = (int32_t)p.C;
    w->bal_kcw = (int32_t)p.kcw;
    PFR_HIP(hipStreamSynchronize(s));
}

// Merge-path partition (layout at pfr_csr::mp_wave) of the CSR with row
// pointers `rowptr`, after Merrill and Garland, "Merge-based parallel sparse
// matrix-vector multiplication" (SC 2016): the row ends and the nonzeros are
// one sequence of M + nnz items (row r's end after its last nonzero), and a
// point on it, a diagonal d, is the coordinate {rows ended, nonzeros taken}
// whose sum is d, found by binary search (the number of row ends i taken
// before nonzero d - i is the first i with rowptr[i + 1] > d - i - 1).
// Workgroup boundaries are placed at row ends where that costs little: the
// smallest capacity C for which a greedy fill -- each workgroup ends at the
// last row end within C items of its start, or at exactly C items when no
// row ends there -- needs at most one workgroup per CU.  So a row is cut
// between workgroups only when it is longer than a share, and every
// workgroup's load stays within a row of C (on the int8 decode weights at
// 30 % with lognormal rows the heaviest holds 1.007 to 1.041 times the
// mean).  Within a workgroup the waves take shares weighted by their issue
// priority (below).  Uploads
// the tables and zeroes the exchange words and arrival counters.  False (no
// partition) when the weight has no column copy in uint16 or x does not fit
// the staged slot.
bool set_merge(pfr_csr* w, const std::vector<int32_t>& rowptr, hipStream_t s) {
    const int64_t M = w->M, nnz = w->nnz, T = M + nnz, W = pfr::kMergeWaves;
    if (w->col16 == nullptr || nnz == 0 || w->K > pfr::kMergeMaxK || nnz > INT32_MAX - 4096) return false;
    const int64_t cu = w->ctx->num_cu > 0 ? w->ctx->num_cu : 256;
    const int64_t P0 = std::max<int64_t>(1, std::min<int64_t>(cu, T / (W * pfr::kMergeMinItems)));
    std::vector<int64_t> ends((size_t)M);  // the diagonal just after row r's end
    for (int64_t r = 0; r < M; ++r) ends[(size_t)r] = rowptr[(size_t)r + 1] + r + 1;
    auto greedy = [&](int64_t C, std::vector<int64_t>* D) {
        int64_t x = 0, n = 0;
        if (D) D->assign(1, 0);
        while (x < T) {
            const auto it = std::upper_bound(ends.begin(), ends.end(), x + C);
            const int64_t e = it == ends.begin() ? -1 : *(it - 1);  // the last row end within C
            x = e > x ? e : std::min(x + C, T);
            ++n;
            if (D) D->push_back(x);
        }
        return n;
    };
    int64_t lo = (T + P0 - 1) / P0, hi = T;
    while (lo < hi) {
        const int64_t mid = lo + (hi - lo) / 2;
        if (greedy(mid, nullptr) <= P0) hi = mid;
        else lo = mid + 1;
    }
    std::vector<int64_t> D;
    const int64_t P = greedy(lo, &D);
    auto search = [&](int64_t d) {
        int64_t i0 = std::max<int64_t>(d - nnz, 0), i1 = std::min<int64_t>(d, M);
        while (i0 < i1) {
            const int64_t mid = i0 + (i1 - i0) / 2;
            if (rowptr[(size_t)mid + 1] <= d - mid - 1) i0 = mid + 1;
            else i1 = mid;
        }
        return make_int2((int)i0, (int)(d - i0));
    };
    // a workgroup's waves start on whole records (a multiple of four
    // nonzeros): the point of the path at that nonzero where every row
    // ending before it has ended, and a row ending exactly there keeps the
    // side the diagonal gave it
    const auto e1 = rowptr.begin() + 1;
    const int64_t Q = P * W;
    // Wave t's share is proportional to kMergeWaveWeight[t].  The 16 waves
    // of a workgroup run four to a SIMD, and the SIMD's issue arbitration
    // favours its older waves: with equal shares, per-wave timestamps on the
    // int8 decode weights showed the walk taking about 4 % longer for each
    // later wave of a SIMD (waves 0-3 fastest, 12-15 slowest, wave 15 a
    // further 4 %), so the youngest waves set the launch time.  The weights
    // give the older waves more: 1 - 0.10 (t / 4 - 1.5), and 0.92 of that for
    // the last wave.  (On the 22016 x 4096 stacked weight the per-position
    // medians of the walk's end then agree within 0.5 us of 14.7 us.)
    double cum[pfr::kMergeWaves + 1];
    cum[0] = 0.0;
    for (int t = 0; t < W; ++t) {
        const double wt = (1.0 - 0.10 * ((t / 4) - 1.5)) * (t == W - 1 ? 0.92 : 1.0);
        cum[t + 1] = cum[t] + wt;
    }
    std::vector<int2> wp((size_t)Q + 1);
    for (int64_t p = 0; p < P; ++p) {
        const int2 end = search(D[(size_t)p + 1]);
        wp[(size_t)(p * W)] = search(D[(size_t)p]);
        for (int64_t t = 1; t < W; ++t) {
            const int2 c = search(D[(size_t)p] + (int64_t)((double)(D[(size_t)p + 1] - D[(size_t)p]) * cum[t] / cum[W]));
            const int2 prev = wp[(size_t)(p * W + t - 1)];
            const int64_t j = std::max<int64_t>(std::min<int64_t>(((int64_t)c.y + 3) / 4 * 4, end.y), prev.y);
            const int64_t lt = std::lower_bound(e1, e1 + M, (int32_t)j) - e1;  // rows ending before j
            const int64_t le = std::upper_bound(e1, e1 + M, (int32_t)j) - e1;  // rows ending at or before j
            const int64_t i = std::max<int64_t>(std::min<int64_t>(std::max<int64_t>(c.x, lt), le), prev.x);
            wp[(size_t)(p * W + t)] = make_int2((int)i, (int)j);
        }
    }
    wp[(size_t)Q] = make_int2((int)M, (int)nnz);
    auto I0 = [&](int64_t p) { return (int64_t)wp[(size_t)(p * W)].x; };
    auto J0 = [&](int64_t p) { return (int64_t)wp[(size_t)(p * W)].y; };
    // the workgroup holding nonzero n, searched back from p (n < J0(p + 1))
    auto holder = [&](int64_t n, int64_t p) {
        while (p > 0 && J0(p) > n) --p;
        return p;
    };
    std::vector<int4> gp((size_t)P, make_int4(-1, -1, -1, 0));
    for (int64_t p = 0; p < P; ++p) {
        const int64_t i0 = I0(p), j0 = J0(p), i1 = I0(p + 1), j1 = J0(p + 1);
        if (i1 > i0 && rowptr[(size_t)i0] < j0) gp[(size_t)p].x = (int)holder(rowptr[(size_t)i0], p - 1);
        if (i1 < M && j1 > std::max<int64_t>(rowptr[(size_t)i1], j0)) {
            int64_t b = p + 1;
            while (I0(b + 1) <= i1) ++b;  // the workgroup that takes row i1's end (b < P: the last ends at M)
            gp[(size_t)p].y = (int)b;
            gp[(size_t)p].z = (int)(rowptr[(size_t)i1] >= j0 ? p : holder(rowptr[(size_t)i1], p - 1));
        }
    }
    // per wave, the rows it shares with other waves of its workgroup: the
    // row whose end it takes after earlier waves began it ("own") and the
    // row it leaves unfinished ("give"), each with the wave where the row
    // starts (-1: before the workgroup), the wave that takes its end (W:
    // after the workgroup) and how many waves add to it, so the last of them
    // can finish it: {own start or -2, give start, give end or -1, own count
    // | give count << 16}
    std::vector<int4> wm((size_t)Q);
    for (int64_t p = 0; p < P; ++p) {
        const int2* c = wp.data() + p * W;  // c[0 .. W]: the workgroup's wave starts and its end
        auto gives = [&](int64_t t) {
            return c[t + 1].x < M && c[t + 1].y > std::max<int64_t>(rowptr[(size_t)c[t + 1].x], c[t].y);
        };
        auto owns = [&](int64_t t) { return c[t].x < c[t + 1].x && rowptr[(size_t)c[t].x] < c[t].y; };
        auto start_wave = [&](int64_t n, int64_t t) {
            while (t > 0 && n < c[t].y) --t;
            return n < c[t].y ? int64_t(-1) : t;
        };
        for (int64_t t = 0; t < W; ++t) {
            int4 m = make_int4(-2, -1, -1, 0);
            if (owns(t)) {
                const int64_t a = start_wave(rowptr[(size_t)c[t].x], t);
                int64_t n = 1;
                for (int64_t u = std::max<int64_t>(a, 0); u < t; ++u) n += gives(u);
                m.x = (int)a;
                m.w |= (int)n;
            }
            if (gives(t)) {
                const int64_t a = start_wave(rowptr[(size_t)c[t + 1].x], t);
                int64_t b = t + 1;
                while (b < W && c[b].x == c[b + 1].x) ++b;  // the next wave that takes a row end
                int64_t n = b < W;
                for (int64_t u = std::max<int64_t>(a, 0); u < b; ++u) n += gives(u);
                m.y = (int)a;
                m.z = (int)b;
                m.w |= (int)n << 16;
            }
            wm[(size_t)(p * W + t)] = m;
        }
    }
    w->mp_wave = walloc_copy(w, wp.data(), Q + 1, s);
    w->mp_wmeta = walloc_copy(w, wm.data(), Q, s);
    w->mp_grp = walloc_copy(w, gp.data(), P, s);
    w->mp_xchg = walloc<unsigned long long>(w, P);
    fill_dev(w->mp_xchg, P, 0ull, s);
    w->mp_carry = walloc<float>(w, 2 * P);
    w->mp_cnt = walloc<uint32_t>(w, P);
    fill_dev(w->mp_cnt, P, 0u, s);
    w->mp_groups = (int32_t)P;
    PFR_HIP(hipStreamSynchronize(s));  // wp and gp outlive the uploads
    return true;
}

// ---- Build from a dense device weight ----------------------------------------

// Device memory freed when it goes out of scope (temporaries of a build).
struct DevTmp {
    void* p = nullptr;
    explicit DevTmp(size_t bytes) { PFR_HIP(hipMalloc(&p, bytes > 0 ? bytes : 4)); }
    ~DevTmp() { if (p) (void)hipFree(p); }
    DevTmp(const DevTmp&) = delete;
    DevTmp& operator=(const DevTmp&) = delete;
    template <class T> T* as() const { return static_cast<T*>(p); }
};


// D[c, r] = A[r, c] (* mask[r, c]) for A rows x cols: the op(W) a CSR of
// W^T is built from, through 32 x 33 LDS tiles (coalesced both ways).
template <bool MASK>
__global__ __launch_bounds__(256) void k_transpose_mask(const float* __restrict__ A, const float* __restrict__ mask,
                                                        int64_t rows, int64_t cols, float* __restrict__ D) {
    __shared__ float t[32][33];
    const int64_t ntc = (cols + 31) / 32;  // one workgroup per 32 x 32 tile
    const int64_t r0 = (int64_t)blockIdx.x / ntc * 32, c0 = (int64_t)blockIdx.x % ntc * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
    for (int i = ty; i < 32; i += 8) {
        const int64_t r = r0 + i, c = c0 + tx;
        if (r < rows && c < cols) {
            float v = A[r * cols + c];
            if constexpr (MASK) v = v * mask[r * cols + c];
            t[i][tx] = v;
        }
    }
    __syncthreads();
    for (int i = ty; i < 32; i += 8) {
        const int64_t c = c0 + i, r = r0 + tx;
        if (r < rows && c < cols) D[c * rows + r] = t[tx][i];
    }
}

// Adds the kept entries of one wave's 64 consecutive columns [kw, kw + 64)
// (bit l of m: column kw + l) to the counts of their chunks of width w.  The
// 64 columns meet at most two chunks: w >= 64 whenever there are two.
__device__ __forceinline__ void count_chunks(int32_t* s, uint64_t m, int64_t kw, int64_t w) {
    const int64_t c = kw / w, b = (c + 1) * w - kw;  // lanes below b are in chunk c
    if (b >= 64) {
        atomicAdd(&s[c], (int)__popcll(m));
    } else {
        const uint64_t lo = m & ((uint64_t(1) << b) - 1), hi = m >> b;
        if (lo) atomicAdd(&s[c], (int)__popcll(lo));
        if (hi) atomicAdd(&s[c + 1], (int)__popcll(hi));
    }
}

// One workgroup per row of D (M x K, row-major): the row's count of
// |v| > thr (the test of to_sparse, sparse_tensor.cpp:578; NaN fails it),
// then its counts per sliced-ELL chunk (nchs of width kc) and per balanced
// chunk (nchb of width kcw): cnt[r * (1 + nchs + nchb) + ...].
__global__ __launch_bounds__(256) void k_dense_count(const float* __restrict__ D, int64_t K, float thr, int kc,
                                                     int nchs, int kcw, int nchb, int32_t* __restrict__ cnt) {
    extern __shared__ int32_t sc[];  // [1 + nchs + nchb]
    const int n = 1 + nchs + nchb;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int i = tid; i < n; i += 256) sc[i] = 0;
    __syncthreads();
    const float* row = D + (int64_t)blockIdx.x * K;
    int tot = 0;
    for (int64_t k0 = 0; k0 < K; k0 += 256) {
        const int64_t k = k0 + tid;
        const bool f = k < K && fabsf(row[k]) > thr;
        const uint64_t m = __ballot(f);
        if (lane == 0 && m) {
            const int64_t kw = k0 + 64 * wave;
            tot += (int)__popcll(m);
            if (nchs) count_chunks(sc + 1, m, kw, kc);
            if (nchb) count_chunks(sc + 1 + nchs, m, kw, kcw);
        }
    }
    if (lane == 0 && tot) atomicAdd(&sc[0], tot);
    __syncthreads();
    for (int i = tid; i < n; i += 256) cnt[(int64_t)blockIdx.x * n + i] = sc[i];
}

// One workgroup per row of D: the kept entries in ascending column order at
// rowptr[r] onward (the order to_sparse emits), as float values and the
// columns as int32 (col) or uint16 (col16), whichever is given.
__global__ __launch_bounds__(256) void k_dense_compact(const float* __restrict__ D, int64_t K, float thr,
                                                       const int32_t* __restrict__ rowptr, int32_t* __restrict__ col,
                                                       uint16_t* __restrict__ col16, float* __restrict__ val) {
    __shared__ int wsum[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float* row = D + (int64_t)blockIdx.x * K;
    int base = rowptr[blockIdx.x];
    for (int64_t k0 = 0; k0 < K; k0 += 256) {
        const int64_t k = k0 + tid;
        const float v = k < K ? row[k] : 0.0f;
        const bool f = k < K && fabsf(v) > thr;
        const uint64_t m = __ballot(f);
        if (lane == 0) wsum[wave] = (int)__popcll(m);
        __syncthreads();
        int off = base, total = 0;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            off += w < wave ? wsum[w] : 0;
            total += wsum[w];
        }
        if (f) {
            const int j = off + (int)__popcll(m & ((uint64_t(1) << lane) - 1));
            val[j] = v;
            if (col) col[j] = (int32_t)k;
            if (col16) col16[j] = (uint16_t)k;
        }
        base += total;
        __syncthreads();
    }
}

// First index in [lo, hi) whose column is >= t, where t starts a chunk of
// columns and the chunk index (column / chunk width) does not decrease over
// [lo, hi) (ascending columns are one such case).
template <class CI>
__device__ __forceinline__ int32_t first_at_least(const CI* __restrict__ col, int32_t lo, int32_t hi, int32_t t) {
    while (lo < hi) {
        const int32_t mid = lo + (hi - lo) / 2;
        if ((int32_t)col[mid] < t) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

// Sliced-ELL fill, one wave per slab position i (row perm[i], slab i / 16,
// lane i % 16; -1 for the lanes of a partial slab past its rows): entry j
// of chunk c is that chunk's step j - (the row's first entry in c); step t
// of slab lane r in chunk c is int4 t / 8 * 64 + 4 r + t % 8 / 2 of the
// (slab, chunk) run, its half t % 2.  blk holds the padding pattern.
template <class CI>
__global__ __launch_bounds__(256) void k_sell_fill(int64_t npos, const int32_t* __restrict__ perm,
                                                   const int32_t* __restrict__ rowptr, const CI* __restrict__ col,
                                                   const float* __restrict__ val, const int64_t* __restrict__ off,
                                                   int nch, int kc, int4* __restrict__ blk) {
    const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (i >= npos) return;
    const int lane = threadIdx.x & 63;
    const int32_t row = perm[i];
    if (row < 0) return;  // a lane of a partial slab past its rows
    const int32_t b = rowptr[row], e = rowptr[row + 1];
    const int64_t sl = i / pfr::kSellRows, r = i % pfr::kSellRows;
    for (int32_t j = b + lane; j < e; j += 64) {
        const int32_t k = (int32_t)col[j], c = k / kc;
        const int32_t step = j - first_at_least(col, b, j, c * kc);
        int32_t* q = reinterpret_cast<int32_t*>(blk + off[sl * nch + c] + (step / 8) * 64 + 4 * r + (step % 8) / 2) +
                     (step % 2) * 2;
        q[0] = (k - c * kc) * 64;
        q[1] = __float_as_int(val[j]);
    }
}

// The 24 orders of the four column classes mod 4, two bits per row of a group.
__constant__ uint8_t kClassPerms[24] = {0xE4, 0xB4, 0xD8, 0x78, 0x9C, 0x6C, 0xE1, 0xB1, 0xC9, 0x39, 0x8D, 0x2D,
                                        0xD2, 0x72, 0xC6, 0x36, 0x4E, 0x1E, 0x93, 0x63, 0x87, 0x27, 0x4B, 0x1B};
// Slab rows (r & 7) of each LDS read group: lanes 4r .. 4r + 3 of the rows
// with r >> 3 == h and an even (group 2h) or odd (2h + 1) number of bits set
// in r & 7 are served together.
__constant__ uint8_t kReadGroupRows[2][4] = {{0, 3, 5, 6}, {1, 2, 4, 7}};

// Fast-mode sliced-ELL fill (pfr_csr::sell_blk_fast), one thread per
// (slab, LDS read group, chunk): the layout of k_sell_fill, but each row of
// the group takes its chunk's entries in an order of its own.  A column's X
// row in the chunk's LDS copy starts 64 (column % kc) bytes in, so its 16
// banks are one quarter of the 64, column % 4.  A step's 16-byte reads
// (lane 4r + q: bytes 16q .. 16q + 15 of slab row r's X row) are served four
// slab rows at a time, the rows {0, 3, 5, 6}, {1, 2, 4, 7}, {8, 11, 13, 14}
// and {9, 10, 12, 15} (measured: a probe of 16-byte reads runs at about 230
// B per clock per CU when each of these groups' rows take distinct
// quarters, whatever else repeats, and at 132 when the consecutive rows
// 4g .. 4g + 3 do instead).  So at each step the group's rows that still
// have entries get, over the 24 orders of the quarters, the assignment with
// the most rows on a quarter of their own (a row past its entries reads the
// zero row, quarter 0, which the others then avoid), ties going to the
// rows' fullest quarters; a row left without a quarter of its own takes its
// fullest one.  Every row still takes one entry per step, so the runs keep
// their lengths and padding; only the order of a row's terms changes, which
// the fast mode's reassociated sums allow.
template <class CI>
__global__ __launch_bounds__(256) void k_sell_fill_fast(int64_t nthr, int nch, int kc,
                                                        const int32_t* __restrict__ perm,
                                                        const int32_t* __restrict__ rowptr, const CI* __restrict__ col,
                                                        const float* __restrict__ val,
                                                        const int32_t* __restrict__ soff, int4* __restrict__ blk) {
    const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (id >= nthr) return;
    const int c = (int)(id % nch);
    const int64_t sg = id / nch, sl = sg / 4;
    const int g = (int)(sg % 4);
    const int32_t k0 = c * kc;
    int sr[4];  // the group's slab rows
    int32_t cur[4][4], cnt[4][4], n[4];
    int32_t T = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        sr[i] = 8 * (g >> 1) + kReadGroupRows[g & 1][i];
        const int32_t row = perm[sl * pfr::kSellRows + sr[i]];
        int32_t b = 0, e = 0;
        if (row >= 0) {
            const int32_t rb = rowptr[row], re = rowptr[row + 1];
            b = first_at_least(col, rb, re, k0);
            e = first_at_least(col, b, re, k0 + kc);
        }
        n[i] = e - b;
        T = max(T, n[i]);
#pragma unroll
        for (int q = 0; q < 4; ++q) cur[i][q] = b, cnt[i][q] = 0;
        for (int32_t j = b; j < e; ++j) {
            const int q = (int)(col[j] & 3);
#pragma unroll
            for (int u = 0; u < 4; ++u) cnt[i][u] += u == q ? 1 : 0;
        }
    }
    int4* run = blk + soff[sl * (nch + 1) + c];
    for (int32_t t = 0; t < T; ++t) {
        const bool pad = n[0] <= t || n[1] <= t || n[2] <= t || n[3] <= t;
        int best = 0, best_score = -1;
        for (int pi = 0; pi < 24; ++pi) {
            const int code = kClassPerms[pi];
            int score = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int q = (code >> (2 * i)) & 3;
                if (t < n[i] && cnt[i][q] > 0 && !(pad && q == 0)) score += (1 << 16) + cnt[i][q];
            }
            if (score > best_score) best_score = score, best = code;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (t >= n[i]) continue;
            int q = (best >> (2 * i)) & 3;
            if (cnt[i][q] == 0 || (pad && q == 0)) {  // no quarter of its own: the fullest
                int m = -1;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int v = cnt[i][u] * 2 + (pad && u == 0 ? 0 : 1);
                    if (cnt[i][u] > 0 && v > m) m = v, q = u;
                }
            }
            int32_t j = cur[i][q];
            while ((int)(col[j] & 3) != q) ++j;
            cur[i][q] = j + 1;
            --cnt[i][q];
            int32_t* dst = reinterpret_cast<int32_t*>(run + (t / 8) * 64 + 4 * sr[i] + (t % 8) / 2) + (t % 2) * 2;
            dst[0] = ((int32_t)col[j] - k0) * 64;
            dst[1] = __float_as_int(val[j]);
        }
    }
}

// Row-chain fill, one wave per sorted position i (row perm[i], slab i / R,
// lane i % R): step t of the row goes to entry t % 4 of quad row
// q0[slab] + t / 4, lane i % R, with its column times mul (4: byte offsets
// into staged x); v and c hold the padding.
template <class CI, class V, class CO>
__global__ __launch_bounds__(256) void k_chain_fill(int64_t M, int R, const int32_t* __restrict__ perm,
                                                    const int32_t* __restrict__ q0, const int32_t* __restrict__ rowptr,
                                                    const CI* __restrict__ col, const V* __restrict__ val,
                                                    int mul, V* __restrict__ v, CO* __restrict__ c) {
    const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (i >= M) return;
    const int lane = threadIdx.x & 63;
    const int32_t row = perm[i], b = rowptr[row], e = rowptr[row + 1];
    const int64_t sl = i / R, ln = i % R, q = q0[sl];
    for (int32_t j = b + lane; j < e; j += 64) {
        const int64_t step = j - b;
        const int64_t at = ((q + step / 4) * R + ln) * 4 + step % 4;
        v[at] = val[j];
        c[at] = (CO)((int32_t)col[j] * mul);
    }
}

// Balanced copy: padding of each (group, chunk) region at that chunk's zero.
__global__ __launch_bounds__(256) void k_bal_pad(int C, int kcw, const int4* __restrict__ meta,
                                                 const int2* __restrict__ cmeta, uint16_t* __restrict__ cidx) {
    const int64_t g = blockIdx.x;
    const int64_t R = int64_t(1) << meta[g].x;
    for (int c = 0; c < C; ++c) {
        const int2 cm = cmeta[g * C + c];
        const uint16_t z = (uint16_t)(4 * (c * (kcw + 1) + kcw));
        for (int64_t e = (int64_t)cm.x * 4 + threadIdx.x; e < ((int64_t)cm.x + R * cm.y) * 4; e += 256) cidx[e] = z;
    }
}

// Balanced fill, one wave per sorted position i (group gpos[i], lane i minus
// the group's first position): entry j is entry k of its row in chunk c, k
// counted from the row's first entry in c, goes to entry k % 4 of record
// cmeta[g, c].x + k / 4 * R + lane with the byte offset of its column in
// the staged chunk.
template <class CI, class V>
__global__ __launch_bounds__(256) void k_bal_fill(int64_t M, int C, int kcw, const int4* __restrict__ meta,
                                                  const int2* __restrict__ cmeta, const int32_t* __restrict__ perm,
                                                  const int32_t* __restrict__ gpos, const int32_t* __restrict__ rowptr,
                                                  const CI* __restrict__ col, const V* __restrict__ val,
                                                  V* __restrict__ v, uint16_t* __restrict__ cidx) {
    const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (i >= M) return;
    const int lane = threadIdx.x & 63;
    const int64_t g = gpos[i];
    const int4 m = meta[g];
    const int64_t R = int64_t(1) << m.x, ln = i - m.y;
    const int32_t row = perm[i], b = rowptr[row], e = rowptr[row + 1];
    for (int32_t j = b + lane; j < e; j += 64) {
        const int32_t kk = (int32_t)col[j], c = kk / kcw;
        const int64_t k = j - first_at_least(col, b, j, c * kcw);
        const int64_t at = ((cmeta[g * C + c].x + (k / 4) * R + ln) * 4) + k % 4;
        v[at] = val[j];
        cidx[at] = (uint16_t)(4 * (c * (kcw + 1) + kk - c * kcw));
    }
}

// Reorders the balanced copy's entries within each row and chunk, one wave
// per (group, chunk), reading the filled copy (tv, tc) and writing v, cidx.
// The batch-8 kernel's 16-byte reads of 32-byte X rows (lane l: half l & 1
// of the X row of its record's entry j, then of its partner's) are served in
// four sets of 16 lanes, the lanes 4r .. 4r + 3 of the slab-row groups the
// sliced-ELL copy's ordering uses (k_sell_fill_fast); the 16 lanes of a set
// hit distinct banks when the eight of each parity take X rows in distinct
// eighths of the banks (column % 8 in the chunk).  One instruction reads
// records q = b G + l >> log2 R of rows l & (R - 1) for a block b of
// G = 64 / R consecutive records; so block by block and entry by entry, each
// set of eight lanes gets, lane by lane (fewest options first), the class
// mod 8 with the most entries left in the lane's row among those not yet
// taken in the set (a lane past its row's entries reads the zero row, whose
// class the others then avoid), or its row's fullest class when none is
// left; a class hands out its entries in their stored order.  Every row
// keeps its cells, so padding and the kernels are unchanged; only the order
// of a row's terms changes (the copy serves the fast mode only).
//
// First each row's entries are sorted by class (stable) into spos, with the
// class counts and first positions in LDS; then the choice runs set by set
// with lane 8i + u of the wave holding class u of the set's entry i, and
// records each cell's position in the sorted list in pick; last the wave
// gathers every cell's entry through pick and spos.  spos and pick are as
// long as the copy.
__device__ inline int set_lane(int set, int i) {
    const int m = (((set >> 1) & 1 ? 0x7421 : 0x6530) >> (4 * (i >> 1))) & 15;  // the read group's slab rows
    return (set >> 2) << 5 | m << 2 | (i & 1) << 1 | (set & 1);
}

template <class V>
__global__ __launch_bounds__(64) void k_bal_order(int C, int kcw, const int4* __restrict__ meta,
                                                  const int2* __restrict__ cmeta, const V* __restrict__ tv,
                                                  const uint16_t* __restrict__ tc, uint16_t* __restrict__ spos,
                                                  uint16_t* __restrict__ pick, V* __restrict__ v,
                                                  uint16_t* __restrict__ cidx) {
    __shared__ int n_l[64], cnt_l[512], ptr_l[512];  // per row: entries; per (row, class): left, next position
    const int g = (int)(blockIdx.x / (unsigned)C), c = (int)(blockIdx.x % (unsigned)C), t = (int)threadIdx.x;
    const int lgR = meta[g].x, R = 1 << lgR, G = 64 >> lgR;
    const int2 cm = cmeta[(int64_t)g * C + c];
    const int64_t rec0 = cm.x;
    const int nq = cm.y, base = c * (kcw + 1), zc = kcw & 7, zero = 4 * (base + kcw);
    const uint64_t lt = (1ull << t) - 1;
    auto cell = [&](int r, int k) { return (rec0 + (int64_t)(k >> 2) * R + r) * 4 + (k & 3); };
    for (int r = 0; r < R; ++r) {
        // the row's entries come before its first padding cell
        int nr = 4 * nq, mine = 0;
        for (int k0 = 0; k0 < nr; k0 += 64) {
            const int k = k0 + t, cv = k < nr ? (int)tc[cell(r, k)] : zero;
            const uint64_t z = __ballot(cv == zero);
            const int lim = z ? k0 + __builtin_ctzll(z) : nr;
            const int u = (cv / 4 - base) & 7;
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int nqc = __builtin_popcountll(__ballot(k < lim && u == q));
                if (t == q) mine += nqc;
            }
            nr = lim;
        }
        int run[8], off = 0;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            run[q] = off;
            off += __builtin_amdgcn_readlane(mine, q);
        }
        if (t < 8) {
            int first = 0;
#pragma unroll
            for (int q = 0; q < 8; ++q) first = t == q ? run[q] : first;
            cnt_l[r * 8 + t] = mine;
            ptr_l[r * 8 + t] = first;
        }
        if (t == 0) n_l[r] = nr;
        for (int k0 = 0; k0 < nr; k0 += 64) {
            const int k = k0 + t;
            const bool in = k < nr;
            const int u = in ? ((int)tc[cell(r, k)] / 4 - base) & 7 : 0;
            int pos = 0;
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const uint64_t m = __ballot(in && u == q);
                if (u == q) pos = run[q] + __builtin_popcountll(m & lt);
                run[q] += __builtin_popcountll(m);
            }
            if (in) spos[cell(r, pos)] = (uint16_t)k;
        }
    }
    __syncthreads();
    const int gi = t >> 3, u = t & 7, nblk = (nq + G - 1) / G;
    for (int b = 0; b < nblk; ++b)
        for (int j = 0; j < 4; ++j)
            for (int set = 0; set < 8; ++set) {
                const int li = set_lane(set, gi), r = li & (R - 1), q = b * G + (li >> lgR);
                const bool inq = q < nq, live = inq && 4 * q + j < n_l[r];
                const uint64_t lv = __ballot(live);
                if (lv == 0) continue;
                int cn = cnt_l[r * 8 + u], pt = ptr_l[r * 8 + u];
                const uint64_t pz = __ballot(live && cn > 0);
                uint32_t used = __ballot(inq && !live) ? 1u << zc : 0u, left = 0, opts = 0;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    left |= (uint32_t)(lv >> (8 * i) & 1) << i;
                    opts |= (uint32_t)__builtin_popcountll((pz >> (8 * i)) & 0xff) << (4 * i);
                }
                while (left) {
                    int bi = 0, bo = 16;  // the live entry with the fewest classes left, first on ties
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const int o = (int)(opts >> (4 * i)) & 15;
                        if ((left >> i & 1) && o < bo) bo = o, bi = i;
                    }
                    left &= ~(1u << bi);
                    // untaken classes first, then the most entries, then the lowest class
                    const int key = gi == bi && cn > 0 ? ((used >> u & 1) ? 0 : 1 << 30) | cn << 3 | (7 - u) : -1;
                    int best = -1;
#pragma unroll
                    for (int w = 0; w < 8; ++w) best = max(best, __builtin_amdgcn_readlane(key, 8 * bi + w));
                    const int bu = 7 - (best & 7), sp = __builtin_amdgcn_readlane(pt, 8 * bi + bu);
                    used |= 1u << bu;
                    const int bl = set_lane(set, bi), br = bl & (R - 1);
                    if (r == br && u == bu) --cn, ++pt;
                    if (t == 0) pick[cell(br, 4 * (b * G + (bl >> lgR)) + j)] = (uint16_t)sp;
                }
                cnt_l[r * 8 + u] = cn;  // lanes of one row hold the same values
                ptr_l[r * 8 + u] = pt;
            }
    __syncthreads();  // pick and spos are read back below
#pragma unroll 4
    for (int e = t; e < 4 * nq * R; e += 64) {  // the task's cells in storage order
        const int r = (e >> 2) & (R - 1), k = (e >> 2 >> lgR) * 4 + (e & 3), nr = n_l[r];
        if (k < nr) {
            const int64_t to = rec0 * 4 + e;
            const int64_t from = cell(r, min((int)spos[cell(r, min((int)pick[to], nr - 1))], nr - 1));
            v[to] = tv[from];
            cidx[to] = tc[from];
        }
    }
}

unsigned waves_grid(int64_t M) { return (unsigned)((M + 3) / 4); }

// Stored-entry bitmap: one wave per row sets the bit of every stored column.
template <class CI>
__global__ __launch_bounds__(256) void k_pattern(int64_t M, const int32_t* __restrict__ rowptr,
                                                 const CI* __restrict__ col, int64_t nw,
                                                 unsigned long long* __restrict__ bm) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= M) return;
    for (int32_t j = rowptr[r] + (int32_t)(threadIdx.x & 63); j < rowptr[r + 1]; j += 64) {
        const int32_t k = (int32_t)col[j];
        atomicOr(&bm[r * nw + k / 64], 1ull << (k % 64));
    }
}

// ---- Copies built on first use ----------------------------------------------

// Each row's chunk index (column / width) does not decrease along it, which
// the chunked copies' fills rely on (always true for ascending columns).
bool chunks_ascend(const std::vector<int32_t>& rowptr, const std::vector<int32_t>& col, int64_t M, int64_t width) {
    for (int64_t r = 0; r < M; ++r)
        for (int32_t j = rowptr[(size_t)r] + 1; j < rowptr[(size_t)r + 1]; ++j)
            if (col[(size_t)j] / width < col[(size_t)j - 1] / width) return false;
    return true;
}

// Keeps what the copies' plans need on the host and marks the copies
// pending: the row-chain copy always, the sliced-ELL and balanced copies
// where their per-row chunk counts are given.
void set_lazy(pfr_csr* w, const std::vector<int32_t>& rowptr, std::vector<int32_t> sell_cnt,
              std::vector<int32_t> bal_cnt) {
    uint32_t bits = 0;
    if (w->M > 0 && w->nnz > 0) {
        bits = pfr::kCopyChain | (sell_cnt.empty() ? 0u : pfr::kCopySell | pfr::kCopySellFast) |
               (bal_cnt.empty() ? 0u : pfr::kCopyBal);
        w->h_rowptr = rowptr;
        w->h_sell_cnt = std::move(sell_cnt);
        w->h_bal_cnt = std::move(bal_cnt);
    }
    w->pending.store(bits, std::memory_order_release);
}

std::vector<int32_t> row_lengths(const pfr_csr* w) {
    std::vector<int32_t> len((size_t)w->M);
    for (int64_t r = 0; r < w->M; ++r) len[(size_t)r] = w->h_rowptr[(size_t)r + 1] - w->h_rowptr[(size_t)r];
    return len;
}

// Sliced-ELL copy (float32 values), planned from the kept chunk counts.
template <class CI>
void fill_sell(pfr_csr* w, const CI* col, hipStream_t s) {
    SellPlan p;
    if (!plan_sell(w->M, w->K, w->h_sell_cnt, &p)) return;
    w->sell_blk = walloc<int4>(w, p.len + pfr::kSellTail);
    const int32_t pad = (int32_t)(p.kc * 64);
    fill_dev(w->sell_blk, p.len + pfr::kSellTail, make_int4(pad, 0, pad, 0), s);
    if (w->sell_perm == nullptr) set_sell(w, p, s);  // else the fast copy's build uploaded them
    int64_t* off = dev_alloc_copy(p.off.data(), (int64_t)p.off.size(), s);
    const int64_t npos = p.nslab * pfr::kSellRows;  // perm's length
    hipLaunchKernelGGL(k_sell_fill<CI>, dim3(waves_grid(npos)), dim3(256), 0, s, npos, w->sell_perm, w->rowptr, col,
                       static_cast<const float*>(w->val), off, (int)p.nch, (int)p.kc, w->sell_blk);
    const hipError_t e = hipGetLastError();
    (void)hipStreamSynchronize(s);
    (void)hipFree(off);
    if (e != hipSuccess) throw pfr::Error(PFR_ERR_HIP, std::string("k_sell_fill: ") + hipGetErrorString(e));
}

// The fast mode's sliced-ELL copy: the same plan and tables (uploaded here
// when the strict copy has not), its runs filled by k_sell_fill_fast.
template <class CI>
void fill_sell_fast(pfr_csr* w, const CI* col, hipStream_t s) {
    SellPlan p;
    if (!plan_sell(w->M, w->K, w->h_sell_cnt, &p)) return;
    w->sell_blk_fast = walloc<int4>(w, p.len + pfr::kSellTail);
    const int32_t pad = (int32_t)(p.kc * 64);
    fill_dev(w->sell_blk_fast, p.len + pfr::kSellTail, make_int4(pad, 0, pad, 0), s);
    if (w->sell_perm == nullptr) set_sell(w, p, s);
    const int64_t nthr = p.nslab * 4 * p.nch;
    hipLaunchKernelGGL(k_sell_fill_fast<CI>, dim3((unsigned)((nthr + 255) / 256)), dim3(256), 0, s, nthr,
                       (int)p.nch, (int)p.kc, w->sell_perm, w->rowptr, col, static_cast<const float*>(w->val),
                       w->sell_soff, w->sell_blk_fast);
    PFR_HIP(hipGetLastError());
    PFR_HIP(hipStreamSynchronize(s));
}

// Row-chain copy; V is the value type (float or int8).
template <class CI, class V>
void fill_chain(pfr_csr* w, const CI* col, hipStream_t s) {
    ChainPlan p;
    if (!plan_chain(w, row_lengths(w), &p)) return;  // the block kernels serve
    // one spare quad row of padding after the last slab: the kernels'
    // clamped loads may touch it
    const int64_t n = ((int64_t)p.q0.back() * p.R + p.R) * 4;
    V* v = walloc<V>(w, n);
    w->chain_val = v;
    fill_dev(v, n, V(0), s);
    set_chain(w, p, s);
    // staged-x form: byte offsets into the LDS copy of x, padding at its
    // zero slot K; otherwise column indices, padding at column 0
    const int mul = p.xlds ? 4 : 1;
    const auto* val = static_cast<const V*>(w->val);
    if (p.c16) {
        auto* c = walloc<uint16_t>(w, n);
        w->chain_col = c;
        fill_dev(c, n, (uint16_t)(p.xlds ? w->K * 4 : 0), s);
        hipLaunchKernelGGL((k_chain_fill<CI, V, uint16_t>), dim3(waves_grid(w->M)), dim3(256), 0, s, w->M, (int)p.R,
                           w->chain_perm, w->chain_q0, w->rowptr, col, val, mul, v, c);
    } else {
        auto* c = walloc<int32_t>(w, n);
        w->chain_col = c;
        fill_dev(c, n, (int32_t)(p.xlds ? w->K * 4 : 0), s);
        hipLaunchKernelGGL((k_chain_fill<CI, V, int32_t>), dim3(waves_grid(w->M)), dim3(256), 0, s, w->M, (int)p.R,
                           w->chain_perm, w->chain_q0, w->rowptr, col, val, mul, v, c);
    }
    PFR_HIP(hipGetLastError());
    PFR_HIP(hipStreamSynchronize(s));
}

// nnz-balanced copy, planned from the kept chunk counts.
template <class CI, class V>
void fill_bal(pfr_csr* w, const CI* col, hipStream_t s) {
    BalPlan p;
    if (!plan_bal(w, row_lengths(w), w->h_bal_cnt, &p)) return;
    const int64_t n = (p.nrec + 64) * 4;  // one spare record per lane after the last group
    V* v = walloc<V>(w, n);
    w->bal_val = v;
    w->bal_col = walloc<uint16_t>(w, n);
    fill_dev(v, n, V(0), s);
    fill_dev(w->bal_col, n, (uint16_t)(4 * p.kcw), s);  // chunk 0's zero
    set_bal(w, p, s);
    int32_t* gpos = dev_alloc_copy(p.gpos.data(), (int64_t)p.gpos.size(), s);
    hipLaunchKernelGGL(k_bal_pad, dim3((unsigned)p.G), dim3(256), 0, s, (int)p.C, (int)p.kcw, w->bal_meta,
                       w->bal_cmeta, w->bal_col);
    hipLaunchKernelGGL((k_bal_fill<CI, V>), dim3(waves_grid(w->M)), dim3(256), 0, s, w->M, (int)p.C, (int)p.kcw,
                       w->bal_meta, w->bal_cmeta, w->bal_perm, gpos, w->rowptr, col, static_cast<const V*>(w->val),
                       v, w->bal_col);
    hipError_t e = hipGetLastError();
    (void)hipStreamSynchronize(s);
    (void)hipFree(gpos);
    if (e != hipSuccess) throw pfr::Error(PFR_ERR_HIP, std::string("k_bal_fill: ") + hipGetErrorString(e));
    // the terms' order against LDS bank conflicts (k_bal_order), from a copy
    // of the filled entries
    const int64_t nt = p.G * p.C;
    V* tv = nullptr;
    uint16_t *tc = nullptr, *sp = nullptr;
    try {
        tv = dev_alloc<V>(n);
        tc = dev_alloc<uint16_t>(n);
        sp = dev_alloc<uint16_t>(2 * n);
    } catch (...) {
        (void)hipFree(tv), (void)hipFree(tc), (void)hipFree(sp);
        throw;
    }
    e = hipMemcpyAsync(tv, v, sizeof(V) * (size_t)n, hipMemcpyDeviceToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(tc, w->bal_col, sizeof(uint16_t) * (size_t)n, hipMemcpyDeviceToDevice, s);
    if (e == hipSuccess && nt > 0) {
        hipLaunchKernelGGL(k_bal_order<V>, dim3((unsigned)nt), dim3(64), 0, s, (int)p.C, (int)p.kcw, w->bal_meta,
                           w->bal_cmeta, tv, tc, sp, sp + n, v, w->bal_col);
        e = hipGetLastError();
    }
    (void)hipStreamSynchronize(s);
    (void)hipFree(tv), (void)hipFree(tc), (void)hipFree(sp);
    if (e != hipSuccess) throw pfr::Error(PFR_ERR_HIP, std::string("k_bal_order: ") + hipGetErrorString(e));
}

template <class CI>
void build_copy(pfr_csr* w, uint32_t bit, const CI* col, hipStream_t s) {
    const bool i8 = w->vdt == PFR_I8;
    if (bit == pfr::kCopySell) fill_sell(w, col, s);  // pending for float32 weights only
    else if (bit == pfr::kCopySellFast) fill_sell_fast(w, col, s);  // likewise
    else if (bit == pfr::kCopyChain) i8 ? fill_chain<CI, int8_t>(w, col, s) : fill_chain<CI, float>(w, col, s);
    else i8 ? fill_bal<CI, int8_t>(w, col, s) : fill_bal<CI, float>(w, col, s);
}

template <class P>
void free_null(P*& p) {
    if (p) (void)hipFree((void*)p);
    p = nullptr;
}

// Frees a copy left part-built by a failed build.
void drop_copy(pfr_csr* w, uint32_t bit) {
    if (bit == pfr::kCopySell || bit == pfr::kCopySellFast) {
        free_null(bit == pfr::kCopySell ? w->sell_blk : w->sell_blk_fast);
        if (w->sell_blk == nullptr && w->sell_blk_fast == nullptr) {  // the tables serve neither copy now
            free_null(w->sell_perm), free_null(w->sell_soff);
            w->sell_nslab = w->sell_nch = w->sell_kc = 0;
            w->sell_len = 0;
        }
    } else if (bit == pfr::kCopyChain) {
        free_null(w->chain_q0), free_null(w->chain_len), free_null(w->chain_perm);
        free_null(w->chain_val), free_null(w->chain_col);
        w->chain_nslab = 0;
    } else {
        free_null(w->bal_meta), free_null(w->bal_cmeta), free_null(w->bal_perm), free_null(w->bal_pair);
        w->bal_npair = 0;
        free_null(w->bal_val), free_null(w->bal_col);
        w->bal_ngroup = w->bal_nchunk = w->bal_kcw = 0;
    }
}

// ---- Builds ------------------------------------------------------------------

// The handle of a host CSR: row pointers, columns (uint16 when K <= 65536),
// values and row scales on the device, the row-block table and the
// merge-path partition; the other copies are built on first use.
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
        w->rowptr = walloc_copy(w, rowptr.data(), M + 1, s);
        // col16 and val hold whole records of four and one spare record;
        // padding entries are value 0 at column K (x's zero slot in the
        // merge-path kernels, which read whole records and point loads past
        // a share at the spare one)
        const int64_t npad = (w->nnz + 3) / 4 * 4 + 4;
        if (K > 65536) {
            w->col = walloc_copy(w, col.data(), w->nnz, s);
        } else {  // allocated (padding only) also without entries: kernels may load a row's first record
            std::vector<uint16_t> c16(col.begin(), col.end());
            c16.resize((size_t)npad, (uint16_t)std::min<int64_t>(K, 65535));
            w->col16 = walloc_copy(w, c16.data(), npad, s);
            PFR_HIP(hipStreamSynchronize(s));  // c16 goes out of scope
        }
        if (vdt == PFR_F32) {
            std::vector<float> v(static_cast<const float*>(vals), static_cast<const float*>(vals) + w->nnz);
            v.resize((size_t)npad, 0.0f);
            w->val = walloc_copy(w, v.data(), npad, s);
            PFR_HIP(hipStreamSynchronize(s));
        } else {
            std::vector<int8_t> v(static_cast<const int8_t*>(vals), static_cast<const int8_t*>(vals) + w->nnz);
            v.resize((size_t)npad, 0);
            w->val = walloc_copy(w, v.data(), npad, s);
            PFR_HIP(hipStreamSynchronize(s));
        }
        if (row_scales) w->row_scale = walloc_copy(w, row_scales, M, s);
        std::vector<int32_t> blocks = spmv_blocks(rowptr, M);
        w->n_spmv_blocks = (int64_t)blocks.size() - 1;
        w->spmv_blocks = walloc_copy(w, blocks.data(), (int64_t)blocks.size(), s);
        bool sorted = true;
        for (int64_t r = 0; r < M && sorted; ++r)
            for (int32_t j = rowptr[r] + 1; j < rowptr[r + 1]; ++j)
                if (col[j] <= col[j - 1]) { sorted = false; break; }
        w->cols_sorted = sorted;
        // per-row chunk counts for the plans of the copies built on first use
        int64_t kc, nchs, nchb = 0, kcw = 1;
        sell_geom(K, &kc, &nchs);
        std::vector<int32_t> cs, cb;
        if (vdt == PFR_F32 && sell_wanted(M, K, w->nnz) && chunks_ascend(rowptr, col, M, kc)) {
            cs.assign((size_t)(M * nchs), 0);
            for (int64_t r = 0; r < M; ++r)
                for (int32_t j = rowptr[r]; j < rowptr[r + 1]; ++j) ++cs[(size_t)(r * nchs + col[j] / kc)];
        }
        if (w->nnz > 0 && bal_geom(K, &nchb, &kcw) && chunks_ascend(rowptr, col, M, kcw)) {
            cb.assign((size_t)(M * nchb), 0);
            for (int64_t r = 0; r < M; ++r)
                for (int32_t j = rowptr[r]; j < rowptr[r + 1]; ++j) ++cb[(size_t)(r * nchb + col[j] / kcw)];
        }
        set_lazy(w, rowptr, std::move(cs), std::move(cb));
        set_merge(w, rowptr, s);
        PFR_HIP(hipStreamSynchronize(s));
        return w;
    } catch (...) {
        (void)hipStreamSynchronize(ctx->stream);
        free_csr(w);
        throw;
    }
}

// The handle of D (M x K, row-major, device), as build() makes it from the
// same entries: counts on the device, copied back (M x a few integers) for
// the row pointers and the copies' plans, then the entries compacted on the
// device, so the nonzeros never leave the GPU.
pfr_csr* build_dense_dev(pfr_ctx* ctx, const float* D, int64_t M, int64_t K, float thr) {
    hipStream_t s = ctx->stream;
    int64_t kc, nchs;
    sell_geom(K, &kc, &nchs);
    if (!sell_wanted(M, K, 1)) nchs = 0;
    int64_t nchb = 0, kcw = 1;
    if (!bal_geom(K, &nchb, &kcw)) nchb = 0, kcw = 1;
    const int64_t stride = 1 + nchs + nchb;
    std::vector<int32_t> cnt((size_t)(M * stride));
    {
        DevTmp dcnt(sizeof(int32_t) * (size_t)(M * stride));
        hipLaunchKernelGGL(k_dense_count, dim3((unsigned)M), dim3(256), (size_t)stride * 4, s, D, K, thr, (int)kc,
                           (int)nchs, (int)kcw, (int)nchb, dcnt.as<int32_t>());
        PFR_HIP(hipGetLastError());
        PFR_HIP(hipMemcpyAsync(cnt.data(), dcnt.p, cnt.size() * 4, hipMemcpyDeviceToHost, s));
        PFR_HIP(hipStreamSynchronize(s));
    }
    std::vector<int32_t> rowptr((size_t)M + 1, 0), len((size_t)M);
    for (int64_t r = 0; r < M; ++r) {
        len[(size_t)r] = cnt[(size_t)(r * stride)];
        pfr::require((int64_t)rowptr[(size_t)r] + len[(size_t)r] < INT32_MAX, "nnz exceeds 32-bit indices");
        rowptr[(size_t)r + 1] = rowptr[(size_t)r] + len[(size_t)r];
    }
    auto* w = new pfr_csr();
    try {
        w->ctx = ctx;
        w->M = M;
        w->K = K;
        w->nnz = rowptr[(size_t)M];
        w->vdt = PFR_F32;
        w->max_row_nnz = M ? *std::max_element(len.begin(), len.end()) : 0;
        w->cols_sorted = true;
        w->rowptr = walloc_copy(w, rowptr.data(), M + 1, s);
        const int64_t npad = (w->nnz + 3) / 4 * 4 + 4;  // whole records and a spare one, as build() pads
        float* val = walloc<float>(w, npad);
        w->val = val;
        fill_dev(val + w->nnz, npad - w->nnz, 0.0f, s);
        if (K > 65536) {
            w->col = walloc<int32_t>(w, w->nnz);
        } else {
            w->col16 = walloc<uint16_t>(w, npad);
            fill_dev(w->col16 + w->nnz, npad - w->nnz, (uint16_t)std::min<int64_t>(K, 65535), s);
        }
        hipLaunchKernelGGL(k_dense_compact, dim3((unsigned)M), dim3(256), 0, s, D, K, thr, w->rowptr, w->col,
                           w->col16, val);
        PFR_HIP(hipGetLastError());
        std::vector<int32_t> blocks = spmv_blocks(rowptr, M);
        w->n_spmv_blocks = (int64_t)blocks.size() - 1;
        w->spmv_blocks = walloc_copy(w, blocks.data(), (int64_t)blocks.size(), s);
        PFR_HIP(hipStreamSynchronize(s));  // blocks goes out of scope
        if (w->nnz == 0) return w;
        std::vector<int32_t> cs, cb;
        if (nchs > 0 && sell_wanted(M, K, w->nnz)) {
            cs.resize((size_t)(M * nchs));
            for (int64_t r = 0; r < M; ++r)
                std::copy(cnt.begin() + r * stride + 1, cnt.begin() + r * stride + 1 + nchs, cs.begin() + r * nchs);
        }
        if (nchb > 0) {
            cb.resize((size_t)(M * nchb));
            for (int64_t r = 0; r < M; ++r)
                std::copy(cnt.begin() + r * stride + 1 + nchs, cnt.begin() + (r + 1) * stride, cb.begin() + r * nchb);
        }
        set_lazy(w, rowptr, std::move(cs), std::move(cb));
        set_merge(w, rowptr, s);
        PFR_HIP(hipStreamSynchronize(s));
        return w;
    } catch (...) {
        (void)hipStreamSynchronize(s);
        free_csr(w);
        throw;
    }
}

}  // namespace

namespace pfr {

void csr_build_copies(pfr_csr* w, uint32_t which) {
    if ((w->pending.load(std::memory_order_acquire) & which) == 0) return;
    std::lock_guard<std::mutex> lock(w->lazy_mu);
    which &= w->pending.load(std::memory_order_acquire);
    if (which == 0) return;
    hipStream_t s = w->ctx->stream;
    // nothing is allocated or synchronized while the stream is captured:
    // the product reads the CSR in place and the copy waits for an eager one
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    PFR_HIP(hipStreamIsCapturing(s, &st));
    if (st != hipStreamCaptureStatusNone) return;
    for (const uint32_t bit : {kCopySell, kCopySellFast, kCopyChain, kCopyBal}) {
        if ((which & bit) == 0) continue;
        const int64_t before = w->dev_bytes;
        try {
            if (w->col16) build_copy(w, bit, w->col16, s);
            else build_copy(w, bit, w->col, s);
        } catch (...) {
            (void)hipStreamSynchronize(s);
            drop_copy(w, bit);
            w->dev_bytes = before;
            throw;  // still pending: the next product tries again
        }
        w->pending.fetch_and(~bit, std::memory_order_release);
    }
    if (w->pending.load(std::memory_order_acquire) == 0) {
        std::vector<int32_t>().swap(w->h_rowptr);
        std::vector<int32_t>().swap(w->h_sell_cnt);
        std::vector<int32_t>().swap(w->h_bal_cnt);
    }
}

}  // namespace pfr

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

int pfr_csr_from_dense_dev(pfr_ctx* ctx, const float* dense, int64_t rows, int64_t cols, int transpose,
                           float threshold, const float* mask, pfr_csr** out) {
    return pfr::guarded([&] {
        pfr::require(out != nullptr, "null output handle");
        *out = nullptr;
        pfr::bind(ctx);
        pfr::require(rows >= 0 && cols >= 0, "negative dimension");
        pfr::require(rows < INT32_MAX && cols < INT32_MAX, "dimension exceeds 32-bit indices");
        pfr::require(dense != nullptr || rows * cols == 0, "null dense weight");
        const int64_t M = transpose ? cols : rows, K = transpose ? rows : cols;
        // one 256-thread workgroup per row; one per 32 x 32 tile for the transpose
        pfr::require(M <= (int64_t(1) << 24) && (rows + 31) / 32 * ((cols + 31) / 32) < (int64_t(1) << 31),
                     "weight too large for the device build");
        if (M == 0 || K == 0) {
            *out = build(ctx, M, K, std::vector<int32_t>((size_t)M + 1, 0), {}, nullptr, PFR_F32, nullptr);
            return;
        }
        hipStream_t s = ctx->stream;
        const float* D = dense;
        std::unique_ptr<DevTmp> tmp;
        if (transpose || mask) {  // op(dense * mask), row-major
            tmp.reset(new DevTmp(sizeof(float) * (size_t)(M * K)));
            if (transpose) {
                const unsigned tiles = (unsigned)((rows + 31) / 32 * ((cols + 31) / 32));
                if (mask)
                    hipLaunchKernelGGL(k_transpose_mask<true>, dim3(tiles), dim3(256), 0, s, dense, mask, rows, cols,
                                       tmp->as<float>());
                else
                    hipLaunchKernelGGL(k_transpose_mask<false>, dim3(tiles), dim3(256), 0, s, dense, mask, rows,
                                       cols, tmp->as<float>());
                PFR_HIP(hipGetLastError());
            } else {
                pfr::apply_mask_dev(s, dense, mask, M * K, tmp->as<float>());
            }
            D = tmp->as<float>();
        }
        *out = build_dense_dev(ctx, D, M, K, threshold);
        PFR_HIP(hipStreamSynchronize(s));  // tmp is freed on return
    });
}

int pfr_csr_dense_semantics(pfr_csr* w) {
    return pfr::guarded([&] {
        pfr::require(w != nullptr, "null CSR handle");
        pfr::bind(w->ctx);
        if (w->pattern != nullptr || w->M == 0 || w->K == 0) return;
        const int64_t nw = (w->K + 63) / 64;
        hipStream_t s = w->ctx->stream;
        auto* bm = dev_alloc<unsigned long long>(w->M * nw);
        try {
            fill_dev(bm, w->M * nw, 0ull, s);
            if (w->nnz > 0) {
                if (w->col16)
                    hipLaunchKernelGGL(k_pattern<uint16_t>, dim3(waves_grid(w->M)), dim3(256), 0, s, w->M, w->rowptr,
                                       w->col16, nw, bm);
                else
                    hipLaunchKernelGGL(k_pattern<int32_t>, dim3(waves_grid(w->M)), dim3(256), 0, s, w->M, w->rowptr,
                                       w->col, nw, bm);
                PFR_HIP(hipGetLastError());
            }
            PFR_HIP(hipStreamSynchronize(s));
        } catch (...) {
            (void)hipStreamSynchronize(s);
            (void)hipFree(bm);
            throw;
        }
        w->pattern = reinterpret_cast<uint64_t*>(bm);
        w->pattern_nw = nw;
        w->dev_bytes += (int64_t)sizeof(unsigned long long) * w->M * nw;
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

int pfr_csr_device_bytes(const pfr_csr* w, int64_t* bytes) {
    return pfr::guarded([&] {
        pfr::require(w != nullptr && bytes != nullptr, "null CSR handle or output");
        *bytes = w->dev_bytes;
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
