// Device-resident CSR weights: upload from the reference's SparseTensor
// arrays or from a dense zero-filled pruned weight, with the range checks the
// reference leaves out, and the row-block table used by the vector kernel.
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
                    (void*)w->chunk_ptr})
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
        if (sorted && M > 0) {
            const int64_t nc = (K + pfr::kChunkK - 1) / pfr::kChunkK;
            w->n_chunks = (int32_t)nc;
            std::vector<int32_t> cp((size_t)(M * (nc + 1)));
            for (int64_t r = 0; r < M; ++r) {
                int32_t j = rowptr[r];
                for (int64_t c = 0; c <= nc; ++c) {
                    const int64_t lim = c * pfr::kChunkK;
                    while (j < rowptr[r + 1] && col[j] < lim) ++j;
                    cp[(size_t)(r * (nc + 1) + c)] = (c == nc) ? rowptr[r + 1] : j;
                }
            }
            w->chunk_ptr = dev_alloc_copy(cp.data(), (int64_t)cp.size(), s);
        }
        PFR_HIP(hipStreamSynchronize(s));
        return w;
    } catch (...) {
        free_csr(w);
        throw;
    }
}

}  // namespace

extern "C" {

int pfr_csr_upload(pfr_ctx* ctx, int64_t M, int64_t K, int64_t nnz, const int64_t* indptr,
                   const int64_t* indices, const void* values, pfr_dtype values_dtype,
                   const float* row_scales, pfr_csr** out) {
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
            int64_t c = indices[j];
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
