/*
 * pfr_oracle.c -- CPU restatement of the reference's pruned-weight
 * MatMul/Gemm path.  TEST INFRASTRUCTURE ONLY (see pfr_oracle.h): the product
 * never links or calls it.
 *
 * Build: gcc -std=c11 -O2 -ffp-contract=off -fPIC -shared (oracle/Makefile).
 * ISO C with contraction off and no -march matches GCC's default for the
 * reference's -std=c++17 Release build: every product and every sum is a
 * separately rounded IEEE single operation.
 */
#include "pfr_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* dense fp32                                                                */
/* ------------------------------------------------------------------------ */

/* math.cpp:268-374.  Output starts at +0 (:309-310); per output the terms
 * a_ik*b_kj are added in ascending k (:327-333, batched :363-369). */
int orc_matmul_f32(const float* a, const float* b, float* out,
                   int64_t batch_a, int64_t batch_b,
                   int64_t M, int64_t K, int64_t N) {
    if (batch_a < 1 || batch_b < 1) return -1;
    if (batch_a != batch_b && batch_a != 1 && batch_b != 1) return -1;
    int64_t total = batch_a > batch_b ? batch_a : batch_b;
    memset(out, 0, sizeof(float) * (size_t)(total * M * N));
    for (int64_t n = 0; n < total; ++n) {
        const float* ab = a + (batch_a == 1 ? 0 : n) * M * K;
        const float* bb = b + (batch_b == 1 ? 0 : n) * K * N;
        float* ob = out + n * M * N;
        for (int64_t i = 0; i < M; ++i) {
            for (int64_t k = 0; k < K; ++k) {
                float a_ik = ab[i * K + k];
                for (int64_t j = 0; j < N; ++j) {
                    ob[i * N + j] += a_ik * bb[k * N + j];
                }
            }
        }
    }
    return 0;
}

/* math.cpp:377-438.  Term is (alpha*a_ik)*b_kj (:421, left to right), bias
 * beta*c[i % c_size] is added after the full sum (:427-435). */
void orc_gemm_f32(const float* A, const float* B, const float* c,
                  int64_t c_size, float* out, int64_t M, int64_t K, int64_t N,
                  float alpha, float beta, int transA, int transB) {
    memset(out, 0, sizeof(float) * (size_t)(M * N));
    for (int64_t i = 0; i < M; ++i) {
        for (int64_t k = 0; k < K; ++k) {
            float a_ik = transA ? A[k * M + i] : A[i * K + k];
            for (int64_t j = 0; j < N; ++j) {
                float b_kj = transB ? B[j * K + k] : B[k * N + j];
                out[i * N + j] += alpha * a_ik * b_kj;
            }
        }
    }
    if (c && c_size > 0) {
        for (int64_t i = 0; i < M * N; ++i) {
            out[i] += beta * c[i % c_size];
        }
    }
}

/* ------------------------------------------------------------------------ */
/* CSR                                                                       */
/* ------------------------------------------------------------------------ */

/* sparse_tensor.cpp:473-519 (CSR branch :500-510). */
void orc_csr_spmm_f32(int64_t m, int64_t k, int64_t n, const int64_t* indptr,
                      const int64_t* indices, const float* values,
                      const float* b, float* out) {
    (void)k;
    memset(out, 0, sizeof(float) * (size_t)(m * n));
    for (int64_t row = 0; row < m; ++row) {
        for (int64_t j = indptr[row]; j < indptr[row + 1]; ++j) {
            int64_t col = indices[j];
            float val = values[j];
            for (int64_t c = 0; c < n; ++c) {
                out[row * n + c] += val * b[col * n + c];
            }
        }
    }
}

/* sparse_tensor.cpp:521-554 (CSR branch :542-549). */
void orc_csr_spmv_f32(int64_t m, int64_t k, const int64_t* indptr,
                      const int64_t* indices, const float* values,
                      const float* x, float* out) {
    (void)k;
    for (int64_t row = 0; row < m; ++row) out[row] = 0.0f;
    for (int64_t row = 0; row < m; ++row) {
        for (int64_t j = indptr[row]; j < indptr[row + 1]; ++j) {
            out[row] += values[j] * x[indices[j]];
        }
    }
}

/* sparse_tensor.cpp:560-610 (CSR branch :570-587): row-major scan, keeps
 * fabs(v) > threshold, so +-0 and NaN are dropped; columns ascend. */
int64_t orc_to_sparse_csr(const float* dense, int64_t rows, int64_t cols,
                          float threshold, int64_t* indptr, int64_t* indices,
                          float* values) {
    int64_t nnz = 0;
    if (indptr) indptr[0] = 0;
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t c = 0; c < cols; ++c) {
            float v = dense[r * cols + c];
            if (fabsf(v) > threshold) {
                if (indices) {
                    indices[nnz] = c;
                    values[nnz] = v;
                }
                ++nnz;
            }
        }
        if (indptr) indptr[r + 1] = nnz;
    }
    return nnz;
}

/* sparse_tensor.cpp:616-631. */
void orc_apply_mask(const float* t, const float* mask, int64_t n, float* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = t[i] * mask[i];
}

/* ------------------------------------------------------------------------ */
/* mask producers                                                            */
/* ------------------------------------------------------------------------ */

/* Ascending, NaN after everything (+inf included).  std::sort's order of
 * NaN importances is unspecified (they break its strict weak ordering);
 * this fixes it to the end, as the GPU's radix select on |w| bit patterns
 * does.  For NaN-free input it is the plain ascending order. */
static int cmp_float_asc(const void* pa, const void* pb) {
    float a = *(const float*)pa, b = *(const float*)pb;
    const int na = a != a, nb = b != b;
    if (na || nb) return na - nb;
    return (a < b) ? -1 : (a > b) ? 1 : 0;
}

/* magnitude_pruning.cpp:22-102. */
int orc_magnitude_mask(const float* w, int64_t n, float sparsity,
                       float* mask) {
    if (sparsity <= 0.0f) {                               /* :31-37 */
        for (int64_t i = 0; i < n; ++i) mask[i] = 1.0f;
        return 0;
    }
    if (sparsity >= 1.0f) {                               /* :39-45 */
        for (int64_t i = 0; i < n; ++i) mask[i] = 0.0f;
        return 0;
    }
    if (n == 0) return -1;                                /* :52-54 */
    float* imp = (float*)malloc(sizeof(float) * (size_t)n);
    float* scores = (float*)malloc(sizeof(float) * (size_t)n);
    if (!imp || !scores) { free(imp); free(scores); return -2; }
    for (int64_t i = 0; i < n; ++i) imp[i] = fabsf(w[i]); /* :8-20 */
    memcpy(scores, imp, sizeof(float) * (size_t)n);
    qsort(scores, (size_t)n, sizeof(float), cmp_float_asc);   /* :65 */
    /* :69-72: index in double, clamped to n-1 */
    size_t idx = (size_t)floor((double)n * (double)sparsity);
    if (idx > (size_t)(n - 1)) idx = (size_t)(n - 1);
    float threshold = scores[idx];
    for (int64_t i = 0; i < n; ++i)                        /* :79-81 */
        mask[i] = (imp[i] > threshold) ? 1.0f : 0.0f;
    /* :84: int64 * float is evaluated in float, then truncated */
    size_t target_zeros = (size_t)((float)n * sparsity);
    size_t actual_zeros = 0;
    for (int64_t i = 0; i < n; ++i)
        if (mask[i] == 0.0f) actual_zeros++;
    if (actual_zeros > target_zeros) {                     /* :91-99 */
        size_t to_restore = actual_zeros - target_zeros;
        for (int64_t i = 0; i < n && to_restore > 0; ++i) {
            if (mask[i] == 0.0f && imp[i] == threshold) {
                mask[i] = 1.0f;
                to_restore--;
            }
        }
    }
    free(imp);
    free(scores);
    return 0;
}

/*
 * libstdc++ (GCC 11.4, bits/stl_heap.h + bits/stl_algo.h) std::partial_sort
 * = __heap_select followed by __sort_heap.  Restated on an index array with
 * the comparator of nm_sparsity.cpp:107-110 / :90-93:
 *     comp(a, b) := |w[base+a]| > |w[base+b]|
 * Which indices end in the first `middle` slots depends on this exact
 * sequence when magnitudes tie, so it is kept step for step.
 */
typedef struct { const float* w; int64_t base; } nm_cmp_ctx;

static int nm_comp(const nm_cmp_ctx* c, int64_t a, int64_t b) {
    return fabsf(c->w[c->base + a]) > fabsf(c->w[c->base + b]);
}

static void heap_push(int64_t* first, int64_t hole, int64_t top, int64_t value,
                      const nm_cmp_ctx* c) {
    int64_t parent = (hole - 1) / 2;
    while (hole > top && nm_comp(c, first[parent], value)) {
        first[hole] = first[parent];
        hole = parent;
        parent = (hole - 1) / 2;
    }
    first[hole] = value;
}

static void heap_adjust(int64_t* first, int64_t hole, int64_t len,
                        int64_t value, const nm_cmp_ctx* c) {
    const int64_t top = hole;
    int64_t second = hole;
    while (second < (len - 1) / 2) {
        second = 2 * (second + 1);
        if (nm_comp(c, first[second], first[second - 1])) second--;
        first[hole] = first[second];
        hole = second;
    }
    if ((len & 1) == 0 && second == (len - 2) / 2) {
        second = 2 * (second + 1);
        first[hole] = first[second - 1];
        hole = second - 1;
    }
    heap_push(first, hole, top, value, c);
}

static void heap_make(int64_t* first, int64_t len, const nm_cmp_ctx* c) {
    if (len < 2) return;
    int64_t parent = (len - 2) / 2;
    for (;;) {
        int64_t value = first[parent];
        heap_adjust(first, parent, len, value, c);
        if (parent == 0) return;
        parent--;
    }
}

static void heap_pop(int64_t* first, int64_t len, int64_t* result,
                     const nm_cmp_ctx* c) {
    int64_t value = *result;
    *result = first[0];
    heap_adjust(first, 0, len, value, c);
}

static void partial_sort_idx(int64_t* idx, int64_t middle, int64_t len,
                             const nm_cmp_ctx* c) {
    heap_make(idx, middle, c);                       /* __heap_select */
    for (int64_t i = middle; i < len; ++i)
        if (nm_comp(c, idx[i], idx[0])) heap_pop(idx, middle, &idx[i], c);
    for (int64_t last = middle; last > 1;) {         /* __sort_heap */
        --last;
        heap_pop(idx, last, &idx[last], c);
    }
}

/* nm_sparsity.cpp:45-120. */
int orc_nm_mask(const float* w, int64_t total, int64_t n, int64_t m,
                float* mask) {
    if (n > m || n == 0 || m == 0) return -1;        /* ctor :9-18 */
    for (int64_t i = 0; i < total; ++i) mask[i] = 0.0f;
    int64_t* idx = (int64_t*)malloc(sizeof(int64_t) * (size_t)m);
    if (!idx) return -2;
    for (int64_t i = 0; i < total; i += m) {
        int64_t gs = (total - i) < m ? (total - i) : m;
        nm_cmp_ctx c = {w, i};
        int64_t keep;
        if (gs < m) {                                /* :82-101 */
            keep = (int64_t)ceilf((float)(gs * n) / (float)m);
            if (keep > gs) keep = gs;
        } else {
            keep = n;                                /* :102-116 */
        }
        for (int64_t j = 0; j < gs; ++j) idx[j] = j;
        partial_sort_idx(idx, keep, gs, &c);
        for (int64_t j = 0; j < keep; ++j) mask[i + idx[j]] = 1.0f;
    }
    free(idx);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* quantization                                                              */
/* ------------------------------------------------------------------------ */

static void quant_range(int qdtype, int32_t* qmin, int32_t* qmax) {
    if (qdtype == ORC_U8) { *qmin = 0; *qmax = 255; }
    else { *qmin = -128; *qmax = 127; }
}

static int32_t clamp_i32(int32_t v, int32_t lo, int32_t hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}

/* static_cast<int32_t>(float) as x86-64 executes it (cvttss2si): truncation,
 * and the "integer indefinite" 0x80000000 for NaN or out-of-range values. */
static int32_t f2i_trunc_x86(float r) {
    if (r >= -2147483648.0f && r < 2147483648.0f) return (int32_t)r;
    return INT32_MIN;
}

static int32_t add_wrap(int32_t a, int32_t b) {
    return (int32_t)((uint32_t)a + (uint32_t)b);
}

/* quant_params.cpp:14-55, then the checks of QuantParams::per_tensor
 * (quant_params.hpp:60-82). */
int orc_params_from_minmax(float min_val, float max_val, int qdtype,
                           int symmetric, float* scale, int32_t* zp) {
    int32_t qmin, qmax;
    quant_range(qdtype, &qmin, &qmax);
    float s;
    int32_t z;
    if (fabsf(max_val - min_val) < 1e-8f) {
        *scale = 1.0f;
        *zp = 0;
        return 0;
    }
    if (symmetric) {
        float a = fabsf(min_val), b = fabsf(max_val);
        float abs_max = (a < b) ? b : a;             /* std::max(a, b) */
        if (qdtype == ORC_I8) { s = abs_max / 127.0f; z = 0; }
        else { s = (2.0f * abs_max) / 255.0f; z = 128; }
    } else {
        s = (max_val - min_val) / (float)(qmax - qmin);
        z = qmin - f2i_trunc_x86(roundf(min_val / s));
        z = clamp_i32(z, qmin, qmax);
    }
    if (s < 1e-10f) s = 1e-10f;
    if (!(s > 0.0f) || !isfinite(s)) return -1;     /* per_tensor check */
    *scale = s;
    *zp = z;
    return 0;
}

/* quant_ops.cpp:288-322. */
int orc_dynamic_params(const float* x, int64_t count, int qdtype,
                       int symmetric, float* scale, int32_t* zp) {
    if (count == 0) { *scale = 1.0f; *zp = 0; return 0; }
    float mn = 3.40282347e+38f, mx = -3.40282347e+38f;
    for (int64_t i = 0; i < count; ++i) {
        float v = x[i];
        if (isfinite(v)) {
            mn = (v < mn) ? v : mn;                    /* std::min(mn, v) */
            mx = (mx < v) ? v : mx;                    /* std::max(mx, v) */
        }
    }
    if (mn > mx) { *scale = 1.0f; *zp = 0; return 0; }
    return orc_params_from_minmax(mn, mx, qdtype, symmetric, scale, zp);
}

/* quant_ops.cpp:324-381 -> quant_params.cpp:57-106. */
int orc_dynamic_params_per_channel(const float* x, int64_t outer,
                                   int64_t channels, int64_t inner,
                                   int qdtype, int symmetric, float* scales,
                                   int32_t* zps) {
    int32_t qmin, qmax;
    quant_range(qdtype, &qmin, &qmax);
    float* mns = (float*)malloc(sizeof(float) * (size_t)channels);
    float* mxs = (float*)malloc(sizeof(float) * (size_t)channels);
    if (!mns || !mxs) { free(mns); free(mxs); return -2; }
    for (int64_t c = 0; c < channels; ++c) {
        mns[c] = 3.40282347e+38f;
        mxs[c] = -3.40282347e+38f;
    }
    for (int64_t o = 0; o < outer; ++o) {
        for (int64_t c = 0; c < channels; ++c) {
            const float* p = x + (o * channels + c) * inner;
            for (int64_t i = 0; i < inner; ++i) {
                float v = p[i];
                if (isfinite(v)) {
                    mns[c] = (v < mns[c]) ? v : mns[c];
                    mxs[c] = (mxs[c] < v) ? v : mxs[c];
                }
            }
        }
    }
    int rc = 0;
    for (int64_t c = 0; c < channels; ++c) {
        if (mns[c] > mxs[c]) { mns[c] = 0.0f; mxs[c] = 0.0f; }
        float mn = mns[c], mx = mxs[c], s;
        int32_t z;
        if (fabsf(mx - mn) < 1e-8f) { scales[c] = 1.0f; zps[c] = 0; continue; }
        if (symmetric) {
            float a = fabsf(mn), b = fabsf(mx);
            float abs_max = (a < b) ? b : a;
            if (qdtype == ORC_I8) { s = abs_max / 127.0f; z = 0; }
            else { s = (2.0f * abs_max) / 255.0f; z = 128; }
        } else {
            s = (mx - mn) / (float)(qmax - qmin);
            z = qmin - f2i_trunc_x86(roundf(mn / s));
            z = clamp_i32(z, qmin, qmax);
        }
        if (s < 1e-10f) s = 1e-10f;
        if (!(s > 0.0f) || !isfinite(s)) rc = -1;      /* per_channel check */
        scales[c] = s;
        zps[c] = z;
    }
    free(mns);
    free(mxs);
    return rc;
}

/* One element of quantize_tensor (quant_ops.cpp:45-47 / :102-105):
 *   q = static_cast<int32_t>(std::round(src * inv_scale)) + zp, clamped. */
static int32_t quant_one(float v, float inv_scale, int32_t zp, int32_t qmin,
                         int32_t qmax) {
    float prod = v * inv_scale;
    int32_t q = add_wrap(f2i_trunc_x86(roundf(prod)), zp);
    return clamp_i32(q, qmin, qmax);
}

/* quant_ops.cpp:15-127. */
int orc_quantize(const float* x, int64_t outer, int64_t channels,
                 int64_t inner, const float* scales, const int32_t* zps,
                 int qdtype, void* out) {
    int32_t qmin, qmax;
    quant_range(qdtype, &qmin, &qmax);
    int8_t* o8 = (int8_t*)out;
    uint8_t* ou8 = (uint8_t*)out;
    if (channels == 0) {                              /* per-tensor :33-57 */
        float scale = scales[0];
        int32_t zp = zps[0];
        if (scale <= 0.0f || !isfinite(scale)) return -1;
        float inv = 1.0f / scale;
        int64_t count = outer * inner;
        for (int64_t i = 0; i < count; ++i) {
            int32_t q = quant_one(x[i], inv, zp, qmin, qmax);
            if (qdtype == ORC_I8) o8[i] = (int8_t)q; else ou8[i] = (uint8_t)q;
        }
        return 0;
    }
    for (int64_t c = 0; c < channels; ++c)            /* :83-90 */
        if (scales[c] <= 0.0f || !isfinite(scales[c])) return -1;
    for (int64_t o = 0; o < outer; ++o) {             /* :92-125 */
        for (int64_t c = 0; c < channels; ++c) {
            float inv = 1.0f / scales[c];
            int32_t zp = zps[c];
            int64_t base = (o * channels + c) * inner;
            for (int64_t i = 0; i < inner; ++i) {
                int32_t q = quant_one(x[base + i], inv, zp, qmin, qmax);
                if (qdtype == ORC_I8) o8[base + i] = (int8_t)q;
                else ou8[base + i] = (uint8_t)q;
            }
        }
    }
    return 0;
}

/* quant_ops.cpp:129-214: x = ((float)q - (float)zp) * scale. */
int orc_dequantize(const void* q, int qdtype, int64_t outer, int64_t channels,
                   int64_t inner, const float* scales, const int32_t* zps,
                   float* out) {
    const int8_t* q8 = (const int8_t*)q;
    const uint8_t* qu8 = (const uint8_t*)q;
    if (channels == 0) {
        float scale = scales[0];
        float zp = (float)zps[0];
        int64_t count = outer * inner;
        for (int64_t i = 0; i < count; ++i) {
            float v = (qdtype == ORC_I8) ? (float)q8[i] : (float)qu8[i];
            out[i] = (v - zp) * scale;
        }
        return 0;
    }
    for (int64_t o = 0; o < outer; ++o) {
        for (int64_t c = 0; c < channels; ++c) {
            float scale = scales[c];
            float zp = (float)zps[c];
            int64_t base = (o * channels + c) * inner;
            for (int64_t i = 0; i < inner; ++i) {
                float v = (qdtype == ORC_I8) ? (float)q8[base + i]
                                             : (float)qu8[base + i];
                out[base + i] = (v - zp) * scale;
            }
        }
    }
    return 0;
}

/* quant_ops.cpp:387-506 without the final requant (:500-503), which is
 * orc_quantize on the returned floats. */
int orc_quantized_matmul(const void* a, int a_dtype, const void* b,
                         int b_dtype, int64_t batch, int64_t M, int64_t K,
                         int64_t N, float a_scale, float b_scale, int32_t a_zp,
                         int32_t b_zp, float* out) {
    if ((a_dtype != ORC_I8 && a_dtype != ORC_U8) ||
        (b_dtype != ORC_I8 && b_dtype != ORC_U8)) return -1;
    float output_scale = a_scale * b_scale;           /* :435 */
    const int8_t* a8 = (const int8_t*)a;
    const uint8_t* au8 = (const uint8_t*)a;
    const int8_t* b8 = (const int8_t*)b;
    const uint8_t* bu8 = (const uint8_t*)b;
    int64_t* acc = (int64_t*)malloc(sizeof(int64_t) * (size_t)N);
    if (!acc) return -2;
    /* The int64 sum of exact integer products is order-independent, so the
     * loops run i-k-j for speed; the float conversion and scaling are per
     * output exactly as :467 / :492. */
    for (int64_t n = 0; n < batch; ++n) {
        for (int64_t i = 0; i < M; ++i) {
            for (int64_t j = 0; j < N; ++j) acc[j] = 0;
            for (int64_t k = 0; k < K; ++k) {
                int64_t ai = n * M * K + i * K + k;
                int32_t av = (a_dtype == ORC_I8 ? (int32_t)a8[ai]
                                                : (int32_t)au8[ai]) - a_zp;
                if (av == 0) continue;
                const int64_t bo = n * K * N + k * N;
                if (b_dtype == ORC_I8) {
                    for (int64_t j = 0; j < N; ++j)
                        acc[j] += (int64_t)av * (int64_t)((int32_t)b8[bo + j] - b_zp);
                } else {
                    for (int64_t j = 0; j < N; ++j)
                        acc[j] += (int64_t)av * (int64_t)((int32_t)bu8[bo + j] - b_zp);
                }
            }
            for (int64_t j = 0; j < N; ++j)
                out[n * M * N + i * N + j] = (float)acc[j] * output_scale;
        }
    }
    free(acc);
    return 0;
}

void orc_int8_matmul_acc(const int8_t* a, const int8_t* b, int64_t M,
                         int64_t K, int64_t N, int32_t* acc) {
    memset(acc, 0, sizeof(int32_t) * (size_t)(M * N));
    for (int64_t i = 0; i < M; ++i) {
        int32_t* row = acc + i * N;
        for (int64_t k = 0; k < K; ++k) {
            int32_t av = a[i * K + k];
            if (av == 0) continue;
            const int8_t* brow = b + k * N;
            for (int64_t j = 0; j < N; ++j) row[j] += av * (int32_t)brow[j];
        }
    }
}

void orc_quantized_matmul_rowscale(const int8_t* a, const int8_t* b,
                                   int64_t M, int64_t K, int64_t N,
                                   const float* a_scales, float b_scale,
                                   float* out) {
    int32_t* acc = (int32_t*)malloc(sizeof(int32_t) * (size_t)N);
    if (!acc) return;
    for (int64_t i = 0; i < M; ++i) {
        float s = a_scales[i] * b_scale;              /* :435 per channel */
        for (int64_t j = 0; j < N; ++j) acc[j] = 0;
        for (int64_t k = 0; k < K; ++k) {
            int32_t av = a[i * K + k];
            if (av == 0) continue;
            const int8_t* brow = b + k * N;
            for (int64_t j = 0; j < N; ++j) acc[j] += av * (int32_t)brow[j];
        }
        for (int64_t j = 0; j < N; ++j) out[i * N + j] = (float)acc[j] * s;
    }
    free(acc);
}

/* quantized_ops.cpp:77-167: int32 accumulator (wrapping as x86 does). */
void orc_cpu_quantized_matmul(const int8_t* a, const int8_t* b, int64_t batch,
                              int64_t M, int64_t K, int64_t N, float a_scale,
                              float b_scale, int64_t a_zp, int64_t b_zp,
                              float* out) {
    float output_scale = a_scale * b_scale;           /* :134 */
    for (int64_t n = 0; n < batch; ++n) {
        const int8_t* ab = a + n * M * K;
        const int8_t* bb = b + n * K * N;
        float* ob = out + n * M * N;
        for (int64_t i = 0; i < M; ++i) {
            for (int64_t j = 0; j < N; ++j) {
                uint32_t acc = 0;
                for (int64_t k = 0; k < K; ++k) {
                    int32_t av = (int32_t)ab[i * K + k] - (int32_t)a_zp;
                    int32_t bv = (int32_t)bb[k * N + j] - (int32_t)b_zp;
                    acc += (uint32_t)(av * bv);
                }
                ob[i * N + j] = (float)(int32_t)acc * output_scale;
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* bf16                                                                      */
/* ------------------------------------------------------------------------ */

/* half_types.cpp:132-174. */
uint16_t orc_bf16_from_float(float v) {
    uint32_t f;
    memcpy(&f, &v, 4);
    if ((f & 0x7F800000u) == 0x7F800000u && (f & 0x007FFFFFu) != 0) {
        uint16_t r = (uint16_t)(f >> 16);             /* NaN :137-144 */
        if ((r & 0x007F) == 0) r |= 0x0040;
        return r;
    }
    if ((f & 0x7F800000u) == 0x7F800000u)             /* inf :148-151 */
        return (uint16_t)(f >> 16);
    uint32_t bias = 0x7FFFu + ((f >> 16) & 1u);       /* :156 */
    uint32_t upper = f >> 16;
    if (upper >= 0x7F7Fu) {                           /* :159-168 */
        uint32_t lower = f & 0xFFFFu;
        if (lower + bias > 0xFFFFu) {
            uint32_t sign = f & 0x80000000u;
            return (uint16_t)((sign >> 16) | 0x7F80u);
        }
    }
    f += bias;
    return (uint16_t)(f >> 16);
}

float orc_bf16_to_float(uint16_t b) {
    uint32_t f = (uint32_t)b << 16;
    float r;
    memcpy(&r, &f, 4);
    return r;
}

void orc_f32_to_bf16(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_bf16_from_float(in[i]);
}

void orc_bf16_to_f32(const uint16_t* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_bf16_to_float(in[i]);
}

/* ------------------------------------------------------------------------ */
/* activations                                                               */
/* ------------------------------------------------------------------------ */

/* activation.cpp:45-60: std::max(0.0f, x). */
void orc_relu(const float* x, int64_t n, float* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = (0.0f < x[i]) ? x[i] : 0.0f;
}

/* activation.cpp:157-237. */
/* activation.cpp:249-256: inner = c * (v + ((0.044715 * v) * v) * v),
 * out = (0.5 * v) * (1 + tanhf(inner)), left to right as written. */
void orc_gelu(const float* x, int64_t n, float* out) {
    const float c = 0.7978845608028654f;
    for (int64_t i = 0; i < n; ++i) {
        const float v = x[i];
        const float inner = c * (v + 0.044715f * v * v * v);
        out[i] = 0.5f * v * (1.0f + tanhf(inner));
    }
}

/* nn.cpp:458-486. */
void orc_layernorm(const float* x, int64_t outer, int64_t norm, const float* scale,
                   const float* bias, float epsilon, float* out) {
    for (int64_t o = 0; o < outer; ++o) {
        const float* xr = x + o * norm;
        float mean = 0;
        for (int64_t i = 0; i < norm; ++i) mean += xr[i];
        mean /= (float)norm;
        float var = 0;
        for (int64_t i = 0; i < norm; ++i) {
            const float d = xr[i] - mean;
            var += d * d;
        }
        var /= (float)norm;
        const float inv_std = 1.0f / sqrtf(var + epsilon);
        for (int64_t i = 0; i < norm; ++i)
            out[o * norm + i] = scale[i] * (xr[i] - mean) * inv_std + bias[i];
    }
}

/* math.cpp:150-224: shapes right-aligned, a dimension of 1 (or a missing
 * one) broadcasts; out[i] = a[ia] + b[ib]. */
int orc_add(const float* a, const int64_t* a_shape, int a_nd, const float* b,
            const int64_t* b_shape, int b_nd, float* out, int64_t* out_shape,
            int* out_nd) {
    const int nd = a_nd > b_nd ? a_nd : b_nd;
    if (nd > 16) return -1;
    int64_t as[16], bs[16];
    for (int d = 0; d < nd; ++d) {
        const int da = d - (nd - a_nd), db = d - (nd - b_nd);
        as[d] = da >= 0 ? a_shape[da] : 1;
        bs[d] = db >= 0 ? b_shape[db] : 1;
        if (as[d] != bs[d] && as[d] != 1 && bs[d] != 1) return -1;
        out_shape[d] = as[d] > bs[d] ? as[d] : bs[d]; /* math.cpp:54-64: the larger */
    }
    *out_nd = nd;
    int64_t n = 1, na = 1, nb = 1;
    for (int d = 0; d < nd; ++d) n *= out_shape[d], na *= as[d], nb *= bs[d];
    if (na == 0 || nb == 0) { /* math.cpp:170-173 returns the new tensor, zeroed by tensor.cpp:47 */
        for (int64_t i = 0; i < n; ++i) out[i] = 0.0f;
        return 0;
    }
    for (int64_t i = 0; i < n; ++i) {
        int64_t rem = i, ia = 0, ib = 0, sa = 1, sb = 1;
        for (int d = nd - 1; d >= 0; --d) {
            const int64_t idx = rem % out_shape[d];
            rem /= out_shape[d];
            if (as[d] != 1) ia += idx * sa;
            if (bs[d] != 1) ib += idx * sb;
            sa *= as[d];
            sb *= bs[d];
        }
        out[i] = a[ia] + b[ib];
    }
    return 0;
}

void orc_softmax(const float* x, int64_t outer, int64_t axis_size,
                 int64_t inner, float* out) {
    if (axis_size == 0) return;
    for (int64_t o = 0; o < outer; ++o) {
        for (int64_t in = 0; in < inner; ++in) {
            float mx = -INFINITY;
            for (int64_t a = 0; a < axis_size; ++a) {
                float v = x[(o * axis_size + a) * inner + in];
                mx = (mx < v) ? v : mx;
            }
            if (isinf(mx) && mx < 0) {
                float u = 1.0f / (float)axis_size;
                for (int64_t a = 0; a < axis_size; ++a)
                    out[(o * axis_size + a) * inner + in] = u;
                continue;
            }
            float sum = 0;
            for (int64_t a = 0; a < axis_size; ++a) {
                int64_t idx = (o * axis_size + a) * inner + in;
                float e = expf(x[idx] - mx);
                out[idx] = e;
                sum += e;
            }
            if (sum == 0.0f) {
                float u = 1.0f / (float)axis_size;
                for (int64_t a = 0; a < axis_size; ++a)
                    out[(o * axis_size + a) * inner + in] = u;
                continue;
            }
            for (int64_t a = 0; a < axis_size; ++a)
                out[(o * axis_size + a) * inner + in] /= sum;
        }
    }
}
