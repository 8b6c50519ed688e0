"""Seeded synthetic inputs for the pruned-weight workloads.

All generators are deterministic numpy draws (PCG64).  CSR arrays follow the
reference's SparseTensor (int64 indptr/indices, float32 values, columns
ascending within a row: the order to_sparse produces, sparse_tensor.cpp:575-585).
"""
from __future__ import annotations

import numpy as np


def csr_from_mask(mask, values):
    """CSR (row-major scan order) of the entries of `values` where mask holds."""
    rows, cols = np.nonzero(mask)
    indptr = np.zeros(mask.shape[0] + 1, np.int64)
    np.cumsum(np.bincount(rows, minlength=mask.shape[0]), out=indptr[1:])
    return indptr, cols.astype(np.int64), np.ascontiguousarray(values[rows, cols], np.float32)


def csr_uniform(M, K, density, std, seed):
    """Each entry kept independently with probability `density`, values
    N(0, std) (the 4096x4096 90 %-sparse SpMM workload uses 0.1 / 0.02)."""
    rng = np.random.default_rng(seed)
    mask = rng.random((M, K), dtype=np.float32) < density
    nnz = int(mask.sum())
    vals = np.zeros((M, K), np.float32)
    vals[mask] = (rng.standard_normal(nnz, dtype=np.float32) * np.float32(std))
    return csr_from_mask(mask, vals)


def csr_lognormal_rows(M, K, mean_density, sigma, std, seed):
    """Per-row nnz ~ lognormal(sigma), scaled to a mean density and capped at
    K; positions uniform within a row (the skewed decode-linear workload)."""
    rng = np.random.default_rng(seed)
    w = rng.lognormal(0.0, sigma, M)
    counts = np.minimum(np.rint(w / w.mean() * mean_density * K).astype(np.int64), K)
    indptr = np.zeros(M + 1, np.int64)
    np.cumsum(counts, out=indptr[1:])
    indices = np.empty(int(indptr[-1]), np.int64)
    for r in range(M):
        c = counts[r]
        if c:
            indices[indptr[r]:indptr[r + 1]] = np.sort(rng.choice(K, size=c, replace=False))
    values = (rng.standard_normal(int(indptr[-1]), dtype=np.float32) * np.float32(std))
    return indptr, indices, values


def dense_normal(shape, std, seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


def csr_to_dense(M, K, indptr, indices, values):
    d = np.zeros((M, K), np.float32)
    rows = np.repeat(np.arange(M), np.diff(indptr))
    d[rows, indices] = values
    return d


def round_half_away(x):
    """std::round on float32 values (half away from zero)."""
    x = np.asarray(x, np.float32)
    return (np.sign(x) * np.floor(np.abs(x) + np.float32(0.5))).astype(np.float32)


def bf16_bits_rne(x):
    """bf16 bit patterns of finite float32 values, rounded to nearest even
    (synthetic bf16 operands; the reference's BFloat16::from_float turns
    about half of all negative values into -inf, half_types.cpp:159-168)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def keep_top2_of_4(w):
    """2:4 along the last axis: keep the two largest |w| of every group of
    four consecutive entries (NMSparsityPruning(2, 4) on continuous draws)."""
    M, K = w.shape
    g = np.abs(w.reshape(M, K // 4, 4))
    order = np.argsort(-g, axis=2, kind="stable")[:, :, :2]
    mask = np.zeros_like(g, dtype=bool)
    np.put_along_axis(mask, order, True, axis=2)
    return np.where(mask.reshape(M, K), w, np.float32(0)).astype(np.float32)


def symmetric_int8_rows(w):
    """Per-row symmetric int8: scale = absmax / 127, q = clamp(round(w / s))."""
    absmax = np.abs(w).max(axis=1).astype(np.float32)
    scale = np.where(absmax > 0, absmax / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    inv = (np.float32(1.0) / scale).astype(np.float32)
    q = np.clip(round_half_away(w * inv[:, None]), -128, 127).astype(np.int8)
    return q, scale


def quantize_per_tensor(x, scale):
    inv = np.float32(1.0) / np.float32(scale)
    return np.clip(round_half_away(np.asarray(x, np.float32) * inv), -128, 127).astype(np.int8)


def sp24_int8_weight(M, K, seed):
    """The 2:4 int8 GEMM weight: N(0,1) draws, top-2-of-4 along K, per-row
    symmetric int8."""
    w = keep_top2_of_4(np.random.default_rng(seed).standard_normal((M, K), dtype=np.float32))
    return symmetric_int8_rows(w)


def csr_int8_lognormal(M, K, mean_density, sigma, std, seed):
    """int8 weight-only CSR: lognormal row lengths (csr_lognormal_rows), values
    N(0, std) quantised per row, symmetric (scale = absmax / 127), entries
    that round to 0 dropped (the dequantised weight's CSR would not hold
    them).  Returns indptr, indices, int8 values, float32 row scales."""
    ip, ix, v = csr_lognormal_rows(M, K, mean_density, sigma, std, seed)
    rows = np.repeat(np.arange(M), np.diff(ip))
    absmax = np.zeros(M, np.float32)
    np.maximum.at(absmax, rows, np.abs(v))
    scale = np.where(absmax > 0, absmax / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    inv = (np.float32(1.0) / scale).astype(np.float32)
    q = np.clip(round_half_away(v * inv[rows]), -127, 127).astype(np.int8)
    keep = q != 0
    counts = np.bincount(rows[keep], minlength=M)
    ip2 = np.zeros(M + 1, np.int64)
    np.cumsum(counts, out=ip2[1:])
    return ip2, ix[keep], q[keep], scale


def dequant_rows(ip, q, scale):
    """float32 values RN((float)q * scale[row]) of an int8 CSR."""
    rows = np.repeat(np.arange(len(ip) - 1), np.diff(ip))
    return (q.astype(np.float32) * scale[rows]).astype(np.float32)


def csr_vstack(parts):
    """Row-wise concatenation of CSR matrices with the same K: parts are
    (indptr, indices, values[, row_scales]) tuples; returns the same tuple
    for the stacked matrix (rows of parts[0] first).  Sibling projections
    that read one activation (q, k and v; gate and up) stacked this way run
    as one product whose output rows are the parts' outputs in order."""
    ips, ixs, vs = [], [], []
    base = 0
    for p in parts:
        ip = np.asarray(p[0], np.int64)
        ips.append(ip[:-1] + base if ips else ip[:-1])
        base += int(ip[-1])
        ixs.append(np.asarray(p[1]))
        vs.append(np.asarray(p[2]))
    indptr = np.concatenate(ips + [np.array([base], np.int64)])
    out = (indptr, np.concatenate(ixs), np.concatenate(vs))
    if all(len(p) > 3 for p in parts):
        out += (np.concatenate([np.asarray(p[3], np.float32) for p in parts]),)
    return out
