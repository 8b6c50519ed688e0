"""ctypes front-end of the oracle libraries (test infrastructure only).

``orc_*`` functions call oracle/libpfr_oracle.so, the C restatement of the
reference's kernels (oracle/pfr_oracle.c).  ``ref_*`` functions call
oracle/_ref/libpfr_ref.so, the reference's own kernel sources compiled where
they lie (oracle/Makefile, target ``ref``); that library only exists where the
reference tree was present at build time, so ``have_ref()`` gates it.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "libpfr_oracle.so")
REF_SO = os.path.join(HERE, "_ref", "libpfr_ref.so")

F32, BF16, I32, I8, U8 = 0, 2, 5, 7, 8

_P = C.c_void_p
_I64 = C.c_int64
_I32 = C.c_int32
_F = C.c_float
_INT = C.c_int

_orc = None
_ref = None


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def lib():
    global _orc
    if _orc is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"oracle library missing: {ORACLE_SO} (run build)")
        L = C.CDLL(ORACLE_SO)
        sig = {
            "orc_matmul_f32": (_INT, [_P, _P, _P, _I64, _I64, _I64, _I64, _I64]),
            "orc_gemm_f32": (None, [_P, _P, _P, _I64, _P, _I64, _I64, _I64, _F, _F, _INT, _INT]),
            "orc_csr_spmm_f32": (None, [_I64, _I64, _I64, _P, _P, _P, _P, _P]),
            "orc_csr_spmv_f32": (None, [_I64, _I64, _P, _P, _P, _P, _P]),
            "orc_to_sparse_csr": (_I64, [_P, _I64, _I64, _F, _P, _P, _P]),
            "orc_apply_mask": (None, [_P, _P, _I64, _P]),
            "orc_magnitude_mask": (_INT, [_P, _I64, _F, _P]),
            "orc_nm_mask": (_INT, [_P, _I64, _I64, _I64, _P]),
            "orc_params_from_minmax": (_INT, [_F, _F, _INT, _INT, _P, _P]),
            "orc_dynamic_params": (_INT, [_P, _I64, _INT, _INT, _P, _P]),
            "orc_dynamic_params_per_channel": (_INT, [_P, _I64, _I64, _I64, _INT, _INT, _P, _P]),
            "orc_quantize": (_INT, [_P, _I64, _I64, _I64, _P, _P, _INT, _P]),
            "orc_dequantize": (_INT, [_P, _INT, _I64, _I64, _I64, _P, _P, _P]),
            "orc_quantized_matmul": (_INT, [_P, _INT, _P, _INT, _I64, _I64, _I64, _I64, _F, _F, _I32, _I32, _P]),
            "orc_quantized_matmul_rowscale": (None, [_P, _P, _I64, _I64, _I64, _P, _F, _P]),
            "orc_int8_matmul_acc": (None, [_P, _P, _I64, _I64, _I64, _P]),
            "orc_cpu_quantized_matmul": (None, [_P, _P, _I64, _I64, _I64, _I64, _F, _F, _I64, _I64, _P]),
            "orc_bf16_from_float": (C.c_uint16, [_F]),
            "orc_bf16_to_float": (_F, [C.c_uint16]),
            "orc_f32_to_bf16": (None, [_P, _P, _I64]),
            "orc_bf16_to_f32": (None, [_P, _P, _I64]),
            "orc_relu": (None, [_P, _I64, _P]),
            "orc_gelu": (None, [_P, _I64, _P]),
            "orc_layernorm": (None, [_P, _I64, _I64, _P, _P, _F, _P]),
            "orc_add": (_INT, [_P, _P, _INT, _P, _P, _INT, _P, _P, C.POINTER(_INT)]),
            "orc_softmax": (None, [_P, _I64, _I64, _I64, _P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _orc = L
    return _orc


def have_ref():
    return os.path.exists(REF_SO)


def ref_lib():
    global _ref
    if _ref is None:
        if not have_ref():
            raise RuntimeError(f"reference library missing: {REF_SO}")
        L = C.CDLL(REF_SO)
        sig = {
            "ref_last_error": (C.c_char_p, []),
            "ref_run_op": (_INT, [C.c_char_p, _INT, _P, _P, _P, _P, _INT, _P, _P, _INT, _P, _P, _P, _I64, _P, _P]),
            "ref_to_sparse_csr": (_INT, [_P, _I64, _I64, _F, _P, _P, _P, _P]),
            "ref_sparse_matmul": (_INT, [_I64, _I64, _I64, _P, _P, _P, _I64, _P, _INT, _P]),
            "ref_time_sparse_matmul": (_INT, [_I64, _I64, _I64, _P, _P, _P, _I64, _P, _INT, _P, _P]),
            "ref_time_sparse_matvec": (_INT, [_I64, _I64, _P, _P, _P, _I64, _P, _INT, _P, _P]),
            "ref_sparse_matvec": (_INT, [_I64, _I64, _P, _P, _P, _I64, _P, _P]),
            "ref_apply_mask": (_INT, [_P, _P, _I64, _P]),
            "ref_magnitude_mask": (_INT, [_P, _I64, _I64, _F, _P]),
            "ref_nm_mask": (_INT, [_P, _I64, _I64, _I64, _P]),
            "ref_params_from_minmax": (_INT, [_F, _F, _INT, _INT, _P, _P]),
            "ref_dynamic_params": (_INT, [_P, _I64, _INT, _INT, _P, _P]),
            "ref_dynamic_params_per_channel": (_INT, [_P, _I64, _I64, _I64, _INT, _INT, _P, _P]),
            "ref_quantize": (_INT, [_P, _I64, _I64, _I64, _P, _P, _INT, _P]),
            "ref_dequantize": (_INT, [_P, _INT, _I64, _I64, _I64, _P, _P, _P]),
            "ref_quantized_matmul": (_INT, [_P, _INT, _P, _INT, _I64, _I64, _I64, _F, _I32, _F, _I32, _INT, _F, _I32, _INT, _P]),
            "ref_bf16_from_float": (C.c_uint16, [_F]),
            "ref_bf16_to_float": (_F, [C.c_uint16]),
            "ref_f32_to_bf16": (None, [_P, _P, _I64]),
            "ref_save_mlp_pfm": (_INT, [C.c_char_p, _I64, _I64, _I64, _I64, _P, _P, _P, _P]),
            "ref_run_pfm": (_INT, [C.c_char_p, C.c_char_p, _P, _P, _INT, _P, _I64, _P]),
            "ref_time_pfm": (_INT, [C.c_char_p, C.c_char_p, _P, _P, _INT, _INT, _P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _ref = L
    return _ref


def _ref_check(rc):
    if rc != 0:
        raise RuntimeError("reference raised: " + ref_lib().ref_last_error().decode())


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


# ---------------------------------------------------------------------------
# oracle (C restatement)
# ---------------------------------------------------------------------------

def orc_matmul(a, b):
    """cpu_matmul (math.cpp:268-374) for [.., M, K] x [.., K, N] with at most
    one leading batch dimension on either side (broadcast if 1 or absent)."""
    a = _c(a, np.float32)
    b = _c(b, np.float32)
    M, K = a.shape[-2:]
    N = b.shape[-1]
    ba = int(np.prod(a.shape[:-2])) if a.ndim > 2 else 1
    bb = int(np.prod(b.shape[:-2])) if b.ndim > 2 else 1
    lead = a.shape[:-2] if ba >= bb else b.shape[:-2]
    out = np.empty(tuple(lead) + (M, N), np.float32)
    rc = lib().orc_matmul_f32(_ptr(a), _ptr(b), _ptr(out), ba, bb, M, K, N)
    if rc:
        raise ValueError("MatMul: batch dimensions are not broadcastable")
    return out


def orc_gemm(A, B, C_=None, alpha=1.0, beta=1.0, transA=0, transB=0):
    A = _c(A, np.float32)
    B = _c(B, np.float32)
    M = A.shape[1] if transA else A.shape[0]
    K = A.shape[0] if transA else A.shape[1]
    N = B.shape[0] if transB else B.shape[1]
    out = np.empty((M, N), np.float32)
    csz = 0
    if C_ is not None:
        C_ = _c(C_, np.float32)
        csz = C_.size
    lib().orc_gemm_f32(_ptr(A), _ptr(B), _ptr(C_), csz, _ptr(out), M, K, N,
                       alpha, beta, int(transA), int(transB))
    return out


def orc_to_sparse_csr(dense, threshold=0.0):
    d = _c(dense, np.float32)
    rows, cols = d.shape
    nnz = lib().orc_to_sparse_csr(_ptr(d), rows, cols, threshold, None, None, None)
    indptr = np.empty(rows + 1, np.int64)
    indices = np.empty(nnz, np.int64)
    values = np.empty(nnz, np.float32)
    lib().orc_to_sparse_csr(_ptr(d), rows, cols, threshold, _ptr(indptr), _ptr(indices), _ptr(values))
    return indptr, indices, values


def orc_csr_spmm(m, k, indptr, indices, values, b):
    b = _c(b, np.float32)
    n = 1 if b.ndim == 1 else b.shape[1]
    out = np.empty((m, n) if b.ndim > 1 else (m,), np.float32)
    lib().orc_csr_spmm_f32(m, k, n, _ptr(_c(indptr, np.int64)), _ptr(_c(indices, np.int64)),
                           _ptr(_c(values, np.float32)), _ptr(b), _ptr(out))
    return out


def orc_csr_spmv(m, k, indptr, indices, values, x):
    out = np.empty(m, np.float32)
    lib().orc_csr_spmv_f32(m, k, _ptr(_c(indptr, np.int64)), _ptr(_c(indices, np.int64)),
                           _ptr(_c(values, np.float32)), _ptr(_c(x, np.float32)), _ptr(out))
    return out


def orc_apply_mask(t, mask):
    t = _c(t, np.float32)
    out = np.empty_like(t)
    lib().orc_apply_mask(_ptr(t), _ptr(_c(mask, np.float32)), t.size, _ptr(out))
    return out


def orc_magnitude_mask(w, sparsity):
    w = _c(w, np.float32)
    mask = np.empty_like(w)
    rc = lib().orc_magnitude_mask(_ptr(w), w.size, sparsity, _ptr(mask))
    if rc:
        raise RuntimeError("Cannot prune empty weight tensor")
    return mask


def orc_nm_mask(w, n=2, m=4):
    w = _c(w, np.float32)
    mask = np.empty_like(w)
    rc = lib().orc_nm_mask(_ptr(w), w.size, n, m, _ptr(mask))
    if rc:
        raise ValueError("invalid N:M")
    return mask


def orc_params_from_minmax(mn, mx, qdtype=I8, symmetric=True):
    s = np.zeros(1, np.float32)
    z = np.zeros(1, np.int32)
    rc = lib().orc_params_from_minmax(mn, mx, qdtype, int(symmetric), _ptr(s), _ptr(z))
    if rc:
        raise ValueError("scale must be positive and finite")
    return float(s[0]), int(z[0])


def orc_dynamic_params(x, qdtype=I8, symmetric=True):
    x = _c(x, np.float32)
    s = np.zeros(1, np.float32)
    z = np.zeros(1, np.int32)
    rc = lib().orc_dynamic_params(_ptr(x), x.size, qdtype, int(symmetric), _ptr(s), _ptr(z))
    if rc:
        raise ValueError("scale must be positive and finite")
    return np.float32(s[0]), int(z[0])


def orc_dynamic_params_per_channel(x3, qdtype=I8, symmetric=True):
    """x3 is viewed as [outer, channels, inner]."""
    x3 = _c(x3, np.float32)
    o, c, i = x3.shape
    s = np.zeros(c, np.float32)
    z = np.zeros(c, np.int32)
    rc = lib().orc_dynamic_params_per_channel(_ptr(x3), o, c, i, qdtype, int(symmetric), _ptr(s), _ptr(z))
    if rc:
        raise ValueError("scale must be positive and finite")
    return s, z


def orc_quantize(x, scales, zps, qdtype=I8, channel_view=None):
    """Per-tensor when channel_view is None, else x viewed as
    channel_view = (outer, channels, inner)."""
    x = _c(x, np.float32)
    scales = _c(np.atleast_1d(scales), np.float32)
    zps = _c(np.atleast_1d(zps), np.int32)
    out = np.empty(x.shape, np.int8 if qdtype == I8 else np.uint8)
    if channel_view is None:
        o, c, i = 1, 0, x.size
    else:
        o, c, i = channel_view
    rc = lib().orc_quantize(_ptr(x), o, c, i, _ptr(scales), _ptr(zps), qdtype, _ptr(out))
    if rc:
        raise ValueError("quantize_tensor: invalid scale")
    return out


def orc_dequantize(q, scales, zps, qdtype=I8, channel_view=None):
    q = np.ascontiguousarray(q)
    scales = _c(np.atleast_1d(scales), np.float32)
    zps = _c(np.atleast_1d(zps), np.int32)
    out = np.empty(q.shape, np.float32)
    if channel_view is None:
        o, c, i = 1, 0, q.size
    else:
        o, c, i = channel_view
    lib().orc_dequantize(_ptr(q), qdtype, o, c, i, _ptr(scales), _ptr(zps), _ptr(out))
    return out


def orc_quantized_matmul(a, b, a_scale, b_scale, a_zp=0, b_zp=0):
    adt = I8 if a.dtype == np.int8 else U8
    bdt = I8 if b.dtype == np.int8 else U8
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    M, K = a.shape[-2:]
    N = b.shape[-1]
    batch = int(np.prod(a.shape[:-2])) if a.ndim > 2 else 1
    out = np.empty(tuple(a.shape[:-2]) + (M, N), np.float32)
    lib().orc_quantized_matmul(_ptr(a), adt, _ptr(b), bdt, batch, M, K, N,
                               a_scale, b_scale, a_zp, b_zp, _ptr(out))
    return out


def orc_quantized_matmul_rowscale(a, b, a_scales, b_scale):
    a = _c(a, np.int8)
    b = _c(b, np.int8)
    M, K = a.shape
    N = b.shape[1]
    out = np.empty((M, N), np.float32)
    lib().orc_quantized_matmul_rowscale(_ptr(a), _ptr(b), M, K, N,
                                        _ptr(_c(a_scales, np.float32)), b_scale, _ptr(out))
    return out


def orc_int8_matmul_acc(a, b):
    a = _c(a, np.int8)
    b = _c(b, np.int8)
    M, K = a.shape
    N = b.shape[1]
    acc = np.empty((M, N), np.int32)
    lib().orc_int8_matmul_acc(_ptr(a), _ptr(b), M, K, N, _ptr(acc))
    return acc


def orc_cpu_quantized_matmul(a, b, a_scale, b_scale, a_zp=0, b_zp=0):
    a = np.ascontiguousarray(a).view(np.int8)
    b = np.ascontiguousarray(b).view(np.int8)
    M, K = a.shape[-2:]
    N = b.shape[-1]
    batch = int(np.prod(a.shape[:-2])) if a.ndim > 2 else 1
    out = np.empty(tuple(a.shape[:-2]) + (M, N), np.float32)
    lib().orc_cpu_quantized_matmul(_ptr(a), _ptr(b), batch, M, K, N, a_scale, b_scale,
                                   a_zp, b_zp, _ptr(out))
    return out


def orc_f32_to_bf16(x):
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_bf16(_ptr(x), _ptr(out), x.size)
    return out


def orc_bf16_to_f32(b):
    b = _c(b, np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().orc_bf16_to_f32(_ptr(b), _ptr(out), b.size)
    return out


def orc_relu(x):
    x = _c(x, np.float32)
    out = np.empty_like(x)
    lib().orc_relu(_ptr(x), x.size, _ptr(out))
    return out


def orc_gelu(x):
    x = _c(x, np.float32)
    out = np.empty_like(x)
    lib().orc_gelu(_ptr(x), x.size, _ptr(out))
    return out


def orc_layernorm(x, scale, bias, epsilon=1e-5, axis=-1):
    x = _c(x, np.float32)
    axis = axis % x.ndim
    outer = int(np.prod(x.shape[:axis]))
    norm = int(np.prod(x.shape[axis:]))
    out = np.empty_like(x)
    lib().orc_layernorm(_ptr(x), outer, norm, _ptr(_c(scale, np.float32)), _ptr(_c(bias, np.float32)),
                        epsilon, _ptr(out))
    return out


def orc_add(a, b):
    a = _c(a, np.float32)
    b = _c(b, np.float32)
    ash = np.array(a.shape, np.int64)
    bsh = np.array(b.shape, np.int64)
    nd = max(a.ndim, b.ndim)
    # capacity: the product of the larger extent per right-aligned axis
    ea = [1] * (nd - a.ndim) + list(a.shape)
    eb = [1] * (nd - b.ndim) + list(b.shape)
    osh = np.zeros(16, np.int64)
    ond = C.c_int(0)
    out = np.empty(max(1, int(np.prod([max(x, y) for x, y in zip(ea, eb)], dtype=np.int64))), np.float32)
    rc = lib().orc_add(_ptr(a), _ptr(ash), a.ndim, _ptr(b), _ptr(bsh), b.ndim, _ptr(out), _ptr(osh),
                       C.byref(ond))
    if rc:
        raise ValueError("Add: shapes are not broadcastable")
    shape = tuple(int(v) for v in osh[:ond.value])
    return out[: int(np.prod(shape, dtype=np.int64))].reshape(shape)


def orc_softmax(x, axis=-1):
    x = _c(x, np.float32)
    axis = axis % x.ndim
    outer = int(np.prod(x.shape[:axis]))
    inner = int(np.prod(x.shape[axis + 1:]))
    out = np.empty_like(x)
    lib().orc_softmax(_ptr(x), outer, x.shape[axis], inner, _ptr(out))
    return out


# ---------------------------------------------------------------------------
# compiled reference (only where oracle/_ref was built)
# ---------------------------------------------------------------------------

def ref_run_op(op_type, inputs, fattrs=None, iattrs=None, out_bytes=None):
    """Run one op registered by the reference's CPU backend."""
    fattrs = fattrs or {}
    iattrs = iattrs or {}
    dt_of = {np.dtype(np.float32): F32, np.dtype(np.int8): I8, np.dtype(np.uint8): U8}
    ins = [np.ascontiguousarray(x) for x in inputs]
    n = len(ins)
    data = (C.c_void_p * n)(*[x.ctypes.data for x in ins])
    dts = (C.c_int * n)(*[dt_of[x.dtype] for x in ins])
    shapes = [np.array(x.shape, np.int64) for x in ins]
    shp = (C.c_void_p * n)(*[s.ctypes.data for s in shapes])
    nd = (C.c_int * n)(*[x.ndim for x in ins])
    fn = list(fattrs)
    inn = list(iattrs)
    fnames = (C.c_char_p * max(1, len(fn)))(*[s.encode() for s in fn])
    fvals = np.array([fattrs[k] for k in fn] or [0], np.float32)
    inames = (C.c_char_p * max(1, len(inn)))(*[s.encode() for s in inn])
    ivals = np.array([iattrs[k] for k in inn] or [0], np.int64)
    cap = out_bytes or (1 << 26)
    out = np.empty(cap, np.uint8)
    oshape = np.zeros(16, np.int64)
    ond = C.c_int(0)
    rc = ref_lib().ref_run_op(op_type.encode(), n, data, dts, shp, nd, len(fn), fnames, _ptr(fvals),
                              len(inn), inames, _ptr(ivals), _ptr(out), cap, _ptr(oshape), C.byref(ond))
    _ref_check(rc)
    return out, tuple(int(v) for v in oshape[:ond.value])


def ref_op_f32(op_type, inputs, fattrs=None, iattrs=None):
    raw, shape = ref_run_op(op_type, inputs, fattrs, iattrs)
    n = int(np.prod(shape)) if shape else 0
    return raw[: 4 * n].view(np.float32).reshape(shape).copy()


def ref_to_sparse_csr(dense, threshold=0.0):
    d = _c(dense, np.float32)
    rows, cols = d.shape
    nnz = np.zeros(1, np.int64)
    _ref_check(ref_lib().ref_to_sparse_csr(_ptr(d), rows, cols, threshold, None, None, None, _ptr(nnz)))
    indptr = np.empty(rows + 1, np.int64)
    indices = np.empty(int(nnz[0]), np.int64)
    values = np.empty(int(nnz[0]), np.float32)
    _ref_check(ref_lib().ref_to_sparse_csr(_ptr(d), rows, cols, threshold, _ptr(indptr), _ptr(indices),
                                           _ptr(values), _ptr(nnz)))
    return indptr, indices, values


def ref_sparse_matmul(m, k, indptr, indices, values, b):
    b = _c(b, np.float32)
    n = 1 if b.ndim == 1 else b.shape[1]
    out = np.empty((m,) if b.ndim == 1 else (m, n), np.float32)
    _ref_check(ref_lib().ref_sparse_matmul(m, k, n, _ptr(_c(indptr, np.int64)), _ptr(_c(indices, np.int64)),
                                           _ptr(_c(values, np.float32)), len(values), _ptr(b),
                                           int(b.ndim == 1), _ptr(out)))
    return out


def ref_time_sparse_matmul(m, k, indptr, indices, values, b, reps):
    """Per-call seconds of the reference sparse_matmul (after one warm-up),
    and its output."""
    b = _c(b, np.float32)
    n = b.shape[1]
    ns = np.zeros(reps, np.int64)
    out = np.empty((m, n), np.float32)
    _ref_check(ref_lib().ref_time_sparse_matmul(m, k, n, _ptr(_c(indptr, np.int64)), _ptr(_c(indices, np.int64)),
                                                _ptr(_c(values, np.float32)), len(values), _ptr(b), reps,
                                                _ptr(ns), _ptr(out)))
    return ns.astype(np.float64) * 1e-9, out


def ref_time_sparse_matvec(m, k, indptr, indices, values, x, reps):
    """Per-call seconds of the reference sparse_matvec (after one warm-up),
    and its output."""
    ns = np.zeros(reps, np.int64)
    out = np.empty(m, np.float32)
    _ref_check(ref_lib().ref_time_sparse_matvec(m, k, _ptr(_c(indptr, np.int64)), _ptr(_c(indices, np.int64)),
                                                _ptr(_c(values, np.float32)), len(values), _ptr(_c(x, np.float32)),
                                                reps, _ptr(ns), _ptr(out)))
    return ns.astype(np.float64) * 1e-9, out


def ref_sparse_matvec(m, k, indptr, indices, values, x):
    out = np.empty(m, np.float32)
    _ref_check(ref_lib().ref_sparse_matvec(m, k, _ptr(_c(indptr, np.int64)), _ptr(_c(indices, np.int64)),
                                           _ptr(_c(values, np.float32)), len(values),
                                           _ptr(_c(x, np.float32)), _ptr(out)))
    return out


def ref_apply_mask(t, mask):
    t = _c(t, np.float32)
    out = np.empty_like(t)
    _ref_check(ref_lib().ref_apply_mask(_ptr(t), _ptr(_c(mask, np.float32)), t.size, _ptr(out)))
    return out


def ref_magnitude_mask(w, sparsity):
    w = _c(w, np.float32)
    w2 = w.reshape(1, -1) if w.ndim == 1 else w.reshape(w.shape[0], -1)
    mask = np.empty_like(w)
    _ref_check(ref_lib().ref_magnitude_mask(_ptr(w2), w2.shape[0], w2.shape[1], sparsity, _ptr(mask)))
    return mask


def ref_nm_mask(w, n=2, m=4):
    w = _c(w, np.float32)
    mask = np.empty_like(w)
    _ref_check(ref_lib().ref_nm_mask(_ptr(w), w.size, n, m, _ptr(mask)))
    return mask


def ref_params_from_minmax(mn, mx, qdtype=I8, symmetric=True):
    s = np.zeros(1, np.float32)
    z = np.zeros(1, np.int32)
    _ref_check(ref_lib().ref_params_from_minmax(mn, mx, qdtype, int(symmetric), _ptr(s), _ptr(z)))
    return float(s[0]), int(z[0])


def ref_dynamic_params(x, qdtype=I8, symmetric=True):
    x = _c(x, np.float32)
    s = np.zeros(1, np.float32)
    z = np.zeros(1, np.int32)
    _ref_check(ref_lib().ref_dynamic_params(_ptr(x), x.size, qdtype, int(symmetric), _ptr(s), _ptr(z)))
    return np.float32(s[0]), int(z[0])


def ref_dynamic_params_per_channel(x3, qdtype=I8, symmetric=True):
    x3 = _c(x3, np.float32)
    o, c, i = x3.shape
    s = np.zeros(c, np.float32)
    z = np.zeros(c, np.int32)
    _ref_check(ref_lib().ref_dynamic_params_per_channel(_ptr(x3), o, c, i, qdtype, int(symmetric),
                                                        _ptr(s), _ptr(z)))
    return s, z


def ref_quantize(x, scales, zps, qdtype=I8, channel_view=None):
    x = _c(x, np.float32)
    scales = _c(np.atleast_1d(scales), np.float32)
    zps = _c(np.atleast_1d(zps), np.int32)
    out = np.empty(x.shape, np.int8 if qdtype == I8 else np.uint8)
    o, c, i = (1, 0, x.size) if channel_view is None else channel_view
    _ref_check(ref_lib().ref_quantize(_ptr(x), o, c, i, _ptr(scales), _ptr(zps), qdtype, _ptr(out)))
    return out


def ref_dequantize(q, scales, zps, qdtype=I8, channel_view=None):
    q = np.ascontiguousarray(q)
    scales = _c(np.atleast_1d(scales), np.float32)
    zps = _c(np.atleast_1d(zps), np.int32)
    out = np.empty(q.shape, np.float32)
    o, c, i = (1, 0, q.size) if channel_view is None else channel_view
    _ref_check(ref_lib().ref_dequantize(_ptr(q), qdtype, o, c, i, _ptr(scales), _ptr(zps), _ptr(out)))
    return out


def ref_quantized_matmul(a, b, a_scale, b_scale, a_zp=0, b_zp=0, out_params=None):
    """quantization::quantized_matmul; out_params=(scale, zp, qdtype) requantizes."""
    adt = I8 if a.dtype == np.int8 else U8
    bdt = I8 if b.dtype == np.int8 else U8
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    M, K = a.shape
    N = b.shape[1]
    if out_params is None:
        out = np.empty((M, N), np.float32)
        rq, os_, oz, odt = 0, 1.0, 0, I8
    else:
        os_, oz, odt = out_params
        out = np.empty((M, N), np.int8 if odt == I8 else np.uint8)
        rq = 1
    _ref_check(ref_lib().ref_quantized_matmul(_ptr(a), adt, _ptr(b), bdt, M, K, N, a_scale, a_zp, b_scale,
                                              b_zp, rq, os_, oz, odt, _ptr(out)))
    return out


def ref_bf16_from_float(x):
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    ref_lib().ref_f32_to_bf16(_ptr(x), _ptr(out), x.size)
    return out


def ref_save_mlp_pfm(path, batch, w1, b1, w2, b2):
    w1, b1, w2, b2 = (_c(t, np.float32) for t in (w1, b1, w2, b2))
    _ref_check(ref_lib().ref_save_mlp_pfm(path.encode(), batch, w1.shape[0], w1.shape[1], w2.shape[1],
                                          _ptr(w1), _ptr(b1), _ptr(w2), _ptr(b2)))


def ref_time_pfm(path, input_name, x, reps):
    """Seconds per CPUExecutor::execute call on a graph loaded once."""
    x = _c(x, np.float32)
    shape = np.array(x.shape, np.int64)
    t = np.zeros(reps, np.int64)
    _ref_check(ref_lib().ref_time_pfm(path.encode(), input_name.encode(), _ptr(x), _ptr(shape), x.ndim, reps,
                                      _ptr(t)))
    return t.astype(np.float64) * 1e-9


def ref_run_pfm(path, input_name, x, out_elems):
    x = _c(x, np.float32)
    shape = np.array(x.shape, np.int64)
    out = np.empty(out_elems, np.float32)
    n = np.zeros(1, np.int64)
    _ref_check(ref_lib().ref_run_pfm(path.encode(), input_name.encode(), _ptr(x), _ptr(shape), x.ndim,
                                     _ptr(out), out_elems, _ptr(n)))
    return out[: int(n[0])]
