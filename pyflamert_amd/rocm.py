"""Python front-end of the gfx950 kernels (thin wrappers over the C ABI).

Host entry points take and return numpy arrays; the ``*_dev`` methods take
device pointers (e.g. ``torch.Tensor.data_ptr()``) and enqueue on the
context's stream without synchronising.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from ._lib import (MODE_FAST, MODE_STRICT, PFR_BF16, PFR_F32, PFR_I8, SP24_OUT_F32, SP24_OUT_I8,
                   SP24_OUT_I32, check)

_MODES = {"strict": MODE_STRICT, "fast": MODE_FAST, MODE_STRICT: MODE_STRICT, MODE_FAST: MODE_FAST}


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def device_count():
    n = C.c_int(0)
    check(_lib.load().pfr_device_count(C.byref(n)))
    return n.value


class Context:
    """One device, one stream, grow-only scratch (pfr_ctx)."""

    def __init__(self, device=0):
        self._lib = _lib.load()
        h = C.c_void_p()
        check(self._lib.pfr_rocm_init(device, C.byref(h)))
        self.handle = h
        self.device = device

    def close(self):
        if self.handle:
            check(self._lib.pfr_rocm_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def stream(self):
        s = C.c_void_p()
        check(self._lib.pfr_ctx_get_stream(self.handle, C.byref(s)))
        return s.value

    def set_stream(self, stream_ptr):
        check(self._lib.pfr_ctx_set_stream(self.handle, stream_ptr))

    def synchronize(self):
        check(self._lib.pfr_synchronize(self.handle))

    # -- weights ---------------------------------------------------------
    def csr_upload(self, M, K, indptr, indices, values, row_scales=None):
        """CSR as the reference's SparseTensor holds it (int64 indptr/indices,
        float32 values) or int8 values with per-row float32 scales."""
        indptr = np.ascontiguousarray(indptr, np.int64)
        indices = np.ascontiguousarray(indices, np.int64)
        values = np.ascontiguousarray(values)
        if values.dtype == np.int8:
            vdt = PFR_I8
            row_scales = np.ascontiguousarray(row_scales, np.float32)
        else:
            values = values.astype(np.float32, copy=False)
            vdt = PFR_F32
            row_scales = None
        h = C.c_void_p()
        check(self._lib.pfr_csr_upload(self.handle, M, K, len(values), _ptr(indptr), _ptr(indices),
                                       _ptr(values), vdt, _ptr(row_scales), C.byref(h)))
        return CsrWeight(self, h)

    def csr_from_dense(self, dense, transpose=False, threshold=0.0):
        dense = np.ascontiguousarray(dense, np.float32)
        rows, cols = dense.shape
        h = C.c_void_p()
        check(self._lib.pfr_csr_from_dense(self.handle, _ptr(dense), rows, cols, int(bool(transpose)),
                                           threshold, C.byref(h)))
        return CsrWeight(self, h)

    def csr_from_dense_dev(self, dense_ptr, rows, cols, transpose=False, threshold=0.0, mask_ptr=None):
        """CSR of op(dense * mask) built on the device from device pointers
        (pfr_csr_from_dense_dev); mask_ptr None: no mask."""
        h = C.c_void_p()
        check(self._lib.pfr_csr_from_dense_dev(self.handle, dense_ptr, rows, cols, int(bool(transpose)),
                                               threshold, mask_ptr, C.byref(h)))
        return CsrWeight(self, h)

    def sp24_pack_dev(self, W_ptr, M, K, dtype, w_scales=None):
        """2:4 weight [M, K] on the device: dtype "i8" (with 1 or M host
        scales) or "bf16" (pfr_sp24_pack_dev)."""
        h = C.c_void_p()
        if dtype == "i8":
            sc = np.ascontiguousarray(np.atleast_1d(w_scales), np.float32)
            check(self._lib.pfr_sp24_pack_dev(self.handle, M, K, W_ptr, PFR_I8, _ptr(sc), sc.size, C.byref(h)))
        elif dtype == "bf16":
            check(self._lib.pfr_sp24_pack_dev(self.handle, M, K, W_ptr, PFR_BF16, None, 0, C.byref(h)))
        else:
            raise TypeError("2:4 weights are int8 or bf16")
        return Sp24Weight(self, h)

    def apply_mask(self, w, mask):
        """apply_mask on the GPU: w * mask elementwise (float32)."""
        w = np.ascontiguousarray(w, np.float32)
        mask = np.ascontiguousarray(mask, np.float32)
        if w.size != mask.size:
            raise ValueError("Tensor and mask must have same number of elements")
        out = np.empty_like(w)
        check(self._lib.pfr_apply_mask(self.handle, _ptr(w), _ptr(mask), w.size, _ptr(out)))
        return out

    def apply_mask_dev(self, w_ptr, mask_ptr, n, out_ptr):
        check(self._lib.pfr_apply_mask_dev(self.handle, w_ptr, mask_ptr, n, out_ptr))

    def gemm_dense_dev(self, A_ptr, M, K, B_ptr, N, Y_ptr, transA=False, alpha=1.0, beta=1.0, C_ptr=None,
                       c_size=0, ldb=None, ldy=None, relu=False, gelu=False):
        """Dense strict product (pfr_gemm_dense_dev), device pointers."""
        act = _lib.ACT_GELU if gelu else (_lib.ACT_RELU if relu else 0)
        check(self._lib.pfr_gemm_dense_dev(self.handle, A_ptr, M, K, int(bool(transA)), B_ptr, N, ldb or N,
                                           alpha, beta, C_ptr, c_size, Y_ptr, ldy or N, act))

    def sp24_pack(self, W, w_scales=None):
        """2:4 weight [M, K]: int8 (with 1 or M symmetric scales) or bf16 bits
        (uint16)."""
        W = np.ascontiguousarray(W)
        M, K = W.shape
        h = C.c_void_p()
        if W.dtype == np.int8:
            sc = np.ascontiguousarray(np.atleast_1d(w_scales), np.float32)
            check(self._lib.pfr_sp24_pack(self.handle, M, K, _ptr(W), PFR_I8, _ptr(sc), sc.size, C.byref(h)))
        elif W.dtype == np.uint16:
            check(self._lib.pfr_sp24_pack(self.handle, M, K, _ptr(W), PFR_BF16, None, 0, C.byref(h)))
        else:
            raise TypeError("2:4 weights are int8 or bf16 bits (uint16)")
        return Sp24Weight(self, h)

    # -- products --------------------------------------------------------
    def gemm_csr(self, A, BT, alpha=1.0, beta=1.0, C_=None, transA=False, mode="strict"):
        """cpu_gemm with the pruned weight in the B position; BT is the CSR of
        op(B)^T (csr_from_dense(B, transpose=not transB))."""
        A = np.ascontiguousarray(A, np.float32)
        Mb = A.shape[1] if transA else A.shape[0]
        K = A.shape[0] if transA else A.shape[1]
        Y = np.empty((Mb, BT.M), np.float32)
        csz = 0
        if C_ is not None:
            C_ = np.ascontiguousarray(C_, np.float32)
            csz = C_.size
        check(self._lib.pfr_gemm_csr(self.handle, _ptr(A), Mb, K, int(bool(transA)), BT.handle,
                                     alpha, beta, _ptr(C_), csz, _ptr(Y), _MODES[mode]))
        return Y

    # -- graph neighbours ------------------------------------------------
    def gelu(self, x):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        check(self._lib.pfr_gelu(self.handle, _ptr(x), x.size, _ptr(y)))
        return y

    def add(self, a, b):
        """a + b with numpy broadcasting (float32)."""
        a = np.ascontiguousarray(a, np.float32)
        b = np.ascontiguousarray(b, np.float32)
        sa = np.asarray(a.shape, np.int64)
        sb = np.asarray(b.shape, np.int64)
        # math.cpp:54-64: right-aligned, the larger extent per axis (an
        # empty operand against a size-1 axis keeps the 1); the library
        # rejects shapes that do not broadcast
        nd = max(a.ndim, b.ndim)
        ea = (1,) * (nd - a.ndim) + a.shape
        eb = (1,) * (nd - b.ndim) + b.shape
        y = np.empty(tuple(max(x, z) for x, z in zip(ea, eb)), np.float32)
        check(self._lib.pfr_add(self.handle, _ptr(a), _ptr(sa), a.ndim, _ptr(b), _ptr(sb), b.ndim, _ptr(y)))
        return y

    def layernorm(self, x, scale, bias, epsilon=1e-5, axis=-1):
        """LayerNormalization over the dimensions from `axis` on."""
        x = np.ascontiguousarray(x, np.float32)
        ax = axis + x.ndim if axis < 0 else axis
        norm = int(np.prod(x.shape[ax:], dtype=np.int64))
        outer = int(np.prod(x.shape[:ax], dtype=np.int64))
        scale = np.ascontiguousarray(scale, np.float32).ravel()
        bias = np.ascontiguousarray(bias, np.float32).ravel()
        if scale.size != norm or bias.size != norm:
            raise ValueError("scale and bias must hold the normalised extent")
        y = np.empty_like(x)
        check(self._lib.pfr_layernorm(self.handle, _ptr(x), outer, norm, _ptr(scale), _ptr(bias),
                                      float(epsilon), _ptr(y)))
        return y

    def add_dev(self, a_ptr, a_shape, b_ptr, b_shape, y_ptr):
        sa = np.asarray(a_shape, np.int64)
        sb = np.asarray(b_shape, np.int64)
        check(self._lib.pfr_add_dev(self.handle, a_ptr, _ptr(sa), sa.size, b_ptr, _ptr(sb), sb.size, y_ptr))

    def layernorm_dev(self, x_ptr, outer, norm, scale_ptr, bias_ptr, epsilon, y_ptr):
        check(self._lib.pfr_layernorm_dev(self.handle, x_ptr, outer, norm, scale_ptr, bias_ptr, float(epsilon), y_ptr))

    # -- per-tensor quantize / dequantize ----------------------------------
    def quantize_linear(self, x, scale, zero_point=0, out="i8"):
        """quantize_tensor with per-tensor parameters: int8 (out="i8") or
        uint8 (out="u8") of x's shape."""
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(x.shape, np.uint8 if out == "u8" else np.int8)
        check(self._lib.pfr_quantize_linear(self.handle, _ptr(x), x.size, float(scale), int(zero_point),
                                            _lib.PFR_U8 if out == "u8" else _lib.PFR_I8, _ptr(y)))
        return y

    def dequantize_linear(self, q, scale, zero_point=0):
        q = np.ascontiguousarray(q)
        dt = {np.dtype(np.int8): _lib.PFR_I8, np.dtype(np.uint8): _lib.PFR_U8}.get(q.dtype, _lib.PFR_F32)
        y = np.empty(q.shape, np.float32)
        check(self._lib.pfr_dequantize_linear(self.handle, _ptr(q), dt, q.size, float(scale), int(zero_point),
                                              _ptr(y)))
        return y

    # -- dynamic activation quantization ----------------------------------
    def dynamic_quantize_linear(self, x):
        """DynamicQuantizeLinear: (uint8 y of x's shape, float32 scale,
        uint8 zero point)."""
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(x.shape, np.uint8)
        scale = np.zeros(1, np.float32)
        zp = np.zeros(1, np.uint8)
        check(self._lib.pfr_dynamic_quantize_linear(self.handle, _ptr(x), x.size, _ptr(y), _ptr(scale), _ptr(zp)))
        return y, scale[0], zp[0]

    # -- pruning masks ---------------------------------------------------
    def magnitude_mask(self, w, sparsity):
        """MagnitudePruning::compute_mask on the GPU (float32 0/1 mask of
        w's shape)."""
        w = np.ascontiguousarray(w, np.float32)
        mask = np.empty_like(w)
        check(self._lib.pfr_magnitude_mask(self.handle, _ptr(w), w.size, float(sparsity), _ptr(mask)))
        return mask

    def magnitude_mask_dev(self, w_ptr, n, sparsity, mask_ptr):
        check(self._lib.pfr_magnitude_mask_dev(self.handle, w_ptr, n, float(sparsity), mask_ptr))

    def nm_mask(self, w, n=2, m=4):
        """NMSparsityPruning::compute_mask on the GPU: n kept of every m
        consecutive elements in flat order."""
        w = np.ascontiguousarray(w, np.float32)
        mask = np.empty_like(w)
        check(self._lib.pfr_nm_mask(self.handle, _ptr(w), w.size, int(n), int(m), _ptr(mask)))
        return mask

    def nm_mask_dev(self, w_ptr, total, n, m, mask_ptr):
        check(self._lib.pfr_nm_mask_dev(self.handle, w_ptr, total, int(n), int(m), mask_ptr))

    def gemm_csr_dev(self, A_ptr, Mb, K, BT, Y_ptr, alpha=1.0, beta=1.0, C_ptr=None, c_size=0,
                     transA=False, mode="strict", relu=False, gelu=False, noalloc=False):
        """Device-pointer Gemm; noalloc=True calls the allocation-free entry
        (pfr_gemm_csr_act_noalloc_dev: op(A)^T in the fixed per-device
        workspace, K * Mb <= 4,194,304 when a copy is needed)."""
        if noalloc:
            act = _lib.ACT_GELU if gelu else _lib.ACT_RELU if relu else _lib.ACT_NONE
            check(self._lib.pfr_gemm_csr_act_noalloc_dev(self.handle, A_ptr, Mb, K, int(bool(transA)), BT.handle,
                                                         alpha, beta, C_ptr, c_size, Y_ptr, _MODES[mode], act))
        elif relu or gelu:
            act = _lib.ACT_GELU if gelu else _lib.ACT_RELU
            check(self._lib.pfr_gemm_csr_act_dev(self.handle, A_ptr, Mb, K, int(bool(transA)), BT.handle,
                                                 alpha, beta, C_ptr, c_size, Y_ptr, _MODES[mode], act))
        else:
            check(self._lib.pfr_gemm_csr_dev(self.handle, A_ptr, Mb, K, int(bool(transA)), BT.handle,
                                             alpha, beta, C_ptr, c_size, Y_ptr, _MODES[mode]))


class CsrWeight:
    """Device-resident CSR weight (pfr_csr)."""

    def __init__(self, ctx, handle):
        self.ctx = ctx
        self.handle = handle
        M, K, nnz = C.c_int64(), C.c_int64(), C.c_int64()
        check(ctx._lib.pfr_csr_info(handle, C.byref(M), C.byref(K), C.byref(nnz)))
        self.M, self.K, self.nnz = M.value, K.value, nnz.value

    def dense_semantics(self):
        """pfr_csr_dense_semantics: products then propagate non-finite
        activations as the dense kernels do."""
        check(self.ctx._lib.pfr_csr_dense_semantics(self.handle))
        return self

    def device_bytes(self):
        """pfr_csr_device_bytes: device memory the handle holds now (the CSR,
        its tables and the derived copies its products have built)."""
        b = C.c_int64()
        check(self.ctx._lib.pfr_csr_device_bytes(self.handle, C.byref(b)))
        return b.value

    def free(self):
        if self.handle:
            check(self.ctx._lib.pfr_csr_free(self.handle))
            self.handle = None

    def __del__(self):
        try:
            if self.ctx.handle:
                self.free()
        except Exception:
            pass

    def spmm(self, X, mode="strict"):
        """Y = W . X with host numpy X of shape [K, N] or [K]."""
        X = np.ascontiguousarray(X, np.float32)
        vec = X.ndim == 1
        N = 1 if vec else X.shape[1]
        if X.shape[0] != self.K:
            raise ValueError(f"Dimension mismatch in sparse matmul: K={self.K}, X has {X.shape[0]} rows")
        Y = np.empty((self.M,) if vec else (self.M, N), np.float32)
        check(self.ctx._lib.pfr_spmm_csr(self.ctx.handle, self.handle, _ptr(X), N, _ptr(Y), _MODES[mode]))
        return Y

    def spmm_dev(self, X_ptr, N, Y_ptr, ldx=None, ldy=None, mode="strict", relu=False, gelu=False):
        if relu or gelu:
            act = _lib.ACT_GELU if gelu else _lib.ACT_RELU
            check(self.ctx._lib.pfr_spmm_csr_act_dev(self.ctx.handle, self.handle, X_ptr, N, ldx or N, Y_ptr,
                                                     ldy or N, _MODES[mode], act))
        else:
            check(self.ctx._lib.pfr_spmm_csr_dev(self.ctx.handle, self.handle, X_ptr, N, ldx or N, Y_ptr,
                                                 ldy or N, _MODES[mode]))


_SP24_OUT = {"i32": SP24_OUT_I32, "f32": SP24_OUT_F32, "i8": SP24_OUT_I8}


class Sp24Weight:
    """Device-resident 2:4 compressed weight (pfr_sp24)."""

    def __init__(self, ctx, handle):
        self.ctx = ctx
        self.handle = handle
        M, K, dt = C.c_int64(), C.c_int64(), C.c_int()
        check(ctx._lib.pfr_sp24_info(handle, C.byref(M), C.byref(K), C.byref(dt)))
        self.M, self.K, self.dtype = M.value, K.value, dt.value

    def free(self):
        if self.handle:
            check(self.ctx._lib.pfr_sp24_free(self.handle))
            self.handle = None

    def __del__(self):
        try:
            if self.ctx.handle:
                self.free()
        except Exception:
            pass

    def gemm_i8(self, X, x_scale=1.0, out="i32", out_scale=1.0, out_zp=0):
        """Y = W . X for int8 X [K, N]; out = "i32" | "f32" | "i8"."""
        X = np.ascontiguousarray(X, np.int8)
        if X.shape[0] != self.K:
            raise ValueError("quantized_matmul: inner dimensions must match")
        N = X.shape[1]
        dt = {"i32": np.int32, "f32": np.float32, "i8": np.int8}[out]
        Y = np.empty((self.M, N), dt)
        check(self.ctx._lib.pfr_sp24_gemm_i8(self.ctx.handle, self.handle, _ptr(X), N, x_scale, _SP24_OUT[out],
                                             out_scale, out_zp, _ptr(Y)))
        return Y

    def gemm_i8_dev(self, X_ptr, N, Y_ptr, x_scale=1.0, out="i32", out_scale=1.0, out_zp=0, ldx=None, ldy=None):
        check(self.ctx._lib.pfr_sp24_gemm_i8_dev(self.ctx.handle, self.handle, X_ptr, N, ldx or N, x_scale,
                                                 _SP24_OUT[out], out_scale, out_zp, Y_ptr, ldy or N))

    def gemm_q(self, X, x_scale=1.0, x_zp=0, out="f32", out_scale=1.0, out_zp=0):
        """Y = W . (X - x_zp) for int8 or uint8 X [K, N] (the activation as
        QuantizeLinear / DynamicQuantizeLinear leave it)."""
        X = np.ascontiguousarray(X)
        if X.dtype not in (np.int8, np.uint8):
            raise ValueError("activation must be int8 or uint8")
        if X.shape[0] != self.K:
            raise ValueError("quantized_matmul: inner dimensions must match")
        N = X.shape[1]
        dt = {"i32": np.int32, "f32": np.float32, "i8": np.int8}[out]
        Y = np.empty((self.M, N), dt)
        xdt = _lib.PFR_U8 if X.dtype == np.uint8 else _lib.PFR_I8
        check(self.ctx._lib.pfr_sp24_gemm_q(self.ctx.handle, self.handle, _ptr(X), xdt, N, x_scale, int(x_zp),
                                            _SP24_OUT[out], out_scale, out_zp, _ptr(Y)))
        return Y

    def gemm_q_dev(self, X_ptr, x_u8, N, Y_ptr, x_scale=1.0, x_zp=0, x_scale_ptr=None, x_zp_ptr=None, out="f32",
                   out_scale=1.0, out_zp=0, ldx=None, ldy=None):
        xdt = _lib.PFR_U8 if x_u8 else _lib.PFR_I8
        check(self.ctx._lib.pfr_sp24_gemm_q_dev(self.ctx.handle, self.handle, X_ptr, xdt, N, ldx or N, x_scale,
                                                int(x_zp), x_scale_ptr, x_zp_ptr, _SP24_OUT[out], out_scale, out_zp,
                                                Y_ptr, ldy or N))

    def gemm_bf16(self, X):
        """Y (float32) = W . X for bf16-bit X [K, N] (uint16)."""
        X = np.ascontiguousarray(X, np.uint16)
        N = X.shape[1]
        Y = np.empty((self.M, N), np.float32)
        check(self.ctx._lib.pfr_sp24_gemm_bf16(self.ctx.handle, self.handle, _ptr(X), N, _ptr(Y)))
        return Y

    def gemm_bf16_dev(self, X_ptr, N, Y_ptr, ldx=None, ldy=None):
        check(self.ctx._lib.pfr_sp24_gemm_bf16_dev(self.ctx.handle, self.handle, X_ptr, N, ldx or N, Y_ptr,
                                                   ldy or N))
