"""ctypes binding of the gfx950 kernel library (include/pfr_rocm.h).

The library is built in-tree by ``__graft_entry__.build()`` into
``pyflamert_amd/lib/libpfr_rocm.so``.  Loading fails loudly when it is
missing: there is no CPU fallback anywhere in this package.
"""
from __future__ import annotations

import ctypes as C
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(HERE, "lib")
ROCM_SO = os.path.join(LIB_DIR, "libpfr_rocm.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "pfr_rocm.h")

PFR_OK = 0
PFR_ERR_INVALID_ARG = 1
PFR_ERR_HIP = 2
PFR_ERR_UNSUPPORTED = 3
PFR_ERR_NO_DEVICE = 4

PFR_F32, PFR_BF16, PFR_I32, PFR_I8, PFR_U8 = 0, 2, 5, 7, 8
MODE_STRICT, MODE_FAST = 0, 1
ACT_NONE, ACT_RELU, ACT_GELU = 0, 1, 2
SP24_OUT_I32, SP24_OUT_F32, SP24_OUT_I8 = 0, 1, 2

_P = C.c_void_p
_PP = C.POINTER(C.c_void_p)
_I64 = C.c_int64
_I32 = C.c_int32
_INT = C.c_int
_F = C.c_float

# name -> (restype, argtypes); every function declared in include/pfr_rocm.h.
SIGNATURES = {
    "pfr_last_error": (C.c_char_p, []),
    "pfr_device_count": (_INT, [C.POINTER(_INT)]),
    "pfr_rocm_init": (_INT, [_INT, _PP]),
    "pfr_rocm_destroy": (_INT, [_P]),
    "pfr_ctx_get_stream": (_INT, [_P, _PP]),
    "pfr_ctx_set_stream": (_INT, [_P, _P]),
    "pfr_synchronize": (_INT, [_P]),
    "pfr_dev_alloc": (_INT, [_P, _I64, _PP]),
    "pfr_dev_free": (_INT, [_P, _P]),
    "pfr_copy_to_device": (_INT, [_P, _P, _P, _I64]),
    "pfr_copy_to_host": (_INT, [_P, _P, _P, _I64]),
    "pfr_csr_upload": (_INT, [_P, _I64, _I64, _I64, _P, _P, _P, _INT, _P, _PP]),
    "pfr_csr_upload_i32": (_INT, [_P, _I64, _I64, _I64, _P, _P, _P, _INT, _P, _PP]),
    "pfr_dynamic_quantize_linear": (_INT, [_P, _P, _I64, _P, _P, _P]),
    "pfr_dynamic_quantize_linear_dev": (_INT, [_P, _P, _I64, _P, _P, _P, _P]),
    "pfr_magnitude_mask": (_INT, [_P, _P, _I64, C.c_float, _P]),
    "pfr_magnitude_mask_dev": (_INT, [_P, _P, _I64, C.c_float, _P]),
    "pfr_nm_mask": (_INT, [_P, _P, _I64, _INT, _INT, _P]),
    "pfr_nm_mask_dev": (_INT, [_P, _P, _I64, _INT, _INT, _P]),
    "pfr_csr_from_dense": (_INT, [_P, _P, _I64, _I64, _INT, _F, _PP]),
    "pfr_csr_from_dense_dev": (_INT, [_P, _P, _I64, _I64, _INT, _F, _P, _PP]),
    "pfr_csr_dense_semantics": (_INT, [_P]),
    "pfr_gemm_dense_dev": (_INT, [_P, _P, _I64, _I64, _INT, _P, _I64, _I64, _F, _F, _P, _I64, _P, _I64, _INT]),
    "pfr_apply_mask": (_INT, [_P, _P, _P, _I64, _P]),
    "pfr_apply_mask_dev": (_INT, [_P, _P, _P, _I64, _P]),
    "pfr_csr_info": (_INT, [_P, C.POINTER(_I64), C.POINTER(_I64), C.POINTER(_I64)]),
    "pfr_csr_device_bytes": (_INT, [_P, C.POINTER(_I64)]),
    "pfr_csr_free": (_INT, [_P]),
    "pfr_spmm_csr": (_INT, [_P, _P, _P, _I64, _P, _INT]),
    "pfr_spmm_csr_dev": (_INT, [_P, _P, _P, _I64, _I64, _P, _I64, _INT]),
    "pfr_spmm_csr_act_dev": (_INT, [_P, _P, _P, _I64, _I64, _P, _I64, _INT, _INT]),
    "pfr_gemm_csr": (_INT, [_P, _P, _I64, _I64, _INT, _P, _F, _F, _P, _I64, _P, _INT]),
    "pfr_gemm_csr_dev": (_INT, [_P, _P, _I64, _I64, _INT, _P, _F, _F, _P, _I64, _P, _INT]),
    "pfr_gemm_csr_act_dev": (_INT, [_P, _P, _I64, _I64, _INT, _P, _F, _F, _P, _I64, _P, _INT, _INT]),
    "pfr_gemm_csr_act_noalloc_dev": (_INT, [_P, _P, _I64, _I64, _INT, _P, _F, _F, _P, _I64, _P, _INT, _INT]),
    "pfr_sp24_pack": (_INT, [_P, _I64, _I64, _P, _INT, _P, _I64, _PP]),
    "pfr_sp24_pack_dev": (_INT, [_P, _I64, _I64, _P, _INT, _P, _I64, _PP]),
    "pfr_sp24_info": (_INT, [_P, C.POINTER(_I64), C.POINTER(_I64), C.POINTER(_INT)]),
    "pfr_sp24_free": (_INT, [_P]),
    "pfr_sp24_gemm_i8": (_INT, [_P, _P, _P, _I64, _F, _INT, _F, _I32, _P]),
    "pfr_sp24_gemm_i8_dev": (_INT, [_P, _P, _P, _I64, _I64, _F, _INT, _F, _I32, _P, _I64]),
    "pfr_sp24_gemm_q": (_INT, [_P, _P, _P, _INT, _I64, _F, _I32, _INT, _F, _I32, _P]),
    "pfr_sp24_gemm_q_dev": (_INT, [_P, _P, _P, _INT, _I64, _I64, _F, _I32, _P, _P, _INT, _F, _I32, _P, _I64]),
    "pfr_sp24_gemm_bf16": (_INT, [_P, _P, _P, _I64, _P]),
    "pfr_sp24_gemm_bf16_dev": (_INT, [_P, _P, _P, _I64, _I64, _P, _I64]),
    "pfr_relu": (_INT, [_P, _P, _I64, _P]),
    "pfr_relu_dev": (_INT, [_P, _P, _I64, _P]),
    "pfr_softmax": (_INT, [_P, _P, _I64, _I64, _I64, _P]),
    "pfr_softmax_dev": (_INT, [_P, _P, _I64, _I64, _I64, _P]),
    "pfr_gelu": (_INT, [_P, _P, _I64, _P]),
    "pfr_gelu_dev": (_INT, [_P, _P, _I64, _P]),
    "pfr_add": (_INT, [_P, _P, _P, _INT, _P, _P, _INT, _P]),
    "pfr_add_dev": (_INT, [_P, _P, _P, _INT, _P, _P, _INT, _P]),
    "pfr_sp24_gemm_qt": (_INT, [_P, _P, _P, _INT, _I64, _F, _I32, _P]),
    "pfr_sp24_gemm_qt_dev": (_INT, [_P, _P, _P, _INT, _I64, _I64, _F, _I32, _P, _P, _P, _I64]),
    "pfr_quantize_linear": (_INT, [_P, _P, _I64, _F, _I32, _INT, _P]),
    "pfr_quantize_linear_dev": (_INT, [_P, _P, _I64, _F, _I32, _INT, _P]),
    "pfr_dequantize_linear": (_INT, [_P, _P, _INT, _I64, _F, _I32, _P]),
    "pfr_dequantize_linear_dev": (_INT, [_P, _P, _INT, _I64, _F, _I32, _P]),
    "pfr_layernorm": (_INT, [_P, _P, _I64, _I64, _P, _P, _F, _P]),
    "pfr_layernorm_dev": (_INT, [_P, _P, _I64, _I64, _P, _P, _F, _P]),
}

_lib = None


class PfrError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"[pfr {code}] {msg}")
        self.code = code


class InvalidArgument(PfrError, ValueError):
    pass


class Unsupported(PfrError):
    pass


class NoDevice(PfrError):
    pass


def header_functions(path=HEADER):
    """Names of the functions declared in the public header."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pfr_[a-z0-9_]+)\s*\(", text)))


def _share_torch_runtime():
    """torch ships its own libamdhip64 (SONAME libamdhip64.so.7) but asks for
    it as "libamdhip64.so", so a process that loads /opt/rocm's runtime first
    and torch second ends up with two HIP runtimes and torch sees no GPU.
    Loading torch first makes this library's libamdhip64.so.7 dependency bind
    to the copy already in the process: one runtime, shared by both."""
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def load(path=ROCM_SO):
    global _lib
    if _lib is None:
        _share_torch_runtime()
        if not os.path.exists(path):
            raise RuntimeError(
                f"gfx950 kernel library not built: {path} is missing "
                "(run __graft_entry__.build()); there is no CPU fallback")
        L = C.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc):
    if rc == PFR_OK:
        return
    msg = load().pfr_last_error().decode(errors="replace")
    cls = {PFR_ERR_INVALID_ARG: InvalidArgument, PFR_ERR_UNSUPPORTED: Unsupported,
           PFR_ERR_NO_DEVICE: NoDevice}.get(rc, PfrError)
    raise cls(rc, msg)
