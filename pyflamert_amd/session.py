"""InferenceSession over the C++ runtime (include/pfr_session.h), with the
Python surface of the reference package (python/pyflame_rt/__init__.py:
InferenceSession(path, options).run(output_names, input_feed) -> list of
numpy arrays; get_inputs/get_outputs/get_providers).  The backend is the
MI355X one: SessionOptions(device="rocm").
"""
from __future__ import annotations

import ctypes as C
import json
import os
from dataclasses import dataclass

import numpy as np

from . import _lib

# PFR_RUNTIME_LIB selects another build of the host runtime (the
# AddressSanitizer/UBSan one, `make -C pyflamert_amd/csrc sanitize`).
RT_SO = os.environ.get("PFR_RUNTIME_LIB") or os.path.join(_lib.LIB_DIR, "libpyflamert.so")

_P = C.c_void_p
_I64 = C.c_int64
_INT = C.c_int
_SIGS = {
    "pfr_session_last_error": (C.c_char_p, []),
    "pfr_session_create": (_INT, [C.c_char_p, C.c_char_p, _INT, _INT, _INT, _INT, C.c_char_p, C.POINTER(_P)]),
    "pfr_session_destroy": (_INT, [_P]),
    "pfr_session_io_count": (_INT, [_P, C.POINTER(_INT), C.POINTER(_INT)]),
    "pfr_session_io_info": (_INT, [_P, _INT, _INT, C.POINTER(C.c_char_p), C.POINTER(_INT), _P, C.POINTER(_INT)]),
    "pfr_session_run": (_INT, [_P, _INT, _P, _P, _P, _P, _P, _INT, _P, C.POINTER(_INT)]),
    "pfr_session_result": (_INT, [_P, _INT, C.POINTER(_INT), _P, C.POINTER(_INT), C.POINTER(_P)]),
    "pfr_session_supported_ops": (_INT, [_P, C.c_char_p, _I64]),
    "pfr_session_device_plan": (_INT, [_P, C.POINTER(_INT), C.POINTER(_INT)]),
    "pfr_session_weight_forms": (_INT, [_P, C.POINTER(_INT), C.POINTER(_INT), C.POINTER(_INT)]),
    "pfr_model_describe": (_INT, [C.c_char_p, C.c_char_p, _I64, C.POINTER(_I64)]),
    "pfr_model_resave": (_INT, [C.c_char_p, C.c_char_p]),
    "pfr_model_quantize": (_INT, [C.c_char_p, C.c_char_p, C.c_char_p, C.POINTER(_INT)]),
}
_DT = {0: np.float32, 1: np.float16, 2: np.uint16, 3: np.float64, 4: np.int64, 5: np.int32, 6: np.int16,
       7: np.int8, 8: np.uint8, 9: np.bool_}
_CODE = {np.dtype(v): k for k, v in _DT.items() if k != 2}
_rt = None


class PyFlameRTError(RuntimeError):
    status = 15


class InvalidModelError(PyFlameRTError):
    status = 10


class ValidationError(PyFlameRTError):
    status = 11


class UnsupportedOperatorError(PyFlameRTError):
    status = 12


class InputError(PyFlameRTError):
    status = 13


class BackendError(PyFlameRTError):
    status = 14


class UnsupportedFormatError(PyFlameRTError):
    status = 16


_BY_STATUS = {c.status: c for c in (PyFlameRTError, InvalidModelError, ValidationError, UnsupportedOperatorError,
                                    InputError, BackendError, UnsupportedFormatError)}


def runtime():
    global _rt
    if _rt is None:
        _lib.load()  # kernel library (and torch's HIP runtime first, if present)
        if not os.path.exists(RT_SO):
            raise RuntimeError(f"runtime library not built: {RT_SO} (run __graft_entry__.build())")
        L = C.CDLL(RT_SO)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _rt = L
    return _rt


def _check(rc):
    if rc:
        raise _BY_STATUS.get(rc, PyFlameRTError)(runtime().pfr_session_last_error().decode(errors="replace"))


@dataclass
class SessionOptions:
    device: str = "rocm"
    strict_math_mode: bool = False
    math_mode: str = "strict"    # "strict": bit-exact fp32 sums; "fast": FMA
    device_id: int = 0
    # OptLevel (types.hpp:119-124): 0 None = node by node through the host
    # OpFuncs, 1 Basic = device-resident plan, 2 Extended (default) and 3 All
    # = plan + Relu fused into the pruned product before it
    optimization_level: int = 2
    # "" or "dynamic_int8": 2:4-pruned MatMul(W, X) nodes run as
    # DynamicQuantizeLinear + per-channel int8 QuantizedMatMul
    quantization: str = ""


@dataclass
class NodeArg:
    name: str
    shape: list
    type: str


def describe_model(path):
    """Summary of a .pfm as loaded and validated by the C++ runtime."""
    need = _I64(0)
    _check(runtime().pfr_model_describe(path.encode(), None, 0, C.byref(need)))
    buf = C.create_string_buffer(need.value)
    _check(runtime().pfr_model_describe(path.encode(), buf, need.value, C.byref(need)))
    return json.loads(buf.value.decode())


def resave_model(src, dst):
    _check(runtime().pfr_model_resave(src.encode(), dst.encode()))


def quantize_model(src, dst, mode="dynamic_int8"):
    """The session's quantization rewrite applied offline; returns the number
    of MatMul nodes replaced."""
    n = _INT(0)
    _check(runtime().pfr_model_quantize(src.encode(), dst.encode(), mode.encode(), C.byref(n)))
    return n.value


class InferenceSession:
    def __init__(self, model_path, options=None, providers=None):
        options = options or SessionOptions()
        L = runtime()
        h = _P()
        mode = {"strict": 0, "fast": 1}[options.math_mode]
        _check(L.pfr_session_create(str(model_path).encode(), options.device.encode(),
                                    int(options.strict_math_mode), mode, options.device_id,
                                    int(options.optimization_level), (options.quantization or "").encode(),
                                    C.byref(h)))
        self._h = h
        self._L = L

    def close(self):
        if getattr(self, "_h", None):
            self._L.pfr_session_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _io(self, is_output):
        ni, no = _INT(), _INT()
        _check(self._L.pfr_session_io_count(self._h, C.byref(ni), C.byref(no)))
        out = []
        for i in range(no.value if is_output else ni.value):
            name, dt, nd = C.c_char_p(), _INT(), _INT()
            shape = (C.c_int64 * 16)()
            _check(self._L.pfr_session_io_info(self._h, int(is_output), i, C.byref(name), C.byref(dt), shape,
                                               C.byref(nd)))
            dims = [None if shape[d] < 0 else shape[d] for d in range(nd.value)]
            out.append(NodeArg(name.value.decode(), dims, f"tensor({np.dtype(_DT[dt.value]).name})"))
        return out

    def get_inputs(self):
        return self._io(False)

    def get_outputs(self):
        return self._io(True)

    def get_providers(self):
        return ["ROCMExecutionProvider"]

    def supported_ops(self):
        buf = C.create_string_buffer(1 << 16)
        _check(self._L.pfr_session_supported_ops(self._h, buf, len(buf)))
        lines = buf.value.decode().split("\n")
        return lines[0], lines[1:]

    def weight_forms(self):
        """{"csr": n, "dense": n, "sp24": n}: the device form of each prepared
        weight (float32 initializers at most half nonzero and CSR records go
        to CSR, denser ones to the dense product)."""
        a, b, c = C.c_int(), C.c_int(), C.c_int()
        _check(self._L.pfr_session_weight_forms(self._h, C.byref(a), C.byref(b), C.byref(c)))
        return {"csr": a.value, "dense": b.value, "sp24": c.value}

    def device_plan(self):
        """(device_resident, kernel_steps) of the last run: whether the graph
        ran with activations kept on the GPU (Relu fused into a product that
        feeds only it), and how many launches that plan makes."""
        res, steps = C.c_int(), C.c_int()
        _check(self._L.pfr_session_device_plan(self._h, C.byref(res), C.byref(steps)))
        return bool(res.value), steps.value

    def run(self, output_names, input_feed):
        names = list(input_feed)
        arrs = [np.ascontiguousarray(input_feed[n]) for n in names]
        n = len(arrs)
        c_names = (C.c_char_p * n)(*[s.encode() for s in names])
        c_data = (C.c_void_p * n)(*[a.ctypes.data for a in arrs])
        c_dt = (C.c_int * n)(*[_CODE[a.dtype] for a in arrs])
        shapes = [np.array(a.shape, np.int64) for a in arrs]
        c_shapes = (C.c_void_p * n)(*[s.ctypes.data for s in shapes])
        c_nd = (C.c_int * n)(*[a.ndim for a in arrs])
        outs = list(output_names or [])
        c_outs = (C.c_char_p * max(1, len(outs)))(*[s.encode() for s in outs])
        nres = _INT()
        _check(self._L.pfr_session_run(self._h, n, c_names, c_data, c_dt, c_shapes, c_nd, len(outs), c_outs,
                                       C.byref(nres)))
        results = []
        for i in range(nres.value):
            dt, nd, ptr = _INT(), _INT(), _P()
            shape = (C.c_int64 * 16)()
            _check(self._L.pfr_session_result(self._h, i, C.byref(dt), shape, C.byref(nd), C.byref(ptr)))
            shp = tuple(shape[d] for d in range(nd.value))
            npdt = np.dtype(_DT[dt.value])
            count = int(np.prod(shp)) if shp else 0
            buf = (C.c_char * (count * npdt.itemsize)).from_address(ptr.value) if count else b""
            results.append(np.frombuffer(bytes(buf), npdt).reshape(shp).copy())
        return results
