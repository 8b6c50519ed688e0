"""CPU checks of the C ABI library: it loads, exports every function the
public header declares, and rejects bad arguments before touching a device."""
import ctypes as C
import os

import numpy as np
import pytest

from pyflamert_amd import _lib


def test_library_exports_every_header_symbol():
    L = _lib.load()
    names = _lib.header_functions()
    assert "pfr_spmm_csr" in names and "pfr_gemm_csr_dev" in names
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    # the ctypes table covers exactly the header
    assert sorted(_lib.SIGNATURES) == names


def test_null_context_is_an_argument_error():
    L = _lib.load()
    h = C.c_void_p()
    ip = np.zeros(2, np.int64)
    rc = L.pfr_csr_upload(None, 1, 1, 0, ip.ctypes.data_as(C.c_void_p), None, None,
                          _lib.PFR_F32, None, C.byref(h))
    assert rc == _lib.PFR_ERR_INVALID_ARG
    assert "null context" in L.pfr_last_error().decode()
    with pytest.raises(_lib.InvalidArgument):
        _lib.check(rc)


def test_init_without_device_reports_no_device():
    L = _lib.load()
    n = C.c_int(-1)
    assert L.pfr_device_count(C.byref(n)) == _lib.PFR_OK
    if n.value > 0:
        pytest.skip("a device is visible")
    h = C.c_void_p()
    assert L.pfr_rocm_init(0, C.byref(h)) == _lib.PFR_ERR_NO_DEVICE
    assert not h.value


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        _lib._lib = None
        try:
            _lib.load(str(tmp_path / "nope.so"))
        finally:
            _lib._lib = None
            _lib.load()


def test_product_does_not_import_oracle():
    """The product never links, loads or imports the checker."""
    import re

    pat = re.compile(r"\b(from|import)\s+oracle\b|pfr_oracle|libpfr_ref|oracle/")
    root = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "pyflamert_amd")
    for dirpath, _, files in os.walk(root):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".hpp", ".h", "Makefile")):
                text = open(os.path.join(dirpath, f), errors="replace").read()
                assert not pat.search(text), os.path.join(dirpath, f)
