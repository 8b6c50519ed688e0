"""The allocation-free Gemm entry (pfr_gemm_csr_act_noalloc_dev) against
the allocating one (pfr_gemm_csr_act_dev), through the C ABI: bit-identical
outputs on two calls in a row, the second with a smaller activation, in the
forms that stage op(A)^T in the workspace (transA = 0, and transA = 1 with
alpha != 1) and the one that reads A directly; strict results also equal the
oracle's.  Sizes beyond the workspace are refused before anything runs."""
import sys

import numpy as np
import pytest

from oracle import oracle as O
from pyflamert_amd import _lib

pytestmark = pytest.mark.gpu

WORKSPACE_FLOATS = 1 << 22


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_noalloc_gemm_matches_allocating_entry():
    import torch

    from pyflamert_amd import rocm

    ctx = rocm.Context(0)
    rng = np.random.default_rng(31)
    K, Nf = 768, 3072
    w = (rng.standard_normal((Nf, K)) * 0.02).astype(np.float32)
    w[rng.random(w.shape) < 0.8] = 0
    BT = ctx.csr_from_dense(w)  # Gemm transB = 1: op(B)^T is w
    bias = (rng.standard_normal(Nf) * 0.1).astype(np.float32)
    dC = torch.from_numpy(bias).cuda()
    for Mb in (1024, 96):  # the second call is smaller than the first
        A = rng.standard_normal((Mb, K)).astype(np.float32)
        dA = torch.from_numpy(A).cuda()
        dAt = torch.from_numpy(np.ascontiguousarray(A.T)).cuda()
        dY0 = torch.empty((Mb, Nf), dtype=torch.float32, device="cuda")
        dY1 = torch.full((Mb, Nf), 7.0, dtype=torch.float32, device="cuda")
        cases = [("transA 0, strict", dA, False, 1.0, "strict", {}),
                 ("transA 0, fast, Gelu", dA, False, 1.0, "fast", {"gelu": True}),
                 ("transA 1, alpha 0.5, strict, Relu", dAt, True, 0.5, "strict", {"relu": True}),
                 ("transA 1, alpha 1, strict", dAt, True, 1.0, "strict", {})]
        for name, src, ta, alpha, mode, act in cases:
            say(f"no-alloc Gemm Mb={Mb} K={K} Nf={Nf}: {name}")
            ctx.gemm_csr_dev(src.data_ptr(), Mb, K, BT, dY0.data_ptr(), alpha, 1.0, dC.data_ptr(), Nf,
                             transA=ta, mode=mode, **act)
            ctx.gemm_csr_dev(src.data_ptr(), Mb, K, BT, dY1.data_ptr(), alpha, 1.0, dC.data_ptr(), Nf,
                             transA=ta, mode=mode, noalloc=True, **act)
            ctx.synchronize()
            y0, y1 = dY0.cpu().numpy(), dY1.cpu().numpy()
            assert bits_equal(y1, y0), (Mb, name)
            if mode == "strict" and not act and Mb <= 96:
                assert bits_equal(y1, O.orc_gemm(A, w, bias, alpha, 1.0, transB=1)), (Mb, name)
    BT.free()
    ctx.close()


def test_noalloc_gemm_allocates_nothing():
    """On a fresh context whose grow-only buffers are still empty, the first
    call is the allocation-free entry in a form that stages op(A)^T
    (transA = 0, 1024 x 768: 3 MiB): device free memory is the same before
    and after it.  Were the staging to go through the context's grow-only
    buffer instead of the fixed workspace, this call would allocate it.  A
    warm-up call on another context loads the kernels first."""
    import torch

    from pyflamert_amd import rocm

    rng = np.random.default_rng(32)
    K, Nf, Mb = 768, 3072, 1024
    w = (rng.standard_normal((Nf, K)) * 0.02).astype(np.float32)
    w[rng.random(w.shape) < 0.8] = 0
    A = rng.standard_normal((Mb, K)).astype(np.float32)
    dA = torch.from_numpy(A).cuda()
    dY = torch.empty((Mb, Nf), dtype=torch.float32, device="cuda")
    dY2 = torch.empty((Mb, Nf), dtype=torch.float32, device="cuda")
    warm = rocm.Context(0)
    BTw = warm.csr_from_dense(w)
    warm.gemm_csr_dev(dA.data_ptr(), Mb, K, BTw, dY2.data_ptr(), noalloc=True)
    warm.synchronize()
    ctx = rocm.Context(0)
    BT = ctx.csr_from_dense(w)
    ctx.synchronize()
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    say(f"no-alloc Gemm on a fresh context, Mb={Mb} K={K}: device free memory {free0}")
    ctx.gemm_csr_dev(dA.data_ptr(), Mb, K, BT, dY.data_ptr(), noalloc=True)
    ctx.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0, (free0, free1)
    assert bits_equal(dY.cpu().numpy(), dY2.cpu().numpy())
    for W_, c in ((BT, ctx), (BTw, warm)):
        W_.free()
        c.close()


def test_noalloc_gemm_rejects_oversize():
    """K * Mb above the workspace is an argument error raised on the host,
    before any kernel is enqueued (the buffers here hold only what a valid
    call would read: A is never read)."""
    import torch

    from pyflamert_amd import rocm

    ctx = rocm.Context(0)
    K = 4096
    Mb = WORKSPACE_FLOATS // K + 1
    w = np.zeros((8, K), np.float32)
    w[:, ::64] = 1.0
    BT = ctx.csr_from_dense(w)
    dA = torch.zeros(16, dtype=torch.float32, device="cuda")
    dY = torch.zeros(16, dtype=torch.float32, device="cuda")
    say(f"no-alloc Gemm K={K} Mb={Mb}: refused")
    with pytest.raises(_lib.InvalidArgument, match="workspace"):
        ctx.gemm_csr_dev(dA.data_ptr(), Mb, K, BT, dY.data_ptr(), noalloc=True)
    with pytest.raises(_lib.InvalidArgument, match="workspace"):
        ctx.gemm_csr_dev(dA.data_ptr(), Mb, K, BT, dY.data_ptr(), alpha=2.0, transA=True, noalloc=True)
    ctx.synchronize()
    BT.free()
    ctx.close()
