"""GPU parity of the device-side prune -> compress chain: apply_mask
(sparse_tensor.cpp:616-631), the CSR of a dense device weight
(to_sparse, sparse_tensor.cpp:560-610, built on the device with the mask
applied on the way) and the 2:4 pack of a device weight.

Bar: apply_mask bit-exact against the oracle (special values included).  A
device-built CSR handle must equal the host-built one for the same weight:
same nnz, and bit-identical products in every kernel family that reads it
(strict N = 1 row chains, strict N = 3 and 8, strict N = 64 column slices,
fast N = 1 and 8 over the balanced copy, whose sums depend on the exact
record placement), and strict products bit-exact against the oracle's
to_sparse + sparse_matmul.  A device-packed 2:4 weight must give the same
GEMM bits as the host-packed one and raise the same error for a weight that
is not 2:4.
"""
import sys

import numpy as np
import pytest

from oracle import oracle as O
from pyflamert_amd import _lib

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def same(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(bits(a), bits(b))


def same_or_nan(a, b):
    """Bits equal, except that a NaN matches any NaN (the device's default
    NaN and x86's differ in sign)."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    if a.shape != b.shape or not np.array_equal(np.isnan(a), np.isnan(b)):
        return False
    ok = ~np.isnan(a)
    return np.array_equal(bits(a[ok]), bits(b[ok]))


@pytest.fixture(scope="module")
def ctx():
    from pyflamert_amd import rocm

    c = rocm.Context(0)
    yield c
    c.close()


def specials(rng, n):
    v = rng.standard_normal(n).astype(np.float32)
    pick = rng.random(n)
    v[pick < 0.02] = np.nan
    v[(pick >= 0.02) & (pick < 0.04)] = np.inf
    v[(pick >= 0.04) & (pick < 0.06)] = -np.inf
    v[(pick >= 0.06) & (pick < 0.10)] = -0.0
    v[(pick >= 0.10) & (pick < 0.20)] = 0.0
    return v


@pytest.mark.parametrize("n", [1, 3, 4, 257, 4096, 100003])
def test_apply_mask(ctx, n):
    """w * mask with NaN, +-inf, +-0 in the weight and 0 / 1 / fractional /
    negative / NaN mask entries; host, device, unaligned and in-place."""
    import torch

    rng = np.random.default_rng(n)
    w = specials(rng, n)
    m = np.where(rng.random(n) < 0.5, 0.0, 1.0).astype(np.float32)
    m[rng.random(n) < 0.05] = 0.5
    m[rng.random(n) < 0.05] = -1.0
    m[rng.random(n) < 0.01] = np.nan
    say(f"apply_mask n={n}")
    want = O.orc_apply_mask(w, m)
    assert same(ctx.apply_mask(w, m), want)
    wp = np.concatenate([[7.0], w]).astype(np.float32)  # one leading float: [1:] is not 16-byte aligned
    mp = np.concatenate([[3.0], m]).astype(np.float32)
    dw, dm = torch.from_numpy(wp).cuda(), torch.from_numpy(mp).cuda()
    out = torch.empty(n + 1, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    ctx.apply_mask_dev(dw.data_ptr(), dm.data_ptr(), n + 1, out.data_ptr())  # aligned: 16-byte path
    ctx.synchronize()
    assert same(out.cpu().numpy(), O.orc_apply_mask(wp, mp))
    ctx.apply_mask_dev(dw.data_ptr() + 4, dm.data_ptr() + 4, n, out.data_ptr() + 4)  # unaligned
    ctx.synchronize()
    assert same(out.cpu().numpy()[1:], want)
    ctx.apply_mask_dev(dw.data_ptr() + 4, dm.data_ptr() + 4, n, dw.data_ptr() + 4)  # in place
    ctx.synchronize()
    assert same(dw.cpu().numpy()[1:], want)


def products(W, rng, K):
    """Every kernel family's output for one handle (strict and fast)."""
    out = {}
    x = rng.standard_normal(K).astype(np.float32)
    X3 = rng.standard_normal((K, 3)).astype(np.float32)
    X8 = rng.standard_normal((K, 8)).astype(np.float32)
    X64 = rng.standard_normal((K, 64)).astype(np.float32)
    for mode in ("strict", "fast"):
        out[("1", mode)] = W.spmm(x, mode=mode)
        out[("8", mode)] = W.spmm(X8, mode=mode)
    out[("3", "strict")] = W.spmm(X3, mode="strict")
    out[("64", "strict")] = W.spmm(X64, mode="strict")
    return out, {"1": x, "3": X3, "8": X8, "64": X64}


def weight(rng, rows, cols, dens, kind):
    w = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
    w[rng.random(w.shape) >= dens] = 0.0
    if kind == "skewed":  # lognormal row lengths, a few empty rows, one full row
        keep = rng.lognormal(0.0, 0.8, rows)
        keep = keep / keep.mean() * dens
        for r in range(rows):
            w[r, rng.random(cols) >= min(keep[r], 1.0)] = 0.0
        w[::17] = 0.0
        w[3] = (rng.standard_normal(cols) * 0.05).astype(np.float32)
    if kind == "special":  # NaN is never kept (|NaN| > t fails), inf is
        w[0, :5] = [np.nan, np.inf, -np.inf, -0.0, 1e-30]
    return w


CASES = [  # rows, cols, transpose, density, kind, threshold, masked
    (300, 700, False, 0.3, "plain", 0.0, False),
    (1000, 3000, False, 0.2, "skewed", 0.0, False),
    (700, 6000, False, 0.1, "skewed", 0.0, True),
    (4096, 600, True, 0.15, "plain", 0.02, False),
    (3000, 900, True, 0.2, "skewed", 0.0, True),
    (120, 20000, False, 0.05, "plain", 0.0, False),
    (1, 4097, False, 0.5, "special", 0.0, False),
    (64, 64, False, 0.0, "plain", 0.0, False),
    (50, 33, False, 0.9, "special", 0.0, True),
]


@pytest.mark.parametrize("rows,cols,transpose,dens,kind,thr,masked", CASES)
def test_csr_from_dense_dev_equals_host_build(ctx, rows, cols, transpose, dens, kind, thr, masked):
    import torch

    rng = np.random.default_rng(rows * 31 + cols)
    w = weight(rng, rows, cols, dens, kind)
    mask = O.orc_magnitude_mask(np.nan_to_num(w).ravel(), 0.5).reshape(rows, cols) if masked else None
    wm = O.orc_apply_mask(w, mask) if masked else w
    say(f"csr_from_dense_dev {rows}x{cols} transpose={transpose} {kind} thr={thr} mask={masked}")
    host = ctx.csr_from_dense(wm, transpose=transpose, threshold=thr)
    dw = torch.from_numpy(w).cuda()
    dm = torch.from_numpy(mask).cuda() if masked else None
    torch.cuda.synchronize()
    dev = ctx.csr_from_dense_dev(dw.data_ptr(), rows, cols, transpose=transpose, threshold=thr,
                                 mask_ptr=dm.data_ptr() if masked else None)
    assert (dev.M, dev.K, dev.nnz) == (host.M, host.K, host.nnz)
    op = np.ascontiguousarray(wm.T if transpose else wm)
    ip, ix, v = O.orc_to_sparse_csr(op, thr)
    assert dev.nnz == len(v)
    if dev.nnz:
        a, xs = products(dev, np.random.default_rng(5), dev.K)
        b, _ = products(host, np.random.default_rng(5), dev.K)
        for key in a:
            assert same(a[key], b[key]), key
        for n in ("1", "3", "8", "64"):
            R = O.orc_csr_spmm(dev.M, dev.K, ip, ix, v, xs[n].reshape(dev.K, -1))
            assert same_or_nan(a[(n, "strict")].reshape(R.shape), R), n
    dev.free()
    host.free()


def test_csr_from_dense_dev_empty_and_errors(ctx):
    import torch

    d = torch.zeros(4, dtype=torch.float32, device="cuda")
    for rows, cols in ((0, 5), (5, 0), (0, 0)):
        W = ctx.csr_from_dense_dev(d.data_ptr(), rows, cols)
        assert (W.M, W.K, W.nnz) == (rows, cols, 0)
        W.free()
    with pytest.raises(_lib.PfrError):
        ctx.csr_from_dense_dev(d.data_ptr(), -1, 4)
    with pytest.raises(_lib.PfrError):
        ctx.csr_from_dense_dev(None, 4, 4)


def rand_24(rng, M, K, dtype):
    K4 = (K + 3) // 4 * 4
    w = rng.standard_normal((M, K4)).astype(np.float32)
    w = O.orc_apply_mask(w, O.orc_nm_mask(w.ravel(), 2, 4).reshape(M, K4))[:, :K]
    w[rng.random(w.shape) < 0.1] = 0.0
    w = np.ascontiguousarray(w)
    if dtype == "i8":
        s, _ = O.orc_dynamic_params_per_channel(w.reshape(1, M, K))
        return np.ascontiguousarray(O.orc_quantize(w, s, np.zeros(M, np.int32), O.I8, (1, M, K))), s
    b = O.orc_f32_to_bf16(w.ravel()).reshape(M, K)
    b[rng.random(b.shape) < 0.01] = 0x8000  # -0: a zero for the 2:4 pattern
    return b, None


@pytest.mark.parametrize("M,K", [(16, 128), (200, 300), (300, 1030), (1024, 4096)])
@pytest.mark.parametrize("dtype", ["i8", "bf16"])
def test_sp24_pack_dev_equals_host_pack(ctx, M, K, dtype):
    import torch

    rng = np.random.default_rng(M + K)
    Wq, s = rand_24(rng, M, K, dtype)
    say(f"sp24_pack_dev {dtype} M={M} K={K}")
    host = ctx.sp24_pack(Wq, s) if dtype == "i8" else ctx.sp24_pack(Wq)
    dW = torch.from_numpy(Wq.view(np.int16) if dtype == "bf16" else Wq).cuda()
    torch.cuda.synchronize()
    dev = ctx.sp24_pack_dev(dW.data_ptr(), M, K, dtype, s)
    N = 70
    if dtype == "i8":
        X = rng.integers(-128, 128, (K, N)).astype(np.int8)
        a, b = dev.gemm_i8(X, out="i32"), host.gemm_i8(X, out="i32")
        assert np.array_equal(a, b)
        assert np.array_equal(a, O.orc_int8_matmul_acc(Wq, X))
        Xq = rng.integers(0, 256, (K, N)).astype(np.uint8)  # zero point: the row sums
        assert same(dev.gemm_q(Xq, x_scale=0.02, x_zp=9), host.gemm_q(Xq, x_scale=0.02, x_zp=9))
    else:
        X = O.orc_f32_to_bf16(rng.standard_normal(K * N).astype(np.float32)).reshape(K, N)
        assert same(dev.gemm_bf16(X), host.gemm_bf16(X))
    dev.free()
    host.free()


def test_sp24_pack_dev_rejects_dense_groups(ctx):
    import torch

    rng = np.random.default_rng(3)
    Wq, s = rand_24(rng, 40, 64, "i8")
    Wq[13, 20:23] = 5  # three nonzeros in group k = 20..23 of row 13
    Wq[30, 0:4] = 1
    msgs = []
    for pack in (lambda: ctx.sp24_pack(Wq, s),
                 lambda: ctx.sp24_pack_dev(torch.from_numpy(Wq).cuda().data_ptr(), 40, 64, "i8", s)):
        with pytest.raises(_lib.PfrError) as e:
            pack()
        msgs.append(str(e.value))
    assert msgs[0] == msgs[1] and "row 13, k 20..23" in msgs[0], msgs


def test_device_prune_pipeline(ctx):
    """Weight on the device -> 2:4 mask -> apply_mask -> CSR and (int8) 2:4
    weight, never leaving the GPU: the CSR product equals the oracle's
    to_sparse(apply_mask(w, nm_mask(w))) product bit for bit, and a
    magnitude-pruned CSR built with the mask fused likewise."""
    import torch

    rng = np.random.default_rng(11)
    M, K = 512, 1024
    w = rng.standard_normal((M, K)).astype(np.float32)
    dw = torch.from_numpy(w).cuda()
    dmask = torch.empty_like(dw)
    dwm = torch.empty_like(dw)
    torch.cuda.synchronize()
    ctx.nm_mask_dev(dw.data_ptr(), M * K, 2, 4, dmask.data_ptr())
    ctx.apply_mask_dev(dw.data_ptr(), dmask.data_ptr(), M * K, dwm.data_ptr())
    W = ctx.csr_from_dense_dev(dwm.data_ptr(), M, K)
    wm = O.orc_apply_mask(w, O.orc_nm_mask(w.ravel(), 2, 4).reshape(M, K))
    ip, ix, v = O.orc_to_sparse_csr(wm)
    X = rng.standard_normal((K, 16)).astype(np.float32)
    assert same(W.spmm(X), O.orc_csr_spmm(M, K, ip, ix, v, X))
    W.free()
    ctx.magnitude_mask_dev(dw.data_ptr(), M * K, 0.8, dmask.data_ptr())
    W = ctx.csr_from_dense_dev(dw.data_ptr(), M, K, mask_ptr=dmask.data_ptr())
    wm = O.orc_apply_mask(w, O.orc_magnitude_mask(w.ravel(), 0.8).reshape(M, K))
    ip, ix, v = O.orc_to_sparse_csr(wm)
    assert W.nnz == len(v)
    assert same(W.spmm(X), O.orc_csr_spmm(M, K, ip, ix, v, X))
    W.free()
