"""The dense kernels' semantics on the GPU: the strict dense product used
for weights above the density gate (pfr_gemm_dense_dev), the non-finite
fix-up of CSR weights that stand for dense initializers
(pfr_csr_dense_semantics), and sessions that route float32 initializers
through the gate.

Bar: finite results bit-exact against the oracle's cpu_gemm / cpu_matmul
(math.cpp:268-438) on the zero-filled weight; with inf and NaN in the
activations or the weight, NaN exactly where the oracle (and, where it is
built, the compiled reference op) has NaN and the other bits equal (a NaN's
sign is not compared: the GPU's default NaN is positive, x86's negative).
Fast mode: the same NaN and inf positions, finite values normwise 1e-5.
"""
import sys

import numpy as np
import pytest

from oracle import oracle as O
from pyflamert_amd import _lib, pfm, session

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def same_or_nan(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    if a.shape != b.shape or not np.array_equal(np.isnan(a), np.isnan(b)):
        return False
    ok = ~np.isnan(a)
    return np.array_equal(bits(a[ok]), bits(b[ok]))


def close_fast(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    if not np.array_equal(np.isnan(a), np.isnan(b)):
        return False
    inf = np.isinf(b)
    if not np.array_equal(a[inf], b[inf]):
        return False
    ok = np.isfinite(b)
    return not ok.any() or np.abs(a[ok] - b[ok]).max() <= 1e-5 * np.abs(b[ok]).max()


@pytest.fixture(scope="module")
def ctx():
    from pyflamert_amd import rocm

    c = rocm.Context(0)
    yield c
    c.close()


def poison(rng, x, frac_inf=0.002, frac_nan=0.001):
    x = x.copy()
    x[rng.random(x.shape) < frac_inf] = np.inf
    x[rng.random(x.shape) < frac_inf] = -np.inf
    x[rng.random(x.shape) < frac_nan] = np.nan
    return x


def pruned(rng, shape, keep):
    w = (rng.standard_normal(shape) * 0.1).astype(np.float32)
    w[rng.random(shape) >= keep] = 0.0
    return w


@pytest.mark.parametrize("M,K,N", [(1, 1, 1), (7, 13, 5), (64, 64, 64), (100, 300, 70), (257, 1000, 129),
                                   (1024, 768, 512)])
def test_gemm_dense_dev_bit_exact(ctx, M, K, N):
    """alpha, beta, a bias broadcast by the flat-index modulo, transA, the
    fused Relu; inf and NaN on both sides."""
    import torch

    rng = np.random.default_rng(M * 3 + K)
    for ta in (0, 1):
        for alpha, beta, csz, act in ((1.0, 1.0, 0, 0), (0.5, 2.0, N, 0), (-3.0, 0.25, 7, _lib.ACT_RELU)):
            A = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
            B = pruned(rng, (K, N), 0.6)
            if M * K > 100:
                A = poison(rng, A)
                B = poison(rng, B, 0.0005, 0.0002)
            Cb = rng.standard_normal(csz).astype(np.float32) if csz else None
            say(f"dense gemm M={M} K={K} N={N} transA={ta} alpha={alpha} c_size={csz} act={act}")
            R = O.orc_gemm(A, B, Cb, alpha, beta, ta, 0)
            if act == _lib.ACT_RELU:
                R = O.orc_relu(R)
            dA, dB = torch.from_numpy(A).cuda(), torch.from_numpy(B).cuda()
            dC = torch.from_numpy(Cb).cuda() if csz else None
            dY = torch.empty((M, N), dtype=torch.float32, device="cuda")
            torch.cuda.synchronize()
            ctx.gemm_dense_dev(dA.data_ptr(), M, K, dB.data_ptr(), N, dY.data_ptr(), transA=ta, alpha=alpha,
                               beta=beta, C_ptr=dC.data_ptr() if csz else None, c_size=csz,
                               relu=act == _lib.ACT_RELU)
            ctx.synchronize()
            assert same_or_nan(dY.cpu().numpy(), R), (ta, alpha, csz, act)


def test_gemm_dense_dev_against_compiled_reference(ctx):
    """The same product against the reference's own Gemm op, non-finite
    values included (where the compiled reference is present)."""
    import torch

    if not O.have_ref():
        pytest.skip("compiled reference not built")
    rng = np.random.default_rng(5)
    M, K, N = 40, 96, 33
    A = poison(rng, rng.standard_normal((M, K)).astype(np.float32), 0.01, 0.005)
    B = pruned(rng, (N, K), 0.3)
    Cb = rng.standard_normal(N).astype(np.float32)
    R = O.ref_op_f32("Gemm", [A, B, Cb], {"alpha": 0.75, "beta": 1.5}, {"transA": 0, "transB": 1})
    Bt = np.ascontiguousarray(B.T)
    dA, dB, dC = (torch.from_numpy(v).cuda() for v in (A, Bt, Cb))
    dY = torch.empty((M, N), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    ctx.gemm_dense_dev(dA.data_ptr(), M, K, dB.data_ptr(), N, dY.data_ptr(), alpha=0.75, beta=1.5,
                       C_ptr=dC.data_ptr(), c_size=N)
    ctx.synchronize()
    assert same_or_nan(dY.cpu().numpy(), R)


@pytest.mark.parametrize("N", [1, 3, 8, 64])
def test_csr_dense_semantics_spmm(ctx, N):
    """Y = W . X with W 80 % zeros as a CSR and inf / NaN in X: with the
    dense semantics on, every output equals cpu_matmul on the zero-filled W
    (strict: bits; fast: NaN and inf positions, finite values normwise);
    without them, inf meeting a pruned weight is skipped (the sparse rule),
    which the check detects."""
    rng = np.random.default_rng(N)
    M, K = 300, 700
    W = pruned(rng, (M, K), 0.2)
    X = rng.standard_normal((K, N)).astype(np.float32)
    X[5, 0] = np.inf          # meets the zeros of column 5: NaN in most rows of column 0
    X[9, N - 1] = -np.inf
    if N > 1:
        X[20, 1] = np.nan     # column 1 is NaN in every row
    R = O.orc_matmul(W, X)
    ip, ix, v = O.orc_to_sparse_csr(W)
    plain = ctx.csr_upload(M, K, ip, ix, v)
    Yp = plain.spmm(X).reshape(M, N)
    assert not same_or_nan(Yp, R)  # the sparse rule differs here
    Wd = ctx.csr_upload(M, K, ip, ix, v).dense_semantics()
    say(f"dense semantics spmm N={N}")
    assert same_or_nan(Wd.spmm(X).reshape(M, N), R)
    assert close_fast(Wd.spmm(X, mode="fast").reshape(M, N), R)
    # finite X: unchanged by the fix-up
    Xf = rng.standard_normal((K, N)).astype(np.float32)
    assert np.array_equal(bits(Wd.spmm(Xf)), bits(plain.spmm(Xf)))
    plain.free()
    Wd.free()


def test_csr_dense_semantics_gemm(ctx):
    """The Gemm form (A activations, pruned B) with transA, alpha, bias and
    the fused Relu / Gelu: outputs NaN (then Relu's +0) where cpu_gemm has
    NaN."""
    import torch

    rng = np.random.default_rng(17)
    Mb, K, Nf = 50, 300, 90
    B = pruned(rng, (K, Nf), 0.25)
    BT = ctx.csr_from_dense(B, transpose=True).dense_semantics()
    bias = rng.standard_normal(Nf).astype(np.float32)
    for ta in (0, 1):
        A = rng.standard_normal((K, Mb) if ta else (Mb, K)).astype(np.float32)
        A = poison(rng, A, 0.003, 0.001)
        for alpha in (1.0, 0.5):
            R = O.orc_gemm(A, B, bias, alpha, 1.0, ta, 0)
            say(f"dense semantics gemm transA={ta} alpha={alpha}")
            assert same_or_nan(ctx.gemm_csr(A, BT, alpha, 1.0, bias, transA=bool(ta)), R)
            dA, dC = torch.from_numpy(A).cuda(), torch.from_numpy(bias).cuda()
            dY = torch.empty((Mb, Nf), dtype=torch.float32, device="cuda")
            torch.cuda.synchronize()
            ctx.gemm_csr_dev(dA.data_ptr(), Mb, K, BT, dY.data_ptr(), alpha, 1.0, dC.data_ptr(), Nf,
                             transA=bool(ta), relu=True)
            ctx.synchronize()
            assert same_or_nan(dY.cpu().numpy(), O.orc_relu(R))
    BT.free()


def session_model(tmp_path, name, nodes, inits, inputs, outputs):
    m = {"name": name, "inputs": inputs, "outputs": outputs, "initializers": inits, "nodes": nodes}
    p = str(tmp_path / (name + ".pfm"))
    pfm.save(m, p)
    return p


@pytest.mark.parametrize("keep", [0.2, 0.8])
def test_session_density_gate(tmp_path, keep):
    """Gemm(x, W1, b) -> Relu -> MatMul(., W2) and MatMul(W3, x2) with the
    weights at density `keep`: 0.2 goes to CSR with the dense semantics, 0.8
    to the dense product.  Finite inputs: bit-exact against the oracle's
    dense kernels; inf / NaN inputs and a NaN weight: NaN where they have
    it; all three optimization levels agree."""
    rng = np.random.default_rng(int(keep * 10))
    T, H, F = 16, 96, 80
    W1 = pruned(rng, (F, H), keep)       # Gemm transB = 1: [F, H]
    b1 = rng.standard_normal(F).astype(np.float32)
    W2 = pruned(rng, (F, 48), keep)
    W3 = pruned(rng, (24, H), keep)
    W2[3, 7] = np.nan                   # a NaN weight: the dense kernel spreads it to column 7
    nodes = [("g", "Gemm", ["x", "w1", "b1"], ["h"], {"transB": 1}),
             ("r", "Relu", ["h"], ["a"], {}),
             ("m", "MatMul", ["a", "w2"], ["y"], {}),
             ("m3", "MatMul", ["w3", "x2"], ["z"], {})]
    p = session_model(tmp_path, f"gate{keep}", nodes, {"w1": W1, "b1": b1, "w2": W2, "w3": W3},
                      [("x", 0, [T, H]), ("x2", 0, [H, 5])], [("y", 0, [T, 48]), ("z", 0, [24, 5])])
    x = rng.standard_normal((T, H)).astype(np.float32)
    x2 = rng.standard_normal((H, 5)).astype(np.float32)
    xb, x2b = poison(rng, x, 0.01, 0.003), poison(rng, x2, 0.01, 0.003)
    xb[2, 0] = np.inf
    x2b[0, 1] = np.nan
    runs = []
    for lvl in (2, 1, 0):
        s = session.InferenceSession(p, session.SessionOptions(optimization_level=lvl))
        say(f"density gate keep={keep} level={lvl}")
        for feed_x, feed_x2 in ((x, x2), (xb, x2b)):
            y, z = s.run(None, {"x": feed_x, "x2": feed_x2})
            Ry = O.orc_matmul(O.orc_relu(O.orc_gemm(feed_x, W1, b1, 1.0, 1.0, 0, 1)), W2)
            Rz = O.orc_matmul(W3, feed_x2)
            assert same_or_nan(y, Ry), lvl
            assert same_or_nan(z, Rz), lvl
            runs.append((y, z))
        forms = s.weight_forms()
        assert forms == ({"csr": 3, "dense": 0, "sp24": 0} if keep < 0.5 else {"csr": 0, "dense": 3, "sp24": 0})
    for i in range(2, len(runs)):  # every level gives the same results per feed
        assert same_or_nan(runs[i][0], runs[i % 2][0]) and same_or_nan(runs[i][1], runs[i % 2][1]), i
    if O.have_ref():  # the reference's own ops on the non-finite inputs
        h = O.ref_op_f32("Gemm", [xb, W1, b1], {}, {"transB": 1})
        y_ref = O.ref_op_f32("MatMul", [O.ref_op_f32("Relu", [h]), W2])
        assert same_or_nan(runs[1][0], y_ref)
        assert same_or_nan(runs[1][1], O.ref_op_f32("MatMul", [W3, x2b]))
