"""GPU parity at the full workload shapes the bench times.

* Llama-2-7B-shaped decode linears: q/k/v/o 4096 x 4096, gate/up 11008 x 4096,
  down 4096 x 11008; 70 % sparsity with lognormal (sigma 0.5) row lengths,
  int8 weight-only with per-row scales; batch 1 and 8.  Strict mode is
  bit-exact against the oracle's sparse_matmul on the dequantised values
  (sparse_tensor.cpp:473-554 after dequantize_tensor, quant_ops.cpp:182-196);
  fast mode is within 1e-5 normwise.
* BERT-base linears at 1024 tokens (batch 8 x seq 128), 80 % unstructured:
  Gemm(x, W, b) with transB = 1 (cpu_gemm, math.cpp:377-438), strict,
  bit-exact; the Gelu-fused epilogue; the MatMul(x, W) form (transB = 0).
* The workgroup-per-row fast kernel (rows with a mean of >= 2048 nonzeros):
  reached by the batch-8 down projection above, by N = 1 with K >= 16384 and
  by the Gemm form with bias and fused activations; NaN and infinities in X.
"""
import sys

import numpy as np
import pytest

from oracle import oracle as O
from pyflamert_amd import workloads

from bounds import gamma_bound_ok

pytestmark = pytest.mark.gpu

DECODE = {"qkvo_4096x4096": (4096, 4096), "gate_up_11008x4096": (11008, 4096),
          "down_4096x11008": (4096, 11008)}
BERT = {"qkvo_768x768": (768, 768), "ffn_up_3072x768": (3072, 768), "ffn_down_768x3072": (768, 3072)}
T_TOKENS = 1024


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def first_diff(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    d = np.nonzero(a.view(np.uint32).ravel() != b.view(np.uint32).ravel())[0]
    return (len(d), d[:5], a.ravel()[d[:5]], b.ravel()[d[:5]]) if len(d) else None


def close_normwise(Y, R, tol=1e-5):
    """NaN exactly where R has NaN, infinities equal, finite entries within
    tol * max|R_finite| of R."""
    Y = np.asarray(Y, np.float32)
    R = np.asarray(R, np.float32)
    if not np.array_equal(np.isnan(Y), np.isnan(R)):
        return False
    inf = np.isinf(R)
    if not np.array_equal(Y[inf], R[inf]):
        return False
    ok = np.isfinite(R)
    if not ok.any():
        return True
    scale = np.abs(R[ok]).max()
    return bool(np.abs(Y[ok].astype(np.float64) - R[ok]).max() <= tol * scale)


@pytest.fixture(scope="module")
def ctx():
    from pyflamert_amd import rocm

    c = rocm.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="module", params=list(DECODE))
def decode_layer(request, ctx):
    """One decode weight at its full shape, generated as the bench does."""
    M, K = DECODE[request.param]
    ip, ix, q, sc = workloads.csr_int8_lognormal(M, K, 0.3, 0.5, 0.02, seed=M + 3 * K)
    vals = workloads.dequant_rows(ip, q, sc)
    W = ctx.csr_upload(M, K, ip, ix, q, row_scales=sc)
    yield request.param, M, K, ip, ix, vals, W
    W.free()


def test_decode_strict_bit_exact(decode_layer):
    name, M, K, ip, ix, vals, W = decode_layer
    assert W.nnz == len(vals)
    for B in (1, 8):
        say(f"decode {name} nnz={len(vals)} batch {B} strict")
        X = workloads.dense_normal((K, B), 1.0, seed=100 + B)
        Xa = X[:, 0].copy() if B == 1 else X
        Y = W.spmm(Xa, mode="strict")
        R = O.orc_csr_spmm(M, K, ip, ix, vals, Xa)
        assert bits_equal(Y, R), (name, B, first_diff(Y, R))


def test_decode_fast_normwise(decode_layer):
    """Fast mode at batch 1, 2, 5 and 8: the row-chain kernel with x in LDS
    (batch 1), X rows in LDS (K = 4096 at batch 2..8) and the wave- or
    workgroup-per-row kernel over uint16 columns (K = 11008 at batch 2..8;
    the down projection's mean row of ~3,250 nonzeros selects a workgroup
    per row).  NaN and -inf in X propagate where the oracle's do."""
    name, M, K, ip, ix, vals, W = decode_layer
    for B in (1, 2, 5, 8):
        X = workloads.dense_normal((K, B), 1.0, seed=200 + B)
        say(f"decode {name} batch {B} fast")
        Xa = X[:, 0].copy() if B == 1 else X
        assert close_normwise(W.spmm(Xa, mode="fast"), O.orc_csr_spmm(M, K, ip, ix, vals, Xa)), (name, B)
        Xb = X.copy()
        Xb[ix[3], B - 1] = np.nan
        Xb[ix[len(ix) // 2], 0] = -np.inf
        Xa = Xb[:, 0].copy() if B == 1 else Xb
        say(f"decode {name} batch {B} fast, NaN and -inf in X")
        assert close_normwise(W.spmm(Xa, mode="fast"), O.orc_csr_spmm(M, K, ip, ix, vals, Xa)), (name, B)


def test_fast_mode_forward_error_bound(ctx, decode_layer):
    """Fast mode against the error bound every summation order meets (not
    against the oracle's own order, which near cancelling rows differs from
    the exact sum by as much): batch 1, 2 and 8 at the decode shapes."""
    name, M, K, ip, ix, vals, W = decode_layer
    for B in (1, 2, 8):
        X = workloads.dense_normal((K, B), 1.0, seed=500 + B)
        Xa = X[:, 0].copy() if B == 1 else X
        say(f"decode {name} batch {B} fast, forward error bound")
        ok, worst = gamma_bound_ok(W.spmm(Xa, mode="fast"), M, K, ip, ix, vals, Xa)
        assert ok, (name, B, worst)


def elementwise_rel(Y, R):
    """The fast-mode metric of the parity contract: max over outputs of
    |y - r| / max(|r|, 1e-6 * max|r|), over finite r."""
    Y = np.asarray(Y, np.float64).ravel()
    R = np.asarray(R, np.float64).ravel()
    ok = np.isfinite(R)
    Y, R = Y[ok], R[ok]
    den = np.maximum(np.abs(R), 1e-6 * np.abs(R).max())
    i = int(np.argmax(np.abs(Y - R) / den))
    return float(np.abs(Y[i] - R[i]) / den[i]), i


def test_fast_mode_elementwise_metric(ctx, decode_layer):
    """Reports the element-wise relative error of fast mode against the
    oracle at the decode shapes, batch 1 and 8, next to the normwise error
    (asserted <= 1e-5).  The element-wise figure is not bounded by 1e-5 for
    a reassociated sum: where a row's terms cancel, the storage-order result
    itself is off the exact sum by up to gamma_n * sum|w x|, so it is
    printed (and documented), not asserted; the largest case is also
    checked against the exact float64 sum."""
    import scipy.sparse as sparse

    name, M, K, ip, ix, vals, W = decode_layer
    A = sparse.csr_matrix((np.asarray(vals, np.float64), np.asarray(ix), np.asarray(ip)), shape=(M, K))
    for B in (1, 8):
        X = workloads.dense_normal((K, B), 1.0, seed=700 + B)
        Xa = X[:, 0].copy() if B == 1 else X
        Y = W.spmm(Xa, mode="fast")
        R = O.orc_csr_spmm(M, K, ip, ix, vals, Xa)
        e, i = elementwise_rel(Y, R)
        nw = float(np.abs(Y.astype(np.float64) - R).max() / np.abs(R).max())
        exact = (A @ np.asarray(Xa, np.float64).reshape(K, -1)).ravel()
        say(f"ELEMENTWISE {name} batch {B}: elementwise {e:.3e} at output {i} (|r| = {abs(float(R.ravel()[i])):.3e}, "
            f"max|r| = {float(np.abs(R).max()):.3e}); normwise {nw:.3e}; oracle vs exact there "
            f"{abs(float(R.ravel()[i]) - exact[i]):.3e}, fast vs exact {abs(float(Y.ravel()[i]) - exact[i]):.3e}")
        assert nw <= 1e-5


def test_fast_mode_elementwise_metric_uniform(ctx):
    """The same report for the 4096 x 4096, 10 % fp32 weight at N = 256 (the
    column-slice kernel's fused multiply-add form against the strict,
    bit-exact result)."""
    M = K = 4096
    ip, ix, v = workloads.csr_uniform(M, K, 0.1, 0.02, seed=1234)
    W = ctx.csr_upload(M, K, ip, ix, v)
    X = workloads.dense_normal((K, 256), 1.0, seed=2024)
    Yf, Ys = W.spmm(X, mode="fast"), W.spmm(X, mode="strict")
    e, i = elementwise_rel(Yf, Ys)
    nw = float(np.abs(Yf.astype(np.float64) - Ys).max() / np.abs(Ys).max())
    say(f"ELEMENTWISE 4096x4096 N=256: elementwise {e:.3e} at output {i} (|r| = {abs(float(Ys.ravel()[i])):.3e}); "
        f"normwise {nw:.3e}")
    assert nw <= 1e-5
    W.free()


@pytest.mark.parametrize("N", [1, 16, 64, 256])
def test_fast_mode_forward_error_bound_uniform(ctx, N):
    """The same bound for the 4096 x 4096, 10 % fp32 weight at N = 1 .. 256
    (the column-slice and balanced kernels with fused multiply-adds)."""
    M = K = 4096
    ip, ix, v = workloads.csr_uniform(M, K, 0.1, 0.02, seed=1234)
    W = ctx.csr_upload(M, K, ip, ix, v)
    try:
        X = workloads.dense_normal((K, N), 1.0, seed=600 + N)
        Xa = X[:, 0].copy() if N == 1 else X
        say(f"uniform 4096x4096 N={N} fast, forward error bound")
        ok, worst = gamma_bound_ok(W.spmm(Xa, mode="fast"), M, K, ip, ix, v, Xa, extra=1)
        assert ok, (N, worst)
    finally:
        W.free()


def test_decode_stacked_siblings(ctx):
    """q, k and v (three different 4096 x 4096 weights) stacked into one
    12288 x 4096 product, as the decode bench's stacked form runs them:
    strict is bit-exact against the oracle on each projection alone, fast
    within 1e-5 normwise; batch 1 and 8."""
    M, K = DECODE["qkvo_4096x4096"]
    parts = [workloads.csr_int8_lognormal(M, K, 0.3, 0.5, 0.02, seed=40 + i) for i in range(3)]
    ip, ix, q, sc = workloads.csr_vstack(parts)
    W = ctx.csr_upload(3 * M, K, ip, ix, q, row_scales=sc)
    try:
        for B in (1, 8):
            X = workloads.dense_normal((K, B), 1.0, seed=300 + B)
            Xa = X[:, 0].copy() if B == 1 else X
            refs = [O.orc_csr_spmm(M, K, p[0], p[1], workloads.dequant_rows(p[0], p[2], p[3]), Xa) for p in parts]
            for mode in ("strict", "fast"):
                say(f"decode stacked q/k/v 12288x4096 batch {B} {mode}")
                Y = W.spmm(Xa, mode=mode)
                for i, R in enumerate(refs):
                    Yi = Y[i * M:(i + 1) * M]
                    if mode == "strict":
                        assert bits_equal(Yi, R), (B, i, first_diff(Yi, R))
                    else:
                        assert close_normwise(Yi, R), (B, i)
    finally:
        W.free()


@pytest.mark.parametrize("count", [2, 3])
def test_decode_stacked_tall_strict(ctx, count):
    """gate and up stacked (22016 x 4096), and three 11008 x 4096 weights
    (33024 rows): tall enough that the row-chain copy takes 32- and 64-row
    slabs for the vector kernel; the 2..8-column strict kernel walks them 16
    rows at a time.  Bit-exact against the oracle at batch 3 and 8."""
    M, K = DECODE["gate_up_11008x4096"]
    parts = [workloads.csr_int8_lognormal(M, K, 0.3, 0.5, 0.02, seed=50 + i) for i in range(count)]
    ip, ix, q, sc = workloads.csr_vstack(parts)
    vals = workloads.dequant_rows(ip, q, sc)
    W = ctx.csr_upload(count * M, K, ip, ix, q, row_scales=sc)
    try:
        for B in (3, 8):
            X = workloads.dense_normal((K, B), 1.0, seed=400 + B)
            say(f"decode stacked {count} x 11008x4096 batch {B} strict")
            Y = W.spmm(X, mode="strict")
            R = O.orc_csr_spmm(count * M, K, ip, ix, vals, X)
            assert bits_equal(Y, R), (count, B, first_diff(Y, R))
    finally:
        W.free()


def test_decode_device_pointers_strided(ctx, decode_layer):
    """The device-pointer entry the bench times: batch 8 with X and Y rows
    padded (ldx 12, ldy 10), both modes."""
    import torch

    name, M, K, ip, ix, vals, W = decode_layer
    X = workloads.dense_normal((K, 12), 1.0, seed=7)
    dX = torch.from_numpy(X).cuda()
    dY = torch.zeros((M, 10), dtype=torch.float32, device="cuda")
    R = O.orc_csr_spmm(M, K, ip, ix, vals, np.ascontiguousarray(X[:, :8]))
    for mode in ("strict", "fast"):
        say(f"decode {name} batch 8 {mode}, ldx 12, ldy 10")
        W.spmm_dev(dX.data_ptr(), 8, dY.data_ptr(), ldx=12, ldy=10, mode=mode)
        ctx.synchronize()
        Y = dY.cpu().numpy()
        assert not Y[:, 8:].any()
        if mode == "strict":
            assert bits_equal(Y[:, :8], R), (name, first_diff(Y[:, :8], R))
        else:
            assert close_normwise(Y[:, :8], R), name


def test_workgroup_per_row_long_k(ctx):
    """N <= 8 fast with K >= 16384 (no LDS copy of x or X) and a mean row of
    about 3,000 nonzeros: the workgroup-per-row kernel over uint16 columns;
    fp32 and int8 values, NaN and inf in x, the Relu epilogue, then N = 3
    and 8 (the eight-wide float4 X reads) with infinities and NaN in X."""
    import torch

    M, K = 600, 20000
    ip, ix, q, sc = workloads.csr_int8_lognormal(M, K, 0.15, 0.5, 0.02, seed=5)
    vals = workloads.dequant_rows(ip, q, sc)
    assert len(vals) >= 2048 * M
    rng = np.random.default_rng(6)
    x = rng.standard_normal(K).astype(np.float32)
    for tag, W in (("int8", ctx.csr_upload(M, K, ip, ix, q, row_scales=sc)),
                   ("fp32", ctx.csr_upload(M, K, ip, ix, vals))):
        say(f"workgroup per row N=1 K={K} {tag}")
        R = O.orc_csr_spmv(M, K, ip, ix, vals, x)
        assert close_normwise(W.spmm(x, mode="fast"), R), tag
        assert bits_equal(W.spmm(x, mode="strict"), R), tag
        xb = x.copy()
        xb[ix[10]] = np.inf
        xb[ix[len(ix) // 2]] = np.nan
        assert close_normwise(W.spmm(xb, mode="fast"), O.orc_csr_spmv(M, K, ip, ix, vals, xb)), tag
        dx = torch.from_numpy(x).cuda()
        dy = torch.empty(M, dtype=torch.float32, device="cuda")
        W.spmm_dev(dx.data_ptr(), 1, dy.data_ptr(), mode="fast", relu=True)
        ctx.synchronize()
        fused = dy.cpu().numpy()
        W.spmm_dev(dx.data_ptr(), 1, dy.data_ptr(), mode="fast")
        ctx.synchronize()
        plain = dy.cpu().numpy()
        assert bits_equal(fused, np.where(plain > 0, plain, np.float32(0))), tag
        for N in (3, 8):
            X = rng.standard_normal((K, N)).astype(np.float32)
            X[ix[10], 0] = np.inf
            X[ix[len(ix) // 3], N - 1] = np.nan
            say(f"workgroup per row N={N} K={K} {tag}")
            assert close_normwise(W.spmm(X, mode="fast"), O.orc_csr_spmm(M, K, ip, ix, vals, X)), (tag, N)
        W.free()


def test_balanced_gemm_epilogues(ctx):
    """The Gemm form y = act(A . B + bias) in fast mode with rows of op(B)^T
    holding ~2,400 nonzeros and K = 6000 (two K chunks of the nnz-balanced
    copy), batch 1, 3 and 8, with bias and Relu / Gelu fused; infinities in
    A.  Normwise against the oracle's sparse product plus bias (and, for the
    finite rows, its dense cpu_gemm), and the fused activations
    bit-identical to the separate device kernels on the unfused result."""
    import torch

    rng = np.random.default_rng(9)
    K, Nf = 6000, 600
    B = (rng.standard_normal((K, Nf)) * 0.05).astype(np.float32)
    B[rng.random(B.shape) >= 0.4] = 0
    BT = ctx.csr_from_dense(B, transpose=True)
    assert BT.nnz >= 2048 * Nf
    ipT, ixT, vT = O.orc_to_sparse_csr(np.ascontiguousarray(B.T))
    bias = rng.standard_normal(Nf).astype(np.float32)
    dC = torch.from_numpy(bias).cuda()
    for Mb in (1, 3, 8):
        A = rng.standard_normal((Mb, K)).astype(np.float32)
        A[0, rng.integers(0, K, 3)] = np.inf
        dA = torch.from_numpy(A).cuda()
        dY = torch.empty((Mb, Nf), dtype=torch.float32, device="cuda")
        say(f"balanced Gemm Mb={Mb} fast, bias, inf in A")
        ctx.gemm_csr_dev(dA.data_ptr(), Mb, K, BT, dY.data_ptr(), 1.0, 1.0, dC.data_ptr(), Nf, mode="fast")
        ctx.synchronize()
        plain = dY.cpu().numpy()
        assert close_normwise(plain, sparse_gemm_ref(A, ipT, ixT, vT, Nf, bias)), Mb
        if Mb > 1:  # the finite rows also equal the dense cpu_gemm
            assert close_normwise(plain[1:], O.orc_gemm(A[1:], B, bias, 1.0, 1.0)), Mb
        for act in ("relu", "gelu"):
            ctx.gemm_csr_dev(dA.data_ptr(), Mb, K, BT, dY.data_ptr(), 1.0, 1.0, dC.data_ptr(), Nf, mode="fast",
                             **{act: True})
            ctx.synchronize()
            fused = dY.cpu().numpy()
            want = np.where(plain > 0, plain, np.float32(0)) if act == "relu" else ctx.gelu(plain)
            assert bits_equal(fused, want), (Mb, act)


def sparse_gemm_ref(A, ipT, ixT, vT, Nf, bias):
    """A . B + bias with B given as the CSR of B^T: the oracle's
    sparse_matmul (pruned terms skipped, so an infinity in A meets only the
    stored weights), then the bias added once in fp32, as cpu_gemm adds
    beta * C after the sum (math.cpp:431-433)."""
    K = A.shape[1]
    return (O.orc_csr_spmm(Nf, K, ipT, ixT, vT, np.ascontiguousarray(A.T)).T + bias).astype(np.float32)


def bert_weight(out_f, in_f, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((out_f, in_f)) * 0.02).astype(np.float32)
    w[rng.random(w.shape) < 0.8] = 0
    return w


@pytest.mark.parametrize("name", list(BERT))
def test_bert_linear_gemm_1024_tokens(ctx, name):
    """Gemm(x, W, b), transB = 1, W [out, in] 80 % zeros, x [1024, in]: the
    full output bit-exact against the oracle's CSR product plus bias (equal
    to cpu_gemm on the zero-filled weight for finite inputs), and the first
    64 token rows against the oracle's dense cpu_gemm itself; the
    Gelu-fused epilogue bit-identical to Gelu on the unfused output."""
    import torch

    out_f, in_f = BERT[name]
    T = T_TOKENS
    w = bert_weight(out_f, in_f, seed=out_f * 7 + in_f)
    rng = np.random.default_rng(out_f + in_f)
    x = rng.standard_normal((T, in_f)).astype(np.float32)
    bias = (rng.standard_normal(out_f) * 0.1).astype(np.float32)
    ip, ix, v = O.orc_to_sparse_csr(w)
    BT = ctx.csr_from_dense(w)  # transB = 1: op(B)^T is W itself
    assert BT.nnz == len(v)
    say(f"BERT {name} Gemm transB=1 bias, T={T}, nnz={len(v)}, strict")
    Y = ctx.gemm_csr(x, BT, 1.0, 1.0, bias)
    R = (O.orc_csr_spmm(out_f, in_f, ip, ix, v, np.ascontiguousarray(x.T)).T + bias).astype(np.float32)
    assert bits_equal(Y, R), (name, first_diff(Y, R))
    R64 = O.orc_gemm(x[:64], w, bias, 1.0, 1.0, transB=1)
    assert bits_equal(R[:64], R64) and bits_equal(Y[:64], R64), name
    dx = torch.from_numpy(x).cuda()
    db = torch.from_numpy(bias).cuda()
    dY = torch.empty((T, out_f), dtype=torch.float32, device="cuda")
    say(f"BERT {name} Gemm + Gelu fused")
    ctx.gemm_csr_dev(dx.data_ptr(), T, in_f, BT, dY.data_ptr(), 1.0, 1.0, db.data_ptr(), out_f, gelu=True)
    ctx.synchronize()
    assert bits_equal(dY.cpu().numpy(), ctx.gelu(Y)), name
    BT.free()


def test_bert_matmul_form_1024_tokens(ctx):
    """MatMul(x, W) with W [in, out] (transB = 0): the CSR of W^T, alpha 1,
    no bias, 1024 tokens on the FFN up projection's shape, bit-exact."""
    in_f, out_f = 768, 3072
    w = bert_weight(out_f, in_f, seed=77).T.copy()  # [in, out]
    x = np.random.default_rng(78).standard_normal((T_TOKENS, in_f)).astype(np.float32)
    BT = ctx.csr_from_dense(w, transpose=True)
    ip, ix, v = O.orc_to_sparse_csr(np.ascontiguousarray(w.T))
    say("BERT MatMul(x, W) 1024 x 768 . 768 x 3072 strict")
    Y = ctx.gemm_csr(x, BT)
    R = O.orc_csr_spmm(out_f, in_f, ip, ix, v, np.ascontiguousarray(x.T)).T
    assert bits_equal(Y, R), first_diff(Y, R)
    assert bits_equal(Y[:32], O.orc_matmul(x[:32], w))
    BT.free()
