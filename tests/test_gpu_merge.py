"""GPU parity of the merge-path fast kernels (k_spmv_merge): fast mode
(reassociated sums) of pruning::sparse_matvec / sparse_matmul
(sparse_tensor.cpp:473-554), checked against the oracle within 1e-5
normwise and within the forward error bound of any summation order, on
weights whose rows the partition cuts in every way it can: rows spanning
several workgroups, runs of empty rows, shares holding only row ends, a
single workgroup, rows ending exactly at a record or batch boundary.  A row
cut by a workgroup boundary is finished by whichever contributor arrives
last, through per-row arrival counters that the last arrival clears: three
calls in a row must give the same bits."""
import sys

import numpy as np
import pytest

from oracle import oracle as O
from pyflamert_amd import workloads

from bounds import gamma_bound_ok

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def close_normwise(Y, R, tol=1e-5):
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
    scale = max(float(np.abs(R[ok]).max()), 1e-30)
    return bool(np.abs(Y[ok].astype(np.float64) - R[ok]).max() <= tol * scale)


@pytest.fixture(scope="module")
def ctx():
    from pyflamert_amd import rocm

    c = rocm.Context(0)
    yield c
    c.close()


def csr_from_lengths(lens, K, rng):
    """CSR with the given row lengths, columns drawn without replacement and
    ascending, values N(0, 0.02)."""
    lens = np.minimum(np.asarray(lens, np.int64), K)
    ip = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    ix = np.empty(int(ip[-1]), np.int64)
    for r, n in enumerate(lens):
        if n:
            ix[ip[r]:ip[r + 1]] = np.sort(rng.choice(K, int(n), replace=False))
    v = (rng.standard_normal(len(ix)) * 0.02).astype(np.float32)
    return ip, ix, v


def shape_case(kind, rng):
    """(M, K, row lengths) of one edge case."""
    if kind == "empty_runs":  # long runs of empty rows between heavy rows
        M, K = 3000, 4096
        lens = np.where(rng.random(M) < 0.04, rng.integers(500, 4096, M), 0)
    elif kind == "one_long_row":  # one full row across every workgroup of a small launch
        M, K = 40, 16000
        lens = rng.integers(0, 4, M)
        lens[7] = K
    elif kind == "full_rows":  # rows of 16000 alternating with empty ones: ~one row per workgroup
        M, K = 600, 16000
        lens = np.where(np.arange(M) % 2 == 0, K, 0)
    elif kind == "tiny":  # one workgroup, shares of a few items
        M, K = 5, 7
        lens = np.array([3, 0, 7, 1, 2])
    elif kind == "short_rows":  # many row ends per wave share
        M, K = 20000, 3000
        lens = rng.integers(0, 30, M)
    elif kind == "record_aligned":  # every row a multiple of four entries (ends on record boundaries)
        M, K = 4000, 2048
        lens = 4 * rng.integers(0, 300, M)
    elif kind == "batch_aligned":  # rows of 512 entries: ends on the 128-record batch boundaries
        M, K = 2048, 4096
        lens = np.full(M, 512)
    else:  # lognormal rows, as the decode weights
        M, K = 2500, 6000
        lens = np.minimum(rng.lognormal(np.log(0.3 * K) - 0.125, 0.5, M).astype(np.int64), K)
    return M, K, lens


KINDS = ["empty_runs", "one_long_row", "full_rows", "tiny", "short_rows", "record_aligned", "batch_aligned",
         "lognormal"]


@pytest.mark.parametrize("N", [1, 2, 3, 8])
@pytest.mark.parametrize("int8", [False, True])
@pytest.mark.parametrize("kind", KINDS)
def test_merge_spmv_edge_shapes(ctx, kind, int8, N):
    """N = 1: the merge-path kernel; N = 2, 3, 8: the fast kernels for few
    columns over the same weights (nnz-balanced or row kernels), on the same
    skewed shapes."""
    rng = np.random.default_rng(2 * KINDS.index(kind) + int(int8))
    M, K, lens = shape_case(kind, rng)
    ip, ix, v = csr_from_lengths(lens, K, rng)
    if int8:
        q = rng.integers(-127, 128, len(ix)).astype(np.int8)
        sc = (rng.random(M) * 0.01 + 1e-3).astype(np.float32)
        W = ctx.csr_upload(M, K, ip, ix, q, row_scales=sc)
        vals = workloads.dequant_rows(ip, q, sc)
    else:
        W = ctx.csr_upload(M, K, ip, ix, v)
        vals = v
    x = rng.standard_normal((K, N) if N > 1 else K).astype(np.float32)
    say(f"merge spmv {kind} int8={int8} M={M} K={K} nnz={len(ix)} N={N}")
    Y = W.spmm(x, mode="fast")
    R = O.orc_csr_spmm(M, K, ip, ix, vals, x)
    assert close_normwise(Y, R), kind
    ok, worst = gamma_bound_ok(Y, M, K, ip, ix, vals, x)
    assert ok, (kind, worst)
    for _ in range(2):  # the arrival counters start from zero again on every call
        Y2 = W.spmm(x, mode="fast")
        assert np.array_equal(Y.view(np.uint32), Y2.view(np.uint32)), kind
    # NaN and -inf in x propagate to the rows that use them, cut or not
    xb = x.copy()
    if len(ix):
        xb[ix[len(ix) // 2], ...] = np.nan
        xb[ix[-1], ...] = -np.inf
    Y = W.spmm(xb, mode="fast")
    R = O.orc_csr_spmm(M, K, ip, ix, vals, xb)
    assert close_normwise(Y, R), (kind, "non-finite x")
    W.free()


def test_merge_gemm_epilogue(ctx):
    """The Gemm form with one activation row (N = 1 of the product): bias,
    beta, alpha and the fused Relu / Gelu on rows cut by workgroup
    boundaries, against the strict kernels' result within 1e-5 normwise."""
    import torch

    rng = np.random.default_rng(11)
    Kb, Nb = 9000, 300
    B = np.zeros((Kb, Nb), np.float32)
    m = rng.random((Kb, Nb)) < 0.6
    B[m] = rng.standard_normal(int(m.sum())).astype(np.float32) * 0.05
    BT = ctx.csr_from_dense(B, transpose=True)
    bias = rng.standard_normal(Nb).astype(np.float32)
    A = rng.standard_normal((1, Kb)).astype(np.float32)
    dA = torch.from_numpy(A).cuda()
    dC = torch.from_numpy(bias).cuda()
    dY = torch.empty((1, Nb), dtype=torch.float32, device="cuda")
    for act in ("none", "relu", "gelu"):
        out = {}
        for mode in ("strict", "fast"):
            say(f"merge gemm Mb=1 act={act} {mode}")
            ctx.gemm_csr_dev(dA.data_ptr(), 1, Kb, BT, dY.data_ptr(), 0.5, 2.0, dC.data_ptr(), Nb, mode=mode,
                             relu=act == "relu", gelu=act == "gelu")
            ctx.synchronize()
            out[mode] = dY.cpu().numpy().copy()
        assert close_normwise(out["fast"], out["strict"], tol=2e-5), act


def test_merge_decode_shapes_deterministic(ctx):
    """The decode shapes at batch 1: every call gives the same bits (rows
    cut by workgroup boundaries summed in workgroup order whatever the
    arrival order), within 1e-5 normwise of the oracle."""
    for M, K in ((4096, 4096), (11008, 4096), (4096, 11008)):
        ip, ix, q, sc = workloads.csr_int8_lognormal(M, K, 0.3, 0.5, 0.02, seed=M + 3 * K)
        W = ctx.csr_upload(M, K, ip, ix, q, row_scales=sc)
        x = workloads.dense_normal((K,), 1.0, seed=7)
        say(f"merge decode {M}x{K} batch 1, five calls")
        Y = W.spmm(x, mode="fast")
        for _ in range(4):
            assert np.array_equal(Y.view(np.uint32), W.spmm(x, mode="fast").view(np.uint32)), (M, K)
        R = O.orc_csr_spmm(M, K, ip, ix, workloads.dequant_rows(ip, q, sc), x)
        assert close_normwise(Y, R), (M, K)
        W.free()
