"""GPU parity of the CSR SpMM/SpMV/Gemm kernels against the oracle and the
golden vectors written by the compiled reference.

Bar: strict mode is bit-exact (fp32 bits compared with array_equal on the
uint32 view).  Fast mode (fused multiply-add, terms in an order the kernel
chooses) is checked with a normwise bound: max|y - r| <= 1e-5 * max|r|.
"""
import sys

import numpy as np
import pytest

from oracle import oracle as O
from pyflamert_amd import _lib, workloads

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def first_diff(a, b):
    d = np.nonzero(a.view(np.uint32).ravel() != b.view(np.uint32).ravel())[0]
    return (len(d), d[:5], a.ravel()[d[:5]], b.ravel()[d[:5]]) if len(d) else None


@pytest.fixture(scope="module")
def ctx():
    from pyflamert_amd import rocm

    c = rocm.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def cfg_weight():
    """4096 x 4096, each entry kept with p = 0.1, values N(0, 0.02)."""
    return workloads.csr_uniform(4096, 4096, 0.1, 0.02, seed=1234)


@pytest.mark.parametrize("N", [1, 16, 64, 128, 256])
def test_spmm_4096_strict_bit_exact(ctx, cfg_weight, N):
    ip, ix, v = cfg_weight
    say(f"spmm 4096x4096 nnz={len(v)} N={N} strict")
    W = ctx.csr_upload(4096, 4096, ip, ix, v)
    X = workloads.dense_normal((4096, N), 1.0, seed=99 + N)
    Y = W.spmm(X if N > 1 else X[:, 0], mode="strict")
    R = O.orc_csr_spmm(4096, 4096, ip, ix, v, X if N > 1 else X[:, 0])
    assert bits_equal(Y, R), first_diff(Y, R)
    W.free()


@pytest.mark.parametrize("N", [2, 3, 8, 17, 33, 63, 65, 100, 130, 257])
def test_spmm_odd_widths_strict(ctx, N):
    ip, ix, v = workloads.csr_uniform(517, 389, 0.12, 0.05, seed=N)
    say(f"spmm 517x389 N={N}")
    W = ctx.csr_upload(517, 389, ip, ix, v)
    X = workloads.dense_normal((389, N), 1.0, seed=7 * N)
    assert bits_equal(W.spmm(X), O.orc_csr_spmm(517, 389, ip, ix, v, X))


@pytest.mark.parametrize("N", [1, 8, 64, 256])
def test_spmm_fast_normwise(ctx, cfg_weight, N):
    ip, ix, v = cfg_weight
    say(f"spmm fast N={N}")
    W = ctx.csr_upload(4096, 4096, ip, ix, v)
    X = workloads.dense_normal((4096, N), 1.0, seed=5 + N)
    Y = W.spmm(X, mode="fast")
    R = O.orc_csr_spmm(4096, 4096, ip, ix, v, X)
    assert np.abs(Y - R).max() <= 1e-5 * np.abs(R).max()


@pytest.mark.parametrize("M,K,N,dens", [(4096, 4096, 16, 0.1), (4096, 4096, 32, 0.1), (4096, 4096, 64, 0.1),
                                        (1500, 3000, 48, 0.2), (700, 5000, 64, 0.05), (33, 2100, 20, 0.5)])
def test_fast_chunk_split(ctx, M, K, N, dens):
    """Fast mode at few columns with K in several chunks (the column-slice
    kernel's chunked walk, several slabs per workgroup, a partial last
    slab).  Within 1e-5 normwise of the oracle and within the forward error bound
    of any summation order, with an odd number of chunks (K = 3000, 5000,
    2100); repeated calls give the same bits; bias and Relu through the
    Gemm form's epilogue against the strict result."""
    from bounds import gamma_bound_ok

    ip, ix, v = workloads.csr_uniform(M, K, dens, 0.02, seed=M + K + N)
    W = ctx.csr_upload(M, K, ip, ix, v)
    X = workloads.dense_normal((K, N), 1.0, seed=N)
    say(f"fast chunk split M={M} K={K} N={N}")
    Y = W.spmm(X, mode="fast")
    R = O.orc_csr_spmm(M, K, ip, ix, v, X)
    assert np.abs(Y - R).max() <= 1e-5 * np.abs(R).max()
    ok, worst = gamma_bound_ok(Y, M, K, ip, ix, v, X)
    assert ok, worst
    Y2 = W.spmm(X, mode="fast")
    assert bits_equal(Y2, Y)
    W.free()
    # Gemm form: Y = relu(A . B + bias), B = W^T, A = X^T (Mb = N rows)
    B = np.zeros((K, M), np.float32)
    rows = np.repeat(np.arange(M), np.diff(ip))
    B[ix, rows] = v
    BT = ctx.csr_from_dense(B, transpose=True)
    import torch

    dA = torch.from_numpy(np.ascontiguousarray(X.T)).cuda()
    dC = torch.from_numpy(workloads.dense_normal((M,), 0.1, seed=3)).cuda()
    out = {}
    for mode in ("fast", "strict"):
        dY = torch.empty((N, M), dtype=torch.float32, device="cuda")
        ctx.gemm_csr_dev(dA.data_ptr(), N, K, BT, dY.data_ptr(), 1.0, 1.0, dC.data_ptr(), M, mode=mode, relu=True)
        ctx.synchronize()
        out[mode] = dY.cpu().numpy()
    assert np.abs(out["fast"] - out["strict"]).max() <= 1e-5 * max(np.abs(out["strict"]).max(), 1e-30)
    assert (out["fast"] >= 0).all()
    BT.free()


def test_golden_csr(ctx, golden):
    g = golden("csr.npz")
    M, K = g["W"].shape
    say("golden csr.npz")
    for tag in ("t0", "t1"):
        W = ctx.csr_upload(M, K, g[f"{tag}_indptr"], g[f"{tag}_indices"], g[f"{tag}_values"])
        if tag == "t0":
            for n in (1, 8, 64):
                X = g[f"X{n}"]
                assert bits_equal(W.spmm(X), g[f"Y{n}"]), n
            assert bits_equal(W.spmm(g["x"]), g["y_matvec"])
            assert bits_equal(W.spmm(g["x"]), g["y_1d"])
        W.free()
    # from the dense weight with to_sparse's threshold rule
    Wd = ctx.csr_from_dense(g["W"], threshold=0.0)
    assert Wd.nnz == len(g["t0_values"])
    assert bits_equal(Wd.spmm(g["X64"]), g["Y64"])
    Wt = ctx.csr_from_dense(g["W"], threshold=0.005)
    assert Wt.nnz == len(g["t1_values"])


def test_golden_gemm(ctx, golden):
    """cpu_gemm cases: alpha/beta, transA/transB, bias broadcast by modulo."""
    g = golden("gemm.npz")
    for i in range(int(g["n"])):
        al, be, ta, tb = (float(x) for x in g[f"c{i}_p"])
        A, B, Cb = g[f"c{i}_A"], g[f"c{i}_B"], g[f"c{i}_C"]
        say(f"golden gemm case {i} A{A.shape} B{B.shape} ta={ta} tb={tb} c={Cb.size}")
        BT = ctx.csr_from_dense(B, transpose=not tb)
        Y = ctx.gemm_csr(A, BT, al, be, Cb if Cb.size else None, transA=bool(ta))
        assert bits_equal(Y, g[f"c{i}_out"]), (i, first_diff(Y, g[f"c{i}_out"]))


def test_golden_matmul_and_kat(ctx, golden):
    """MatMul(X, W) with a pruned W as the Gemm form (alpha 1, no bias); the
    batched case [3,4,5] x [5,6] flattens the broadcast batch into rows."""
    g = golden("matmul.npz")
    a, b = g["c0_a"], g["c0_b"]
    BT = ctx.csr_from_dense(b, transpose=True)
    Y = ctx.gemm_csr(a.reshape(-1, a.shape[-1]), BT).reshape(g["c0_out"].shape)
    assert bits_equal(Y, g["c0_out"])
    a, b = g["c3_a"], g["c3_b"]
    assert bits_equal(ctx.gemm_csr(a, ctx.csr_from_dense(b, transpose=True)), g["c3_out"])
    k = golden("kat_matmul.npz")
    Y = ctx.gemm_csr(k["a"], ctx.csr_from_dense(k["b"], transpose=True))
    assert Y.tolist() == [[22.0, 28.0], [49.0, 64.0]]


@pytest.mark.parametrize("Mb", [1, 5, 32, 100, 1024])
def test_gemm_form_vs_oracle(ctx, Mb):
    rng = np.random.default_rng(Mb)
    K, Nf = 768, 300
    B = rng.normal(0, 0.02, (K, Nf)).astype(np.float32)
    B[rng.random(B.shape) < 0.8] = 0.0
    A = rng.standard_normal((Mb, K)).astype(np.float32)
    bias = rng.standard_normal(Nf).astype(np.float32)
    BT = ctx.csr_from_dense(B, transpose=True)
    # alpha != 1 scales A as it is staged (Mb >= 16: the column-slice kernel
    # reads A in place) or in the transposed copy
    for alpha, beta in ((1.0, 1.0), (0.37, -0.5)):
        say(f"gemm form Mb={Mb} alpha={alpha} beta={beta}")
        Y = ctx.gemm_csr(A, BT, alpha, beta, bias)
        R = O.orc_gemm(A, B, bias, alpha, beta)
        assert bits_equal(Y, R), (alpha, first_diff(Y, R))


def test_edge_cases(ctx):
    say("edge: empty matrix, empty rows, long row, many tiny rows, skewed rows")
    # nnz == 0: all +0
    W = ctx.csr_upload(5, 7, np.zeros(6, np.int64), np.zeros(0, np.int64), np.zeros(0, np.float32))
    Y = W.spmm(np.ones((7, 3), np.float32))
    assert bits_equal(Y, np.zeros((5, 3), np.float32))
    assert bits_equal(W.spmm(np.ones(7, np.float32)), np.zeros(5, np.float32))
    # one row longer than the vector kernel's LDS chunk, plus empty rows
    K = 9000
    ip = np.array([0, 0, 8500, 8500, 8600], np.int64)
    rng = np.random.default_rng(3)
    ix = np.concatenate([np.sort(rng.choice(K, 8500, replace=False)), np.sort(rng.choice(K, 100, replace=False))])
    v = rng.standard_normal(8600).astype(np.float32)
    W = ctx.csr_upload(4, K, ip, ix, v)
    for n in (1, 2, 64):
        X = rng.standard_normal((K, n)).astype(np.float32)
        assert bits_equal(W.spmm(X), O.orc_csr_spmm(4, K, ip, ix, v, X)), n
    # many rows with one entry each (64-row vector blocks)
    M = 10000
    ip = np.arange(M + 1, dtype=np.int64)
    ix = rng.integers(0, 50, M).astype(np.int64)
    v = rng.standard_normal(M).astype(np.float32)
    W = ctx.csr_upload(M, 50, ip, ix, v)
    x = rng.standard_normal(50).astype(np.float32)
    assert bits_equal(W.spmm(x), O.orc_csr_spmv(M, 50, ip, ix, v, x))
    # lognormal row lengths (skewed), vector and matrix
    ip, ix, v = workloads.csr_lognormal_rows(2000, 3000, 0.3, 0.8, 0.02, seed=11)
    W = ctx.csr_upload(2000, 3000, ip, ix, v)
    for n in (1, 8, 64):
        X = rng.standard_normal((3000, n)).astype(np.float32)
        assert bits_equal(W.spmm(X), O.orc_csr_spmm(2000, 3000, ip, ix, v, X)), n
    # unsorted / duplicate columns: storage order is the summation order
    ip = np.array([0, 4], np.int64)
    ix = np.array([3, 1, 3, 0], np.int64)
    v = np.array([1e8, 1.0, -1e8, 0.5], np.float32)
    W = ctx.csr_upload(1, 4, ip, ix, v)
    X = np.array([[1.0], [1.0], [0.0], [1.0]], np.float32)
    assert bits_equal(W.spmm(X[:, 0]), O.orc_csr_spmv(1, 4, ip, ix, v, X[:, 0]))


def test_rejects_bad_csr(ctx):
    say("argument errors")
    with pytest.raises(_lib.InvalidArgument, match="out of range"):
        ctx.csr_upload(2, 3, np.array([0, 1, 2]), np.array([0, 3]), np.ones(2, np.float32))
    with pytest.raises(_lib.InvalidArgument, match="non-decreasing"):
        ctx.csr_upload(3, 3, np.array([0, 2, 1, 2]), np.array([0, 1]), np.ones(2, np.float32))
    with pytest.raises(_lib.InvalidArgument, match="indptr"):
        ctx.csr_upload(2, 3, np.array([0, 1, 3]), np.array([0, 1]), np.ones(2, np.float32))
    BT = ctx.csr_from_dense(np.ones((4, 3), np.float32), transpose=True)
    with pytest.raises(_lib.InvalidArgument, match="incompatible dimensions"):
        ctx.gemm_csr(np.ones((2, 5), np.float32), BT)


def test_device_pointer_variant(ctx, cfg_weight):
    import torch

    ip, ix, v = cfg_weight
    say("spmm_dev via torch device tensors")
    W = ctx.csr_upload(4096, 4096, ip, ix, v)
    X = workloads.dense_normal((4096, 256), 1.0, seed=17)
    dX = torch.from_numpy(X).cuda()
    dY = torch.empty((4096, 300), dtype=torch.float32, device="cuda")  # ldy > N
    torch.cuda.synchronize()
    W.spmm_dev(dX.data_ptr(), 256, dY.data_ptr(), ldx=256, ldy=300)
    ctx.synchronize()
    Y = dY[:, :256].cpu().numpy()
    assert bits_equal(Y, O.orc_csr_spmm(4096, 4096, ip, ix, v, X))


def shuffle_within(ix, ip, block):
    """Permute each row's columns inside every `block`-wide K range, keeping
    the ranges in order (storage order then differs from column order)."""
    rng = np.random.default_rng(5)
    out = ix.copy()
    for r in range(len(ip) - 1):
        seg = out[ip[r]:ip[r + 1]]
        for b in np.unique(seg // block):
            m = np.nonzero(seg // block == b)[0]
            seg[m] = seg[rng.permutation(m)]
    return out


def test_column_slice_layout_cases(ctx):
    """The column-slice kernel (N >= 16): several K chunks, storage order
    unsorted inside chunks, a weight that must fall back to the row kernels,
    ragged column counts, unaligned leading dimensions, empty slabs, and
    infinities in X."""
    import torch

    M, K = 16 * 21 + 3, 5000
    ip, ix, v = workloads.csr_uniform(M, K, 0.08, 0.05, seed=21)
    cnt = np.diff(ip)
    cnt[16 * 4:16 * 6] = 0  # two slabs' worth of empty rows
    ip = np.zeros(M + 1, np.int64)
    np.cumsum(cnt, out=ip[1:])
    rng = np.random.default_rng(8)
    ix = np.concatenate([np.sort(rng.choice(K, c, replace=False)) for c in cnt]).astype(np.int64)
    v = (rng.standard_normal(len(ix)) * 0.05).astype(np.float32)
    cases = {"sorted": ix, "shuffled in chunks": shuffle_within(ix, ip, 1024),
             "shuffled across chunks": shuffle_within(ix, ip, K)}
    for name, cols in cases.items():
        W = ctx.csr_upload(M, K, ip, cols, v)
        for N in (16, 48, 50):
            say(f"column slice: {name} N={N}")
            X = rng.standard_normal((K, N)).astype(np.float32)
            assert bits_equal(W.spmm(X), O.orc_csr_spmm(M, K, ip, cols, v, X)), (name, N)
    # unaligned leading dimensions through the device-pointer entry
    W = ctx.csr_upload(M, K, ip, ix, v)
    N = 37
    X = rng.standard_normal((K, N + 3)).astype(np.float32)
    dX = torch.from_numpy(X).cuda()
    dY = torch.zeros((M, N + 5), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    say("column slice: ldx=40 ldy=42")
    W.spmm_dev(dX.data_ptr(), N, dY.data_ptr(), ldx=N + 3, ldy=N + 5)
    ctx.synchronize()
    R = O.orc_csr_spmm(M, K, ip, ix, v, np.ascontiguousarray(X[:, :N]))
    assert bits_equal(dY[:, :N].cpu().numpy(), R)
    assert not dY[:, N:].cpu().numpy().any()  # columns past N untouched
    # infinities: products inf and inf - inf = nan exactly where the oracle has them
    X = rng.standard_normal((K, 32)).astype(np.float32)
    X[rng.integers(0, K, 40), rng.integers(0, 32, 40)] = np.inf
    say("column slice: infinities")
    Y, R = W.spmm(X), O.orc_csr_spmm(M, K, ip, ix, v, X)
    assert np.array_equal(np.isnan(Y), np.isnan(R))
    fin = ~np.isnan(R)
    assert np.array_equal(Y[fin].view(np.uint32), R[fin].view(np.uint32))


def test_column_slice_placed_slabs(ctx):
    """Slab placement: 4087 rows (256 slabs, one of them holding 7 rows) are
    dealt out to workgroups by length, so the partial slab sits inside the
    slab array.  The copy built from host arrays and the one built from a
    dense device weight both match the oracle bit for bit through the 16-,
    8- and 4-wave launches (N = 256, 128, 64)."""
    import torch

    M, K = 4087, 4096
    ip, ix, v = workloads.csr_uniform(M, K, 0.1, 0.02, seed=77)
    dW = torch.from_numpy(workloads.csr_to_dense(M, K, ip, ix, v)).cuda()
    torch.cuda.synchronize()
    weights = {"host": ctx.csr_upload(M, K, ip, ix, v), "device": ctx.csr_from_dense_dev(dW.data_ptr(), M, K)}
    rng = np.random.default_rng(9)
    for N in (256, 128, 64):
        X = rng.standard_normal((K, N)).astype(np.float32)
        R = O.orc_csr_spmm(M, K, ip, ix, v, X)
        for name, W in weights.items():
            say(f"placed slabs: {name} N={N}")
            assert bits_equal(W.spmm(X), R), (name, N)


def check_fast(Y, R):
    """Fast-mode bar: NaN exactly where the oracle has it, infinities equal,
    the finite entries normwise within 1e-5 of the oracle's largest."""
    assert np.array_equal(np.isnan(Y), np.isnan(R))
    fin = ~np.isnan(R)
    assert np.array_equal(Y[np.isinf(R)], R[np.isinf(R)])
    ok = fin & np.isfinite(R)
    if ok.any():
        scale = np.abs(R[ok]).max()
        assert np.abs(Y[ok] - R[ok]).max() <= 1e-5 * scale


def test_fast_vector_balanced(ctx):
    """The fast N <= 8 kernels over the nnz-balanced copy (x staged in LDS):
    long and short rows, int8 with row scales and fp32, empty rows (groups
    with no quad rows), a strided x, NaN and infinity in x, and the fused
    bias / activation epilogue; then matrices with enough rows for 32- and
    64-row slabs of the row-chain copy, strict (bit-exact) and fast.  Fast
    results are normwise within 1e-5 of the strict oracle, with NaN exactly
    where the oracle has it."""
    import torch

    rng = np.random.default_rng(12)
    check = check_fast

    cases = [("int8 long rows", 600, 6000, True), ("fp32 long rows", 700, 5000, False),
             ("int8 short rows", 3000, 2000, True)]
    for name, M, K, i8 in cases:
        dens = 0.3 if "long" in name else 0.1
        if i8:
            ip, ix, q, sc = workloads.csr_int8_lognormal(M, K, dens, 0.5, 0.02, seed=M)
            vals = workloads.dequant_rows(ip, q, sc)
        else:
            ip, ix, vals = workloads.csr_lognormal_rows(M, K, dens, 0.5, 0.02, seed=M)
        cnt = np.diff(ip)
        cnt[-40:] = 0  # empty rows: sorted last, a group of them holds no quad rows
        mask = np.ones(len(ix), bool)
        for r in range(M - 40, M):
            mask[ip[r]:ip[r + 1]] = False
        ix, vals = ix[mask], vals[mask]
        if i8:
            q = q[mask]
        ip = np.zeros(M + 1, np.int64)
        np.cumsum(cnt, out=ip[1:])
        W = ctx.csr_upload(M, K, ip, ix, q, row_scales=sc) if i8 else ctx.csr_upload(M, K, ip, ix, vals)
        x = rng.standard_normal(K).astype(np.float32)
        say(f"fast balanced: {name} M={M} K={K}")
        check(W.spmm(x, mode="fast"), O.orc_csr_spmv(M, K, ip, ix, vals, x))
        x2 = x.copy()
        x2[ix[0]] = np.nan
        x2[ix[len(ix) // 2]] = np.inf
        check(W.spmm(x2, mode="fast"), O.orc_csr_spmv(M, K, ip, ix, vals, x2))
        # strided x (every third element of a device buffer), relu epilogue
        dX = torch.from_numpy(np.repeat(x[:, None], 3, axis=1)).cuda()
        dY = torch.zeros((M, 2), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        W.spmm_dev(dX.data_ptr(), 1, dY.data_ptr(), ldx=3, ldy=2, mode="fast", relu=True)
        ctx.synchronize()
        R = O.orc_csr_spmv(M, K, ip, ix, vals, x)
        check(dY[:, 0].cpu().numpy(), relu_ref(R))
        assert not dY[:, 1].cpu().numpy().any()
        # 2 <= N <= 8 (X staged in LDS chunk by chunk as rows of eight)
        for N in (2, 5, 8):
            X = rng.standard_normal((K, N)).astype(np.float32)
            X[ix[1], N - 1] = np.nan
            X[ix[len(ix) // 3], 0] = -np.inf
            say(f"fast balanced: {name} N={N}")
            check(W.spmm(X, mode="fast"), O.orc_csr_spmm(M, K, ip, ix, vals, X))
        W.free()
    # 32- and 64-row slabs: more rows than 16-row (32-row) slabs give four
    # workgroups per CU
    cu = torch.cuda.get_device_properties(0).multi_processor_count
    for rows, M, K, dens in ((32, 16 * 4 * cu + 300, 1300, 0.3), (64, 32 * 4 * cu + 100, 300, 0.05)):
        ip, ix, vals = workloads.csr_uniform(M, K, dens, 0.02, seed=rows)
        W = ctx.csr_upload(M, K, ip, ix, vals)
        x = rng.standard_normal(K).astype(np.float32)
        say(f"row chains: {rows}-row slabs M={M} K={K}")
        R = O.orc_csr_spmv(M, K, ip, ix, vals, x)
        check(W.spmm(x, mode="fast"), R)
        assert bits_equal(W.spmm(x), R)
        W.free()


def test_balanced_copy_edges(ctx):
    """Shapes at the edges of the nnz-balanced copy, fast mode, N = 1..8
    against the oracle: one row holding every column beside empty rows (the
    budget search's largest single row), fewer rows than one group, a
    single row, K at one chunk exactly (4096), one column past it (two
    chunks, the second one column wide), the largest K whose staged x fits
    64 KiB (16380: four chunks of 4095), and K one past that (no balanced
    copy: the wave-per-row kernel), int8 and fp32, with a strided X."""
    import torch

    rng = np.random.default_rng(21)
    cases = [("one full row", 300, 3000), ("few rows", 5, 9000), ("single row", 1, 4096),
             ("one chunk", 700, 4096), ("ragged chunk", 700, 4097), ("largest K", 400, 16380),
             ("past largest K", 400, 16381)]
    for name, M, K in cases:
        dens = 0.2
        ip, ix, q, sc = workloads.csr_int8_lognormal(M, K, dens, 0.8, 0.02, seed=M + K)
        if name == "one full row":
            cnt = np.diff(ip)
            rows = [np.arange(K) if r == 7 else (np.array([], np.int64) if r % 3 == 0 else ix[ip[r]:ip[r + 1]])
                    for r in range(M)]
            qs = [rng.integers(-127, 128, len(c)).astype(np.int8) for c in rows]
            ip = np.zeros(M + 1, np.int64)
            np.cumsum([len(c) for c in rows], out=ip[1:])
            ix = np.concatenate(rows).astype(np.int64)
            q = np.concatenate(qs)
        vals = workloads.dequant_rows(ip, q, sc)
        for tag, W in (("int8", ctx.csr_upload(M, K, ip, ix, q, row_scales=sc)),
                       ("fp32", ctx.csr_upload(M, K, ip, ix, vals))):
            for N in (1, 2, 3, 8):
                X = rng.standard_normal((K, N)).astype(np.float32)
                if len(ix):
                    X[ix[len(ix) // 2], 0] = np.inf
                say(f"balanced edges: {name} M={M} K={K} {tag} N={N}")
                R = O.orc_csr_spmm(M, K, ip, ix, vals, X)
                check_fast(W.spmm(X, mode="fast").reshape(M, N), R.reshape(M, N))
                # X as the first N columns of a K x (2N + 1) device buffer
                # (its other columns NaN), Y rows of stride N + 3
                Xw = np.full((K, 2 * N + 1), np.nan, np.float32)
                Xw[:, :N] = X
                dX = torch.from_numpy(Xw).cuda()
                dY = torch.zeros((M, N + 3), dtype=torch.float32, device="cuda")
                torch.cuda.synchronize()
                W.spmm_dev(dX.data_ptr(), N, dY.data_ptr(), ldx=2 * N + 1, ldy=N + 3, mode="fast")
                ctx.synchronize()
                Yw = dY.cpu().numpy()
                check_fast(Yw[:, :N], R.reshape(M, N))
                assert not Yw[:, N:].any()
            W.free()


def test_strict_vector_row_chains(ctx):
    """The strict N = 1 kernel over the row-sorted chain copy: row lengths at
    the 4-step and 256-step chunk edges and past several chunks, empty rows,
    a row count that is not a multiple of 64, int32 columns (K > 65536),
    +-inf and NaN in x at column 0 (the column padding steps point at: their
    products must not reach any sum), a strided x, and the Gemm form with
    one activation row, bias and fused activations.  Bit-exact against the
    oracle."""
    import torch

    rng = np.random.default_rng(17)
    lens = [0, 1, 3, 4, 5, 255, 256, 257, 511, 512, 513, 1024, 1500, 0, 7, 64, 300, 2, 9, 777] * 5
    lens = lens[:97]
    for K in (4096, 70000):
        ip = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
        ix = np.concatenate([np.sort(rng.choice(K, n, replace=False)) for n in lens]).astype(np.int64)
        v = rng.standard_normal(len(ix)).astype(np.float32)
        M = len(lens)
        W = ctx.csr_upload(M, K, ip, ix, v)
        x = rng.standard_normal(K).astype(np.float32)
        say(f"strict SpMV row chains M={M} K={K}")
        assert bits_equal(W.spmm(x), O.orc_csr_spmv(M, K, ip, ix, v, x)), K
        for bad in (np.inf, -np.inf, np.nan):
            xb = x.copy()
            xb[0] = bad
            assert bits_equal(W.spmm(xb), O.orc_csr_spmv(M, K, ip, ix, v, xb)), (K, bad)
        # int8 values with per-row scales
        q = rng.integers(-127, 128, len(ix)).astype(np.int8)
        q[q == 0] = 1
        sc = (rng.random(M) * 0.01 + 1e-3).astype(np.float32)
        Wq = ctx.csr_upload(M, K, ip, ix, q, row_scales=sc)
        vals = workloads.dequant_rows(ip, q, sc)
        assert bits_equal(Wq.spmm(x), O.orc_csr_spmv(M, K, ip, ix, vals, x)), K
        # strided x (column 1 of a K x 3 matrix), strided y
        X3 = rng.standard_normal((K, 3)).astype(np.float32)
        dX = torch.from_numpy(X3).cuda()
        dY = torch.zeros((M, 2), device="cuda")
        W.spmm_dev(dX.data_ptr() + 4, 1, dY.data_ptr(), ldx=3, ldy=2)
        ctx.synchronize()
        assert bits_equal(dY.cpu().numpy()[:, 0], O.orc_csr_spmv(M, K, ip, ix, v, X3[:, 1].copy())), K
        # 2 .. 8 columns (one in-order chain per row and column), with +-inf
        # and NaN in the first and last x rows (padding steps clamp there)
        for n in (2, 3, 4, 5, 8):
            Xn = rng.standard_normal((K, n)).astype(np.float32)
            Xn[0, 0], Xn[K - 1, n - 1], Xn[K - 1, 0] = np.inf, np.nan, -np.inf
            say(f"strict row chains M={M} K={K} N={n}")
            assert bits_equal(W.spmm(Xn), O.orc_csr_spmm(M, K, ip, ix, v, Xn)), (K, n)
            assert bits_equal(Wq.spmm(Xn), O.orc_csr_spmm(M, K, ip, ix, vals, Xn)), (K, n)
        # strided X and Y for several columns
        X9 = rng.standard_normal((K, 9)).astype(np.float32)
        dX = torch.from_numpy(X9).cuda()
        dY = torch.zeros((M, 11), device="cuda")
        W.spmm_dev(dX.data_ptr(), 8, dY.data_ptr(), ldx=9, ldy=11)
        ctx.synchronize()
        assert bits_equal(dY.cpu().numpy()[:, :8], O.orc_csr_spmm(M, K, ip, ix, v, X9[:, :8].copy())), K
        W.free()
        Wq.free()
    # long rows (mean >= 1024: the 16-row slab layout and its 1..8-column
    # kernels), empty and single-entry rows among them
    K = 6000
    lens = list(rng.integers(1024, 3000, 90)) + [0, 1, 5999, 6000, 4, 1023, 1024, 1025]
    M = len(lens)
    ip = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    ix = np.concatenate([np.sort(rng.choice(K, n, replace=False)) for n in lens]).astype(np.int64)
    v = rng.standard_normal(len(ix)).astype(np.float32)
    q = rng.integers(-127, 128, len(ix)).astype(np.int8)
    q[q == 0] = 3
    sc = (rng.random(M) * 0.01 + 1e-3).astype(np.float32)
    vals = workloads.dequant_rows(ip, q, sc)
    W = ctx.csr_upload(M, K, ip, ix, v)
    Wq = ctx.csr_upload(M, K, ip, ix, q, row_scales=sc)
    for n in (1, 2, 3, 4, 7, 8):
        Xn = rng.standard_normal((K, n)).astype(np.float32)
        Xn[0, 0], Xn[K - 1, n - 1] = np.inf, np.nan
        Xa = Xn[:, 0].copy() if n == 1 else Xn
        say(f"strict long-row chains M={M} K={K} N={n}")
        assert bits_equal(W.spmm(Xa), O.orc_csr_spmm(M, K, ip, ix, v, Xa)), n
        assert bits_equal(Wq.spmm(Xa), O.orc_csr_spmm(M, K, ip, ix, vals, Xa)), n
    W.free()
    Wq.free()
    # Gemm form, one activation row: y = a . B + bias, then Relu / Gelu
    K, Nf = 3000, 700
    B = rng.standard_normal((K, Nf)).astype(np.float32)
    B[rng.random(B.shape) >= 0.2] = 0
    BT = ctx.csr_from_dense(B, transpose=True)
    a = rng.standard_normal((1, K)).astype(np.float32)
    bias = rng.standard_normal(Nf).astype(np.float32)
    ref = O.orc_gemm(a, B, bias, 1.0, 1.0)
    say("Gemm form, one row, bias")
    assert bits_equal(ctx.gemm_csr(a, BT, 1.0, 1.0, bias), ref)
    dA = torch.from_numpy(a).cuda()
    dB = torch.from_numpy(bias).cuda()
    dY = torch.empty((1, Nf), device="cuda")
    ctx.gemm_csr_dev(dA.data_ptr(), 1, K, BT, dY.data_ptr(), 1.0, 1.0, dB.data_ptr(), Nf, relu=True)
    ctx.synchronize()
    assert bits_equal(dY.cpu().numpy(), relu_ref(ref))
    ctx.gemm_csr_dev(dA.data_ptr(), 1, K, BT, dY.data_ptr(), 1.0, 1.0, dB.data_ptr(), Nf, gelu=True)
    ctx.synchronize()
    assert bits_equal(dY.cpu().numpy(), ctx.gelu(ref))


def test_int8_csr_dequant_fused(ctx):
    """int8 CSR values with per-row scales: every product uses
    RN((float)q * scale[row]), i.e. dequantize_tensor followed by the fp32
    CSR kernels, bit for bit.  Skewed (lognormal) rows, N = 1 .. 100, and the
    Gemm form with an int8 weight in the B position."""
    ip, ix, q, sc = workloads.csr_int8_lognormal(1500, 2100, 0.3, 0.5, 0.02, seed=31)
    vals = workloads.dequant_rows(ip, q, sc)
    # the dequantised values are what the oracle's dequantize_tensor gives
    dense_q = np.zeros((1500, 2100), np.int8)
    dense_q[np.repeat(np.arange(1500), np.diff(ip)), ix] = q
    dq = O.orc_dequantize(dense_q, sc, np.zeros(1500, np.int32), O.I8, (1, 1500, 2100))
    assert np.array_equal(dq[dense_q != 0].view(np.uint32),
                          vals.view(np.uint32)[np.argsort(np.repeat(np.arange(1500), np.diff(ip)) * 2100 + ix,
                                                          kind="stable")])
    W = ctx.csr_upload(1500, 2100, ip, ix, q, row_scales=sc)
    rng = np.random.default_rng(4)
    for N in (1, 2, 8, 64, 100):
        say(f"int8 CSR N={N}")
        X = rng.standard_normal((2100, N)).astype(np.float32)
        Xa = X[:, 0] if N == 1 else X
        assert bits_equal(W.spmm(Xa), O.orc_csr_spmm(1500, 2100, ip, ix, vals, Xa)), N
    # fast mode (reassociated wave sums for N <= 8): normwise within 1e-5
    for N in (1, 3, 8):
        X = rng.standard_normal((2100, N)).astype(np.float32)
        Xa = X[:, 0] if N == 1 else X
        R = O.orc_csr_spmm(1500, 2100, ip, ix, vals, Xa)
        Y = W.spmm(Xa, mode="fast")
        assert np.abs(Y - R).max() <= 1e-5 * np.abs(R).max(), N
    # Gemm form: Y = A . B with B = dequantised W^T (the CSR is of B^T)
    A = rng.standard_normal((37, 2100)).astype(np.float32)
    bias = rng.standard_normal(1500).astype(np.float32)
    Bd = np.zeros((2100, 1500), np.float32)
    Bd[ix, np.repeat(np.arange(1500), np.diff(ip))] = vals
    say("int8 CSR Gemm form")
    assert bits_equal(ctx.gemm_csr(A, W, 1.0, 1.0, bias), O.orc_gemm(A, Bd, bias, 1.0, 1.0))


def relu_ref(y):
    """activation.cpp:45-60: std::max(0.0f, v) = (0 < v) ? v : +0, so -0 and
    NaN map to +0."""
    return np.where(y > 0, y, np.float32(0)).astype(np.float32)


def test_fused_relu_epilogue(ctx, cfg_weight):
    """The Relu fused into the product epilogue (PFR_ACT_RELU) equals the
    product followed by a separate Relu, bit for bit, on every kernel the
    dispatch picks: the small-N and vector SpMV forms, the row kernels and
    the column-slice kernel, in both math modes; infinities and NaNs in the
    sums included."""
    import torch

    ip, ix, v = cfg_weight
    W = ctx.csr_upload(4096, 4096, ip, ix, v)
    rng = np.random.default_rng(8)
    for N in (1, 3, 8, 40, 256):
        X = rng.standard_normal((4096, N)).astype(np.float32)
        X[0, :] = np.inf
        X[1, :] = -np.inf
        dX = torch.from_numpy(X).cuda()
        dY = torch.empty((4096, N), dtype=torch.float32, device="cuda")
        for mode in ("strict", "fast"):
            say(f"fused relu spmm N={N} {mode}")
            W.spmm_dev(dX.data_ptr(), N, dY.data_ptr(), mode=mode)
            ctx.synchronize()
            plain = dY.cpu().numpy()
            W.spmm_dev(dX.data_ptr(), N, dY.data_ptr(), mode=mode, relu=True)
            ctx.synchronize()
            fused = dY.cpu().numpy()
            assert np.isnan(plain).any() and (plain < 0).any()
            assert bits_equal(fused, relu_ref(plain)), (N, mode, first_diff(fused, relu_ref(plain)))
            if mode == "strict":
                ref = O.orc_csr_spmm(4096, 4096, ip, ix, v, X)
                assert bits_equal(fused, relu_ref(ref)), (N, first_diff(fused, relu_ref(ref)))
    # Gemm form with bias and beta: Y = relu(alpha * A . B + beta * C)
    B = np.zeros((600, 700), np.float32)
    m = rng.random((600, 700)) < 0.2
    B[m] = rng.standard_normal(int(m.sum())).astype(np.float32) * 0.1
    BT = ctx.csr_from_dense(B, transpose=True)
    bias = rng.standard_normal(700).astype(np.float32)
    dC = torch.from_numpy(bias).cuda()
    for Mb in (1, 5, 32, 200):
        A = rng.standard_normal((Mb, 600)).astype(np.float32)
        dA = torch.from_numpy(A).cuda()
        dY = torch.empty((Mb, 700), dtype=torch.float32, device="cuda")
        for mode in ("strict", "fast"):
            say(f"fused relu gemm Mb={Mb} {mode}")
            ctx.gemm_csr_dev(dA.data_ptr(), Mb, 600, BT, dY.data_ptr(), 0.5, 2.0, dC.data_ptr(), 700, mode=mode)
            ctx.synchronize()
            plain = dY.cpu().numpy()
            ctx.gemm_csr_dev(dA.data_ptr(), Mb, 600, BT, dY.data_ptr(), 0.5, 2.0, dC.data_ptr(), 700, mode=mode,
                             relu=True)
            ctx.synchronize()
            fused = dY.cpu().numpy()
            assert bits_equal(fused, relu_ref(plain)), (Mb, mode)
            if mode == "strict":
                ref = O.orc_gemm(A, B, bias, 0.5, 2.0)
                assert bits_equal(fused, relu_ref(ref)), (Mb, first_diff(fused, relu_ref(ref)))
    # int8 CSR weight (dequantisation and Relu both in the kernel)
    ip8, ix8, q, sc = workloads.csr_int8_lognormal(900, 1000, 0.2, 0.5, 0.02, seed=3)
    W8 = ctx.csr_upload(900, 1000, ip8, ix8, q, row_scales=sc)
    vals = workloads.dequant_rows(ip8, q, sc)
    for N in (1, 8, 64):
        X = rng.standard_normal((1000, N)).astype(np.float32)
        dX = torch.from_numpy(X).cuda()
        dY = torch.empty((900, N), dtype=torch.float32, device="cuda")
        say(f"fused relu int8 spmm N={N}")
        W8.spmm_dev(dX.data_ptr(), N, dY.data_ptr(), relu=True)
        ctx.synchronize()
        ref = relu_ref(O.orc_csr_spmm(900, 1000, ip8, ix8, vals, X))
        assert bits_equal(dY.cpu().numpy(), ref), N
