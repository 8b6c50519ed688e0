"""Derived copies built on first use, through pfr_csr_device_bytes: a handle
starts with the CSR itself (uint16 columns when K <= 65536, values, row
pointers, row scales), the row-block table and the merge-path partition;
the first product that runs on the nnz-balanced copy (fast, 2 <= N <= 8),
the row-chain copy (strict, N <= 8) or the sliced-ELL copy (float32,
N >= 16) builds it, and later products reuse it.  Products match the oracle
as everywhere else (strict bit for bit, fast within 1e-5 normwise).  A
product captured into a HIP graph while its copy is still pending builds
nothing and reads the CSR in place: in strict mode the same bits as the
copy's kernel, on every replay, before and after the copy exists."""
import sys

import numpy as np
import pytest

from oracle import oracle as O
from pyflamert_amd import workloads

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def close_normwise(Y, R, tol=1e-5):
    Y = np.asarray(Y, np.float64)
    R = np.asarray(R, np.float64)
    scale = max(float(np.abs(R).max()), 1e-30)
    return bool(np.abs(Y - R).max() <= tol * scale)


@pytest.fixture(scope="module")
def ctx():
    from pyflamert_amd import rocm

    c = rocm.Context(0)
    yield c
    c.close()


def test_int8_decode_weight_footprint(ctx):
    """4096 x 4096 int8 decode weight at 30 % (lognormal rows): about 3 bytes
    per nonzero after upload, unchanged by batch-1 fast products (the
    merge-path kernel reads the CSR in place); the first batch-8 fast product
    adds the balanced copy (int8 value + uint16 offset per padded entry), the
    first strict product the row-chain copy, each once."""
    M, K = 4096, 4096
    ip, ix, q, sc = workloads.csr_int8_lognormal(M, K, 0.3, 0.5, 0.02, seed=41)
    nnz = len(ix)
    vals = workloads.dequant_rows(ip, q, sc)
    W = ctx.csr_upload(M, K, ip, ix, q, row_scales=sc)
    rng = np.random.default_rng(42)
    x1 = rng.standard_normal(K).astype(np.float32)
    x8 = rng.standard_normal((K, 8)).astype(np.float32)
    b0 = W.device_bytes()
    say(f"int8 {M}x{K} nnz={nnz}: {b0 / nnz:.4f} B/nnz after upload")
    assert 3 * nnz <= b0 <= 3.1 * nnz
    Y = W.spmm(x1, mode="fast")
    assert W.device_bytes() == b0
    assert close_normwise(Y, O.orc_csr_spmm(M, K, ip, ix, vals, x1))
    Y8 = W.spmm(x8, mode="fast")
    b1 = W.device_bytes()
    say(f"after the first batch-8 fast product: {b1 / nnz:.4f} B/nnz")
    assert 3 * nnz <= b1 - b0 <= 3.2 * nnz
    assert close_normwise(Y8, O.orc_csr_spmm(M, K, ip, ix, vals, x8))
    assert np.array_equal(bits(W.spmm(x8, mode="fast")), bits(Y8))
    assert W.device_bytes() == b1
    Ys = W.spmm(x1, mode="strict")
    b2 = W.device_bytes()
    say(f"after the first strict product: {b2 / nnz:.4f} B/nnz")
    assert 3 * nnz <= b2 - b1 <= 3.3 * nnz
    assert np.array_equal(bits(Ys), bits(O.orc_csr_spmm(M, K, ip, ix, vals, x1)))
    Ys8 = W.spmm(x8, mode="strict")
    assert W.device_bytes() == b2
    assert np.array_equal(bits(Ys8), bits(O.orc_csr_spmm(M, K, ip, ix, vals, x8)))
    W.free()


@pytest.mark.parametrize("K", [3000, 70000])
def test_float_weight_copies_on_first_use(ctx, K):
    """Float32 weights, uint16 columns (K = 3000) and int32 ones (K =
    70000, past uint16): 6 and 8 bytes per nonzero after upload; N = 64
    builds the sliced-ELL copy, strict N = 3 the row-chain copy, fast N = 4
    the balanced copy (where K allows it); every product against the
    oracle."""
    M = 1500
    ip, ix, v = workloads.csr_uniform(M, K, 0.05 if K < 10000 else 0.004, 0.02, seed=K)
    nnz = len(ix)
    W = ctx.csr_upload(M, K, ip, ix, v)
    per = 6 if K <= 65536 else 8
    b = W.device_bytes()
    say(f"float32 {M}x{K} nnz={nnz}: {b / nnz:.4f} B/nnz after upload")
    assert per * nnz <= b <= per * nnz + 64 * M + (1 << 20)
    rng = np.random.default_rng(K + 1)
    for N, mode in ((64, "strict"), (64, "fast"), (3, "strict"), (4, "fast"), (1, "strict"), (8, "fast")):
        X = rng.standard_normal((K, N)).astype(np.float32)
        Y = W.spmm(X, mode=mode)
        R = O.orc_csr_spmm(M, K, ip, ix, v, X)
        nb = W.device_bytes()
        say(f"  N={N} {mode}: {nb / nnz:.4f} B/nnz")
        assert nb >= b
        b = nb
        if mode == "strict":
            assert np.array_equal(bits(Y), bits(R)), (N, mode)
        else:
            assert close_normwise(Y, R), (N, mode)
    W.free()


def test_capture_before_copy_reads_in_place(ctx):
    """Strict batch-1 and batch-4 products and a fast batch-8 one captured
    on a fresh int8 handle: the capture allocates nothing (device bytes
    unchanged), and each replay -- before the eager products build the
    copies and after -- gives the strict copies' bits and the fast result
    within 1e-5 normwise of the oracle."""
    import torch

    M, K = 2048, 3000
    ip, ix, q, sc = workloads.csr_int8_lognormal(M, K, 0.3, 0.5, 0.02, seed=43)
    vals = workloads.dequant_rows(ip, q, sc)
    W = ctx.csr_upload(M, K, ip, ix, q, row_scales=sc)
    g = torch.Generator(device="cuda").manual_seed(44)
    x1 = torch.randn((K, 1), device="cuda", generator=g)
    x4 = torch.randn((K, 4), device="cuda", generator=g)
    x8 = torch.randn((K, 8), device="cuda", generator=g)
    out = {k: torch.empty((M, n), device="cuda") for k, n in (("s1", 1), ("s4", 4), ("f8", 8))}

    def run(o):
        W.spmm_dev(x1.data_ptr(), 1, o["s1"].data_ptr(), mode="strict")
        W.spmm_dev(x4.data_ptr(), 4, o["s4"].data_ptr(), mode="strict")
        W.spmm_dev(x8.data_ptr(), 8, o["f8"].data_ptr(), mode="fast")

    main = torch.cuda.current_stream().cuda_stream
    torch.cuda.synchronize()
    b0 = W.device_bytes()
    graph = torch.cuda.CUDAGraph()
    say(f"capture on a fresh {M}x{K} int8 handle")
    with torch.cuda.graph(graph):
        ctx.set_stream(torch.cuda.current_stream().cuda_stream)
        run(out)
    ctx.set_stream(main)
    assert W.device_bytes() == b0
    R = {"s1": O.orc_csr_spmm(M, K, ip, ix, vals, x1.cpu().numpy()),
         "s4": O.orc_csr_spmm(M, K, ip, ix, vals, x4.cpu().numpy()),
         "f8": O.orc_csr_spmm(M, K, ip, ix, vals, x8.cpu().numpy())}
    eager = {k: torch.empty_like(v) for k, v in out.items()}
    for rep in range(3):
        for v in out.values():
            v.fill_(7)
        graph.replay()
        torch.cuda.synchronize()
        if rep == 1:
            run(eager)  # builds the row-chain and balanced copies
            torch.cuda.synchronize()
            assert W.device_bytes() > b0
            for k in ("s1", "s4"):
                assert np.array_equal(bits(eager[k].cpu().numpy()), bits(R[k])), k
            assert close_normwise(eager["f8"].cpu().numpy(), R["f8"])
        say(f"replay {rep}")
        for k in ("s1", "s4"):
            assert np.array_equal(bits(out[k].cpu().numpy()), bits(R[k])), (rep, k)
        assert close_normwise(out["f8"].cpu().numpy(), R["f8"]), rep
    del graph
    W.free()
