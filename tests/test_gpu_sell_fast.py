"""The fast mode's reordered copies: the sliced-ELL copy's fast runs (the
column-slice kernel, N >= 16; each row's terms reordered so that the four
slab rows whose X reads the LDS serves together take different bank
quarters) and the nnz-balanced copy (2 <= N <= 8; each row's terms reordered
so that the lanes the LDS serves together read X rows in different eighths
of the banks).

With small-integer weights and activations every product and partial sum is
an integer below 2^24, so any order of the terms gives the same fp32 bits:
the fast results must equal the oracle's exactly, which pins that a
reordered copy holds every stored term once (a dropped, repeated or moved
term changes an output by at least 1).  Also: a fresh handle's first fast
product builds only the fast copy and its tables, a strict product then adds
only the storage-order runs, and the footprint is the same in either order.
"""
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


@pytest.fixture(scope="module")
def ctx():
    from pyflamert_amd import rocm

    c = rocm.Context(0)
    yield c
    c.close()


def int_weight(M, K, density, seed, skew=False):
    """CSR with values in {-3 .. 3} minus 0; uniform or lognormal row lengths."""
    rng = np.random.default_rng(seed)
    if skew:
        ip, ix, _ = workloads.csr_lognormal_rows(M, K, density, 0.8, 1.0, seed)
    else:
        ip, ix, _ = workloads.csr_uniform(M, K, density, 1.0, seed)
    v = rng.integers(1, 4, len(ix)).astype(np.float32) * rng.choice(np.float32([-1, 1]), len(ix))
    return ip, ix, v


@pytest.mark.parametrize("M,K,density,skew", [(4096, 4096, 0.1, False), (1000, 4097, 0.08, True),
                                              (333, 2500, 0.3, True)])
def test_fast_copy_exact_on_integers(ctx, M, K, density, skew):
    """4096 x 4096 (four chunks, 16-wave launches at N = 256), 1000 x 4097
    (a partial slab, a one-row last chunk, skewed rows) and 333 x 2500 (one
    chunk, dense rows): N = 16, 64, 128, 256 in fast mode equal the oracle
    bit for bit on integer data."""
    ip, ix, v = int_weight(M, K, density, seed=M + K, skew=skew)
    W = ctx.csr_upload(M, K, ip, ix, v)
    rng = np.random.default_rng(K)
    for N in (16, 64, 128, 256):
        X = rng.integers(-4, 5, (K, N)).astype(np.float32)
        say(f"fast {M}x{K} nnz={len(ix)} N={N}")
        Y = W.spmm(X, mode="fast")
        R = O.orc_csr_spmm(M, K, ip, ix, v, X)
        assert np.abs(R).max() < 2 ** 24
        assert np.array_equal(bits(Y), bits(R)), N
    W.free()


def test_fast_copy_footprint_either_order(ctx):
    """Fast then strict, and strict then fast, on fresh handles of the same
    weight: each mode's first N = 64 product adds its own runs (the first
    one also the slab tables), and both handles end at the same size."""
    M, K = 2048, 3000
    ip, ix, v = int_weight(M, K, 0.1, seed=7)
    nnz = len(ix)
    rng = np.random.default_rng(8)
    X = rng.integers(-4, 5, (K, 64)).astype(np.float32)
    R = O.orc_csr_spmm(M, K, ip, ix, v, X)
    ends = []
    for order in (("fast", "strict"), ("strict", "fast")):
        W = ctx.csr_upload(M, K, ip, ix, v)
        b = [W.device_bytes()]
        for mode in order:
            assert np.array_equal(bits(W.spmm(X, mode=mode)), bits(R)), (order, mode)
            b.append(W.device_bytes())
            assert np.array_equal(bits(W.spmm(X, mode=mode)), bits(R)), (order, mode)
            assert W.device_bytes() == b[-1]  # built once
        say(f"{order}: {[(x - b[0]) / nnz for x in b]} B/nnz added")
        runs = b[2] - b[1]  # the second copy: its runs only
        assert runs >= 8 * nnz
        assert b[1] - b[0] > runs  # the first copy brought the tables too
        ends.append(b[2])
        W.free()
    assert ends[0] == ends[1]


@pytest.mark.parametrize("M,K,i8", [(4096, 4096, True), (1000, 11008, True), (777, 5000, False)])
def test_balanced_copy_exact_on_integers(ctx, M, K, i8):
    """Fast N = 2, 5, 8 (the nnz-balanced copy, reordered) on skewed rows:
    int8 weights with unit row scales over one chunk (4096 x 4096) and
    three (1000 x 11008), and an integer-valued float32 weight, all bit for
    bit against the oracle."""
    rng = np.random.default_rng(M + K)
    ip, ix, _ = workloads.csr_lognormal_rows(M, K, 0.3, 0.5, 1.0, seed=M * 3 + K)
    q = (rng.integers(1, 100, len(ix)) * rng.choice([-1, 1], len(ix))).astype(np.int8)
    v = q.astype(np.float32)
    if i8:
        W = ctx.csr_upload(M, K, ip, ix, q, row_scales=np.ones(M, np.float32))
    else:
        W = ctx.csr_upload(M, K, ip, ix, v)
    for N in (2, 5, 8):
        X = rng.integers(-4, 5, (K, N)).astype(np.float32)
        say(f"balanced fast {M}x{K} nnz={len(ix)} N={N} i8={i8}")
        Y = W.spmm(X, mode="fast")
        R = O.orc_csr_spmm(M, K, ip, ix, v, X)
        assert np.abs(R).max() < 2 ** 24
        assert np.array_equal(bits(Y), bits(R)), N
    W.free()


def test_balanced_copy_skewed_classes(ctx):
    """The balanced copy's term order where the choice is hardest, fast
    N = 2 and 8 bit for bit against the oracle: rows whose columns all fall
    in one class mod 8 of their chunk, rows with two classes, empty rows,
    rows confined to the first of three chunks (the others hold no terms of
    theirs), and one row with every column (a group of its own), as int8
    (unit scales) and integer-valued float32."""
    M, K = 600, 9000  # three chunks of 3000 columns
    rng = np.random.default_rng(77)
    rows = []
    for r in range(M):
        kind = r % 5
        if r == 7:
            c = np.arange(K)
        elif kind == 0:
            c = np.array([], np.int64)
        elif kind == 1:  # class 3 of chunk 0 only
            c = np.sort(rng.choice(np.arange(3, 3000, 8), int(rng.integers(1, 300)), replace=False))
        elif kind == 2:  # classes 0 and 5 of every chunk
            base = np.concatenate([np.arange(ch * 3000, ch * 3000 + 3000, 8) for ch in range(3)])
            pool = np.concatenate([base, base + 5])
            c = np.sort(rng.choice(pool, int(rng.integers(1, 1200)), replace=False))
        else:
            c = np.sort(rng.choice(K, int(rng.integers(0, 2700)), replace=False))
        rows.append(c.astype(np.int64))
    ip = np.zeros(M + 1, np.int64)
    np.cumsum([len(c) for c in rows], out=ip[1:])
    ix = np.concatenate(rows)
    q = (rng.integers(1, 100, len(ix)) * rng.choice([-1, 1], len(ix))).astype(np.int8)
    v = q.astype(np.float32)
    for tag, W in (("int8", ctx.csr_upload(M, K, ip, ix, q, row_scales=np.ones(M, np.float32))),
                   ("fp32", ctx.csr_upload(M, K, ip, ix, v))):
        for N in (2, 8):
            X = rng.integers(-4, 5, (K, N)).astype(np.float32)
            say(f"balanced skewed classes {tag} N={N} nnz={len(ix)}")
            Y = W.spmm(X, mode="fast")
            R = O.orc_csr_spmm(M, K, ip, ix, v, X)
            assert np.abs(R).max() < 2 ** 24
            assert np.array_equal(bits(Y), bits(R)), (tag, N)
        W.free()
