"""GPU pruning-mask producers against the reference's masks.

Bar: bit-exact (the float 0/1 masks compared as arrays).  Pins: the golden
masks written by the compiled reference (magnitude at 0.9 on the MLP
weights, tie-heavy vectors at five sparsities and six N:M ratios, a
Gaussian matrix), the oracle restatement on tie-heavy, boundary-crossing
and full-size inputs, and the compiled reference itself where it is built.
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


def same(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.fixture(scope="module")
def ctx():
    from pyflamert_amd import rocm

    c = rocm.Context(0)
    yield c
    c.close()


def test_masks_golden(ctx, golden):
    g = golden("masks.npz")
    say("masks: golden vectors")
    for w, key, n_el in ((g["w1"], "w1_mask90", 784 * 512), (g["w2"], "w2_mask90", 512 * 10)):
        m = ctx.magnitude_mask(w, 0.9)
        assert m.shape == w.shape
        assert np.array_equal(m.ravel() != 0, np.unpackbits(g[key])[:n_el].astype(bool)), key
    assert int(ctx.magnitude_mask(g["w1"], 0.9).sum()) == 40141
    t = g["ties"]
    for s in (0.1, 0.3, 0.5, 0.9, 0.999):
        assert same(ctx.magnitude_mask(t, s), g[f"ties_mag_{s}"]), s
    for n, m in ((2, 4), (1, 4), (3, 8), (2, 3), (5, 7), (4, 4)):
        assert same(ctx.nm_mask(t, n, m), g[f"ties_nm_{n}_{m}"]), (n, m)
    assert same(ctx.nm_mask(g["gauss"], 2, 4), g["gauss_nm_2_4"])
    assert same(ctx.magnitude_mask(g["gauss"], 0.8), g["gauss_mag_0.8"])


def tie_heavy(rng, n):
    """Small integers (many equal magnitudes), signed zeros and infinities."""
    w = rng.integers(-6, 7, n).astype(np.float32)
    w[rng.random(n) < 0.05] = -0.0
    w[rng.random(n) < 0.002] = np.inf
    w[rng.random(n) < 0.002] = -np.inf
    return w


@pytest.mark.parametrize("n", [1, 2, 5, 4095, 4096, 4097, 3 * 4096 + 17, 100003])
def test_magnitude_ties_and_block_boundaries(ctx, n):
    rng = np.random.default_rng(n)
    w = tie_heavy(rng, n)
    say(f"magnitude mask n={n}")
    for s in (0.05, 0.3, 0.5, 0.7, 0.9, 0.9999):
        assert same(ctx.magnitude_mask(w, s), O.orc_magnitude_mask(w, s)), (n, s)
    for s in (0.0, -0.5, 1.0, 1.5):  # all ones / all zeros
        assert same(ctx.magnitude_mask(w, s), O.orc_magnitude_mask(w, s)), (n, s)


@pytest.mark.parametrize("total", [1, 3, 4, 5, 255, 4097, 100003])
def test_nm_ratios_and_partial_groups(ctx, total):
    rng = np.random.default_rng(total + 1)
    w = tie_heavy(rng, total)
    say(f"N:M mask total={total}")
    for n, m in ((2, 4), (1, 4), (3, 8), (2, 3), (5, 7), (4, 4), (7, 16), (1, 16), (16, 16), (1, 1)):
        assert same(ctx.nm_mask(w, n, m), O.orc_nm_mask(w, n, m)), (total, n, m)


def test_nm24_every_tie_pattern(ctx):
    """The closed-form 2:4 kernel on every group of four drawn from nine
    values (signed zeros, +-1, +-2, +-inf, NaN): 6561 groups, every pattern
    of ties the comparator |a| > |b| can meet, against the oracle's heap
    select and, where it is built, the reference's compute_mask."""
    vals = np.array([0.0, -0.0, 1.0, -1.0, 2.0, -2.0, np.inf, -np.inf, np.nan], np.float32)
    grid = np.stack(np.meshgrid(*([np.arange(len(vals))] * 4), indexing="ij"), -1).reshape(-1, 4)
    w = np.ascontiguousarray(vals[grid].ravel())
    say(f"2:4 mask, every tie pattern: {w.size // 4} groups")
    got = ctx.nm_mask(w, 2, 4)
    assert same(got, O.orc_nm_mask(w, 2, 4))
    if O.have_ref():
        assert same(got, O.ref_nm_mask(w, 2, 4))


@pytest.mark.parametrize("frac,s", [(0.01, 0.5), (0.01, 0.995), (0.2, 0.9), (0.3, 0.05)])
def test_magnitude_nan_weights(ctx, frac, s):
    """A NaN weight is never kept and counts among the zeros (the
    reference's comparisons); the threshold may fall on finite values or on
    a NaN.  Bit-identical to the oracle."""
    rng = np.random.default_rng(int(frac * 1000) + int(s * 1000))
    for n in (1000, 4096 * 3 + 5):
        w = tie_heavy(rng, n)
        w[rng.random(n) < frac] = np.nan
        say(f"magnitude mask with NaN n={n} frac={frac} s={s}")
        got = ctx.magnitude_mask(w, s)
        assert same(got, O.orc_magnitude_mask(w, s)), (n, frac, s)
        assert not got[np.isnan(w)].any()


def test_full_size_and_compiled_reference(ctx):
    """A 2:4 and a 70 % magnitude mask of a 4096 x 4096 N(0, 1) weight, and
    an 11008 x 4096 2:4 mask, against the oracle and (where it is built)
    the reference's own compute_mask."""
    import torch

    rng = np.random.default_rng(7)
    w = rng.standard_normal((4096, 4096)).astype(np.float32)
    say("full size: 4096 x 4096")
    m24 = ctx.nm_mask(w, 2, 4)
    assert same(m24, O.orc_nm_mask(w, 2, 4))
    assert np.all(m24.reshape(-1, 4).sum(1) == 2)
    mm = ctx.magnitude_mask(w, 0.7)
    assert same(mm, O.orc_magnitude_mask(w, 0.7))
    if O.have_ref():
        assert same(m24, O.ref_nm_mask(w, 2, 4))
        assert same(mm, O.ref_magnitude_mask(w, 0.7))
    # device-pointer entry points, 11008 x 4096 (config 3's weight)
    big = rng.standard_normal((11008, 4096)).astype(np.float32)
    dw = torch.from_numpy(big).cuda()
    dm = torch.empty_like(dw)
    ctx.nm_mask_dev(dw.data_ptr(), big.size, 2, 4, dm.data_ptr())
    ctx.synchronize()
    assert same(dm.cpu().numpy(), O.orc_nm_mask(big, 2, 4))


def test_mask_errors(ctx):
    with pytest.raises(_lib.InvalidArgument, match="Cannot prune empty weight tensor"):
        ctx.magnitude_mask(np.zeros(0, np.float32), 0.5)
    assert ctx.magnitude_mask(np.zeros(0, np.float32), 1.0).size == 0
    with pytest.raises(_lib.InvalidArgument, match="0 < n <= m"):
        ctx.nm_mask(np.ones(8, np.float32), 5, 4)
    with pytest.raises(_lib.InvalidArgument, match="larger than 16"):
        ctx.nm_mask(np.ones(64, np.float32), 2, 32)
