"""Pin the CPU oracle to the reference: every golden vector (written by the
compiled reference sources) must be reproduced bit-for-bit, and the
mathematical checks below cover what the vectors leave open.  CPU only."""
import gzip
import hashlib
import json
import os

import numpy as np
import pytest

from oracle import oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a


def same(a, b):
    return np.array_equal(bits(a), bits(b))


def test_manifest_hashes():
    man = json.load(open(os.path.join(GOLD, "MANIFEST.json")))
    for name, meta in man.items():
        if name.startswith("_"):
            continue
        data = open(os.path.join(GOLD, name), "rb").read()
        assert hashlib.sha256(data).hexdigest() == meta["sha256"], name


def test_kat_matmul(golden):
    # tests/cpp/test_executor.cpp:162-208
    g = golden("kat_matmul.npz")
    out = O.orc_matmul(g["a"], g["b"])
    assert same(out, g["out"])
    assert out.tolist() == [[22.0, 28.0], [49.0, 64.0]]


def test_gemm_golden(golden):
    g = golden("gemm.npz")
    for i in range(int(g["n"])):
        al, be, ta, tb = g[f"c{i}_p"]
        C = g[f"c{i}_C"]
        out = O.orc_gemm(g[f"c{i}_A"], g[f"c{i}_B"], C if C.size else None, al, be, int(ta), int(tb))
        assert same(out, g[f"c{i}_out"]), i


def test_matmul_golden(golden):
    g = golden("matmul.npz")
    for i in range(int(g["n"])):
        out = O.orc_matmul(g[f"c{i}_a"], g[f"c{i}_b"])
        assert same(out, g[f"c{i}_out"]), i


def test_csr_golden(golden):
    g = golden("csr.npz")
    W = g["W"]
    for tag, thr in (("t0", 0.0), ("t1", 0.005)):
        ip, ix, v = O.orc_to_sparse_csr(W, thr)
        assert np.array_equal(ip, g[f"{tag}_indptr"])
        assert np.array_equal(ix, g[f"{tag}_indices"])
        assert same(v, g[f"{tag}_values"])
    ip, ix, v = g["t0_indptr"], g["t0_indices"], g["t0_values"]
    M, K = W.shape
    for n in (1, 8, 64):
        assert same(O.orc_csr_spmm(M, K, ip, ix, v, g[f"X{n}"]), g[f"Y{n}"]), n
    assert same(O.orc_csr_spmv(M, K, ip, ix, v, g["x"]), g["y_matvec"])
    assert same(O.orc_csr_spmm(M, K, ip, ix, v, g["x"]), g["y_1d"])
    zi, zx, _ = O.orc_to_sparse_csr(np.zeros((3, 4), np.float32))
    assert np.array_equal(zi, g["zero_indptr"]) and len(zx) == int(g["zero_nnz"]) == 0


def test_masks_golden(golden):
    g = golden("masks.npz")
    for w, key, n_el in ((g["w1"], "w1_mask90", 784 * 512), (g["w2"], "w2_mask90", 512 * 10)):
        m = O.orc_magnitude_mask(w, 0.9)
        ref = np.unpackbits(g[key])[:n_el].astype(bool)
        assert np.array_equal(m.ravel() != 0, ref), key
    # 784x512 at 0.9 keeps 40,141; 512x10 keeps 512 (float target_zeros).
    assert int(O.orc_magnitude_mask(g["w1"], 0.9).sum()) == 40141
    assert int(O.orc_magnitude_mask(g["w2"], 0.9).sum()) == 512
    t = g["ties"]
    for s in (0.1, 0.3, 0.5, 0.9, 0.999):
        assert same(O.orc_magnitude_mask(t, s), g[f"ties_mag_{s}"]), s
    for n, m in ((2, 4), (1, 4), (3, 8), (2, 3), (5, 7), (4, 4)):
        assert same(O.orc_nm_mask(t, n, m), g[f"ties_nm_{n}_{m}"]), (n, m)
    assert same(O.orc_nm_mask(g["gauss"], 2, 4), g["gauss_nm_2_4"])
    assert same(O.orc_magnitude_mask(g["gauss"], 0.8), g["gauss_mag_0.8"])
    assert same(O.orc_apply_mask(g["am_t"], g["am_mask"]), g["am_out"])


def test_quant_golden(golden):
    g = golden("quant.npz")
    xs = g["x"]
    for dt, zp in ((O.I8, 0), (O.I8, -3), (O.U8, 128), (O.U8, 7)):
        assert np.array_equal(O.orc_quantize(xs, [0.05], [zp], dt), g[f"q_{dt}_{zp}"]), (dt, zp)
    v = (3, 5, 7)
    assert np.array_equal(O.orc_quantize(g["xc"], g["xc_scales"], g["xc_zps"], O.I8, v), g["qc_i8"])
    assert np.array_equal(O.orc_quantize(g["xc"], g["xc_scales"], np.array([128, 120, 130, 0, 255]),
                                         O.U8, v), g["qc_u8"])
    assert same(O.orc_dequantize(np.arange(-128, 128, dtype=np.int8), [0.05], [3], O.I8), g["dq_i8"])
    assert same(O.orc_dequantize(np.arange(0, 256, dtype=np.uint8), [0.1], [128], O.U8), g["dq_u8"])
    assert same(O.orc_dequantize(g["qcv"], g["xc_scales"], g["xc_zps"], O.I8, v), g["dqc_i8"])
    for mn, mx, dt, sym, sc, z in g["minmax"]:
        s2, z2 = O.orc_params_from_minmax(float(mn), float(mx), int(dt), bool(sym))
        assert np.float32(s2) == np.float32(sc) and z2 == int(z), (mn, mx, dt, sym)
    for dt, sym, sc, z in g["dyn"]:
        s2, z2 = O.orc_dynamic_params(g["dyn_x"], int(dt), bool(sym))
        assert np.float32(s2) == np.float32(sc) and z2 == int(z)
    for dt in (O.I8, O.U8):
        for sym in (True, False):
            s2, z2 = O.orc_dynamic_params_per_channel(g["pc_x"], dt, sym)
            assert same(s2, g[f"pc_{dt}_{int(sym)}_s"]) and np.array_equal(z2, g[f"pc_{dt}_{int(sym)}_z"])


def test_qmatmul_golden(golden):
    g = golden("qmatmul.npz")
    a, b = g["a"], g["b"]
    assert same(O.orc_quantized_matmul(a, b, 0.02, 0.05), g["f_zp0"])
    assert same(O.orc_quantized_matmul(a, b, 0.02, 0.05, 3, -2), g["f_zp"])
    sc, z = g["rq_params"]
    f = O.orc_quantized_matmul(a, b, 0.02, 0.05)
    assert np.array_equal(O.orc_quantize(f, [sc], [int(z)], O.I8), g["rq_i8"])
    assert same(O.orc_quantized_matmul(g["au"], b, 0.02, 0.05, 128, 0), g["f_u8"])
    assert same(O.orc_cpu_quantized_matmul(a, b, 0.02, 0.05, 1, -1), g["op_qmm"])
    assert same(O.orc_cpu_quantized_matmul(g["au"], b, 0.02, 0.05, 0, 0), g["op_qmm_u8"])
    # 2:4 weight path with a per-tensor weight scale
    w = g["sp_w"]
    assert same(O.orc_apply_mask(w, O.orc_nm_mask(w, 2, 4)), w)
    ws, _ = O.orc_dynamic_params(w)
    assert np.float32(ws) == g["sp_ws"]
    assert np.array_equal(O.orc_quantize(w, [ws], [0]), g["sp_wq"])
    yf = O.orc_quantized_matmul(g["sp_wq"], g["sp_xq"], float(ws), 0.05)
    assert same(yf, g["sp_yf"])
    ys, yz = g["sp_y_params"]
    assert np.array_equal(O.orc_quantize(yf, [ys], [int(yz)]), g["sp_yq"])
    # per-row generalisation with all row scales equal == the reference kernel
    rows = np.full(w.shape[0], g["sp_ws"], np.float32)
    assert same(O.orc_quantized_matmul_rowscale(g["sp_wq"], g["sp_xq"], rows, 0.05), g["sp_yf"])


def test_quantized_matmul_rowscale_distinct_scales():
    """The per-row form with a different scale on every row: each output is
    (float)acc * RN(s_row * x_scale) (quant_ops.cpp:435, :456-466), with acc
    the exact integer accumulator.  A wrong row index for the scale (say row
    0's on every row, or the transposed operand) fails this: every row's
    scale is distinct and the accumulators are checked exactly."""
    rng = np.random.default_rng(31)
    M, K, N = 37, 300, 23
    a = rng.integers(-128, 128, (M, K)).astype(np.int8)
    b = rng.integers(-128, 128, (K, N)).astype(np.int8)
    s = (rng.random(M) * 0.02 + 1e-3).astype(np.float32)
    assert len(np.unique(s)) == M
    acc = a.astype(np.int64) @ b.astype(np.int64)  # exact
    scale = (s * np.float32(0.05)).astype(np.float32)  # one float32 rounding per row
    ref = (acc.astype(np.float32) * scale[:, None]).astype(np.float32)
    got = O.orc_quantized_matmul_rowscale(a, b, s, 0.05)
    assert same(got, ref)
    # rows are not interchangeable: swapping two scales changes those rows only
    s2 = s.copy()
    s2[[3, 4]] = s2[[4, 3]]
    got2 = O.orc_quantized_matmul_rowscale(a, b, s2, 0.05)
    diff = np.nonzero((got2 != got).any(axis=1))[0]
    assert set(diff) <= {3, 4} and len(diff) > 0


def test_bf16_golden(golden):
    g = golden("bf16.npz")
    assert np.array_equal(O.orc_f32_to_bf16(g["x"]), g["bf16"])


def test_mlp_pfm_golden(golden):
    g = golden("mlp.npz")
    raw = gzip.open(os.path.join(GOLD, "mlp_784_512_10.pfm.gz")).read()
    assert hashlib.sha256(raw).digest() == bytes(g["pfm_sha256"])
    assert list(g["nnz"]) == [40141, 512]


# ---------------------------------------------------------------------------
# Checks fixed by mathematics, not by the reference's outputs.
# ---------------------------------------------------------------------------

def test_csr_equals_dense_on_zero_filled_weight():
    """Skipped terms are (+-0)*x, and s + (+-0) == s, so CSR SpMM over the
    kept entries equals the dense i-k-j product bit-for-bit (finite x)."""
    rng = np.random.default_rng(1)
    W = rng.normal(0, 0.02, (128, 256)).astype(np.float32)
    W[rng.random(W.shape) >= 0.1] = 0.0
    W[rng.random(W.shape) < 0.02] = -0.0
    X = rng.standard_normal((256, 33)).astype(np.float32)
    ip, ix, v = O.orc_to_sparse_csr(W)
    assert same(O.orc_csr_spmm(128, 256, ip, ix, v, X), O.orc_matmul(W, X))
    x = X[:, 0].copy()
    assert same(O.orc_csr_spmv(128, 256, ip, ix, v, x), O.orc_matmul(W, x[:, None])[:, 0])


def test_spmm_against_float64_and_sequential_rounding():
    """A transposed operand or a wrong index breaks the float64 match; the
    sequential fp32 recurrence fixes the exact bits."""
    rng = np.random.default_rng(2)
    W = rng.standard_normal((9, 13)).astype(np.float32)
    W[rng.random(W.shape) < 0.5] = 0
    X = rng.standard_normal((13, 4)).astype(np.float32)
    ip, ix, v = O.orc_to_sparse_csr(W)
    Y = O.orc_csr_spmm(9, 13, ip, ix, v, X)
    np.testing.assert_allclose(Y, W.astype(np.float64) @ X.astype(np.float64), rtol=1e-5, atol=1e-6)
    ref = np.zeros((9, 4), np.float32)
    for r in range(9):
        for j in range(ip[r], ip[r + 1]):
            ref[r] = (ref[r] + np.float32(v[j]) * X[ix[j]]).astype(np.float32)
    assert same(Y, ref)


def test_gemm_closed_form():
    rng = np.random.default_rng(3)
    A = rng.standard_normal((5, 7)).astype(np.float32)
    B = rng.standard_normal((7, 3)).astype(np.float32)
    c = rng.standard_normal(3).astype(np.float32)
    out = O.orc_gemm(A, B, c, 0.5, 2.0)
    np.testing.assert_allclose(out, 0.5 * (A.astype(np.float64) @ B) + 2.0 * c, rtol=1e-5, atol=1e-5)
    # transA/transB only re-index
    assert same(O.orc_gemm(A.T.copy(), B.T.copy(), c, 0.5, 2.0, 1, 1), out)


def test_quantize_round_half_away_and_clamp():
    x = np.array([0.025, -0.025, 0.075, 0.125, -0.125, 100.0, -100.0, 6.35], np.float32)
    q = O.orc_quantize(x, [0.05], [0], O.I8)
    # (x * 20) rounds half away from zero: 0.5->1, -0.5->-1, 1.5->2, 2.5->3
    assert q.tolist() == [1, -1, 2, 3, -3, 127, -128, 127]
    # cvttss2si of an out-of-range value is INT32_MIN -> clamps low for either sign
    assert O.orc_quantize(np.array([3e9, -3e9, np.nan], np.float32), [1.0], [0], O.I8).tolist() == [-128, -128, -128]


def test_symmetric_scale_closed_form():
    rng = np.random.default_rng(4)
    x = rng.standard_normal(1000).astype(np.float32)
    s, z = O.orc_dynamic_params(x)
    assert z == 0 and s == np.float32(np.float32(np.abs(x).max()) / np.float32(127.0))
    w = rng.standard_normal((6, 11)).astype(np.float32)
    sc, zc = O.orc_dynamic_params_per_channel(w.reshape(1, 6, 11))
    assert np.array_equal(sc, (np.abs(w).max(axis=1) / np.float32(127)).astype(np.float32))
    assert not zc.any()


def test_int8_matmul_exact():
    rng = np.random.default_rng(5)
    a = rng.integers(-128, 128, (17, 300)).astype(np.int8)
    b = rng.integers(-128, 128, (300, 11)).astype(np.int8)
    exact = a.astype(np.int64) @ b.astype(np.int64)
    assert np.array_equal(O.orc_int8_matmul_acc(a, b), exact)
    s = np.float32(0.02) * np.float32(0.05)
    assert same(O.orc_quantized_matmul(a, b, 0.02, 0.05), exact.astype(np.float32) * s)


def test_nm_mask_invariants():
    rng = np.random.default_rng(6)
    w = rng.standard_normal(4 * 1000).astype(np.float32)
    m = O.orc_nm_mask(w, 2, 4).reshape(-1, 4)
    assert (m.sum(axis=1) == 2).all()
    g = np.abs(w.reshape(-1, 4))
    top2 = np.argsort(-g, axis=1, kind="stable")[:, :2]
    ref = np.zeros_like(m)
    np.put_along_axis(ref, top2, 1.0, axis=1)
    assert np.array_equal(m, ref)


def magnitude_mask_textbook(w, s):
    """magnitude_pruning.cpp:22-102 written from its definition with numpy:
    threshold = the sorted |w| at min(floor(n s), n - 1) (np.sort puts NaN
    last), keep |w| > threshold, then restore threshold ties in flat order
    while more than (size_t)((float)n * s) are pruned."""
    imp = np.abs(w.astype(np.float32))
    n = imp.size
    idx = min(int(np.floor(np.float64(n) * np.float64(np.float32(s)))), n - 1)
    thr = np.sort(imp)[idx]
    m = (imp > thr).astype(np.float32)
    target = int(np.float32(n) * np.float32(s))
    extra = int((m == 0).sum()) - target
    for i in np.nonzero((m == 0) & (imp == thr))[0]:
        if extra <= 0:
            break
        m[i] = 1.0
        extra -= 1
    return m


def test_magnitude_mask_nan_weights():
    """NaN weights: never kept (NaN > t is false), counted among the zeros,
    never restored (NaN == t is false); their place in the sort is taken
    after +inf.  The oracle against the definition above, with the
    threshold among the finite values, at a NaN, and with ties."""
    rng = np.random.default_rng(4)
    for n, frac, s in ((1000, 0.01, 0.5), (1000, 0.01, 0.995), (257, 0.2, 0.9), (64, 0.0, 0.3)):
        w = rng.standard_normal(n).astype(np.float32)
        w[rng.integers(0, n, n // 10)] = np.float32(0.5)  # ties
        w[rng.random(n) < frac] = np.nan
        w[3] = -np.inf
        got = O.orc_magnitude_mask(w, s)
        assert np.array_equal(got, magnitude_mask_textbook(w, s)), (n, frac, s)
        assert not got[np.isnan(w)].any()


def test_bf16_rne_on_positive_finite_values():
    """For positive finite values the reference conversion is plain RNE."""
    import torch

    rng = np.random.default_rng(7)
    x = np.abs(rng.standard_normal(10000) * np.exp(rng.uniform(-20, 20, 10000))).astype(np.float32)
    ours = O.orc_f32_to_bf16(x)
    tb = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, tb)
    assert np.array_equal(O.orc_bf16_to_f32(ours), (ours.astype(np.uint32) << 16).view(np.float32))


def test_bf16_reference_sign_quirk():
    """half_types.cpp:159-168 tests `upper >= 0x7F7F` on the raw bits, sign
    included, so a negative value whose rounding carries out of the low half
    becomes -inf; a negative value that rounds down is plain RNE."""
    neg_carry = np.array([0xBF80C000], np.uint32).view(np.float32)   # -1.00585938
    neg_down = np.array([0xBF803FFF], np.uint32).view(np.float32)
    assert O.orc_f32_to_bf16(neg_carry)[0] == 0xFF80
    assert O.orc_f32_to_bf16(neg_down)[0] == 0xBF80


def test_softmax_and_relu_closed_form():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((4, 10)).astype(np.float32)
    y = O.orc_softmax(x)
    e = np.exp(x.astype(np.float64) - x.max(axis=1, keepdims=True))
    np.testing.assert_allclose(y, e / e.sum(axis=1, keepdims=True), rtol=1e-6)
    assert (O.orc_softmax(np.full((1, 3), -np.inf, np.float32)) == np.float32(1 / 3)).all()
    r = O.orc_relu(np.array([-1.0, -0.0, 0.0, 2.0, np.nan], np.float32))
    assert r[:4].tolist() == [0.0, 0.0, 0.0, 2.0] and r[4] == 0.0


@pytest.mark.skipif(not O.have_ref(), reason="compiled reference not present")
def test_oracle_matches_reference_random():
    """Fresh random cases straight against the compiled reference."""
    rng = np.random.default_rng(9)
    W = rng.standard_normal((50, 70)).astype(np.float32)
    W[rng.random(W.shape) < 0.85] = 0
    X = rng.standard_normal((70, 5)).astype(np.float32)
    ip, ix, v = O.ref_to_sparse_csr(W)
    assert same(O.orc_csr_spmm(50, 70, ip, ix, v, X), O.ref_sparse_matmul(50, 70, ip, ix, v, X))
    w = rng.integers(-2, 3, 999).astype(np.float32)
    for n, m in ((2, 4), (3, 5)):
        assert same(O.orc_nm_mask(w, n, m), O.ref_nm_mask(w, n, m))


@pytest.mark.skipif(not O.have_ref(), reason="compiled reference not present")
def test_nm_mask_every_tie_pattern_against_reference():
    """Every group of four drawn from nine values (signed zeros, +-1, +-2,
    +-inf, NaN) through the compiled reference's compute_mask and the
    oracle's heap select: the same mask bit for bit, for 2:4 and for 1:4
    and 3:4 on the same groups."""
    vals = np.array([0.0, -0.0, 1.0, -1.0, 2.0, -2.0, np.inf, -np.inf, np.nan], np.float32)
    grid = np.stack(np.meshgrid(*([np.arange(len(vals))] * 4), indexing="ij"), -1).reshape(-1, 4)
    w = np.ascontiguousarray(vals[grid].ravel())
    for n in (1, 2, 3):
        assert same(O.orc_nm_mask(w, n, 4), O.ref_nm_mask(w, n, 4)), n


def test_neighbours_golden(golden):
    """Gelu, LayerNormalization and Add restated against the reference ops'
    outputs, bit for bit (same libm tanhf as the reference build)."""
    g = golden("neighbours.npz")
    assert same(O.orc_gelu(g["gelu_x"]), g["gelu_y"])
    assert same(O.orc_layernorm(g["ln_x"], g["ln_scale"], g["ln_bias"], 1e-5), g["ln_y"])
    assert same(O.orc_layernorm(g["ln_x"], g["ln_scale"], g["ln_bias"], 1e-12), g["ln_y_eps12"])
    assert same(O.orc_layernorm(g["ln3_x"], g["ln3_scale"], g["ln3_bias"], 1e-5, axis=1), g["ln3_y"])
    for k in ("same", "bias", "scalar", "mid"):
        assert same(O.orc_add(g["add_a"], g[f"add_b_{k}"]), g[f"add_y_{k}"]), k
    assert same(O.orc_add(g["add2_a"], g["add2_b"]), g["add2_y"])
    # an empty operand: the output takes the larger extent per axis (0 vs 1
    # gives 1, not numpy's 0) and holds zeros
    y0 = O.orc_add(g["add0_a"], g["add0_b"])
    assert y0.shape == (2, 1, 3) and same(y0, g["add0_y"]) and not np.any(y0)
    with pytest.raises(ValueError, match="not broadcastable"):
        O.orc_add(np.zeros((3, 4), np.float32), np.zeros(3, np.float32))
    # the bar is sensitive to rounding order: the same formula in float64
    # (another summation and rounding sequence) does not give these bits
    x, sc, bi = g["ln_x"].astype(np.float64), g["ln_scale"], g["ln_bias"]
    d = x - x.mean(1, keepdims=True)
    ln64 = (sc * d / np.sqrt((d * d).mean(1, keepdims=True) + 1e-5) + bi).astype(np.float32)
    assert not same(ln64, g["ln_y"])


def test_forward_error_bound_helper():
    """The bound the fast-mode GPU tests use: the oracle's storage-order sums
    and a reversed-order float32 sum (another summation order) meet it; an
    output off by 1e-4 of the largest fails it."""
    from bounds import gamma_bound_ok
    from pyflamert_amd import workloads

    M = K = 512
    ip, ix, v = workloads.csr_uniform(M, K, 0.2, 0.02, seed=11)
    X = workloads.dense_normal((K, 4), 1.0, seed=12)
    R = O.orc_csr_spmm(M, K, ip, ix, v, X)
    assert gamma_bound_ok(R, M, K, ip, ix, v, X, extra=1)[0]
    rev = np.zeros_like(R)
    for r in range(M):
        acc = np.zeros(4, np.float32)
        for j in range(ip[r + 1] - 1, ip[r] - 1, -1):
            acc = (acc + v[j] * X[ix[j]]).astype(np.float32)
        rev[r] = acc
    assert gamma_bound_ok(rev, M, K, ip, ix, v, X, extra=1)[0]
    bad = R.copy()
    bad[7, 2] += np.float32(1e-4) * np.abs(R).max()
    assert not gamma_bound_ok(bad, M, K, ip, ix, v, X, extra=1)[0]
