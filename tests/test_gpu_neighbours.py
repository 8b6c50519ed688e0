"""Gelu, Add and LayerNormalization on the GPU, and a BERT-shaped FFN block
(pruned Gemm -> Gelu -> pruned Gemm -> residual Add -> LayerNormalization)
on the device-resident plan.

Bars: Add and LayerNormalization bit-exact against the golden vectors
written by the compiled reference and against the oracle; Gelu within
|d| <= 2.4e-7 * |x| + 1e-6 * |y| of the reference (the device tanhf against
glibc's: a few ulp of tanh, which 0.5 * x * (1 + tanh) carries as an absolute
error proportional to |x| where 1 + tanh cancels), the special values (NaN,
+-inf, signed zero) identical.  Fusing Gelu into the product's epilogue
changes no bit.
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
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def gelu_close(x, got, want):
    x, got, want = (np.asarray(v, np.float64) for v in (x, got, want))
    fin = np.isfinite(want)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(got[~fin & ~np.isnan(want)], want[~fin & ~np.isnan(want)])
    d = np.abs(got[fin] - want[fin])
    bound = 2.4e-7 * np.abs(x[fin]) + 1e-6 * np.abs(want[fin])
    assert np.all(d <= bound), float((d - bound).max())
    return float(d.max()) if d.size else 0.0


@pytest.fixture(scope="module")
def ctx():
    from pyflamert_amd import rocm

    c = rocm.Context(0)
    yield c
    c.close()


def test_gelu(ctx, golden):
    g = golden("neighbours.npz")
    say("Gelu: golden vectors")
    y = ctx.gelu(g["gelu_x"])
    say("  max |d| vs reference", gelu_close(g["gelu_x"], y, g["gelu_y"]))
    zi = np.flatnonzero(g["gelu_x"] == 0)
    assert same(y[zi], g["gelu_y"][zi])  # +0 -> +0, -0 -> -0
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(1 << 20) * 4).astype(np.float32)
    say("Gelu: 1M N(0, 16) values against the oracle")
    gelu_close(x, ctx.gelu(x), O.orc_gelu(x))
    assert ctx.gelu(np.zeros(0, np.float32)).size == 0


def test_add(ctx, golden):
    g = golden("neighbours.npz")
    say("Add: golden vectors")
    for k in ("same", "bias", "scalar", "mid"):
        assert same(ctx.add(g["add_a"], g[f"add_b_{k}"]), g[f"add_y_{k}"]), k
    assert same(ctx.add(g["add2_a"], g["add2_b"]), g["add2_y"])
    y0 = ctx.add(g["add0_a"], g["add0_b"])
    assert y0.shape == (2, 1, 3) and same(y0, g["add0_y"])
    rng = np.random.default_rng(6)
    cases = [((3, 1, 4, 1, 2), (5, 4, 1, 1)), ((1,), (7, 9)), ((), (4, 3)), ((), ()), ((2, 3, 4, 5, 6, 7, 1, 2), (1, 2)),
             ((4096, 768), (768,)), ((1024, 1), (1, 3072))]
    for sa, sb in cases:
        say(f"Add {sa} + {sb}")
        a = rng.standard_normal(sa).astype(np.float32)
        b = rng.standard_normal(sb).astype(np.float32)
        assert same(ctx.add(a, b), O.orc_add(a, b)), (sa, sb)
        assert same(ctx.add(b, a), O.orc_add(b, a)), (sb, sa)
    with pytest.raises(_lib.InvalidArgument, match="Add: shapes are not broadcastable"):
        ctx.add(np.zeros((3, 4), np.float32), np.zeros(3, np.float32))
    with pytest.raises(_lib.InvalidArgument, match="at most 8"):
        ctx.add(np.zeros((1,) * 9, np.float32), np.zeros(1, np.float32))


def test_layernorm(ctx, golden):
    g = golden("neighbours.npz")
    say("LayerNormalization: golden vectors")
    assert same(ctx.layernorm(g["ln_x"], g["ln_scale"], g["ln_bias"], 1e-5), g["ln_y"])
    assert same(ctx.layernorm(g["ln_x"], g["ln_scale"], g["ln_bias"], 1e-12), g["ln_y_eps12"])
    assert same(ctx.layernorm(g["ln3_x"], g["ln3_scale"], g["ln3_bias"], 1e-5, axis=1), g["ln3_y"])
    rng = np.random.default_rng(7)
    for shape, axis in (((4096, 768), -1), ((3, 5, 7), 0), ((1, 1), -1), ((130, 1024), 1), ((7, 3), 1)):
        say(f"LayerNormalization {shape} axis={axis}")
        x = (rng.standard_normal(shape) * 3 + 1).astype(np.float32)
        nrm = int(np.prod(shape[axis % len(shape):]))
        sc = rng.standard_normal(nrm).astype(np.float32)
        bi = rng.standard_normal(nrm).astype(np.float32)
        assert same(ctx.layernorm(x, sc, bi, 1e-5, axis), O.orc_layernorm(x, sc, bi, 1e-5, axis)), shape
    # a constant row: variance 0, inv_std = 1 / sqrt(eps)
    x = np.full((2, 16), 3.25, np.float32)
    assert same(ctx.layernorm(x, np.ones(16), np.zeros(16), 1e-5), O.orc_layernorm(x, np.ones(16), np.zeros(16)))


def test_device_entry_points(ctx):
    """The _dev forms on device buffers give the host forms' bits."""
    import torch

    rng = np.random.default_rng(8)
    x = rng.standard_normal((512, 768)).astype(np.float32)
    sc = rng.standard_normal(768).astype(np.float32)
    bi = rng.standard_normal(768).astype(np.float32)
    dx, ds, db = (torch.from_numpy(v).cuda() for v in (x, sc, bi))
    dy = torch.empty_like(dx)
    lib, h = ctx._lib, ctx.handle
    say("device forms: Gelu, Add (row broadcast), LayerNormalization")
    assert lib.pfr_gelu_dev(h, dx.data_ptr(), x.size, dy.data_ptr()) == 0
    ctx.synchronize()
    assert same(dy.cpu().numpy(), ctx.gelu(x))
    sa = np.array(x.shape, np.int64)
    sb = np.array(sc.shape, np.int64)
    assert lib.pfr_add_dev(h, dx.data_ptr(), sa.ctypes.data, 2, ds.data_ptr(), sb.ctypes.data, 1, dy.data_ptr()) == 0
    ctx.synchronize()
    assert same(dy.cpu().numpy(), O.orc_add(x, sc))
    assert lib.pfr_layernorm_dev(h, dx.data_ptr(), 512, 768, ds.data_ptr(), db.data_ptr(), 1e-12, dy.data_ptr()) == 0
    ctx.synchronize()
    assert same(dy.cpu().numpy(), O.orc_layernorm(x, sc, bi, 1e-12))


def ffn_model(rng, T, H, F, keep, outputs):
    def pruned(shape):
        w = (rng.standard_normal(shape) * 0.05).astype(np.float32)
        w[rng.random(shape) >= keep] = 0
        return w

    w1, w2 = pruned((F, H)), pruned((H, F))  # [out, in], as a Linear exports them (transB = 1)
    b1 = (rng.standard_normal(F) * 0.1).astype(np.float32)
    b2 = (rng.standard_normal(H) * 0.1).astype(np.float32)
    ln_s = (1 + rng.standard_normal(H) * 0.1).astype(np.float32)
    ln_b = (rng.standard_normal(H) * 0.1).astype(np.float32)
    inits = {"w1": w1, "b1": b1, "w2": w2, "b2": b2, "ln_s": ln_s, "ln_b": ln_b}
    nodes = [("fc1", "Gemm", ["x", "w1", "b1"], ["h"], {"transB": 1}),
             ("act", "Gelu", ["h"], ["g"], {}),
             ("fc2", "Gemm", ["g", "w2", "b2"], ["f"], {"transB": 1}),
             ("res", "Add", ["f", "x"], ["r"], {}),
             ("ln", "LayerNormalization", ["r", "ln_s", "ln_b"], ["y"], {"epsilon": 1e-12, "axis": -1})]
    shapes = {"y": [T, H], "g": [T, F], "h": [T, F]}
    m = {"name": "ffn", "inputs": [("x", 0, [T, H])], "outputs": [(n, 0, shapes[n]) for n in outputs],
         "initializers": inits, "nodes": nodes}
    return m, inits


def test_bert_ffn_block(tmp_path):
    """A BERT-base FFN block (768 -> 3072 -> 768, 90 % pruned, Gelu, residual
    Add, LayerNormalization eps 1e-12) on the device-resident plan.  With
    fc1's output exposed (no fusion) every product, Add and LayerNorm is
    bit-exact against the oracle applied to the GPU's own Gelu output, and
    Gelu is within its bar; with the Gelu output exposed it is fused into
    fc1's epilogue and gives the same bits; with only y requested, levels
    Extended (fused), Basic and None give the same bits."""
    from pyflamert_amd import pfm, session

    T, H, F = 64, 768, 3072
    rng = np.random.default_rng(12)
    m, w = ffn_model(rng, T, H, F, 0.1, ["y", "g", "h"])
    x = rng.standard_normal((T, H)).astype(np.float32)
    p = str(tmp_path / "ffn_h.pfm")
    pfm.save(m, p)
    say("BERT FFN block, fc1 output exposed")
    s = session.InferenceSession(p)
    y, g, h = s.run(["y", "g", "h"], {"x": x})
    assert s.device_plan() == (True, 5)
    assert same(h, O.orc_gemm(x, w["w1"], w["b1"], transB=1))
    say("  Gelu max |d|", gelu_close(h, g, O.orc_gelu(h)))
    f = O.orc_gemm(g, w["w2"], w["b2"], transB=1)
    y_ref = O.orc_layernorm(O.orc_add(f, x), w["ln_s"], w["ln_b"], 1e-12)
    assert same(y, y_ref)

    mg = dict(m, outputs=[("y", 0, [T, H]), ("g", 0, [T, F])])
    pg = str(tmp_path / "ffn_g.pfm")
    pfm.save(mg, pg)
    say("BERT FFN block, Gelu output exposed (fused into fc1)")
    s = session.InferenceSession(pg)
    yg, gg = s.run(["y", "g"], {"x": x})
    assert s.device_plan() == (True, 4)
    assert same(gg, g) and same(yg, y)

    m1 = dict(m, outputs=[("y", 0, [T, H])])
    p1 = str(tmp_path / "ffn.pfm")
    pfm.save(m1, p1)
    for lvl, plan in ((2, (True, 4)), (1, (True, 5)), (0, (False, 0))):
        say(f"BERT FFN block, optimization level {lvl}")
        s = session.InferenceSession(p1, session.SessionOptions(optimization_level=lvl))
        (yl,) = s.run(None, {"x": x})
        assert s.device_plan() == plan, lvl
        assert same(yl, y), lvl


def test_fused_gelu_epilogue_spmm(ctx):
    """The CSR kernels' Gelu epilogue (SpMM, Gemm) equals Gelu applied to
    the unfused product, bit for bit, on every kernel path the shapes
    select (N = 1, 8, 256; strict and fast)."""
    import torch

    rng = np.random.default_rng(13)
    W = rng.standard_normal((1024, 2048)).astype(np.float32)
    W[rng.random(W.shape) >= 0.1] = 0
    Wc = ctx.csr_from_dense(W)
    for N in (1, 8, 256):
        for mode in ("strict", "fast"):
            say(f"CSR SpMM Gelu epilogue N={N} {mode}")
            X = torch.from_numpy(rng.standard_normal((2048, N)).astype(np.float32)).cuda()
            Y0 = torch.empty((1024, N), device="cuda")
            Y1 = torch.empty((1024, N), device="cuda")
            Wc.spmm_dev(X.data_ptr(), N, Y0.data_ptr(), mode=mode)
            Wc.spmm_dev(X.data_ptr(), N, Y1.data_ptr(), mode=mode, gelu=True)
            ctx.synchronize()
            assert same(Y1.cpu().numpy(), ctx.gelu(Y0.cpu().numpy())), (N, mode)
