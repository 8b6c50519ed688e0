"""The quantized path's GPU pieces against the reference.

DynamicQuantizeLinear: bit-exact against the oracle's compute_dynamic_params
+ quantize_tensor (pinned by the quant golden vectors) and, where it is
built, the reference's own cpu_dynamic_quantize_linear op.  The 2:4 GEMM on
quantized activations: int8 or uint8 X with a zero point, per-tensor or
per-channel weight scales, bit-exact against quantization::quantized_matmul
(oracle, pinned by the qmatmul golden vectors); a per-channel scale is the
per-tensor product of that row with its own scale, so each row is checked
against the oracle's single-row product.
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


@pytest.fixture(scope="module")
def ctx():
    from pyflamert_amd import rocm

    c = rocm.Context(0)
    yield c
    c.close()


def dql_oracle(x):
    s, z = O.orc_dynamic_params(x, O.U8, symmetric=False)
    q = O.orc_quantize(x, s, z, O.U8)
    return q.astype(np.uint8), np.float32(s), np.uint8(z)


def dql_cases(rng):
    yield "normal", rng.standard_normal((64, 300)).astype(np.float32)
    yield "positive", (rng.random(5000) * 7 + 3).astype(np.float32)  # zero point clamps to 0
    yield "negative", (-rng.random(777) * 2 - 1).astype(np.float32)  # zero point clamps to 255
    x = rng.standard_normal(10000).astype(np.float32)
    x[::97] = np.nan
    x[::101] = np.inf
    x[::103] = -np.inf
    yield "non-finite", x
    yield "constant", np.full(333, 2.5, np.float32)  # |max - min| < 1e-8: scale 1
    yield "all non-finite", np.array([np.nan, np.inf, -np.inf], np.float32)
    yield "one", np.array([-3.25], np.float32)
    yield "empty", np.zeros(0, np.float32)
    yield "large", rng.standard_normal(3_000_001).astype(np.float32) * 40
    yield "tiny range", (1000.0 + rng.random(4096) * 1e-3).astype(np.float32)


def test_dynamic_quantize_linear(ctx):
    rng = np.random.default_rng(3)
    for name, x in dql_cases(rng):
        say(f"DynamicQuantizeLinear {name} n={x.size}")
        y, s, z = ctx.dynamic_quantize_linear(x)
        ry, rs, rz = dql_oracle(x.ravel())
        assert np.array_equal(y.ravel(), ry), name
        assert np.array_equal(np.float32(s).view(np.uint32), rs.view(np.uint32)), (name, s, rs)
        assert z == rz, (name, z, rz)
        if O.have_ref() and x.size:
            # the reference op itself (its first output, the quantized tensor)
            raw, shape = O.ref_run_op("DynamicQuantizeLinear", [x.ravel()], out_bytes=x.size)
            assert shape == (x.size,) and np.array_equal(raw[: x.size], y.ravel()), name


def test_dynamic_quantize_linear_scale_error(ctx):
    # max - min overflows to +inf: QuantParams::per_tensor rejects the scale
    x = np.array([-3e38, 3e38], np.float32)
    with pytest.raises(_lib.InvalidArgument, match="scale must be positive and finite"):
        ctx.dynamic_quantize_linear(x)


def rand_24(rng, M, K):
    w = rng.standard_normal((M, K)).astype(np.float32)
    w = O.orc_apply_mask(w, O.orc_nm_mask(w.ravel(), 2, 4).reshape(M, K))
    s, _ = O.orc_dynamic_params_per_channel(w.reshape(1, M, K))
    q = O.orc_quantize(w, s, np.zeros(M, np.int32), O.I8, (1, M, K))
    return q, s.astype(np.float32)


@pytest.mark.parametrize("M,K,N", [(200, 512, 128), (96, 300, 70), (256, 4096, 512)])
def test_sp24_quantized_activation(ctx, M, K, N):
    rng = np.random.default_rng(M + K + N)
    q, s = rand_24(rng, M, K)
    x = rng.standard_normal((K, N)).astype(np.float32) * 3
    xq, xs, xz = dql_oracle(x.ravel())
    xq = xq.reshape(K, N)
    say(f"2:4 GEMM on uint8 activations M={M} K={K} N={N} zp={xz}")
    # per-tensor weight scale: quantization::quantized_matmul exactly
    W1 = ctx.sp24_pack(q, s[:1])
    Y = W1.gemm_q(xq, float(xs), int(xz), out="f32")
    assert np.array_equal(bits(Y), bits(O.orc_quantized_matmul(q, xq, s[0], xs, 0, int(xz))))
    acc = W1.gemm_q(xq, float(xs), int(xz), out="i32")
    ref = (q.astype(np.int64) @ (xq.astype(np.int64) - int(xz))).astype(np.int32)
    assert np.array_equal(acc, ref)
    # per-channel weight scales: row m is the per-tensor product with s[m]
    W = ctx.sp24_pack(q, s)
    Y = W.gemm_q(xq, float(xs), int(xz), out="f32")
    rows = rng.choice(M, size=min(M, 24), replace=False)
    for m in rows:
        r = O.orc_quantized_matmul(q[m:m + 1], xq, s[m], xs, 0, int(xz))
        assert np.array_equal(bits(Y[m:m + 1]), bits(r)), m
    # int8 activations with a nonzero zero point, and requantised output
    xi = rng.integers(-128, 128, (K, N)).astype(np.int8)
    Yi = W1.gemm_q(xi, 0.05, -7, out="f32")
    assert np.array_equal(bits(Yi), bits(O.orc_quantized_matmul(q, xi, s[0], np.float32(0.05), 0, -7)))


def test_sp24_device_scale_and_zero_point(ctx):
    """The activation's scale and zero point read from device scalars (as
    pfr_dynamic_quantize_linear_dev leaves them) give the host-value result."""
    import torch

    rng = np.random.default_rng(9)
    M, K, N = 512, 1024, 256
    q, s = rand_24(rng, M, K)
    x = rng.standard_normal((K, N)).astype(np.float32)
    xq, xs, xz = dql_oracle(x.ravel())
    W = ctx.sp24_pack(q, s)
    dX = torch.from_numpy(xq.reshape(K, N)).cuda()
    dS = torch.tensor([xs], dtype=torch.float32, device="cuda")
    dZ = torch.tensor([xz], dtype=torch.uint8, device="cuda")
    dY = torch.empty((M, N), dtype=torch.float32, device="cuda")
    W.gemm_q_dev(dX.data_ptr(), True, N, dY.data_ptr(), x_scale_ptr=dS.data_ptr(), x_zp_ptr=dZ.data_ptr())
    ctx.synchronize()
    assert np.array_equal(bits(dY.cpu().numpy()), bits(W.gemm_q(xq.reshape(K, N), float(xs), int(xz))))


def test_dynamic_int8_session(tmp_path):
    """A session with quantization="dynamic_int8": each 2:4 MatMul(W, X) runs
    as DynamicQuantizeLinear + per-channel QuantizedMatMul on the GPU, the
    other MatMul stays fp32; results bit-exact against the oracle applied
    node by node (per-row weight quantization, the activation's dynamic
    parameters, the quantized product row by row), on the device-resident
    plan and node by node alike."""
    from pyflamert_amd import pfm, session

    sys.path.insert(0, str(__import__("pathlib").Path(__file__).parent))
    from test_runtime_cpu import quant_graph

    rng = np.random.default_rng(11)
    m, w1, w2 = quant_graph(rng, K=512, M1=384, M2=256, N=64)
    p = str(tmp_path / "q.pfm")
    pfm.save(m, p)
    x = rng.standard_normal((512, 64)).astype(np.float32)

    def qrows(w):
        M, K = w.shape
        s, _ = O.orc_dynamic_params_per_channel(w.reshape(1, M, K))
        q = O.orc_quantize(w, s, np.zeros(M, np.int32), O.I8, (1, M, K))
        return q, np.asarray(s, np.float32)

    def qmm(w, act):
        q, s = qrows(w)
        aq, xs, xz = dql_oracle(act.ravel())
        aq = aq.reshape(act.shape)
        return np.concatenate([O.orc_quantized_matmul(q[r:r + 1], aq, s[r], xs, 0, int(xz)) for r in range(len(q))])

    h = qmm(w1, x)
    y_ref = qmm(w2, O.orc_relu(h))
    z_ref = O.orc_matmul(m["initializers"]["w3"], x)
    for lvl in (2, 0):
        say(f"dynamic int8 session, optimization level {lvl}")
        s = session.InferenceSession(p, session.SessionOptions(quantization="dynamic_int8", optimization_level=lvl))
        y, z = s.run(None, {"x": x})
        assert s.device_plan() == ((True, 6) if lvl else (False, 0))
        assert np.array_equal(bits(y), bits(y_ref)), lvl
        assert np.array_equal(bits(z), bits(z_ref)), lvl


def test_two_input_quantized_matmul_zero_point(tmp_path):
    """The reference form of QuantizedMatMul (two inputs, attributes) with a
    nonzero b_zero_point and per-channel a_scales, int8 and uint8 B (whose
    bytes the reference reads as int8): cpu_quantized_matmul's result (the
    oracle restatement, and the reference op itself for a per-tensor scale)."""
    from pyflamert_amd import pfm, session

    rng = np.random.default_rng(21)
    M, K, N = 128, 256, 40
    q, s = rand_24(rng, M, K)
    for bdt, code in ((np.int8, 7), (np.uint8, 8)):
        b = rng.integers(-128, 128, (K, N)).astype(np.int8).view(bdt)
        for per_channel in (False, True):
            attrs = {"b_scale": 0.04, "b_zero_point": -9}
            attrs.update({"a_scales": [float(v) for v in s]} if per_channel else {"a_scale": float(s[0])})
            m = {"name": "q2", "inputs": [("b", code, [K, N])], "outputs": [("y", 0, [M, N])],
                 "initializers": {"w": q}, "nodes": [("qmm", "QuantizedMatMul", ["w", "b"], ["y"], attrs)]}
            p = str(tmp_path / "q2.pfm")
            pfm.save(m, p)
            say(f"QuantizedMatMul two inputs B={np.dtype(bdt).name} per_channel={per_channel}")
            for lvl in (2, 0):
                (y,) = session.InferenceSession(p, session.SessionOptions(optimization_level=lvl)).run(None, {"b": b})
                if per_channel:
                    for r in rng.choice(M, 16, replace=False):
                        ref = O.orc_cpu_quantized_matmul(q[r:r + 1], b, np.float32(s[r]), np.float32(0.04), 0, -9)
                        assert np.array_equal(bits(y[r:r + 1]), bits(ref)), (r, lvl)
                else:
                    ref = O.orc_cpu_quantized_matmul(q, b, np.float32(s[0]), np.float32(0.04), 0, -9)
                    assert np.array_equal(bits(y), bits(ref)), lvl
                    if O.have_ref():
                        got = O.ref_op_f32("QuantizedMatMul", [q, b], fattrs={"a_scale": float(s[0]), "b_scale": 0.04},
                                           iattrs={"b_zero_point": -9})
                        assert np.array_equal(bits(y), bits(got)), lvl


def test_quantize_dequantize_per_tensor(ctx, golden):
    """Per-tensor quantize_tensor / dequantize_tensor on the GPU: bit-exact
    against the golden vectors written by the compiled reference (edge
    values: +-0, halves, overflow, +-inf, NaN) and the oracle on large
    random inputs; the reference's parameter checks and texts."""
    g = golden("quant.npz")
    xs = g["x"]
    say("QuantizeLinear golden vectors")
    for dt, zp in ((O.I8, 0), (O.I8, -3), (O.U8, 128), (O.U8, 7)):
        q = ctx.quantize_linear(xs, 0.05, zp, "u8" if dt == O.U8 else "i8")
        assert np.array_equal(q, g[f"q_{dt}_{zp}"]), (dt, zp)
    say("DequantizeLinear golden vectors")
    assert np.array_equal(bits(ctx.dequantize_linear(np.arange(-128, 128, dtype=np.int8), 0.05, 3)),
                          bits(g["dq_i8"]))
    assert np.array_equal(bits(ctx.dequantize_linear(np.arange(0, 256, dtype=np.uint8), 0.1, 128)),
                          bits(g["dq_u8"]))
    rng = np.random.default_rng(31)
    x = (rng.standard_normal(1 << 20) * 9).astype(np.float32)
    x[::1009] = np.nan
    x[::1013] = np.inf
    for dt, zp, sc in ((O.I8, 0, 0.07), (O.I8, 100, 3e-3), (O.U8, 128, 0.11), (O.U8, 255, 1e-30), (O.I8, -7, 7e30)):
        say(f"quantize 1M values dtype={dt} zp={zp} scale={sc}")
        q = ctx.quantize_linear(x, sc, zp, "u8" if dt == O.U8 else "i8")
        assert np.array_equal(q, O.orc_quantize(x, [sc], [zp], dt)), (dt, zp, sc)
        q8 = rng.integers(0 if dt == O.U8 else -128, 256 if dt == O.U8 else 128, 100000).astype(
            np.uint8 if dt == O.U8 else np.int8)
        assert np.array_equal(bits(ctx.dequantize_linear(q8, sc, zp)), bits(O.orc_dequantize(q8, [sc], [zp], dt)))
    for bad in (0.0, -1.0, np.inf, np.nan):
        with pytest.raises(_lib.InvalidArgument, match="scale must be positive and finite"):
            ctx.quantize_linear(x[:10], bad)
        with pytest.raises(_lib.InvalidArgument, match="scale must be positive and finite"):
            ctx.dequantize_linear(np.zeros(4, np.int8), bad)
    with pytest.raises(_lib.InvalidArgument, match="dtype must be Int8 or UInt8"):
        ctx.dequantize_linear(np.zeros(4, np.float32), 0.5)
    assert ctx.quantize_linear(np.zeros(0, np.float32), 0.5).size == 0


def test_quantize_ops_in_sessions(tmp_path):
    """Quantize / Dequantize (attributes) and QuantizeLinear /
    DequantizeLinear (scale and zero-point inputs, constant or produced by a
    DynamicQuantizeLinear) in device-resident plans and node by node: the
    oracle's per-tensor results bit for bit."""
    from pyflamert_amd import pfm, session

    rng = np.random.default_rng(41)
    x = (rng.standard_normal((64, 300)) * 4).astype(np.float32)
    sc = np.array([0.03], np.float32)
    zp = np.array([5], np.int8)
    m = {"name": "qdq", "inputs": [("x", 0, [64, 300])],
         "outputs": [("a", 7, [64, 300]), ("b", 0, [64, 300]), ("c", 8, [64, 300]), ("d", 0, [64, 300]),
                     ("e", 0, [64, 300])],
         "initializers": {"s": sc, "z": zp},
         "nodes": [("q1", "QuantizeLinear", ["x", "s", "z"], ["a"], {}),
                   ("d1", "DequantizeLinear", ["a", "s", "z"], ["b"], {}),
                   ("q2", "Quantize", ["x"], ["c"], {"scale": 0.07, "zero_point": 128, "dtype": "uint8"}),
                   ("d2", "Dequantize", ["c"], ["d"], {"scale": 0.07, "zero_point": 128}),
                   ("dq", "DynamicQuantizeLinear", ["x"], ["y", "ys", "yz"], {}),
                   ("d3", "DequantizeLinear", ["y", "ys", "yz"], ["e"], {})]}
    p = str(tmp_path / "qdq.pfm")
    pfm.save(m, p)
    a_ref = O.orc_quantize(x, sc, [5], O.I8)
    b_ref = O.orc_dequantize(a_ref, sc, [5], O.I8)
    c_ref = O.orc_quantize(x, [0.07], [128], O.U8)
    d_ref = O.orc_dequantize(c_ref, [0.07], [128], O.U8)
    ys, yz = O.orc_dynamic_params(x.ravel(), O.U8, symmetric=False)
    e_ref = O.orc_dequantize(O.orc_quantize(x, [ys], [yz], O.U8), [ys], [yz], O.U8)
    for lvl in (2, 0):
        say(f"quantize ops session, optimization level {lvl}")
        s = session.InferenceSession(p, session.SessionOptions(optimization_level=lvl))
        a, b, c, d, e = s.run(None, {"x": x})
        assert s.device_plan()[0] == (lvl > 0)
        assert a.dtype == np.int8 and np.array_equal(a, a_ref)
        assert np.array_equal(bits(b), bits(b_ref))
        assert c.dtype == np.uint8 and np.array_equal(c, c_ref)
        assert np.array_equal(bits(d), bits(d_ref))
        assert np.array_equal(bits(e), bits(e_ref))


def test_dynamic_int8_session_xw(tmp_path):
    """quantization="dynamic_int8" on the x . W form (Gemm with transB and a
    bias, MatMul(x, W)): DynamicQuantizeLinear + QuantizedMatMul with the 2:4
    weight as the second operand, on the device-resident plan and node by
    node, bit-exact against the oracle applied node by node (per output
    column: quantization::quantized_matmul of the quantized activation with
    that column); the Gemm whose bias is not a vector stays fp32."""
    from pyflamert_amd import pfm, session

    sys.path.insert(0, str(__import__("pathlib").Path(__file__).parent))
    from test_runtime_cpu import xw_graph

    rng = np.random.default_rng(13)
    T, K, N1, N2 = 70, 512, 384, 256
    m, w1, b1, w2 = xw_graph(rng, T=T, K=K, N1=N1, N2=N2)
    p = str(tmp_path / "xw.pfm")
    pfm.save(m, p)
    x = rng.standard_normal((T, K)).astype(np.float32)

    def qmm_xw(act, wt):
        N, Kk = wt.shape
        s, _ = O.orc_dynamic_params_per_channel(wt.reshape(1, N, Kk))
        q = O.orc_quantize(wt, s, np.zeros(N, np.int32), O.I8, (1, N, Kk))
        aq, xs, xz = dql_oracle(act.ravel())
        aq = aq.reshape(act.shape)
        cols = [O.orc_quantized_matmul(aq, np.ascontiguousarray(q[n:n + 1].T), xs, np.float32(s[n]), int(xz), 0)
                for n in range(N)]
        return np.concatenate(cols, axis=1)

    h = O.orc_add(qmm_xw(x, w1), b1)
    y_ref = qmm_xw(O.orc_relu(h), np.ascontiguousarray(w2.T))
    z_ref = O.orc_gemm(x, m["initializers"]["w4"], m["initializers"]["c4"])
    for lvl in (2, 0):
        say(f"dynamic int8 x . W session, optimization level {lvl}")
        s = session.InferenceSession(p, session.SessionOptions(quantization="dynamic_int8", optimization_level=lvl))
        y, z = s.run(None, {"x": x})
        assert s.device_plan()[0] == (lvl > 0)
        assert np.array_equal(bits(y), bits(y_ref)), lvl
        assert np.array_equal(bits(z), bits(z_ref)), lvl


def test_sp24_xw_entry_point(ctx):
    """pfr_sp24_gemm_qt directly: int8 and uint8 activations with zero points,
    row counts that are not multiples of the tile, against the per-column
    oracle."""
    rng = np.random.default_rng(17)
    for T, K, M in ((1, 512, 256), (37, 300, 200), (130, 1024, 512)):
        q, s = rand_24(rng, M, K)
        W = ctx.sp24_pack(q, s)
        for u8 in (False, True):
            act = (rng.integers(0, 256, (T, K)).astype(np.uint8) if u8
                   else rng.integers(-128, 128, (T, K)).astype(np.int8))
            zp = 131 if u8 else -5
            say(f"2:4 x . W T={T} K={K} M={M} {'uint8' if u8 else 'int8'}")
            Y = np.empty((T, M), np.float32)
            _lib.check(ctx._lib.pfr_sp24_gemm_qt(ctx.handle, W.handle, act.ctypes.data, _lib.PFR_U8 if u8 else _lib.PFR_I8,
                                                 T, 0.03, zp, Y.ctypes.data))
            for n in rng.choice(M, 8, replace=False):
                ref = O.orc_quantized_matmul(act, np.ascontiguousarray(q[n:n + 1].T), np.float32(0.03), np.float32(s[n]),
                                             zp, 0)
                assert np.array_equal(bits(Y[:, n:n + 1]), bits(ref)), (T, n, u8)
