"""End-to-end sessions on the MI355X backend: the 784-512-10 MLP model
written by the compiled reference, run with device="rocm", against the
reference executor's outputs; plus MatMul / QuantizedMatMul graphs and the
backend's error paths."""
import gzip
import os
import sys

import numpy as np
import pytest

from oracle import oracle as O
from pyflamert_amd import pfm, session

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def mlp(tmp_path_factory):
    p = tmp_path_factory.mktemp("m") / "mlp.pfm"
    p.write_bytes(gzip.open(os.path.join(GOLD, "mlp_784_512_10.pfm.gz")).read())
    return str(p)


def test_mlp_against_reference_executor(mlp, golden, tmp_path):
    g = golden("mlp.npz")
    say("MLP 784-512-10 on device=rocm")
    s = session.InferenceSession(mlp, session.SessionOptions(device="rocm"))
    assert s.get_providers() == ["ROCMExecutionProvider"]
    assert [i.name for i in s.get_inputs()] == ["x"] and s.get_inputs()[0].shape == [32, 784]
    (y,) = s.run(None, {"x": g["x"]})
    # device-resident plan: Gemm+Relu fused, Gemm, Softmax
    assert s.device_plan() == (True, 3)
    # Softmax uses the device expf: a few ulp from glibc's
    assert np.abs(y - g["y"]).max() <= 4e-7
    assert np.array_equal(np.argmax(y, 1), np.argmax(g["y"], 1))
    # The pruned Gemm itself is bit-exact: expose h1 as a graph output.
    m = pfm.load(mlp)
    m["outputs"].append(("h1", 0, [32, 512]))
    p2 = str(tmp_path / "mlp_h1.pfm")
    pfm.save(m, p2)
    s2 = session.InferenceSession(p2, session.SessionOptions(device="rocm"))
    y2, h1 = s2.run(["y", "h1"], {"x": g["x"]})
    assert s2.device_plan() == (True, 4)  # h1 is an output: the Relu runs on its own
    assert np.array_equal(bits(h1), bits(g["h1"]))
    assert np.array_equal(bits(y2), bits(y))
    # OptLevel None: node by node through the host OpFuncs; Basic: the
    # device-resident plan without fusion.  Same bits either way.
    for lvl, plan in ((0, (False, 0)), (1, (True, 4))):
        sl = session.InferenceSession(mlp, session.SessionOptions(device="rocm", optimization_level=lvl))
        (yl,) = sl.run(None, {"x": g["x"]})
        assert sl.device_plan() == plan, lvl
        assert np.array_equal(bits(yl), bits(y)), lvl
    # relu and the second Gemm exactly as the oracle computes them from h1
    a1 = O.orc_relu(h1)
    w2, b2 = m["initializers"]["fc2.weight"], m["initializers"]["fc2.bias"]
    z2 = O.orc_gemm(a1, w2, b2)
    assert np.abs(y - O.orc_softmax(z2)).max() <= 4e-7
    # fast mode: same graph with fused multiply-add sums
    s3 = session.InferenceSession(mlp, session.SessionOptions(device="rocm", math_mode="fast"))
    (y3,) = s3.run(None, {"x": g["x"]})
    assert np.abs(y3 - g["y"]).max() <= 1e-5
    s4 = session.InferenceSession(mlp, session.SessionOptions(device="rocm", math_mode="fast", optimization_level=0))
    (y4,) = s4.run(None, {"x": g["x"]})
    assert np.array_equal(bits(y4), bits(y3))


def test_kat_and_batched_matmul(tmp_path, golden):
    k = golden("kat_matmul.npz")
    say("MatMul KAT through a session")
    m = {"name": "kat", "inputs": [("a", 0, [2, 3])], "outputs": [("c", 0, [2, 2])],
         "initializers": {"b": k["b"]}, "nodes": [("matmul_0", "MatMul", ["a", "b"], ["c"], {})]}
    p = str(tmp_path / "kat.pfm")
    pfm.save(m, p)
    (c,) = session.InferenceSession(p).run(None, {"a": k["a"]})
    assert c.tolist() == [[22.0, 28.0], [49.0, 64.0]]
    g = golden("matmul.npz")
    a, b, ref = g["c0_a"], g["c0_b"], g["c0_out"]      # [3,4,5] x [5,6]
    m = {"name": "bm", "inputs": [("a", 0, list(a.shape))], "outputs": [("c", 0, list(ref.shape))],
         "initializers": {"w": b}, "nodes": [("mm", "MatMul", ["a", "w"], ["c"], {})]}
    p = str(tmp_path / "bm.pfm")
    pfm.save(m, p)
    (c,) = session.InferenceSession(p).run(None, {"a": a})
    assert np.array_equal(bits(c), bits(ref))
    # pruned weight in the first position: Y = W . X
    rng = np.random.default_rng(1)
    W = rng.standard_normal((64, 48)).astype(np.float32)
    W[rng.random(W.shape) < 0.9] = 0
    X = rng.standard_normal((48, 7)).astype(np.float32)
    m = {"name": "wx", "inputs": [("x", 0, [48, 7])], "outputs": [("y", 0, [64, 7])],
         "initializers": {"w": W}, "nodes": [("mm", "MatMul", ["w", "x"], ["y"], {})]}
    p = str(tmp_path / "wx.pfm")
    pfm.save(m, p)
    (y,) = session.InferenceSession(p).run(None, {"x": X})
    assert np.array_equal(bits(y), bits(O.orc_matmul(W, X)))


def test_quantized_matmul_24(tmp_path, golden):
    """QuantizedMatMul(W int8 2:4 initializer, X int8) -> float, against the
    reference op's output."""
    g = golden("qmatmul.npz")
    say("QuantizedMatMul with a 2:4 initializer")
    wq, xq, ws = g["sp_wq"], g["sp_xq"], float(g["sp_ws"])
    m = {"name": "q", "inputs": [("x", 7, list(xq.shape))], "outputs": [("y", 0, [wq.shape[0], xq.shape[1]])],
         "initializers": {"w": wq},
         "nodes": [("qmm", "QuantizedMatMul", ["w", "x"], ["y"], {"a_scale": ws, "b_scale": 0.05})]}
    p = str(tmp_path / "q.pfm")
    pfm.save(m, p)
    (y,) = session.InferenceSession(p).run(None, {"x": xq})
    ref = O.orc_cpu_quantized_matmul(wq, xq, np.float32(ws), np.float32(0.05))
    assert np.array_equal(bits(y), bits(ref))
    assert np.array_equal(bits(y), bits(g["sp_yf"]))


def run_levels(m, tmp_path, feed, inter):
    """Run model dict m at OptLevel Extended (device-resident plan with Relu
    fused), Basic (plan, no fusion) and None (node by node through the host
    OpFuncs): all three give the same bits.  inter lists (name, shape) of
    intermediates, returned from a copy of the model that exposes them as
    graph outputs (which keeps their Relu unfused)."""
    p = str(tmp_path / (m["name"] + ".pfm"))
    pfm.save(m, p)
    runs = []
    for lvl in (2, 1, 0):
        s = session.InferenceSession(p, session.SessionOptions(optimization_level=lvl))
        runs.append((s.run(None, feed), s.device_plan()))
    for outs, _ in runs[1:]:
        for a, b in zip(runs[0][0], outs):
            assert a.shape == b.shape and np.array_equal(bits(a), bits(b))
    assert runs[2][1] == (False, 0)
    m2 = dict(m, name=m["name"] + "_x", outputs=list(m["outputs"]) + [(n, 0, sh) for n, sh in inter])
    p2 = str(tmp_path / (m2["name"] + ".pfm"))
    pfm.save(m2, p2)
    s = session.InferenceSession(p2)
    res = s.run([n for n, *_ in m2["outputs"]], feed)
    for a, b in zip(runs[0][0], res):
        assert np.array_equal(bits(a), bits(b))
    return runs[0][0], res[len(m["outputs"]):], runs[0][1], runs[1][1]


def test_device_plan_graphs(tmp_path, golden):
    """Graphs of pruned MatMuls in both operand positions, batched MatMul,
    fused and unfused Relu, Softmax over axis 0 and a 2:4 QuantizedMatMul
    run on the device-resident plan: the same bits as the node-by-node run,
    the products bit-exact against the oracle."""
    rng = np.random.default_rng(21)

    def pruned(shape, keep):
        w = rng.standard_normal(shape).astype(np.float32)
        w[rng.random(shape) >= keep] = 0
        return w

    W1, W2 = pruned((48, 64), 0.2), pruned((30, 10), 0.5)
    x = rng.standard_normal((10, 48)).astype(np.float32)
    m = {"name": "g1", "inputs": [("x", 0, [10, 48])], "outputs": [("y", 0, [30, 64])],
         "initializers": {"w1": W1, "w2": W2},
         "nodes": [("mm1", "MatMul", ["x", "w1"], ["h"], {}), ("r1", "Relu", ["h"], ["a"], {}),
                   ("mm2", "MatMul", ["w2", "a"], ["z"], {}), ("r2", "Relu", ["z"], ["r"], {}),
                   ("sm", "Softmax", ["r"], ["y"], {"axis": 0})]}
    say("device plan: MatMul(x,W)+Relu, MatMul(W,a)+Relu, Softmax(axis 0)")
    (y,), (h, z), plan, basic = run_levels(m, tmp_path, {"x": x}, [("h", [10, 64]), ("z", [30, 64])])
    assert plan == (True, 3) and basic == (True, 5)
    assert np.array_equal(bits(h), bits(O.orc_matmul(x, W1)))
    z_ref = O.orc_matmul(W2, O.orc_relu(h))
    assert np.array_equal(bits(z), bits(z_ref))
    assert np.abs(y - O.orc_softmax(O.orc_relu(z_ref), axis=0)).max() <= 4e-7

    xb = rng.standard_normal((2, 5, 48)).astype(np.float32)
    m = {"name": "g2", "inputs": [("x", 0, [2, 5, 48])], "outputs": [("y", 0, [2, 5, 64])],
         "initializers": {"w1": W1},
         "nodes": [("mm", "MatMul", ["x", "w1"], ["h"], {}), ("r", "Relu", ["h"], ["y"], {})]}
    say("device plan: batched MatMul + Relu")
    (y,), (h,), plan, basic = run_levels(m, tmp_path, {"x": xb}, [("h", [2, 5, 64])])
    assert plan == (True, 1) and basic == (True, 2) and y.shape == (2, 5, 64)
    assert np.array_equal(bits(y), bits(O.orc_relu(O.orc_matmul(xb, W1))))

    g = golden("qmatmul.npz")
    wq, xq, ws = g["sp_wq"], g["sp_xq"], float(g["sp_ws"])
    m = {"name": "g3", "inputs": [("x", 7, list(xq.shape))], "outputs": [("y", 0, [wq.shape[0], xq.shape[1]])],
         "initializers": {"w": wq},
         "nodes": [("qmm", "QuantizedMatMul", ["w", "x"], ["q"], {"a_scale": ws, "b_scale": 0.05}),
                   ("r", "Relu", ["q"], ["y"], {})]}
    say("device plan: QuantizedMatMul 2:4 + Relu")
    (y,), (q,), plan, basic = run_levels(m, tmp_path, {"x": xq}, [("q", [wq.shape[0], xq.shape[1]])])
    assert plan == (True, 2) and basic == (True, 2)
    assert np.array_equal(bits(q), bits(g["sp_yf"]))
    assert np.array_equal(bits(y), bits(O.orc_relu(g["sp_yf"])))


def test_backend_errors(tmp_path):
    say("rocm backend error paths")
    base = {"name": "e", "inputs": [("a", 0, [2, 3]), ("b", 0, [3, 2])], "outputs": [("c", 0, [2, 2])],
            "initializers": {}}
    m = dict(base, nodes=[("conv", "Conv", ["a", "b"], ["c"], {})])
    p = str(tmp_path / "conv.pfm")
    pfm.save(m, p)
    s = session.InferenceSession(p)
    with pytest.raises(session.UnsupportedOperatorError, match="'Conv' is not supported by the 'rocm' backend"):
        s.run(None, {"a": np.ones((2, 3), np.float32), "b": np.ones((3, 2), np.float32)})
    m = dict(base, nodes=[("mm", "MatMul", ["a", "b"], ["c"], {})])
    p = str(tmp_path / "act.pfm")
    pfm.save(m, p)
    s = session.InferenceSession(p)
    with pytest.raises(session.BackendError, match=r"\[mm\] MatMul: neither operand"):
        s.run(None, {"a": np.ones((2, 3), np.float32), "b": np.ones((3, 2), np.float32)})
    with pytest.raises(session.PyFlameRTError, match="Missing required input 'b'"):
        s.run(None, {"a": np.ones((2, 3), np.float32)})
    with pytest.raises(session.PyFlameRTError, match="dimension 1 has size 4 but expected 3"):
        s.run(None, {"a": np.ones((2, 4), np.float32), "b": np.ones((3, 2), np.float32)})
    with pytest.raises(session.PyFlameRTError, match="has dtype int8 but expected float32"):
        s.run(None, {"a": np.ones((2, 3), np.int8), "b": np.ones((3, 2), np.float32)})
    name, ops = s.supported_ops()
    assert name == "rocm" and {"MatMul", "Gemm", "QuantizedMatMul", "Relu", "Softmax"} <= set(ops)


def test_sparse_record_sessions(mlp, golden, tmp_path):
    """Version-2 .pfm models whose pruned weights are sparse records run
    without a dense copy and give the results of the dense models: the MLP
    with CSR weights (same bits as the dense file), int8 CSR weights in
    both operand positions with per-row, per-column and per-tensor scales
    (bit-exact against the oracle on the dequantised matrix), Gemm with
    transB, a 2:4 record under QuantizedMatMul, and a record used as a plain
    tensor."""
    g = golden("mlp.npz")
    m = pfm.load(mlp)
    inits = dict(m["initializers"])
    sp = {k: pfm.csr_record(inits.pop(k)) for k in ("fc1.weight", "fc2.weight")}
    ms = dict(m, initializers=inits, sparse_initializers=sp)
    p = str(tmp_path / "mlp_sparse.pfm")
    pfm.save(ms, p)
    assert os.path.getsize(p) < os.path.getsize(mlp) / 3
    say("MLP with CSR records")
    for lvl in (2, 0):
        s = session.InferenceSession(p, session.SessionOptions(optimization_level=lvl))
        (y,) = s.run(None, {"x": g["x"]})
        s_dense = session.InferenceSession(mlp, session.SessionOptions(optimization_level=lvl))
        (yd,) = s_dense.run(None, {"x": g["x"]})
        assert np.array_equal(bits(y), bits(yd)), lvl

    rng = np.random.default_rng(12)
    M, K, N = 96, 200, 5
    q = rng.integers(-127, 128, (M, K)).astype(np.int8)
    q[rng.random(q.shape) < 0.7] = 0
    ip = np.concatenate([[0], np.cumsum((q != 0).sum(1))]).astype(np.int64)
    ix = np.nonzero(q)[1].astype(np.int32)
    x = rng.standard_normal((K, N)).astype(np.float32)
    xt = rng.standard_normal((N, M)).astype(np.float32)
    bias = rng.standard_normal(K).astype(np.float32)
    for scales, axis, tag in ((rng.random(M) + 0.01, 0, "row"), (rng.random(K) + 0.01, 1, "col"),
                              (np.array([0.02]), 0, "tensor")):
        rec = pfm.csr_record_int8((M, K), ip, ix, q[q != 0], scales.astype(np.float32), axis)
        Wd = pfm.record_to_dense(rec)
        say(f"int8 CSR record, scales per {tag}: W.x, x.W, Gemm transB")
        mm = {"name": "q", "inputs": [("x", 0, [K, N]), ("xt", 0, [N, M])],
              "outputs": [("y", 0, [M, N]), ("z", 0, [N, K]), ("u", 0, [N, M])],
              "initializers": {"bias": bias}, "sparse_initializers": {"w": rec},
              "nodes": [("wx", "MatMul", ["w", "x"], ["y"], {}),
                        ("xw", "MatMul", ["xt", "w"], ["z0"], {}), ("r", "Relu", ["z0"], ["z"], {}),
                        ("gm", "Gemm", ["x", "w", "bias"], ["u0"], {"transA": 1, "transB": 1, "alpha": 0.5}),
                        ("r2", "Relu", ["u0"], ["u"], {})]}
        pq = str(tmp_path / f"q_{tag}.pfm")
        pfm.save(mm, pq)
        for lvl in (2, 0):
            s = session.InferenceSession(pq, session.SessionOptions(optimization_level=lvl))
            y, z, u = s.run(None, {"x": x, "xt": xt})
            assert np.array_equal(bits(y), bits(O.orc_matmul(Wd, x))), (tag, lvl)
            assert np.array_equal(bits(z), bits(O.orc_relu(O.orc_matmul(xt, Wd)))), (tag, lvl)
            ref_u = O.orc_relu(O.orc_gemm(x, Wd, bias, 0.5, 1.0, transA=1, transB=1))
            assert np.array_equal(bits(u), bits(ref_u)), (tag, lvl)

    gq = golden("qmatmul.npz")
    wq, xq, ws = gq["sp_wq"], gq["sp_xq"], float(gq["sp_ws"])
    rec24 = pfm.nm24_record(wq)
    assert np.array_equal(pfm.record_to_dense(rec24), wq)
    f = rng.standard_normal((6, 8)).astype(np.float32)
    f[f < 0] = 0
    m24 = {"name": "q24", "inputs": [("x", 7, list(xq.shape))],
           "outputs": [("y", 0, [wq.shape[0], xq.shape[1]]), ("fr", 0, [6, 8])],
           "initializers": {}, "sparse_initializers": {"w": rec24, "f": pfm.csr_record(f)},
           "nodes": [("qmm", "QuantizedMatMul", ["w", "x"], ["y"], {"a_scale": ws, "b_scale": 0.05}),
                     ("rf", "Relu", ["f"], ["fr"], {})]}
    p24 = str(tmp_path / "q24.pfm")
    pfm.save(m24, p24)
    say("2:4 record under QuantizedMatMul; a record as a plain tensor")
    for lvl in (2, 0):
        s = session.InferenceSession(p24, session.SessionOptions(optimization_level=lvl))
        y, fr = s.run(None, {"x": xq})
        assert np.array_equal(bits(y), bits(gq["sp_yf"])), lvl
        assert np.array_equal(bits(fr), bits(f)), lvl
