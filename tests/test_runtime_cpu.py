"""Host logic of the C++ runtime, on the CPU: the .pfm loader against the
model written by the compiled reference, writer round trips (read back by
the reference's own loader where it is built), graph validation, options and
device errors, corrupt files and unsafe paths."""
import gzip
import os

import numpy as np
import pytest

from oracle import oracle as O
from pyflamert_amd import pfm, session

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def mlp_path(tmp_path_factory):
    p = tmp_path_factory.mktemp("m") / "mlp.pfm"
    p.write_bytes(gzip.open(os.path.join(GOLD, "mlp_784_512_10.pfm.gz")).read())
    return str(p)


def test_loader_reads_reference_model(mlp_path):
    d = session.describe_model(mlp_path)
    py = pfm.load(mlp_path)
    assert d["name"] == py["name"] == "mlp"
    assert d["inputs"] == [{"name": "x", "dtype": 0, "shape": [32, 784]}]
    assert d["outputs"] == [{"name": "y", "dtype": 0, "shape": [32, 10]}]
    assert d["initializers"]["fc1.weight"] == {"dtype": 0, "shape": [784, 512], "nnz": 40141}
    assert d["initializers"]["fc2.weight"]["nnz"] == 512
    assert [n["op"] for n in d["nodes"]] == ["Gemm", "Relu", "Gemm", "Softmax"]
    g1 = d["nodes"][0]
    assert g1["inputs"] == ["x", "fc1.weight", "fc1.bias"]
    assert g1["attrs"] == {"alpha": 1.0, "beta": 1.0, "transA": 0, "transB": 0}
    assert d["nodes"][3]["attrs"] == {"axis": -1}
    for name, arr in py["initializers"].items():
        assert d["initializers"][name]["shape"] == list(arr.shape)


def test_resave_roundtrip(mlp_path, tmp_path):
    out = str(tmp_path / "again.pfm")
    session.resave_model(mlp_path, out)
    a, b = pfm.load(mlp_path), pfm.load(out)
    assert a["name"] == b["name"] and a["inputs"] == b["inputs"] and a["outputs"] == b["outputs"]
    assert sorted(a["initializers"]) == sorted(b["initializers"])
    for k in a["initializers"]:
        assert np.array_equal(a["initializers"][k], b["initializers"][k])
    assert [n[:4] for n in a["nodes"]] == [n[:4] for n in b["nodes"]]
    assert session.describe_model(out) == session.describe_model(mlp_path)
    # byte-reproducible writer
    out2 = str(tmp_path / "again2.pfm")
    session.resave_model(out, out2)
    assert open(out, "rb").read() == open(out2, "rb").read()


@pytest.mark.skipif(not O.have_ref(), reason="compiled reference not present")
def test_reference_loader_runs_our_files(mlp_path, tmp_path, golden):
    """Files written by this runtime's writer and by the Python writer load
    and run in the reference's own loader/executor with identical results."""
    g = golden("mlp.npz")
    out = str(tmp_path / "resaved.pfm")
    session.resave_model(mlp_path, out)
    y = O.ref_run_pfm(out, "x", g["x"], 320).reshape(32, 10)
    assert np.array_equal(y.view(np.uint32), g["y"].view(np.uint32))
    m = pfm.load(mlp_path)
    p2 = str(tmp_path / "py.pfm")
    pfm.save(m, p2)
    y2 = O.ref_run_pfm(p2, "x", g["x"], 320).reshape(32, 10)
    assert np.array_equal(y2.view(np.uint32), g["y"].view(np.uint32))


def write(tmp_path, name, model):
    p = str(tmp_path / name)
    pfm.save(model, p)
    return p


def small_model(nodes, inits=None, outputs=(("y", 0, [2, 2]),)):
    return {"name": "t", "inputs": [("a", 0, [2, 3])], "outputs": list(outputs),
            "initializers": inits or {"b": np.ones((3, 2), np.float32)}, "nodes": nodes}


def test_graph_validation_errors(tmp_path):
    p = write(tmp_path, "missing.pfm", small_model([("mm", "MatMul", ["a", "nope"], ["y"], {})]))
    with pytest.raises(session.ValidationError, match="input 'nope' not found"):
        session.describe_model(p)
    p = write(tmp_path, "cycle.pfm", small_model([("n1", "Relu", ["z"], ["y"], {}), ("n2", "Relu", ["y"], ["z"], {})]))
    with pytest.raises(session.ValidationError, match="cycle"):
        session.describe_model(p)
    p = write(tmp_path, "noout.pfm", small_model([("mm", "MatMul", ["a", "b"], ["q"], {})]))
    with pytest.raises(session.ValidationError, match="Graph output 'y' not produced"):
        session.describe_model(p)


def test_corrupt_files(tmp_path, mlp_path):
    raw = open(mlp_path, "rb").read()
    cases = {
        "magic.pfm": (b"XFM\0" + raw[4:], "Invalid magic"),
        "trunc.pfm": (raw[: len(raw) // 2], "Incomplete read"),
        "version.pfm": (raw[:4] + (3).to_bytes(4, "little") + raw[8:], "Unsupported version"),
        "v2nosparse.pfm": (raw[:4] + (2).to_bytes(4, "little") + raw[8:], "Incomplete read"),
    }
    for name, (data, msg) in cases.items():
        p = tmp_path / name
        p.write_bytes(data)
        with pytest.raises(session.InvalidModelError, match=msg):
            session.describe_model(str(p))
    # a string length far beyond the limit
    bad = bytearray(raw)
    bad[8:16] = (1 << 40).to_bytes(8, "little")
    p = tmp_path / "biglen.pfm"
    p.write_bytes(bytes(bad))
    with pytest.raises(session.InvalidModelError, match="String size exceeds limit"):
        session.describe_model(str(p))
    # an unknown attribute type code
    m = small_model([("mm", "MatMul", ["a", "b"], ["y"], {"k": 1})])
    data = bytearray(pfm.dumps(m))
    i = data.rfind(b"\x01\x00\x00\x00\x00\x00\x00\x00k")  # len-1 string "k"
    j = i + 9
    data[j:j + 4] = (7).to_bytes(4, "little")
    p = tmp_path / "attr.pfm"
    p.write_bytes(bytes(data))
    with pytest.raises(session.InvalidModelError, match="Unknown attribute type 7"):
        session.describe_model(str(p))


def test_paths_and_formats(tmp_path):
    with pytest.raises(session.InvalidModelError, match="traversal"):
        session.describe_model("../x.pfm")
    with pytest.raises(session.UnsupportedFormatError, match=".onnx"):
        session.describe_model(str(tmp_path / "m.onnx"))
    with pytest.raises(session.InvalidModelError, match="Cannot open file"):
        session.describe_model(str(tmp_path / "absent.pfm"))


def test_session_options_and_device_errors(mlp_path):
    with pytest.raises(session.PyFlameRTError, match="Invalid device: tpu"):
        session.InferenceSession(mlp_path, session.SessionOptions(device="tpu"))
    with pytest.raises(session.PyFlameRTError, match="not provided by this runtime"):
        session.InferenceSession(mlp_path, session.SessionOptions(device="cpu"))


def test_session_without_gpu_raises_backend_error(mlp_path):
    from pyflamert_amd import rocm

    if rocm.device_count() > 0:
        pytest.skip("a device is visible")
    with pytest.raises(session.BackendError, match="cannot initialise ROCm device"):
        session.InferenceSession(mlp_path, session.SessionOptions(device="rocm"))


def sparse_model(rng):
    """A graph with every sparse record form: float32 CSR, int8 CSR with
    per-row, per-column and per-tensor scales, and a 2:4 int8 record."""
    f = rng.standard_normal((40, 24)).astype(np.float32)
    f[rng.random(f.shape) < 0.8] = 0
    q = rng.integers(-127, 128, (30, 70000 // 1000)).astype(np.int8)
    q[rng.random(q.shape) < 0.7] = 0
    ip = np.concatenate([[0], np.cumsum((q != 0).sum(1))]).astype(np.int64)
    ix = np.nonzero(q)[1].astype(np.int32)
    qv = q[q != 0]
    wide = np.zeros((3, 70000), np.float32)  # cols > 65535: int32 indices on disk
    wide[0, [5, 69999]] = [1.5, -2.0]
    wide[2, 65536] = 3.0
    d24 = rng.integers(-100, 100, (8, 32)).astype(np.int8)
    g = d24.reshape(8, 8, 4)
    for r in range(8):
        for k in range(8):
            g[r, k, rng.permutation(4)[: 2 + (k % 3 == 0)]] = 0
    recs = {
        "f32": pfm.csr_record(f),
        "i8_row": pfm.csr_record_int8(q.shape, ip, ix, qv, rng.random(30).astype(np.float32) + 0.01, 0),
        "i8_col": pfm.csr_record_int8(q.shape, ip, ix, qv, rng.random(70).astype(np.float32) + 0.01, 1),
        "i8_one": pfm.csr_record_int8(q.shape, ip, ix, qv, [0.25], 0),
        "wide": pfm.csr_record(wide),
        "w24": pfm.nm24_record(g.reshape(8, 32)),
    }
    nodes = [("mm", "MatMul", ["a", "f32"], ["y"], {})]
    return {"name": "sp", "inputs": [("a", 0, [2, 40])], "outputs": [("y", 0, [2, 24])],
            "initializers": {"dense_b": np.ones((2, 2), np.float32)}, "sparse_initializers": recs,
            "nodes": nodes}


def test_sparse_records_roundtrip(tmp_path):
    """Version-2 sparse initializers: the C++ loader reads what the Python
    writer wrote, reports them, counts their stored bytes against the
    initializer limit, and writes the same bytes back; a model without them
    stays version 1."""
    rng = np.random.default_rng(3)
    m = sparse_model(rng)
    p = write(tmp_path, "sp.pfm", m)
    raw = open(p, "rb").read()
    assert raw[4:8] == (2).to_bytes(4, "little")
    d = session.describe_model(p)
    sp = d["sparse_initializers"]
    assert sorted(sp) == sorted(m["sparse_initializers"])
    stored = 16  # the dense 2x2 float32 initializer
    for name, rec in m["sparse_initializers"].items():
        rows, cols = rec["shape"]
        assert sp[name]["shape"] == [rows, cols]
        dense = pfm.record_to_dense(rec)
        if rec["format"] == "csr":
            nnz = len(rec["values"])
            assert sp[name]["format"] == "csr" and sp[name]["nnz"] == nnz
            b = 8 * (rows + 1) + 4 * nnz + rec["values"].nbytes + 4 * len(rec.get("scales", []))
        else:
            assert sp[name]["format"] == "2:4" and sp[name]["nnz"] == int(np.count_nonzero(dense))
            b = rows * cols // 2 + rows * cols // 4
        assert sp[name]["stored_bytes"] == b
        stored += b
    assert d["total_initializer_bytes"] == stored
    out = str(tmp_path / "sp2.pfm")
    session.resave_model(p, out)
    assert open(out, "rb").read() == raw
    back = pfm.load(out)
    for name, rec in m["sparse_initializers"].items():
        assert np.array_equal(pfm.record_to_dense(back["sparse_initializers"][name]), pfm.record_to_dense(rec))
    # the wide record keeps int32 indices on disk, the others uint16
    assert int(np.max(back["sparse_initializers"]["wide"]["indices"])) == 69999
    dense_only = dict(m, sparse_initializers={})
    p1 = write(tmp_path, "d.pfm", dense_only)
    assert open(p1, "rb").read()[4:8] == (1).to_bytes(4, "little")
    session.resave_model(p1, str(tmp_path / "d2.pfm"))
    assert open(str(tmp_path / "d2.pfm"), "rb").read()[4:8] == (1).to_bytes(4, "little")


def test_sparse_record_validation(tmp_path):
    """Malformed sparse records are rejected at load with the tensor named."""
    rng = np.random.default_rng(4)
    f = rng.standard_normal((5, 6)).astype(np.float32)
    f[rng.random(f.shape) < 0.5] = 0
    f[:, 0] = 1.0
    f[:, 5] = 2.0
    base = pfm.csr_record(f)

    def check(rec, msg, name="w"):
        m = {"name": "v", "inputs": [], "outputs": [], "initializers": {}, "nodes": [],
             "sparse_initializers": {name: rec}}
        p = write(tmp_path, "bad.pfm", m)
        with pytest.raises(session.InvalidModelError, match=msg):
            session.describe_model(p)

    r = dict(base, indices=base["indices"].copy())
    r["indices"][1], r["indices"][0] = r["indices"][0], r["indices"][1]
    check(r, "Sparse initializer 'w': column indices must ascend within row 0")
    r = dict(base, indices=base["indices"].copy())
    r["indices"][-1] = 6
    check(r, "column index 6 out of range")
    r = dict(base, indptr=base["indptr"].copy())
    r["indptr"][2] = r["indptr"][3] + 1
    check(r, "indptr must be non-decreasing")
    r = dict(base, indptr=base["indptr"].copy())
    r["indptr"][0] = 1
    check(r, "indptr")
    q = pfm.csr_record_int8((5, 6), base["indptr"], base["indices"], np.ones(len(base["values"]), np.int8),
                            np.ones(4, np.float32), 0)
    check(q, "int8 values need 1 scale or one per row")
    q["scales"] = np.array([1, 1, -1, 1, 1], np.float32)
    check(q, "scales must be positive and finite")
    w24 = pfm.nm24_record(np.zeros((2, 8), np.int8))
    w24["positions"] = w24["positions"].copy()
    w24["positions"][1, 1] = 1 | (1 << 2)  # both kept slots at offset 1
    check(w24, "2:4 group 3 has invalid positions")
    with pytest.raises(ValueError, match="more than 2 nonzeros"):
        pfm.nm24_record(np.ones((1, 4), np.int8))
    # a sparse record whose name is also a dense initializer
    m = {"name": "v", "inputs": [], "outputs": [], "initializers": {"w": f}, "nodes": [],
         "sparse_initializers": {"w": base}}
    p = write(tmp_path, "dup.pfm", m)
    with pytest.raises(session.InvalidModelError, match="already a dense initializer"):
        session.describe_model(p)


def quant_graph(rng, K=64, M1=48, M2=32, N=5, keep_dense=False):
    """MatMul(W1, x) -> Relu -> MatMul(W2, .) with 2:4-pruned W1 (CSR record)
    and W2 (dense), plus a MatMul whose weight is not 2:4 (left alone)."""
    def pruned24(m, k):
        w = rng.standard_normal((m, k)).astype(np.float32)
        return O.orc_apply_mask(w, O.orc_nm_mask(w.ravel(), 2, 4).reshape(m, k))
    w1, w2 = pruned24(M1, K), pruned24(M2, M1)
    w1[3, :] = 0.0  # an all-zero row: scale 1 (quant_params.cpp:78-82)
    dense3 = rng.standard_normal((7, K)).astype(np.float32)
    m = {"name": "q", "inputs": [("x", 0, [K, N])], "outputs": [("y", 0, [M2, N]), ("z", 0, [7, N])],
         "initializers": {"w2": w2, "w3": dense3},
         "sparse_initializers": {} if keep_dense else {"w1": pfm.csr_record(w1)},
         "nodes": [("mm1", "MatMul", ["w1", "x"], ["h"], {}), ("r", "Relu", ["h"], ["a"], {}),
                   ("mm2", "MatMul", ["w2", "a"], ["y"], {}), ("mm3", "MatMul", ["w3", "x"], ["z"], {})]}
    if keep_dense:
        m["initializers"]["w1"] = w1
    return m, w1, w2


def xw_graph(rng, T=6, K=64, N1=48, N2=32):
    """The x . W form: Gemm(x, W1 N1 x K, transB 1, bias) -> Relu ->
    MatMul(., W2 N1 x N2), both 2:4 along K, plus a Gemm whose bias is not a
    vector of N (left alone)."""
    def pruned24(m, k):
        w = rng.standard_normal((m, k)).astype(np.float32)
        return O.orc_apply_mask(w, O.orc_nm_mask(w.ravel(), 2, 4).reshape(m, k))
    w1 = pruned24(N1, K)                          # stored N x K (transB = 1)
    w2 = np.ascontiguousarray(pruned24(N2, N1).T)  # stored K x N, groups along K
    b1 = rng.standard_normal(N1).astype(np.float32)
    w4 = np.ascontiguousarray(pruned24(9, K).T)
    m = {"name": "xw", "inputs": [("x", 0, [T, K])], "outputs": [("y", 0, [T, N2]), ("z", 0, [T, 9])],
         "initializers": {"w1": w1, "b1": b1, "w2": w2, "w4": w4, "c4": np.ones((T, 9), np.float32)},
         "nodes": [("fc1", "Gemm", ["x", "w1", "b1"], ["h"], {"transB": 1}), ("r", "Relu", ["h"], ["a"], {}),
                   ("fc2", "MatMul", ["a", "w2"], ["y"], {}), ("fc4", "Gemm", ["x", "w4", "c4"], ["z"], {})]}
    return m, w1, b1, w2


def test_dynamic_int8_rewrite_xw(tmp_path):
    """The x . W form of the rewrite: Gemm(x, W, b) with transB and
    MatMul(x, W) become DynamicQuantizeLinear + QuantizedMatMul(X_q, W_q^T)
    (transB 1, per-output-column b_scales) [+ Add(bias)], with W_q^T the
    per-column quantization of W (oracle, on W^T's rows); a Gemm whose bias is
    not a vector of N stays."""
    rng = np.random.default_rng(3)
    m, w1, b1, w2 = xw_graph(rng)
    p = write(tmp_path, "xw.pfm", m)
    out = str(tmp_path / "xw_int8.pfm")
    assert session.quantize_model(p, out) == 2
    q = pfm.load(out)
    ops = [n[1] for n in q["nodes"]]
    assert ops == ["DynamicQuantizeLinear", "QuantizedMatMul", "Add", "Relu", "DynamicQuantizeLinear",
                   "QuantizedMatMul", "Gemm"]
    assert q["nodes"][2][3] == ["h"] and q["nodes"][2][2][1] == "b1" and q["nodes"][5][3] == ["y"]
    assert "w1" not in q["initializers"] and "w2" not in q["initializers"] and "w4" in q["initializers"]
    for dq, node in ((q["nodes"][0], q["nodes"][1]), (q["nodes"][4], q["nodes"][5])):
        assert node[2][0] == dq[3][0] and node[2][2:] == dq[3][1:]  # X_q, X_scale, X_zero_point
    for wt, node in ((w1, q["nodes"][1]), (np.ascontiguousarray(w2.T), q["nodes"][5])):
        N, K = wt.shape
        s_ref, _ = O.orc_dynamic_params_per_channel(wt.reshape(1, N, K))
        q_ref = O.orc_quantize(wt, s_ref, np.zeros(N, np.int32), O.I8, (1, N, K))
        rec = q["sparse_initializers"][node[2][1]]
        assert rec["format"] == "2:4" and np.array_equal(pfm.record_to_dense(rec), q_ref)
        assert np.array_equal(np.array(node[4]["b_scales"], np.float32).view(np.uint32),
                              np.asarray(s_ref, np.float32).view(np.uint32))
        assert node[4]["transB"] == 1 and node[4]["b_zero_point"] == 0


def test_dynamic_int8_rewrite(tmp_path):
    """The rewrite replaces the 2:4 MatMul(W, X) nodes by
    DynamicQuantizeLinear + QuantizedMatMul with the per-row int8 weights and
    scales of compute_dynamic_params_per_channel + quantize_tensor (oracle),
    stores them as 2:4 records, keeps the other nodes, and drops the float
    weights it replaced."""
    rng = np.random.default_rng(2)
    m, w1, w2 = quant_graph(rng)
    p = write(tmp_path, "q.pfm", m)
    out = str(tmp_path / "q_int8.pfm")
    assert session.quantize_model(p, out) == 2
    q = pfm.load(out)
    ops = [(n[1], n[2]) for n in q["nodes"]]
    assert [o for o, _ in ops] == ["DynamicQuantizeLinear", "QuantizedMatMul", "Relu", "DynamicQuantizeLinear",
                                   "QuantizedMatMul", "MatMul"]
    assert "w1" not in q["sparse_initializers"] and "w2" not in q["initializers"] and "w3" in q["initializers"]
    for w, node in ((w1, q["nodes"][1]), (w2, q["nodes"][4])):
        M, K = w.shape
        s_ref, _ = O.orc_dynamic_params_per_channel(w.reshape(1, M, K))
        q_ref = O.orc_quantize(w, s_ref, np.zeros(M, np.int32), O.I8, (1, M, K))
        name = node[2][0]
        rec = q["sparse_initializers"][name]
        assert rec["format"] == "2:4"
        assert np.array_equal(pfm.record_to_dense(rec), q_ref)
        assert np.array_equal(np.array(node[4]["a_scales"], np.float32).view(np.uint32),
                              np.asarray(s_ref, np.float32).view(np.uint32))
        assert node[4]["a_zero_point"] == 0
    # the quantizer output is itself a loadable, re-savable model
    session.resave_model(out, str(tmp_path / "again.pfm"))
    assert open(out, "rb").read() == open(str(tmp_path / "again.pfm"), "rb").read()
    with pytest.raises(session.PyFlameRTError, match="Invalid quantization mode"):
        session.quantize_model(p, out, "static_int4")
