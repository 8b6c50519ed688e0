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
        "version.pfm": (raw[:4] + (2).to_bytes(4, "little") + raw[8:], "Unsupported version"),
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
