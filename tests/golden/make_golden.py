"""Write the golden vectors under tests/golden/ from the COMPILED REFERENCE.

Run in the build container (where /root/reference exists) after
``make -C oracle ref``:

    python tests/golden/make_golden.py

Every expected output below is produced by the reference's own kernel
functions (oracle/_ref/libpfr_ref.so, built from the reference sources where
they lie), never by the oracle or by the product.  Inputs are seeded numpy
draws.  The files hold data only: inputs and expected outputs, plus one
reference-written .pfm model (gzip) for the loader and end-to-end MLP tests.
MANIFEST.json records the SHA-256 of every file.
"""
from __future__ import annotations

import gzip
import hashlib
import json
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402


def f32(a):
    return np.ascontiguousarray(a, np.float32)


def save(name, **arrays):
    path = os.path.join(HERE, name)
    np.savez_compressed(path, **arrays)
    return name


def gen_kat():
    # tests/cpp/test_executor.cpp:162-208
    a = f32([[1, 2, 3], [4, 5, 6]])
    b = f32([[1, 2], [3, 4], [5, 6]])
    return save("kat_matmul.npz", a=a, b=b, out=O.ref_op_f32("MatMul", [a, b]))


def gen_gemm(rng):
    cases = {}
    specs = [
        # (M, K, N, alpha, beta, transA, transB, bias_kind)
        (7, 5, 3, 1.0, 1.0, 0, 0, "N"),
        (7, 5, 3, 0.7, 1.3, 1, 0, "N"),
        (6, 9, 4, -1.5, 0.5, 0, 1, "MN"),
        (5, 8, 6, 2.0, -1.0, 1, 1, "one"),
        (4, 16, 10, 1.0, 1.0, 0, 0, "odd"),
        (8, 12, 5, 1.0, 1.0, 0, 0, "none"),
        (32, 784, 64, 1.0, 1.0, 0, 0, "N"),
    ]
    for i, (M, K, N, al, be, ta, tb, bk) in enumerate(specs):
        A = f32(rng.standard_normal((K, M) if ta else (M, K)))
        B = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
        B[rng.random(B.shape) < 0.8] = 0.0
        B[rng.random(B.shape) < 0.05] = -0.0
        csz = {"N": N, "MN": M * N, "one": 1, "odd": 7, "none": 0}[bk]
        ins = [A, f32(B)]
        if csz:
            Cb = f32(rng.standard_normal(csz))
            ins.append(Cb)
        else:
            Cb = np.zeros(0, np.float32)
        out = O.ref_op_f32("Gemm", ins, {"alpha": al, "beta": be}, {"transA": ta, "transB": tb})
        cases.update({f"c{i}_A": A, f"c{i}_B": f32(B), f"c{i}_C": Cb,
                      f"c{i}_p": np.array([al, be, ta, tb], np.float32), f"c{i}_out": out})
    cases["n"] = np.array(len(specs))
    return save("gemm.npz", **cases)


def gen_matmul(rng):
    cases = {}
    shapes = [((3, 4, 5), (5, 6)), ((4, 5), (3, 5, 6)), ((2, 3, 4), (2, 4, 5)),
              ((16, 64), (64, 32))]
    for i, (sa, sb) in enumerate(shapes):
        a = f32(rng.standard_normal(sa))
        b = rng.standard_normal(sb).astype(np.float32)
        b[rng.random(sb) < 0.9] = 0.0
        cases[f"c{i}_a"] = a
        cases[f"c{i}_b"] = f32(b)
        cases[f"c{i}_out"] = O.ref_op_f32("MatMul", [a, f32(b)])
    cases["n"] = np.array(len(shapes))
    return save("matmul.npz", **cases)


def gen_csr(rng):
    out = {}
    M, K = 200, 300
    W = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
    W[rng.random((M, K)) >= 0.1] = 0.0
    W[5, :] = 0.0                                   # empty row
    W[7, rng.random(K) < 0.05] = -0.0               # signed zeros are dropped
    W[9, :10] = np.float32(0.005)                   # at the 0.005 threshold
    out["W"] = W
    for tag, thr in (("t0", 0.0), ("t1", 0.005)):
        ip, ix, v = O.ref_to_sparse_csr(W, thr)
        out[f"{tag}_indptr"], out[f"{tag}_indices"], out[f"{tag}_values"] = ip, ix, v
    ip, ix, v = out["t0_indptr"], out["t0_indices"], out["t0_values"]
    for n in (1, 8, 64):
        X = f32(rng.standard_normal((K, n)))
        out[f"X{n}"] = X
        out[f"Y{n}"] = O.ref_sparse_matmul(M, K, ip, ix, v, X)
    x = f32(rng.standard_normal(K))
    out["x"] = x
    out["y_matvec"] = O.ref_sparse_matvec(M, K, ip, ix, v, x)
    out["y_1d"] = O.ref_sparse_matmul(M, K, ip, ix, v, x)
    Z = np.zeros((3, 4), np.float32)
    zi, zx, zv = O.ref_to_sparse_csr(Z)
    out["zero_indptr"] = zi
    out["zero_nnz"] = np.array(len(zx))
    return save("csr.npz", **out)


def gen_masks(rng):
    out = {}
    w1 = f32(rng.normal(0.0, 0.05, (784, 512)))
    w2 = f32(rng.normal(0.0, 0.05, (512, 10)))
    out["w1"] = w1
    out["w2"] = w2
    out["w1_mask90"] = np.packbits(O.ref_magnitude_mask(w1, 0.9).ravel() != 0)
    out["w2_mask90"] = np.packbits(O.ref_magnitude_mask(w2, 0.9).ravel() != 0)
    ties = f32(rng.integers(-3, 4, size=1003))
    out["ties"] = ties
    for s in (0.1, 0.3, 0.5, 0.9, 0.999):
        out[f"ties_mag_{s}"] = O.ref_magnitude_mask(ties, s)
    for n, m in ((2, 4), (1, 4), (3, 8), (2, 3), (5, 7), (4, 4)):
        out[f"ties_nm_{n}_{m}"] = O.ref_nm_mask(ties, n, m)
    g = f32(rng.standard_normal((64, 64)))
    out["gauss"] = g
    out["gauss_nm_2_4"] = O.ref_nm_mask(g, 2, 4)
    out["gauss_mag_0.8"] = O.ref_magnitude_mask(g, 0.8)
    t = f32(rng.standard_normal(257))
    mk = f32(rng.random(257) < 0.5)
    out["am_t"], out["am_mask"] = t, mk
    out["am_out"] = O.ref_apply_mask(t, mk)
    return save("masks.npz", **out)


def gen_quant(rng):
    out = {}
    s = np.float32(0.05)
    edge = f32([0.0, -0.0, 0.025, -0.025, 0.075, -0.075, 6.35, -6.4, 6.375, -6.425,
                1e10, -1e10, 3e9, np.inf, -np.inf, np.nan, 1e-30, 0.02499999])
    xs = np.concatenate([edge, f32(rng.standard_normal(500) * 3)])
    out["x"] = xs
    for dt, zp in ((O.I8, 0), (O.I8, -3), (O.U8, 128), (O.U8, 7)):
        out[f"q_{dt}_{zp}"] = O.ref_quantize(xs, [s], [zp], dt)
    xc = f32(rng.standard_normal((3, 5, 7)) * 2)
    scales = f32([0.01, 0.02, 0.05, 0.1, 1.0])
    zps = np.array([0, 1, -2, 3, 0], np.int32)
    out["xc"], out["xc_scales"], out["xc_zps"] = xc, scales, zps
    out["qc_i8"] = O.ref_quantize(xc, scales, zps, O.I8, (3, 5, 7))
    out["qc_u8"] = O.ref_quantize(xc, scales, np.array([128, 120, 130, 0, 255], np.int32), O.U8, (3, 5, 7))
    qv = np.arange(-128, 128, dtype=np.int8)
    out["dq_i8"] = O.ref_dequantize(qv, [0.05], [3], O.I8)
    qu = np.arange(0, 256, dtype=np.uint8)
    out["dq_u8"] = O.ref_dequantize(qu, [0.1], [128], O.U8)
    qcv = rng.integers(-128, 128, size=(3, 5, 7)).astype(np.int8)
    out["qcv"] = qcv
    out["dqc_i8"] = O.ref_dequantize(qcv, scales, zps, O.I8, (3, 5, 7))
    mm = [(-1.0, 1.0), (-0.3, 2.7), (0.5, 0.5), (0.0, 1e-9), (-1e-12, 1e-12), (-5.0, -1.0),
          (1e-12, 3e-11), (-100.0, 0.25)]
    res = []
    for mn, mx in mm:
        for dt in (O.I8, O.U8):
            for sym in (True, False):
                sc, z = O.ref_params_from_minmax(mn, mx, dt, sym)
                res.append([mn, mx, dt, int(sym), sc, z])
    out["minmax"] = np.array(res, np.float64)
    dyn = f32(rng.standard_normal(1000) * 0.7)
    dyn[[3, 10]] = [np.nan, np.inf]
    out["dyn_x"] = dyn
    rows = []
    for dt in (O.I8, O.U8):
        for sym in (True, False):
            sc, z = O.ref_dynamic_params(dyn, dt, sym)
            rows.append([dt, int(sym), sc, z])
    out["dyn"] = np.array(rows, np.float64)
    pc = f32(rng.standard_normal((2, 6, 9)))
    pc[:, 2, :] = 0.5                                   # constant channel
    pc[:, 4, :] = np.nan                                # all non-finite channel
    out["pc_x"] = pc
    for dt in (O.I8, O.U8):
        for sym in (True, False):
            sc, z = O.ref_dynamic_params_per_channel(pc, dt, sym)
            out[f"pc_{dt}_{int(sym)}_s"] = sc
            out[f"pc_{dt}_{int(sym)}_z"] = z
    return save("quant.npz", **out)


def gen_qmatmul(rng):
    out = {}
    M, K, N = 48, 64, 40
    a = rng.integers(-128, 128, size=(M, K)).astype(np.int8)
    b = rng.integers(-128, 128, size=(K, N)).astype(np.int8)
    out["a"], out["b"] = a, b
    out["f_zp0"] = O.ref_quantized_matmul(a, b, 0.02, 0.05)
    out["f_zp"] = O.ref_quantized_matmul(a, b, 0.02, 0.05, 3, -2)
    sc, z = O.ref_dynamic_params(out["f_zp0"])
    out["rq_params"] = np.array([sc, z], np.float64)
    out["rq_i8"] = O.ref_quantized_matmul(a, b, 0.02, 0.05, out_params=(float(sc), z, O.I8))
    au = rng.integers(0, 256, size=(M, K)).astype(np.uint8)
    out["au"] = au
    out["f_u8"] = O.ref_quantized_matmul(au, b, 0.02, 0.05, 128, 0)
    out["op_qmm"] = O.ref_op_f32("QuantizedMatMul", [a, b], {"a_scale": 0.02, "b_scale": 0.05},
                                 {"a_zero_point": 1, "b_zero_point": -1})
    out["op_qmm_u8"] = O.ref_op_f32("QuantizedMatMul", [au, b], {"a_scale": 0.02, "b_scale": 0.05},
                                    {"a_zero_point": 0, "b_zero_point": 0})
    # 2:4 int8 weight, per-tensor scale (the reference kernel uses scales[0]):
    Mw, Kw, Nw = 64, 256, 48
    w = f32(rng.standard_normal((Mw, Kw)))
    w = O.ref_apply_mask(w, O.ref_nm_mask(w, 2, 4))
    ws, _ = O.ref_dynamic_params(w)
    wq = O.ref_quantize(w, [ws], [0], O.I8)
    xq = O.ref_quantize(f32(rng.standard_normal((Kw, Nw))), [0.05], [0], O.I8)
    yf = O.ref_quantized_matmul(wq, xq, float(ws), 0.05)
    ys, yz = O.ref_dynamic_params(yf)
    out["sp_w"], out["sp_wq"], out["sp_ws"], out["sp_xq"] = w, wq, np.float32(ws), xq
    out["sp_yf"] = yf
    out["sp_y_params"] = np.array([ys, yz], np.float64)
    out["sp_yq"] = O.ref_quantized_matmul(wq, xq, float(ws), 0.05, out_params=(float(ys), yz, O.I8))
    return save("qmatmul.npz", **out)


def gen_bf16(rng):
    sp = np.array([0x00000000, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0xFFC00000,
                   0x7F800001, 0x7F810000, 0xFF800001, 0x7FFF0000, 0x7F7F0000, 0x7F7F7FFF,
                   0x7F7F8000, 0x7F7FFFFF, 0xFF7FFFFF, 0x7F7E8000, 0x3F808000, 0x3F818000,
                   0x3F807FFF, 0x3F80C000, 0x00000001, 0x00008000, 0x00018000, 0x807FFFFF,
                   0x3F800000, 0xBF800000, 0x7F000000, 0x00800000], np.uint32)
    x = np.concatenate([sp.view(np.float32),
                        f32(rng.standard_normal(2000) * np.exp(rng.uniform(-30, 30, 2000)))])
    return save("bf16.npz", x=x, bf16=O.ref_bf16_from_float(x))


def gen_mlp(rng):
    """The 784-512-10 MLP: N(0,0.05) weights magnitude-pruned to 90 % by the
    reference mask producer, zero biases, x ~ U(0,1) [32,784]; the model is
    written by the reference .pfm writer and run by the reference executor."""
    w1 = f32(rng.normal(0.0, 0.05, (784, 512)))
    w2 = f32(rng.normal(0.0, 0.05, (512, 10)))
    w1 = O.ref_apply_mask(w1, O.ref_magnitude_mask(w1, 0.9))
    w2 = O.ref_apply_mask(w2, O.ref_magnitude_mask(w2, 0.9))
    b1 = np.zeros(512, np.float32)
    b2 = np.zeros(10, np.float32)
    x = f32(rng.uniform(0.0, 1.0, (32, 784)))
    with tempfile.TemporaryDirectory() as td:
        p = os.path.join(td, "mlp.pfm")
        O.ref_save_mlp_pfm(p, 32, w1, b1, w2, b2)
        y = O.ref_run_pfm(p, "x", x, 32 * 10).reshape(32, 10)
        raw = open(p, "rb").read()
    with open(os.path.join(HERE, "mlp_784_512_10.pfm.gz"), "wb") as fo:
        with gzip.GzipFile(filename="", mode="wb", compresslevel=9, fileobj=fo, mtime=0) as f:
            f.write(raw)
    # Intermediate h1 = Gemm(x, W1, b1) through the reference Gemm op.
    h1 = O.ref_op_f32("Gemm", [x, w1, b1], {"alpha": 1.0, "beta": 1.0}, {"transA": 0, "transB": 0})
    n1 = save("mlp.npz", x=x, y=y, h1=h1, pfm_sha256=np.frombuffer(hashlib.sha256(raw).digest(), np.uint8),
              nnz=np.array([np.count_nonzero(w1), np.count_nonzero(w2)]))
    return [n1, "mlp_784_512_10.pfm.gz"]


def gen_neighbours(rng):
    """The products' graph neighbours on the BERT-shaped workload: Gelu
    (activation.cpp:239-259) over a wide range and special values,
    LayerNormalization (nn.cpp:419-490) on [1024, 768]-like rows with random
    scale and bias, two epsilons and a normalisation over the last two axes,
    and Add (math.cpp:150-224) with equal shapes, a bias broadcast over the
    last axis, a scalar and a middle-axis broadcast."""
    g = np.concatenate([f32(rng.normal(0, 3, 4000)), f32(np.linspace(-12, 12, 2001)),
                        f32([0.0, -0.0, 1e-30, -1e-30, 20.0, -20.0, 88.0, -88.0, np.inf, -np.inf, np.nan])])
    out = {"gelu_x": g, "gelu_y": O.ref_op_f32("Gelu", [g])}
    x = f32(rng.normal(0.5, 2.0, (64, 768)))
    sc = f32(rng.normal(1.0, 0.2, 768))
    bi = f32(rng.normal(0.0, 0.2, 768))
    out.update(ln_x=x, ln_scale=sc, ln_bias=bi,
               ln_y=O.ref_op_f32("LayerNormalization", [x, sc, bi], {"epsilon": 1e-5}, {"axis": -1}),
               ln_y_eps12=O.ref_op_f32("LayerNormalization", [x, sc, bi], {"epsilon": 1e-12}, {"axis": -1}))
    x3 = f32(rng.normal(0, 1, (4, 6, 32)))
    sc3 = f32(rng.normal(1, 0.1, 6 * 32))
    bi3 = f32(rng.normal(0, 0.1, 6 * 32))
    out.update(ln3_x=x3, ln3_scale=sc3, ln3_bias=bi3,
               ln3_y=O.ref_op_f32("LayerNormalization", [x3, sc3, bi3], {"epsilon": 1e-5}, {"axis": 1}))
    a = f32(rng.normal(0, 1, (8, 16, 32)))
    out.update(add_a=a, add_b_same=f32(rng.normal(0, 1, (8, 16, 32))), add_b_bias=f32(rng.normal(0, 1, 32)),
               add_b_scalar=f32([0.375]), add_b_mid=f32(rng.normal(0, 1, (16, 1))))
    for k in ("same", "bias", "scalar", "mid"):
        out[f"add_y_{k}"] = O.ref_op_f32("Add", [a, out[f"add_b_{k}"]])
    # both operands broadcast, and an empty operand against a size-1 one
    # (the output takes the larger extent per axis and stays zero)
    out.update(add2_a=f32(rng.normal(0, 1, (4, 1, 5))), add2_b=f32(rng.normal(0, 1, (3, 1))))
    out["add2_y"] = O.ref_op_f32("Add", [out["add2_a"], out["add2_b"]])
    out.update(add0_a=np.zeros((2, 0, 3), np.float32), add0_b=f32(rng.normal(0, 1, (1, 3))))
    out["add0_y"] = O.ref_op_f32("Add", [out["add0_a"], out["add0_b"]])
    return save("neighbours.npz", **out)


def main():
    if not O.have_ref():
        raise SystemExit("build the reference library first: make -C oracle ref")
    rng = np.random.default_rng(20261201)
    names = [gen_kat(), gen_gemm(rng), gen_matmul(rng), gen_csr(rng), gen_masks(rng),
             gen_quant(rng), gen_qmatmul(rng), gen_bf16(rng)]
    names += gen_mlp(rng)
    names.append(gen_neighbours(rng))
    manifest = {}
    for n in names:
        data = open(os.path.join(HERE, n), "rb").read()
        manifest[n] = {"sha256": hashlib.sha256(data).hexdigest(), "bytes": len(data)}
    manifest["_generator"] = {
        "script": "tests/golden/make_golden.py",
        "expected_outputs_from": "oracle/_ref/libpfr_ref.so (reference sources, g++ -std=c++17 -O3 -DNDEBUG)",
        "seed": 20261201,
    }
    with open(os.path.join(HERE, "MANIFEST.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
    print(json.dumps(manifest, indent=1))


if __name__ == "__main__":
    main()
