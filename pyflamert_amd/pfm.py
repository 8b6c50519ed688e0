"""Reader and writer of the .pfm model format in Python, for building and
inspecting models.  Version 1 is the reference's format
(src/io/pyflame_format.cpp:392-498: magic "PFM\\0", u32 version, graph name,
inputs, outputs, initializers, nodes; little-endian; strings as u64 length +
bytes).  Version 2 appends a section of sparse initializers: pruned weights
kept as CSR (float32, or int8 with symmetric scales) or 2:4-compressed int8,
so a pruned model is stored and loaded without its dense form.  A model
without sparse initializers is written as version 1.

A model is a dict:
    {"name": str,
     "inputs":  [(name, dtype_code, shape)],   shape entries -1 = dynamic
     "outputs": [(name, dtype_code, shape)],
     "initializers": {name: numpy array},
     "sparse_initializers": {name: record},    optional (csr_record, nm24_record)
     "nodes": [(name, op_type, [inputs], [outputs], {attr: value})]}
Attribute values: int -> int64, float -> float32, str, list of int,
list of float (the format's types 0-4).

A CSR record stands for the float32 matrix rows x cols whose row r holds
values[j] at column indices[j], j in [indptr[r], indptr[r+1]) (indices
ascending); int8 values stand for (float)q * scale, the scale per tensor,
per row (scale_axis 0) or per column (scale_axis 1).  A 2:4 record stands for
the int8 matrix whose group g of four columns in row r holds values[r, 2g]
and values[r, 2g+1] at offsets positions[r, g] & 3 and positions[r, g] >> 2.
"""
from __future__ import annotations

import struct

import numpy as np

MAGIC = b"PFM\x00"
VERSION = 2
CSR, NM24 = 1, 2
F32, F16, BF16, F64, I64, I32, I16, I8, U8, BOOL = range(10)
_NP = {F32: np.float32, F16: np.float16, F64: np.float64, I64: np.int64, I32: np.int32, I16: np.int16,
       I8: np.int8, U8: np.uint8, BOOL: np.bool_, BF16: np.uint16}
_CODE = {np.dtype(v): k for k, v in _NP.items() if k != BF16}


def dtype_code(arr):
    return _CODE[np.asarray(arr).dtype]


class _W:
    def __init__(self):
        self.b = bytearray()

    def u32(self, v):
        self.b += struct.pack("<I", v)

    def u64(self, v):
        self.b += struct.pack("<Q", v)

    def i64(self, v):
        self.b += struct.pack("<q", v)

    def f32(self, v):
        self.b += struct.pack("<f", v)

    def s(self, t):
        raw = t.encode()
        self.u64(len(raw))
        self.b += raw


def csr_record(dense, threshold=0.0):
    """CSR record of a dense float32 matrix, keeping |v| > threshold in
    row-major order (to_sparse, sparse_tensor.cpp:560-610)."""
    d = np.ascontiguousarray(dense, np.float32)
    keep = np.abs(d) > threshold
    r, c = np.nonzero(keep)
    indptr = np.zeros(d.shape[0] + 1, np.int64)
    np.cumsum(np.bincount(r, minlength=d.shape[0]), out=indptr[1:])
    return {"format": "csr", "shape": tuple(d.shape), "indptr": indptr, "indices": c.astype(np.int32),
            "values": d[keep]}


def csr_record_int8(shape, indptr, indices, q, scales, scale_axis=0):
    """CSR record of int8 values with symmetric scales (1, one per row with
    scale_axis 0, or one per column with scale_axis 1)."""
    return {"format": "csr", "shape": tuple(shape), "indptr": np.asarray(indptr, np.int64),
            "indices": np.asarray(indices, np.int32), "values": np.asarray(q, np.int8),
            "scales": np.asarray(scales, np.float32).ravel(), "scale_axis": int(scale_axis)}


def nm24_record(dense):
    """2:4 record of an int8 matrix with at most two nonzeros in every group
    of four consecutive columns."""
    d = np.ascontiguousarray(dense, np.int8)
    rows, cols = d.shape
    if cols % 4:
        raise ValueError("2:4 needs cols divisible by 4")
    g = d.reshape(rows, cols // 4, 4)
    nz = g != 0
    if (nz.sum(-1) > 2).any():
        r, k = np.argwhere(nz.sum(-1) > 2)[0]
        raise ValueError(f"group {k} of row {r} has more than 2 nonzeros")
    # the kept offsets: nonzeros first (ascending), padded with the lowest
    # unused offsets, then the two chosen offsets sorted
    key = np.where(nz, 0, 1) * 4 + np.arange(4)
    pick = np.sort(np.argsort(key, axis=-1, kind="stable")[..., :2], axis=-1)
    vals = np.take_along_axis(g, pick, -1).reshape(rows, cols // 2)
    pos = (pick[..., 0] | (pick[..., 1] << 2)).astype(np.uint8)
    return {"format": "2:4", "shape": (rows, cols), "values": vals, "positions": pos}


def record_to_dense(rec):
    """The matrix a sparse record stands for."""
    rows, cols = rec["shape"]
    if rec["format"] == "2:4":
        out = np.zeros((rows, cols // 4, 4), np.int8)
        p = np.asarray(rec["positions"])
        v = np.asarray(rec["values"]).reshape(rows, cols // 4, 2)
        np.put_along_axis(out, np.stack([p & 3, p >> 2], -1).astype(np.int64), v, -1)
        return out.reshape(rows, cols)
    out = np.zeros((rows, cols), np.float32)
    ip = np.asarray(rec["indptr"])
    r = np.repeat(np.arange(rows), np.diff(ip))
    c = np.asarray(rec["indices"]).astype(np.int64)
    v = np.asarray(rec["values"])
    if v.dtype == np.int8:
        s = np.asarray(rec["scales"], np.float32)
        sc = s[0] if s.size == 1 else s[c if rec.get("scale_axis", 0) else r]
        v = (v.astype(np.float32) * sc).astype(np.float32)
    out[r, c] = v
    return out


def _dump_sparse(w, name, rec):
    rows, cols = (int(x) for x in rec["shape"])
    w.s(name)
    if rec["format"] == "csr":
        vals = np.ascontiguousarray(rec["values"])
        w.u32(CSR)
        w.u32(dtype_code(vals))
        w.i64(rows)
        w.i64(cols)
        w.u64(vals.size)
        narrow = cols <= 65536
        w.u32(2 if narrow else 4)
        w.b += np.ascontiguousarray(rec["indptr"], np.int64).tobytes()
        w.b += np.ascontiguousarray(rec["indices"], np.uint16 if narrow else np.int32).tobytes()
        w.b += vals.tobytes()
        sc = np.ascontiguousarray(rec.get("scales", np.zeros(0, np.float32)), np.float32).ravel()
        w.u32(int(rec.get("scale_axis", 0)))
        w.u64(sc.size)
        w.b += sc.tobytes()
    elif rec["format"] == "2:4":
        w.u32(NM24)
        w.u32(I8)
        w.i64(rows)
        w.i64(cols)
        w.b += np.ascontiguousarray(rec["values"], np.int8).tobytes()
        w.b += np.ascontiguousarray(rec["positions"], np.uint8).tobytes()
    else:
        raise ValueError(f"unknown sparse format {rec['format']!r}")


def dumps(model):
    w = _W()
    w.b += MAGIC
    sparse = model.get("sparse_initializers") or {}
    w.u32(VERSION if sparse else 1)
    w.s(model.get("name", ""))
    for key in ("inputs", "outputs"):
        w.u64(len(model[key]))
        for name, dt, shape in model[key]:
            w.s(name)
            w.u32(dt)
            w.u64(len(shape))
            for d in shape:
                w.i64(-1 if d is None else int(d))
    inits = model.get("initializers", {})
    w.u64(len(inits))
    for name in sorted(inits):
        a = np.ascontiguousarray(inits[name])
        w.s(name)
        w.u32(dtype_code(a))
        w.u64(a.ndim)
        for d in a.shape:
            w.i64(d)
        raw = a.tobytes()
        w.u64(len(raw))
        w.b += raw
    w.u64(len(model["nodes"]))
    for name, op, ins, outs, attrs in model["nodes"]:
        w.s(name)
        w.s(op)
        w.u64(len(ins))
        for x in ins:
            w.s(x)
        w.u64(len(outs))
        for x in outs:
            w.s(x)
        w.u64(len(attrs))
        for k in sorted(attrs):
            v = attrs[k]
            w.s(k)
            if isinstance(v, (bool, int, np.integer)):
                w.u32(0)
                w.i64(int(v))
            elif isinstance(v, (float, np.floating)):
                w.u32(1)
                w.f32(float(v))
            elif isinstance(v, str):
                w.u32(2)
                w.s(v)
            elif all(isinstance(x, (int, np.integer)) for x in v):
                w.u32(3)
                w.u64(len(v))
                for x in v:
                    w.i64(int(x))
            else:
                w.u32(4)
                w.u64(len(v))
                for x in v:
                    w.f32(float(x))
    if sparse:
        w.u64(len(sparse))
        for name in sorted(sparse):
            _dump_sparse(w, name, sparse[name])
    return bytes(w.b)


def save(model, path):
    with open(path, "wb") as f:
        f.write(dumps(model))


class _R:
    def __init__(self, b):
        self.b = memoryview(b)
        self.p = 0

    def take(self, n):
        if self.p + n > len(self.b):
            raise ValueError("Incomplete read")
        v = self.b[self.p:self.p + n]
        self.p += n
        return v

    def u32(self):
        return struct.unpack("<I", self.take(4))[0]

    def u64(self):
        return struct.unpack("<Q", self.take(8))[0]

    def i64(self):
        return struct.unpack("<q", self.take(8))[0]

    def f32(self):
        return struct.unpack("<f", self.take(4))[0]

    def s(self):
        return bytes(self.take(self.u64())).decode()


def _load_sparse(r):
    name, fmt, dt = r.s(), r.u32(), r.u32()
    rows, cols = r.i64(), r.i64()
    if fmt == CSR:
        nnz, width = r.u64(), r.u32()
        indptr = np.frombuffer(bytes(r.take(8 * (rows + 1))), np.int64).copy()
        idx = np.frombuffer(bytes(r.take(width * nnz)), np.uint16 if width == 2 else np.int32).astype(np.int32)
        vals = np.frombuffer(bytes(r.take(nnz * np.dtype(_NP[dt]).itemsize)), _NP[dt]).copy()
        axis, ns = r.u32(), r.u64()
        rec = {"format": "csr", "shape": (rows, cols), "indptr": indptr, "indices": idx, "values": vals}
        if ns:
            rec["scales"] = np.frombuffer(bytes(r.take(4 * ns)), np.float32).copy()
            rec["scale_axis"] = axis
        return name, rec
    if fmt == NM24:
        vals = np.frombuffer(bytes(r.take(rows * (cols // 2))), np.int8).reshape(rows, cols // 2).copy()
        pos = np.frombuffer(bytes(r.take(rows * (cols // 4))), np.uint8).reshape(rows, cols // 4).copy()
        return name, {"format": "2:4", "shape": (rows, cols), "values": vals, "positions": pos}
    raise ValueError(f"Unknown sparse format {fmt}")


def loads(data):
    r = _R(data)
    if bytes(r.take(4)) != MAGIC:
        raise ValueError("Invalid magic bytes")
    version = r.u32()
    if version > VERSION:
        raise ValueError("Unsupported version")
    m = {"name": r.s(), "inputs": [], "outputs": [], "initializers": {}, "nodes": []}
    for key in ("inputs", "outputs"):
        for _ in range(r.u64()):
            name, dt, nd = r.s(), r.u32(), r.u64()
            m[key].append((name, dt, [None if d < 0 else d for d in (r.i64() for _ in range(nd))]))
    for _ in range(r.u64()):
        name, dt, nd = r.s(), r.u32(), r.u64()
        shape = [r.i64() for _ in range(nd)]
        raw = bytes(r.take(r.u64()))
        m["initializers"][name] = np.frombuffer(raw, _NP[dt]).reshape(shape).copy()
    for _ in range(r.u64()):
        name, op = r.s(), r.s()
        ins = [r.s() for _ in range(r.u64())]
        outs = [r.s() for _ in range(r.u64())]
        attrs = {}
        for _ in range(r.u64()):
            k, t = r.s(), r.u32()
            if t == 0:
                attrs[k] = r.i64()
            elif t == 1:
                attrs[k] = r.f32()
            elif t == 2:
                attrs[k] = r.s()
            elif t == 3:
                attrs[k] = [r.i64() for _ in range(r.u64())]
            elif t == 4:
                attrs[k] = [r.f32() for _ in range(r.u64())]
            elif t != 255:
                raise ValueError(f"Unknown attribute type {t}")
        m["nodes"].append((name, op, ins, outs, attrs))
    if version >= 2:
        m["sparse_initializers"] = dict(_load_sparse(r) for _ in range(r.u64()))
    return m


def load(path):
    with open(path, "rb") as f:
        return loads(f.read())
