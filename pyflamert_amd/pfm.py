"""Reader and writer of the .pfm v1 model format in Python, for building and
inspecting models (the format of src/io/pyflame_format.cpp:392-498:
magic "PFM\\0", u32 version, graph name, inputs, outputs, initializers,
nodes; little-endian; strings as u64 length + bytes).

A model is a dict:
    {"name": str,
     "inputs":  [(name, dtype_code, shape)],   shape entries -1 = dynamic
     "outputs": [(name, dtype_code, shape)],
     "initializers": {name: numpy array},
     "nodes": [(name, op_type, [inputs], [outputs], {attr: value})]}
Attribute values: int -> int64, float -> float32, str, list of int,
list of float (the format's types 0-4).
"""
from __future__ import annotations

import struct

import numpy as np

MAGIC = b"PFM\x00"
VERSION = 1
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


def dumps(model):
    w = _W()
    w.b += MAGIC
    w.u32(VERSION)
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


def loads(data):
    r = _R(data)
    if bytes(r.take(4)) != MAGIC:
        raise ValueError("Invalid magic bytes")
    if r.u32() > VERSION:
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
    return m


def load(path):
    with open(path, "rb") as f:
        return loads(f.read())
