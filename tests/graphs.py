"""Pure-Python writer of schema-3 model directories for tests.

Plays the role of the reference tests' WireGraphBuilder
(tests/unit/cpu_backend_tests.cpp:77-365): tensors get consecutive IDs,
weights 256-byte-aligned offsets in weights.bin, every activation its own
256-byte-aligned arena slot born at its producing node, and metadata.pb
carries the same checkpoint SHA as graph.pb. The protobuf encoding is
written here independently of the C++ codec (field numbers from the
reference proto/mlvc_model.proto), so loading these files also
cross-checks the C++ wire decoder.
"""

from __future__ import annotations

import hashlib
import pathlib
import struct

import numpy as np

FP16, INT32, INT64 = 1, 2, 3
OPS = dict(ADD=1, SUB=2, MUL=3, CLIP=4, CONCAT=5, CONV=6, DEPTH_TO_SPACE=7, GATHER=8, LEAKY_RELU=9, RECIPROCAL=10,
           ROUND=11, SIGMOID=12, SLICE=13, SPACE_TO_DEPTH=14)


def varint(v: int) -> bytes:
    v &= (1 << 64) - 1
    out = bytearray()
    while v >= 0x80:
        out.append((v & 0x7F) | 0x80)
        v >>= 7
    out.append(v)
    return bytes(out)


def tag(field: int, wt: int) -> bytes:
    return varint((field << 3) | wt)


def f_varint(field: int, v: int, always=False) -> bytes:
    return tag(field, 0) + varint(v) if (v or always) else b""


def f_bytes(field: int, b: bytes, always=False) -> bytes:
    return tag(field, 2) + varint(len(b)) + b if (b or always) else b""


def f_packed(field: int, vals, packed=True) -> bytes:
    if not vals:
        return b""
    if packed:
        return f_bytes(field, b"".join(varint(int(v)) for v in vals))
    return b"".join(tag(field, 0) + varint(int(v)) for v in vals)


def f_float(field: int, v: float) -> bytes:
    b = struct.pack("<f", v)
    return tag(field, 5) + b if b != b"\0\0\0\0" else b""


def zigzag(v: int) -> int:
    return (v << 1) ^ (v >> 31)


class Graph:
    def __init__(self, packed: bool = True):
        self.tensors = []  # dicts: id, name, dtype, shape, storage
        self.nodes = []
        self.inputs, self.outputs = [], []
        self.weights = bytearray()
        self.arena = 0
        self.packed = packed
        self.schema = 3
        self.checkpoint = b"k" * 32
        self.weights_sha = b"w" * 32
        self.arena_alignment = 256

    def _tensor(self, name, dtype, shape):
        t = dict(id=len(self.tensors) + 1, name=name, dtype=dtype, shape=list(shape), storage=None)
        self.tensors.append(t)
        return t["id"]

    def input(self, name, shape, dtype=FP16):
        i = self._tensor(name, dtype, shape)
        self.inputs.append(i)
        return i

    def weight(self, name, arr: np.ndarray, dtype=FP16):
        raw = np.ascontiguousarray(arr).tobytes()
        off = (len(self.weights) + 255) // 256 * 256
        self.weights.extend(b"\0" * (off - len(self.weights)))
        self.weights.extend(raw)
        i = self._tensor(name, dtype, arr.shape)
        self.tensors[i - 1]["storage"] = ("weight", off, len(raw))
        return i

    def weight_fp16(self, name, values: np.ndarray):
        return self.weight(name, np.asarray(values, np.float32).astype(np.float16).view(np.uint16))

    def _activation(self, name, shape, node_index, dtype=FP16):
        i = self._tensor(name, dtype, shape)
        size = (int(np.prod(shape)) * (2 if dtype == FP16 else 4) + 255) // 256 * 256
        self.tensors[i - 1]["storage"] = ["arena", self.arena, size, node_index, 0]
        self.arena += size
        return i

    def node(self, op, inputs, out_name, out_shape, attr=None):
        idx = len(self.nodes)
        out = self._activation(out_name, out_shape, idx)
        self.nodes.append(dict(op=OPS[op], inputs=list(inputs), outputs=[out], attr=attr))
        return out

    def shape(self, tid):
        return self.tensors[tid - 1]["shape"]

    def conv(self, name, x, w, b, stride=(1, 1), pads=(0, 0, 0, 0), groups=1):
        xs, ws = self.shape(x), self.shape(w)
        oh = (xs[2] + pads[0] + pads[2] - ws[2]) // stride[0] + 1
        ow = (xs[3] + pads[1] + pads[3] - ws[3]) // stride[1] + 1
        return self.node("CONV", [x, w, b], name, [xs[0], ws[0], oh, ow],
                         ("conv", list(stride), list(pads), [1, 1], groups))

    def leaky_relu(self, name, x, alpha=0.01):
        return self.node("LEAKY_RELU", [x], name, self.shape(x), ("activation", alpha))

    def binary(self, op, name, a, b):
        return self.node(op, [a, b], name, self.shape(a))

    def pixel(self, op, name, x, block):
        s = self.shape(x)
        if op == "DEPTH_TO_SPACE":
            out = [s[0], s[1] // (block * block), s[2] * block, s[3] * block]
        else:
            out = [s[0], s[1] * block * block, s[2] // block, s[3] // block]
        return self.node(op, [x], name, out, ("pixel", block))

    def concat(self, name, xs, axis=1):
        s = list(self.shape(xs[0]))
        s[axis] = sum(self.shape(x)[axis] for x in xs)
        return self.node("CONCAT", xs, name, s, ("axis", axis))

    def output(self, tid):
        self.outputs.append(tid)

    # ---- serialisation -------------------------------------------------
    def encode(self) -> bytes:
        n_nodes = len(self.nodes)
        out = f_varint(1, self.schema) + f_bytes(2, self.checkpoint)
        for t in self.tensors:
            body = f_varint(1, t["id"]) + f_bytes(2, t["name"].encode()) + f_varint(3, t["dtype"])
            body += f_packed(4, t["shape"], self.packed)
            st = t["storage"]
            if st and st[0] == "weight":
                body += f_bytes(6, f_varint(1, st[1]) + f_varint(2, st[2]), always=True)
            elif st and st[0] == "arena":
                death = st[4] if st[4] else n_nodes
                body += f_bytes(5, f_varint(1, st[1]) + f_varint(2, st[2]) + f_varint(3, st[3]) + f_varint(4, death),
                                always=True)
            out += f_bytes(3, body, always=True)
        out += f_packed(4, self.inputs, self.packed) + f_packed(5, self.outputs, self.packed)
        for n in self.nodes:
            body = f_varint(1, n["op"]) + f_packed(2, n["inputs"], self.packed) + f_packed(3, n["outputs"], self.packed)
            a = n["attr"]
            if a is not None:
                if a[0] == "conv":
                    ab = f_packed(1, a[1], self.packed) + f_packed(2, a[2], self.packed) + f_packed(3, a[3], self.packed)
                    ab += f_varint(4, a[4])
                    body += f_bytes(4, ab, always=True)
                elif a[0] == "axis":
                    body += f_bytes(5, f_varint(1, zigzag(a[1])), always=True)
                elif a[0] == "activation":
                    body += f_bytes(6, f_float(1, a[1]), always=True)
                elif a[0] == "pixel":
                    body += f_bytes(7, f_varint(1, a[1]), always=True)
            out += f_bytes(6, body, always=True)
        out += f_varint(7, max(self.arena, 256)) + f_varint(8, self.arena_alignment)
        w = bytes(self.weights) if self.weights else b"\0" * 256
        out += f_varint(9, len(w)) + f_bytes(10, self.weights_sha)
        return out

    def metadata(self) -> bytes:
        return (f_varint(1, 1) + f_bytes(2, b"test") + f_bytes(3, b"v1") + f_bytes(4, self.checkpoint) +
                f_varint(5, 16) + f_varint(6, 16) + f_float(7, 255.0))

    def write(self, directory, model: str) -> pathlib.Path:
        d = pathlib.Path(directory)
        g = d / "aot" / model
        g.mkdir(parents=True, exist_ok=True)
        w = bytes(self.weights) if self.weights else b"\0" * 256
        if self.weights_sha == b"w" * 32:
            self.weights_sha = hashlib.sha256(w).digest()
        (g / "graph.pb").write_bytes(self.encode())
        (g / "weights.bin").write_bytes(w)
        (d / "metadata.pb").write_bytes(self.metadata())
        return d


def half(a) -> np.ndarray:
    """float array -> raw binary16 bits (RNE)."""
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def to_float(h) -> np.ndarray:
    return np.asarray(h, np.uint16).view(np.float16).astype(np.float32)


def single_conv_graph(directory, model, n, ic, h, w, oc, k, stride, pad, groups=1, epilogue=None, s2d=0, d2s=0,
                      concat_ic=0, seed=0, wstd=None, zero_sum=False):
    """One conv (optionally fed by SPACE_TO_DEPTH or CONCAT, followed by
    LeakyReLU / residual ADD and DEPTH_TO_SPACE). Returns the input shapes.
    zero_sum: each output channel's weights sum to zero (before FP16
    rounding) and the bias is small, so an input with a large constant part
    gives partial sums far larger than the result."""
    rng = np.random.default_rng(seed)
    g = Graph()
    inputs = []
    if s2d:
        x0 = g.input("x", [n, ic // (s2d * s2d), h * s2d, w * s2d])
        inputs.append(g.shape(x0))
        x = g.pixel("SPACE_TO_DEPTH", "x_s2d", x0, s2d)
    elif concat_ic:
        xa = g.input("xa", [n, concat_ic, h, w])
        xb = g.input("xb", [n, ic - concat_ic, h, w])
        inputs += [g.shape(xa), g.shape(xb)]
        x = g.concat("x_cat", [xa, xb], 1)
    else:
        x = g.input("x", [n, ic, h, w])
        inputs.append(g.shape(x))
    icg = ic // groups
    std = wstd if wstd is not None else 1.0 / np.sqrt(icg * k * k)
    wv = rng.normal(0, std, (oc, icg, k, k))
    if zero_sum:
        wv -= wv.mean(axis=(1, 2, 3), keepdims=True)
    wt = g.weight_fp16("w", wv)
    bt = g.weight_fp16("b", rng.normal(0, 0.001 if zero_sum else 0.1, (oc,)))
    y = g.conv("y", x, wt, bt, (stride, stride), (pad, pad, pad, pad), groups)
    if epilogue == "lrelu":
        y = g.leaky_relu("y_act", y, 0.01)
    elif epilogue == "residual":
        r = g.input("r", g.shape(y))
        inputs.append(g.shape(r))
        y = g.binary("ADD", "y_res", y, r)
    if d2s:
        y = g.pixel("DEPTH_TO_SPACE", "y_d2s", y, d2s)
    g.output(y)
    g.write(directory, model)
    return inputs
