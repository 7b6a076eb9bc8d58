"""Build `.tosa` FlatBuffer graphs in memory.

The reference builds graphs either by reading a `.tosa` file or directly as a
`Graph` value (`Interpreter::new(Graph)`, src/interpreter.rs:109). Here the
in-memory graph is serialized to the same FlatBuffer format
(schema/tosa.fbs:695-768) and handed to `Interpreter.from_flatbuffer`, so the
one C++ reader sees both kinds of input.

Layout: the root offset and the "TOSA" file identifier, then every object
after the object that refers to it (FlatBuffers offsets are unsigned and point
forward), each table preceded by its vtable.

    g = GraphBuilder()
    g.input("x", [1, 8, 8, 4], "INT8")
    g.const("w", w_array, "INT8")
    g.op("CONV2D", ["x", "w", ...], ["y"], pad=[...], stride=[...], dilation=[...], acc_type="INT32")
    g.tensor("y", [1, 8, 8, 16], "INT32")
    data = g.build(outputs=["y"])
"""

from __future__ import annotations

import struct

import numpy as np

# schema/tosa.fbs:26-46
DTYPES = ["UNKNOWN", "BOOL", "INT4", "INT8", "INT16", "INT32", "INT48", "FP32", "FP16", "BF16", "SHAPE",
          "FP8E4M3", "FP8E5M2", "FP6E2M3", "FP6E3M2", "FP4E2M1", "FP8UE8M0", "INT64", "MXINT8"]
DTYPE = {n: i for i, n in enumerate(DTYPES)}

# schema/tosa.fbs:88-191 (subset): operator code == its attribute union tag.
OPS = {"AVG_POOL2D": 2, "CONV2D": 3, "CONV3D": 4, "DEPTHWISE_CONV2D": 5, "MATMUL": 7, "MAX_POOL2D": 8,
       "TRANSPOSE_CONV2D": 10, "CLAMP": 11, "ADD": 15, "RESHAPE": 57, "TRANSPOSE": 61, "CAST": 65, "RESCALE": 66,
       "CONST": 67, "IDENTITY": 68, "CONST_SHAPE": 75, "MATMUL_T": 100}
ROUNDING = {"SINGLE_ROUND": 1, "INEXACT_ROUND": 2, "DOUBLE_ROUND": 3}
NAN_MODE = {"PROPAGATE": 1, "IGNORE": 2}


# ---------------------------------------------------------------------------
# Serializer
# ---------------------------------------------------------------------------

class _Table:
    def __init__(self, fields):
        # fields: list of (index, kind, value); kind in u8 bool u32 i32 off
        self.fields = fields


class _Vec:
    def __init__(self, kind, items, align=4):
        self.kind = kind  # "i32", "u8", "off"
        self.items = items
        self.align = align


class _Str:
    def __init__(self, s):
        self.s = s.encode()


_SIZE = {"u8": 1, "bool": 1, "u32": 4, "i32": 4, "off": 4}
_FMT = {"u8": "<B", "bool": "<B", "u32": "<I", "i32": "<i"}


class _Writer:
    def __init__(self):
        self.buf = bytearray()

    def pad(self, a, extra=0):
        self.buf += b"\0" * ((-(len(self.buf) + extra)) % a)

    def place(self, node) -> int:
        if isinstance(node, _Table):
            return self._table(node)
        if isinstance(node, _Vec):
            return self._vec(node)
        if isinstance(node, _Str):
            self.pad(4)
            pos = len(self.buf)
            self.buf += struct.pack("<I", len(node.s)) + node.s + b"\0"
            return pos
        raise TypeError(node)

    def _table(self, t) -> int:
        fields = sorted(t.fields, key=lambda f: -_SIZE[f[1]])  # big fields first: no padding needed
        nslots = (max(f[0] for f in t.fields) + 1) if t.fields else 0
        vt_size = 4 + 2 * nslots
        offsets, off = {}, 4
        for idx, kind, _ in fields:
            sz = _SIZE[kind]
            off += (-off) % sz
            offsets[idx] = off
            off += sz
        table_size = off + (-off) % 4
        self.pad(8, vt_size)
        vt_pos = len(self.buf)
        vt = [vt_size, table_size] + [offsets.get(i, 0) for i in range(nslots)]
        self.buf += struct.pack(f"<{len(vt)}H", *vt)
        pos = len(self.buf)
        body = bytearray(table_size)
        struct.pack_into("<i", body, 0, pos - vt_pos)
        children = []
        for idx, kind, val in fields:
            if kind == "off":
                children.append((pos + offsets[idx], val))
            else:
                struct.pack_into(_FMT[kind], body, offsets[idx], int(val))
        self.buf += body
        for at, child in children:
            cpos = self.place(child)
            struct.pack_into("<I", self.buf, at, cpos - at)
        return pos

    def _vec(self, v) -> int:
        if v.kind == "off":
            self.pad(4)
            pos = len(self.buf)
            self.buf += struct.pack("<I", len(v.items)) + b"\0" * (4 * len(v.items))
            for i, child in enumerate(v.items):
                at = pos + 4 + 4 * i
                cpos = self.place(child)
                struct.pack_into("<I", self.buf, at, cpos - at)
            return pos
        esz = 4 if v.kind == "i32" else 1
        self.pad(max(4, v.align, esz), 4)  # elements aligned, length just before
        pos = len(self.buf)
        data = np.asarray(v.items, dtype="<i4" if v.kind == "i32" else np.uint8).tobytes() if v.kind == "i32" \
            else bytes(v.items)
        self.buf += struct.pack("<I", len(data) // esz) + data
        return pos


def _strvec(names):
    return _Vec("off", [_Str(n) for n in names])


# ---------------------------------------------------------------------------
# Graph builder
# ---------------------------------------------------------------------------

def encode_values(values, dtype: str) -> bytes:
    """Raw serialized bytes of a CONST (src/tensor.rs:86-167 reads them):
    little-endian; INT4 two per byte low nibble first; INT48 six bytes;
    BF16/FP16 as 16-bit patterns; SHAPE as int64."""
    a = np.asarray(values)
    if dtype == "INT4":
        v = (a.reshape(-1).astype(np.int64) & 0xF).astype(np.uint8)
        if v.size % 2:
            v = np.concatenate([v, np.zeros(1, np.uint8)])
        return (v[0::2] | (v[1::2] << 4)).astype(np.uint8).tobytes()
    if dtype == "INT48":
        v = a.reshape(-1).astype("<i8").view(np.uint8).reshape(-1, 8)[:, :6]
        return v.tobytes()
    st = {"BOOL": np.uint8, "INT8": np.int8, "INT16": "<i2", "INT32": "<i4", "INT64": "<i8", "SHAPE": "<i8",
          "FP32": "<f4", "FP16": "<u2", "BF16": "<u2", "FP8E4M3": np.uint8, "FP8E5M2": np.uint8}[dtype]
    if dtype == "FP16" and a.dtype == np.float16:
        a = a.view(np.uint16)
    return np.ascontiguousarray(a.astype(st)).tobytes()


class GraphBuilder:
    def __init__(self, name: str = "main"):
        self.name = name
        self.tensors = []      # (name, shape, dtype, data | None)
        self.operators = []    # (op, inputs, outputs, attr_fields | None)
        self.inputs = []
        self._known = set()

    def tensor(self, name, shape, dtype, data: bytes | None = None):
        if name in self._known:
            return name
        self._known.add(name)
        self.tensors.append((name, list(shape), dtype, data))
        return name

    def input(self, name, shape, dtype):
        self.inputs.append(name)
        return self.tensor(name, shape, dtype)

    def const(self, name, values, dtype, shape=None):
        a = np.asarray(values)
        shape = list(a.shape) if shape is None else list(shape)
        self.tensor(name, shape, dtype, encode_values(a, dtype))
        self.operators.append(("CONST", [], [name], None))
        return name

    def const_shape(self, name, dims):
        dims = [int(d) for d in dims]
        self.tensor(name, [len(dims)], "SHAPE", encode_values(np.array(dims, np.int64), "SHAPE"))
        self.operators.append(("CONST_SHAPE", [], [name], None))
        return name

    def op(self, op, inputs, outputs, **attr):
        self.operators.append((op, list(inputs), list(outputs), attr))
        return outputs[0] if len(outputs) == 1 else outputs

    @staticmethod
    def _attribute(op, a):
        """(union tag, attribute table) with the field order of schema/tosa.fbs:298-520."""
        code = OPS[op]
        if op in ("CONV2D", "CONV3D", "DEPTHWISE_CONV2D"):
            return code, _Table([(0, "off", _Vec("i32", a["pad"])), (1, "off", _Vec("i32", a["stride"])),
                                 (2, "off", _Vec("i32", a["dilation"])), (3, "bool", a.get("local_bound", 0)),
                                 (4, "u32", DTYPE[a["acc_type"]])])
        if op == "AVG_POOL2D":
            return code, _Table([(0, "off", _Vec("i32", a["kernel"])), (1, "off", _Vec("i32", a["stride"])),
                                 (2, "off", _Vec("i32", a["pad"])), (3, "u32", DTYPE[a["acc_type"]])])
        if op == "MAX_POOL2D":
            return code, _Table([(0, "off", _Vec("i32", a["kernel"])), (1, "off", _Vec("i32", a["stride"])),
                                 (2, "off", _Vec("i32", a["pad"])),
                                 (3, "u32", NAN_MODE[a.get("nan_mode", "PROPAGATE")])])
        if op == "TRANSPOSE_CONV2D":
            return code, _Table([(0, "off", _Vec("i32", a["out_pad"])), (1, "off", _Vec("i32", a["stride"])),
                                 (2, "bool", a.get("local_bound", 0)), (3, "u32", DTYPE[a["acc_type"]])])
        if op == "CAST":
            return code, _Table([(0, "bool", a.get("input_unsigned", 0))])
        if op == "CLAMP":
            return code, _Table([(0, "off", _Vec("u8", a["min_val"], align=8)),
                                 (1, "off", _Vec("u8", a["max_val"], align=8)),
                                 (2, "u32", NAN_MODE[a.get("nan_mode", "PROPAGATE")])])
        if op == "RESCALE":
            return code, _Table([(0, "bool", a["scale32"]), (1, "u32", ROUNDING[a["rounding_mode"]]),
                                 (2, "bool", a["per_channel"]), (3, "bool", a.get("input_unsigned", 0)),
                                 (4, "bool", a.get("output_unsigned", 0))])
        if op == "TRANSPOSE":
            return code, _Table([(0, "off", _Vec("i32", a["perms"]))])
        return code, _Table([])

    def build(self, outputs, version=(1, 0, 0)) -> bytes:
        tensors = []
        for name, shape, dtype, data in self.tensors:
            f = [(0, "off", _Str(name)), (1, "off", _Vec("i32", shape)), (2, "u32", DTYPE[dtype])]
            if data is not None:
                f.append((3, "off", _Vec("u8", data, align=8)))
            tensors.append(_Table(f))
        ops = []
        for op, ins, outs, attr in self.operators:
            tag, table = self._attribute(op, attr or {})
            ops.append(_Table([(0, "u32", OPS[op]), (1, "u8", tag), (2, "off", table),
                               (3, "off", _strvec(ins)), (4, "off", _strvec(outs))]))
        block = _Table([(0, "off", _Str(self.name)), (1, "off", _Vec("off", ops)), (2, "off", _Vec("off", tensors)),
                        (3, "off", _strvec(self.inputs)), (4, "off", _strvec(outputs))])
        region = _Table([(0, "off", _Str(self.name)), (1, "off", _Vec("off", [block]))])
        ver = _Table([(0, "i32", version[0]), (1, "i32", version[1]), (2, "i32", version[2]), (3, "bool", 0)])
        graph = _Table([(0, "off", ver), (1, "off", _Vec("off", [region]))])
        w = _Writer()
        w.buf += b"\0\0\0\0TOSA"
        root = w.place(graph)
        struct.pack_into("<I", w.buf, 0, root)
        return bytes(w.buf)
