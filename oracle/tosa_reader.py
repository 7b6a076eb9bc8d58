"""Test-side reader for `.tosa` FlatBuffer graphs and `.npy` fixtures.

TEST INFRASTRUCTURE ONLY: this module belongs to the oracle. It is imported by
`tests/`, by `__graft_entry__.smoke()` and by `bench.py`'s CPU-baseline leg,
never by the product (`tosa_amd/`), whose own C++ reader lives in
`tosa_amd/csrc/flatbuffer.cpp`. Having two independent readers lets the tests
check one against the other.

The layout follows the TOSA schema (schema/tosa.fbs:695-768) and the
reference's parse (src/ir.rs:592-885): a TosaGraph holds regions, a region
holds basic blocks, a block holds operators, tensors, shapes and its input
and output names. Field numbers below are schema declaration order.
"""

from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

# schema/tosa.fbs:26-46
DTYPE_NAMES = [
    "UNKNOWN", "BOOL", "INT4", "INT8", "INT16", "INT32", "INT48", "FP32", "FP16",
    "BF16", "SHAPE", "FP8E4M3", "FP8E5M2", "FP6E2M3", "FP6E3M2", "FP4E2M1",
    "FP8UE8M0", "INT64", "MXINT8",
]

# schema/tosa.fbs:88-191 (the Attribute union at :193-295 has the same order)
OP_NAMES = [
    "UNKNOWN", "ARGMAX", "AVG_POOL2D", "CONV2D", "CONV3D", "DEPTHWISE_CONV2D",
    "FFT2D", "MATMUL", "MAX_POOL2D", "RFFT2D", "TRANSPOSE_CONV2D", "CLAMP", "ERF",
    "SIGMOID", "TANH", "ADD", "ARITHMETIC_RIGHT_SHIFT", "BITWISE_AND", "BITWISE_OR",
    "BITWISE_XOR", "INTDIV", "LOGICAL_AND", "LOGICAL_LEFT_SHIFT",
    "LOGICAL_RIGHT_SHIFT", "LOGICAL_OR", "LOGICAL_XOR", "MAXIMUM", "MINIMUM", "MUL",
    "POW", "SUB", "TABLE", "ABS", "BITWISE_NOT", "CEIL", "CLZ", "COS", "EXP", "FLOOR",
    "LOG", "LOGICAL_NOT", "NEGATE", "RECIPROCAL", "RSQRT", "SIN", "SELECT", "EQUAL",
    "GREATER", "GREATER_EQUAL", "REDUCE_ALL", "REDUCE_ANY", "REDUCE_MAX",
    "REDUCE_MIN", "REDUCE_PRODUCT", "REDUCE_SUM", "CONCAT", "PAD", "RESHAPE",
    "REVERSE", "SLICE", "TILE", "TRANSPOSE", "GATHER", "SCATTER", "RESIZE", "CAST",
    "RESCALE", "CONST", "IDENTITY", "CUSTOM", "COND_IF", "WHILE_LOOP", "VARIABLE",
    "VARIABLE_WRITE", "VARIABLE_READ", "CONST_SHAPE", "MATMUL_T_BLOCK_SCALED",
    "CAST_FROM_BLOCK_SCALED", "CAST_TO_BLOCK_SCALED", "DIM", "CONCAT_SHAPE",
    "ADD_SHAPE", "SUB_SHAPE", "MUL_SHAPE", "SLICE_SHAPE", "EXP2_SHAPE",
    "LOG2_CEIL_SHAPE", "LOG2_FLOOR_SHAPE", "MAX_SHAPE", "MIN_SHAPE", "MOD_SHAPE",
    "DIV_CEIL_SHAPE", "DIV_FLOOR_SHAPE", "ASSERT_EQUAL_SHAPE", "CONV2D_BLOCK_SCALED",
    "MAX_POOL2D_ADAPTIVE", "AVG_POOL2D_ADAPTIVE", "RESHAPE_BLOCK_SCALED",
    "ROW_GATHER_BLOCK_SCALED", "ROW_GATHER", "MATMUL_T", "ARGMIN",
]
OP_CODE = {n: i for i, n in enumerate(OP_NAMES)}
DTYPE_CODE = {n: i for i, n in enumerate(DTYPE_NAMES)}

# Attribute tables on the hot path: name -> list of (field, kind), in schema
# order (schema/tosa.fbs:298-520). kinds: "i32v" vector of int32, "u8v" vector
# of ubyte, "bool", "u32" enum, "i32" scalar.
_ATTR_FIELDS = {
    "AVG_POOL2D": [("kernel", "i32v"), ("stride", "i32v"), ("pad", "i32v"), ("acc_type", "u32")],
    "CONV2D": [("pad", "i32v"), ("stride", "i32v"), ("dilation", "i32v"), ("local_bound", "bool"), ("acc_type", "u32")],
    "CONV3D": [("pad", "i32v"), ("stride", "i32v"), ("dilation", "i32v"), ("local_bound", "bool"), ("acc_type", "u32")],
    "DEPTHWISE_CONV2D": [("pad", "i32v"), ("stride", "i32v"), ("dilation", "i32v"), ("local_bound", "bool"), ("acc_type", "u32")],
    "MAX_POOL2D": [("kernel", "i32v"), ("stride", "i32v"), ("pad", "i32v"), ("nan_mode", "u32")],
    "TRANSPOSE_CONV2D": [("out_pad", "i32v"), ("stride", "i32v"), ("local_bound", "bool"), ("acc_type", "u32")],
    "CLAMP": [("min_val", "u8v"), ("max_val", "u8v"), ("nan_mode", "u32")],
    "RESCALE": [("scale32", "bool"), ("rounding_mode", "u32"), ("per_channel", "bool"),
                ("input_unsigned", "bool"), ("output_unsigned", "bool")],
    "MAXIMUM": [("nan_mode", "u32")],
    "MINIMUM": [("nan_mode", "u32")],
    "TRANSPOSE": [("perms", "i32v")],
    "CONCAT": [("axis", "i32")],
}


class FlatBufferError(ValueError):
    pass


class _Buf:
    def __init__(self, data: bytes):
        self.b = bytes(data)

    def _need(self, pos: int, n: int) -> None:
        if pos < 0 or pos + n > len(self.b):
            raise FlatBufferError(f"read of {n} bytes at {pos} outside buffer of {len(self.b)}")

    def u8(self, p):
        self._need(p, 1)
        return self.b[p]

    def u16(self, p):
        self._need(p, 2)
        return struct.unpack_from("<H", self.b, p)[0]

    def u32(self, p):
        self._need(p, 4)
        return struct.unpack_from("<I", self.b, p)[0]

    def i32(self, p):
        self._need(p, 4)
        return struct.unpack_from("<i", self.b, p)[0]

    def table(self, pos):
        """Return a field accessor for the table at `pos`."""
        vt = pos - self.i32(pos)
        vt_len = self.u16(vt)

        def field_pos(idx):
            off = 4 + 2 * idx
            if off + 2 > vt_len:
                return None
            o = self.u16(vt + off)
            return None if o == 0 else pos + o

        return field_pos

    def deref(self, p):
        return p + self.u32(p)

    def string(self, p):
        s = self.deref(p)
        n = self.u32(s)
        self._need(s + 4, n)
        return self.b[s + 4:s + 4 + n].decode("utf-8")

    def vector(self, p):
        v = self.deref(p)
        return v + 4, self.u32(v)


@dataclass
class TensorDef:
    name: str
    shape: list
    dtype: str
    data: bytes | None
    is_variable: bool = False


@dataclass
class Operator:
    op: str
    attribute_type: int
    attr: dict
    inputs: list
    outputs: list


@dataclass
class Block:
    name: str
    operators: list = field(default_factory=list)
    tensors: list = field(default_factory=list)
    inputs: list = field(default_factory=list)
    outputs: list = field(default_factory=list)

    def tensor(self, name):
        for t in self.tensors:
            if t.name == name:
                return t
        return None


def _strings(buf, fp):
    if fp is None:
        return []
    start, n = buf.vector(fp)
    return [buf.string(start + 4 * i) for i in range(n)]


def _attr(buf, op_name, fpos):
    spec = _ATTR_FIELDS.get(op_name)
    if spec is None or fpos is None:
        return {}
    f = buf.table(buf.deref(fpos))
    out = {}
    for i, (name, kind) in enumerate(spec):
        p = f(i)
        if kind == "i32v":
            if p is None:
                out[name] = []
            else:
                s, n = buf.vector(p)
                out[name] = [buf.i32(s + 4 * k) for k in range(n)]
        elif kind == "u8v":
            if p is None:
                out[name] = b""
            else:
                s, n = buf.vector(p)
                buf._need(s, n)
                out[name] = buf.b[s:s + n]
        elif kind == "bool":
            out[name] = bool(buf.u8(p)) if p is not None else False
        elif kind == "u32":
            out[name] = buf.u32(p) if p is not None else 0
        elif kind == "i32":
            out[name] = buf.i32(p) if p is not None else 0
    return out


def parse_graph(data: bytes) -> list:
    """Parse a `.tosa` buffer into a list of regions, each (name, [Block])."""
    buf = _Buf(data)
    if len(data) < 8:
        raise FlatBufferError("buffer too small")
    g = buf.table(buf.u32(0))
    if g(0) is None:
        raise FlatBufferError("TosaGraph.version is required")
    regions = []
    rp = g(1)
    if rp is not None:
        rs, rn = buf.vector(rp)
        for ri in range(rn):
            r = buf.table(buf.deref(rs + 4 * ri))
            rname = buf.string(r(0)) if r(0) is not None else ""
            blocks = []
            if r(1) is not None:
                bs, bn = buf.vector(r(1))
                for bi in range(bn):
                    blocks.append(_parse_block(buf, buf.deref(bs + 4 * bi)))
            regions.append((rname, blocks))
    return regions


def _parse_block(buf, pos):
    f = buf.table(pos)
    blk = Block(name=buf.string(f(0)) if f(0) is not None else "")
    if f(2) is not None:
        ts, tn = buf.vector(f(2))
        for i in range(tn):
            t = buf.table(buf.deref(ts + 4 * i))
            name = buf.string(t(0)) if t(0) is not None else ""
            shape = []
            if t(1) is not None:
                s, n = buf.vector(t(1))
                shape = [buf.i32(s + 4 * k) for k in range(n)]
            dtype = DTYPE_NAMES[buf.u32(t(2))] if t(2) is not None else "UNKNOWN"
            data = None
            if t(3) is not None:
                s, n = buf.vector(t(3))
                buf._need(s, n)
                data = buf.b[s:s + n]
            var = bool(buf.u8(t(4))) if t(4) is not None else False
            blk.tensors.append(TensorDef(name, shape, dtype, data, var))
    if f(5) is not None:  # shapes become SHAPE tensors of shape [rank] (src/ir.rs:637-652)
        ss, sn = buf.vector(f(5))
        for i in range(sn):
            t = buf.table(buf.deref(ss + 4 * i))
            name = buf.string(t(0)) if t(0) is not None else ""
            rank = buf.u32(t(1)) if t(1) is not None else 0
            data = None
            if t(2) is not None:
                s, n = buf.vector(t(2))
                data = buf.b[s:s + n]
            blk.tensors.append(TensorDef(name, [rank], "SHAPE", data))
    if f(1) is not None:
        os_, on = buf.vector(f(1))
        for i in range(on):
            o = buf.table(buf.deref(os_ + 4 * i))
            code = buf.u32(o(0)) if o(0) is not None else 0
            name = OP_NAMES[code] if code < len(OP_NAMES) else f"UNKNOWN({code})"
            atype = buf.u8(o(1)) if o(1) is not None else 0
            # The attribute is only decoded when the union holds this op's table.
            attr = _attr(buf, name, o(2)) if atype == code else {}
            blk.operators.append(Operator(name, atype, attr, _strings(buf, o(3)), _strings(buf, o(4))))
    blk.inputs = _strings(buf, f(3))
    blk.outputs = _strings(buf, f(4))
    return blk


def main_block(data: bytes) -> Block:
    regions = parse_graph(data)
    if not regions or not regions[0][1]:
        raise FlatBufferError("no main block")
    return regions[0][1][0]


# ---------------------------------------------------------------------------
# Element decoding (src/tensor.rs:86-167; src/npy.rs:171-197)
# ---------------------------------------------------------------------------

def decode_raw(dtype: str, raw: bytes | None, count: int) -> np.ndarray:
    """CONST payload -> numpy array. INT4 packs two per byte, low nibble first;
    INT48 is 6 bytes per element; BF16 is returned as uint16 bit patterns."""
    if raw is None:
        raw = b""
        if dtype not in ("INT4", "INT48"):
            return np.zeros(count, dtype=np_dtype(dtype))
    if dtype == "INT4":
        b = np.frombuffer(raw[: (count + 1) // 2], dtype=np.uint8)
        nib = np.empty(count, dtype=np.uint8)
        nib[0::2] = b[: (count + 1) // 2] & 0xF
        nib[1::2] = (b[: count // 2] >> 4) & 0xF
        return ((nib.astype(np.int8) << 4) >> 4).astype(np.int8)
    if dtype == "INT48":
        b = np.frombuffer(raw[: 6 * count], dtype=np.uint8).reshape(count, 6)
        full = np.zeros((count, 8), dtype=np.uint8)
        full[:, :6] = b
        full[:, 6:] = np.where(b[:, 5:6] & 0x80, 0xFF, 0)
        return full.view("<i8").reshape(count)
    dt = np.dtype(np_dtype(dtype))
    if len(raw) < count * dt.itemsize:
        raise FlatBufferError(f"{dtype} tensor of {count} elements needs {count * dt.itemsize} bytes")
    return np.frombuffer(raw[: count * dt.itemsize], dtype=dt).copy()


def np_dtype(dtype: str):
    return {
        "BOOL": np.bool_, "INT4": np.int8, "INT8": np.int8, "INT16": np.int16,
        "INT32": np.int32, "INT48": np.int64, "INT64": np.int64, "SHAPE": np.int64,
        "FP32": np.float32, "FP16": np.float16, "BF16": np.uint16,
        "FP8E4M3": np.uint8, "FP8E5M2": np.uint8,
    }[dtype]


def load_npy(path: str, dtype: str) -> np.ndarray:
    """Read a fixture `.npy` as the TOSA dtype `dtype` (bf16 stays as uint16 bits)."""
    a = np.load(path, allow_pickle=False)
    a = a.reshape(a.shape).copy(order="C")  # keeps rank 0 (ascontiguousarray would not)
    if a.dtype.kind == "V":  # raw bit patterns: bf16 '<V2', fp8 '<V1'
        a = a.view(np.uint16 if a.dtype.itemsize == 2 else np.uint8)
    if dtype in ("BF16", "FP8E4M3", "FP8E5M2"):
        return a.view(np.uint16 if dtype == "BF16" else np.uint8) if a.dtype.itemsize == np.dtype(np_dtype(dtype)).itemsize else a.astype(np_dtype(dtype))
    if dtype in ("INT4", "INT8"):
        return a.astype(np.int8)
    return a.astype(np_dtype(dtype))
