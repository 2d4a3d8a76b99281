"""ONNX model files without the ``onnx`` package: a reader and writer of the
protobuf wire format for the messages a model file holds.

The reference loads models with ``onnx.load`` (``nn/ONNXImport.py:60``); the
``onnx`` package is not part of this build, so the messages of ``onnx.proto``
(public ONNX IR spec) are decoded here directly.  Only the fields an inference
graph uses are kept; unknown fields are skipped, so files written by other
tools load as long as they stay within that subset (no external data, no
sparse initializers, no subgraph attributes).

Field numbers (onnx.proto):
  ModelProto          1 ir_version, 2 producer_name, 3 producer_version, 4 domain,
                      5 model_version, 6 doc_string, 7 graph, 8 opset_import
  OperatorSetIdProto  1 domain, 2 version
  GraphProto          1 node, 2 name, 5 initializer, 10 doc_string, 11 input,
                      12 output, 13 value_info
  NodeProto           1 input, 2 output, 3 name, 4 op_type, 5 attribute,
                      6 doc_string, 7 domain
  AttributeProto      1 name, 2 f, 3 i, 4 s, 5 t, 7 floats, 8 ints, 9 strings,
                      10 tensors, 20 type
  TensorProto         1 dims, 2 data_type, 4 float_data, 5 int32_data,
                      7 int64_data, 8 name, 9 raw_data, 10 double_data,
                      11 uint64_data
  ValueInfoProto      1 name, 2 type -> TypeProto 1 tensor_type -> 1 elem_type,
                      2 shape -> 1 dim -> 1 dim_value / 2 dim_param
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple, Union

import numpy as np

# TensorProto.DataType
FLOAT, UINT8, INT8, UINT16, INT16, INT32, INT64, STRING, BOOL, FLOAT16, DOUBLE = 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11
UINT32, UINT64, BFLOAT16, FLOAT8E4M3FN, FLOAT8E5M2, INT4 = 12, 13, 16, 17, 19, 22

# element type -> (numpy storage type, typed field used when raw_data is absent)
_STORAGE = {
    FLOAT: (np.float32, 4), UINT8: (np.uint8, 5), INT8: (np.int8, 5), UINT16: (np.uint16, 5),
    INT16: (np.int16, 5), INT32: (np.int32, 5), INT64: (np.int64, 7), BOOL: (np.uint8, 5),
    FLOAT16: (np.uint16, 5), DOUBLE: (np.float64, 10), UINT32: (np.uint32, 11), UINT64: (np.uint64, 11),
    BFLOAT16: (np.uint16, 5), FLOAT8E4M3FN: (np.uint8, 5), FLOAT8E5M2: (np.uint8, 5), INT4: (np.int8, 5),
}

# AttributeProto.AttributeType
A_FLOAT, A_INT, A_STRING, A_TENSOR, A_FLOATS, A_INTS, A_STRINGS, A_TENSORS = 1, 2, 3, 4, 6, 7, 8, 9


# ------------------------------------------------------------------ wire format ---
def _read_varint(buf: bytes, pos: int) -> Tuple[int, int]:
    result, shift = 0, 0
    while True:
        if pos >= len(buf):
            raise ValueError("truncated varint")
        b = buf[pos]
        pos += 1
        result |= (b & 0x7F) << shift
        if b < 0x80:
            return result, pos
        shift += 7
        if shift > 70:
            raise ValueError("varint too long")


def _signed64(v: int) -> int:
    return v - (1 << 64) if v >= (1 << 63) else v


def _fields(buf: bytes) -> List[Tuple[int, int, Union[int, bytes]]]:
    """All (field number, wire type, value) of one message, in order."""
    out = []
    pos, n = 0, len(buf)
    while pos < n:
        key, pos = _read_varint(buf, pos)
        fno, wt = key >> 3, key & 7
        if wt == 0:
            v, pos = _read_varint(buf, pos)
        elif wt == 1:
            v = buf[pos:pos + 8]
            pos += 8
        elif wt == 2:
            ln, pos = _read_varint(buf, pos)
            v = buf[pos:pos + ln]
            if len(v) != ln:
                raise ValueError("truncated field")
            pos += ln
        elif wt == 5:
            v = buf[pos:pos + 4]
            pos += 4
        else:
            raise ValueError(f"unsupported wire type {wt}")
        out.append((fno, wt, v))
    return out


def _ints(vals: list, wt: int, v) -> None:
    """Append a repeated integer field given packed (wt 2) or one-by-one (wt 0)."""
    if wt == 0:
        vals.append(_signed64(v))
        return
    pos = 0
    while pos < len(v):
        x, pos = _read_varint(v, pos)
        vals.append(_signed64(x))


def _enc_varint(v: int) -> bytes:
    if v < 0:
        v += 1 << 64
    out = bytearray()
    while True:
        b = v & 0x7F
        v >>= 7
        if v:
            out.append(b | 0x80)
        else:
            out.append(b)
            return bytes(out)


def _key(fno: int, wt: int) -> bytes:
    return _enc_varint((fno << 3) | wt)


def _w_varint(fno: int, v: int) -> bytes:
    return _key(fno, 0) + _enc_varint(int(v))


def _w_bytes(fno: int, b: bytes) -> bytes:
    return _key(fno, 2) + _enc_varint(len(b)) + b


def _w_str(fno: int, s: str) -> bytes:
    return _w_bytes(fno, s.encode("utf-8"))


def _w_packed_varints(fno: int, vals) -> bytes:
    return _w_bytes(fno, b"".join(_enc_varint(int(x)) for x in vals))


# ------------------------------------------------------------------- messages ---
@dataclass
class TensorProto:
    name: str = ""
    data_type: int = FLOAT
    dims: List[int] = field(default_factory=list)
    raw_data: Optional[bytes] = None
    typed: list = field(default_factory=list)      # float_data / int32_data / int64_data / double / uint64

    def numpy(self) -> np.ndarray:
        """Element array in storage form (float16 / bfloat16 as uint16 bits, fp8 as uint8 codes)."""
        if self.data_type not in _STORAGE:
            raise ValueError(f"tensor {self.name!r}: data type {self.data_type} not supported")
        st, _ = _STORAGE[self.data_type]
        shape = tuple(int(d) for d in self.dims)
        if self.raw_data is not None:
            return np.frombuffer(self.raw_data, dtype=st).reshape(shape).copy()
        if self.data_type in (FLOAT16, BFLOAT16):
            return np.asarray(self.typed, dtype=np.int64).astype(np.uint16).reshape(shape)
        return np.asarray(self.typed).astype(st).reshape(shape)

    @staticmethod
    def from_numpy(arr: np.ndarray, name: str, data_type: int) -> "TensorProto":
        st, _ = _STORAGE[data_type]
        a = np.ascontiguousarray(np.asarray(arr).astype(st, copy=False))
        return TensorProto(name=name, data_type=data_type, dims=list(a.shape), raw_data=a.tobytes())

    @staticmethod
    def parse(buf: bytes) -> "TensorProto":
        t = TensorProto()
        floats: list = []
        for fno, wt, v in _fields(buf):
            if fno == 1:
                _ints(t.dims, wt, v)
            elif fno == 2:
                t.data_type = int(v)
            elif fno == 8:
                t.name = v.decode("utf-8")
            elif fno == 9:
                t.raw_data = bytes(v)
            elif fno == 4:           # float_data: packed fixed32 or one fixed32
                floats.extend(struct.unpack(f"<{len(v) // 4}f", v))
            elif fno in (5, 7, 11):  # int32_data / int64_data / uint64_data (varints)
                _ints(t.typed, wt, v)
            elif fno == 10:          # double_data: packed fixed64
                floats.extend(struct.unpack(f"<{len(v) // 8}d", v))
        if floats:
            t.typed = floats
        return t

    def serialize(self) -> bytes:
        out = b"".join(_w_varint(1, d) for d in self.dims)
        out += _w_varint(2, self.data_type)
        if self.name:
            out += _w_str(8, self.name)
        if self.raw_data is not None:
            out += _w_bytes(9, self.raw_data)
        elif self.typed:
            fno = _STORAGE[self.data_type][1]
            if fno == 4:
                out += _w_bytes(4, struct.pack(f"<{len(self.typed)}f", *self.typed))
            elif fno == 10:
                out += _w_bytes(10, struct.pack(f"<{len(self.typed)}d", *self.typed))
            else:
                out += _w_packed_varints(fno, self.typed)
        return out


@dataclass
class AttributeProto:
    name: str
    type: int
    value: object

    @staticmethod
    def parse(buf: bytes) -> "AttributeProto":
        name, typ = "", 0
        f = i = s = t = None
        floats: list = []
        ints: list = []
        strings: list = []
        tensors: list = []
        for fno, wt, v in _fields(buf):
            if fno == 1:
                name = v.decode("utf-8")
            elif fno == 20:
                typ = int(v)
            elif fno == 2:
                f = struct.unpack("<f", v)[0]
            elif fno == 3:
                i = _signed64(v)
            elif fno == 4:
                s = bytes(v)
            elif fno == 5:
                t = TensorProto.parse(v)
            elif fno == 7:
                floats.extend(struct.unpack(f"<{len(v) // 4}f", v))
            elif fno == 8:
                _ints(ints, wt, v)
            elif fno == 9:
                strings.append(bytes(v))
            elif fno == 10:
                tensors.append(TensorProto.parse(v))
        if not typ:   # files that omit the type field: infer it from what is present
            typ = (A_FLOAT if f is not None else A_INT if i is not None else A_STRING if s is not None else
                   A_TENSOR if t is not None else A_FLOATS if floats else A_INTS if ints else
                   A_STRINGS if strings else A_TENSORS if tensors else 0)
        value = {A_FLOAT: f, A_INT: i, A_STRING: s, A_TENSOR: t, A_FLOATS: floats, A_INTS: ints,
                 A_STRINGS: strings, A_TENSORS: tensors}.get(typ)
        return AttributeProto(name, typ, value)

    def serialize(self) -> bytes:
        out = _w_str(1, self.name) + _w_varint(20, self.type)
        v = self.value
        if self.type == A_FLOAT:
            out += _key(2, 5) + struct.pack("<f", float(v))
        elif self.type == A_INT:
            out += _w_varint(3, int(v))
        elif self.type == A_STRING:
            out += _w_bytes(4, v if isinstance(v, bytes) else str(v).encode("utf-8"))
        elif self.type == A_TENSOR:
            out += _w_bytes(5, v.serialize())
        elif self.type == A_FLOATS:
            out += b"".join(_key(7, 5) + struct.pack("<f", float(x)) for x in v)
        elif self.type == A_INTS:
            out += b"".join(_w_varint(8, int(x)) for x in v)
        elif self.type == A_STRINGS:
            out += b"".join(_w_bytes(9, x if isinstance(x, bytes) else str(x).encode("utf-8")) for x in v)
        elif self.type == A_TENSORS:
            out += b"".join(_w_bytes(10, x.serialize()) for x in v)
        return out


def make_attribute(name: str, value) -> AttributeProto:
    """Attribute from a Python value (int, float, str, list of int / float, TensorProto)."""
    if isinstance(value, TensorProto):
        return AttributeProto(name, A_TENSOR, value)
    if isinstance(value, bool) or isinstance(value, (int, np.integer)):
        return AttributeProto(name, A_INT, int(value))
    if isinstance(value, (float, np.floating)):
        return AttributeProto(name, A_FLOAT, float(value))
    if isinstance(value, (str, bytes)):
        return AttributeProto(name, A_STRING, value if isinstance(value, bytes) else value.encode("utf-8"))
    value = list(value)
    if all(isinstance(x, (int, np.integer)) for x in value):
        return AttributeProto(name, A_INTS, [int(x) for x in value])
    return AttributeProto(name, A_FLOATS, [float(x) for x in value])


@dataclass
class NodeProto:
    op_type: str
    inputs: List[str]
    outputs: List[str]
    name: str = ""
    domain: str = ""
    attributes: List[AttributeProto] = field(default_factory=list)

    def attr(self, name: str, default=None):
        for a in self.attributes:
            if a.name == name:
                return a.value
        return default

    @staticmethod
    def parse(buf: bytes) -> "NodeProto":
        n = NodeProto("", [], [])
        for fno, wt, v in _fields(buf):
            if fno == 1:
                n.inputs.append(v.decode("utf-8"))
            elif fno == 2:
                n.outputs.append(v.decode("utf-8"))
            elif fno == 3:
                n.name = v.decode("utf-8")
            elif fno == 4:
                n.op_type = v.decode("utf-8")
            elif fno == 5:
                n.attributes.append(AttributeProto.parse(v))
            elif fno == 7:
                n.domain = v.decode("utf-8")
        return n

    def serialize(self) -> bytes:
        out = b"".join(_w_str(1, s) for s in self.inputs) + b"".join(_w_str(2, s) for s in self.outputs)
        if self.name:
            out += _w_str(3, self.name)
        out += _w_str(4, self.op_type)
        out += b"".join(_w_bytes(5, a.serialize()) for a in self.attributes)
        if self.domain:
            out += _w_str(7, self.domain)
        return out


@dataclass
class ValueInfoProto:
    name: str
    elem_type: int = 0
    shape: Optional[List[Union[int, str]]] = None      # dim_value, or dim_param for symbolic dims

    @staticmethod
    def parse(buf: bytes) -> "ValueInfoProto":
        vi = ValueInfoProto("")
        for fno, wt, v in _fields(buf):
            if fno == 1:
                vi.name = v.decode("utf-8")
            elif fno == 2:
                for tf, _, tv in _fields(v):
                    if tf != 1:
                        continue
                    for ef, _, ev in _fields(tv):
                        if ef == 1:
                            vi.elem_type = int(ev)
                        elif ef == 2:
                            vi.shape = []
                            for df, _, dv in _fields(ev):
                                if df != 1:
                                    continue
                                dim: Union[int, str] = "?"
                                for xf, _, xv in _fields(dv):
                                    if xf == 1:
                                        dim = _signed64(xv)
                                    elif xf == 2:
                                        dim = xv.decode("utf-8")
                                vi.shape.append(dim)
        return vi

    def serialize(self) -> bytes:
        tensor = _w_varint(1, self.elem_type)
        if self.shape is not None:
            dims = b"".join(_w_bytes(1, _w_varint(1, d) if isinstance(d, int) else _w_str(2, str(d)))
                            for d in self.shape)
            tensor += _w_bytes(2, dims)
        return _w_str(1, self.name) + _w_bytes(2, _w_bytes(1, tensor))


@dataclass
class GraphProto:
    name: str = ""
    nodes: List[NodeProto] = field(default_factory=list)
    initializers: List[TensorProto] = field(default_factory=list)
    inputs: List[ValueInfoProto] = field(default_factory=list)
    outputs: List[ValueInfoProto] = field(default_factory=list)
    value_info: List[ValueInfoProto] = field(default_factory=list)

    @staticmethod
    def parse(buf: bytes) -> "GraphProto":
        g = GraphProto()
        for fno, wt, v in _fields(buf):
            if fno == 1:
                g.nodes.append(NodeProto.parse(v))
            elif fno == 2:
                g.name = v.decode("utf-8")
            elif fno == 5:
                g.initializers.append(TensorProto.parse(v))
            elif fno == 11:
                g.inputs.append(ValueInfoProto.parse(v))
            elif fno == 12:
                g.outputs.append(ValueInfoProto.parse(v))
            elif fno == 13:
                g.value_info.append(ValueInfoProto.parse(v))
        return g

    def serialize(self) -> bytes:
        out = b"".join(_w_bytes(1, n.serialize()) for n in self.nodes)
        out += _w_str(2, self.name)
        out += b"".join(_w_bytes(5, t.serialize()) for t in self.initializers)
        out += b"".join(_w_bytes(11, v.serialize()) for v in self.inputs)
        out += b"".join(_w_bytes(12, v.serialize()) for v in self.outputs)
        out += b"".join(_w_bytes(13, v.serialize()) for v in self.value_info)
        return out


@dataclass
class ModelProto:
    graph: GraphProto
    ir_version: int = 8
    opset_import: List[Tuple[str, int]] = field(default_factory=lambda: [("", 17)])
    producer_name: str = ""
    producer_version: str = ""
    domain: str = ""
    model_version: int = 0
    doc_string: str = ""

    @staticmethod
    def parse(buf: bytes) -> "ModelProto":
        m = ModelProto(GraphProto(), opset_import=[])
        for fno, wt, v in _fields(buf):
            if fno == 1:
                m.ir_version = int(v)
            elif fno == 2:
                m.producer_name = v.decode("utf-8")
            elif fno == 3:
                m.producer_version = v.decode("utf-8")
            elif fno == 4:
                m.domain = v.decode("utf-8")
            elif fno == 5:
                m.model_version = _signed64(v)
            elif fno == 6:
                m.doc_string = v.decode("utf-8")
            elif fno == 7:
                m.graph = GraphProto.parse(v)
            elif fno == 8:
                dom, ver = "", 0
                for of, _, ov in _fields(v):
                    if of == 1:
                        dom = ov.decode("utf-8")
                    elif of == 2:
                        ver = _signed64(ov)
                m.opset_import.append((dom, ver))
        return m

    def serialize(self) -> bytes:
        out = _w_varint(1, self.ir_version)
        if self.producer_name:
            out += _w_str(2, self.producer_name)
        if self.producer_version:
            out += _w_str(3, self.producer_version)
        if self.domain:
            out += _w_str(4, self.domain)
        if self.model_version:
            out += _w_varint(5, self.model_version)
        if self.doc_string:
            out += _w_str(6, self.doc_string)
        out += _w_bytes(7, self.graph.serialize())
        for dom, ver in self.opset_import:
            out += _w_bytes(8, (_w_str(1, dom) if dom else b"") + _w_varint(2, ver))
        return out


def load(path_or_bytes: Union[str, bytes]) -> ModelProto:
    """ModelProto from a file path or the file's bytes (``onnx.load`` without external data)."""
    if isinstance(path_or_bytes, (bytes, bytearray)):
        return ModelProto.parse(bytes(path_or_bytes))
    with open(path_or_bytes, "rb") as f:
        return ModelProto.parse(f.read())


def save(model: ModelProto, path: str) -> None:
    with open(path, "wb") as f:
        f.write(model.serialize())
