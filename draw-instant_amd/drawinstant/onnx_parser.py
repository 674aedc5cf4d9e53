"""ONNX protobuf parser: the reference's onnx-parser.js (parseONNXGraph,
parseONNXWeights, parseTensor), producing the executor's Graph / Node /
TensorProto objects.

The file is read as raw protobuf wire format (varint, fixed64, length-
delimited, fixed32), with no protobuf library.  ModelProto.graph (field 7)
is walked for nodes (1), initializers (5), inputs (11) and outputs (12);
everything else is skipped by length, so weight payloads are sliced, never
scanned.  Like the reference the parser is tolerant: a desynchronised walk
records a warning and stops, and when the walk yields nothing (or too
little) it falls back to scanning for the graph tag and for initializer
records that validate (printable name, known element type, payload length =
element count x element size) (onnx-parser.js:302-356, :417-540).

Superset of the reference, stated: TensorProto int32_data (5), int64_data
(7) and double_data (10) are decoded as well as float_data (4) and raw_data
(9); ValueInfo dims keep their symbolic names as -1 like the reference.
"""
from __future__ import annotations

import mmap
from dataclasses import dataclass, field
from typing import Callable, Dict, List, Optional, Tuple

import numpy as np

from .executor import Attr, Graph, Node, TensorProto

# TensorProto.DataType (onnx-parser.js:28-39)
DTYPE = {1: "float32", 2: "uint8", 3: "int8", 4: "uint16", 5: "int16", 6: "int32", 7: "int64",
         9: "bool", 10: "float16", 11: "float64"}
# element sizes the initializer scan accepts (onnx-parser.js:310)
ELEM_SIZE = {1: 4, 6: 4, 7: 8, 9: 1, 10: 2, 11: 8}


class ProtoError(ValueError):
    """Malformed or desynchronised protobuf."""


class _Reader:
    """Cursor over buf[p:end] with the protobuf wire-format primitives."""

    __slots__ = ("b", "p", "end")

    def __init__(self, b, p: int = 0, end: Optional[int] = None):
        self.b, self.p = b, p
        self.end = len(b) if end is None else end

    def eof(self) -> bool:
        return self.p >= self.end

    def varint(self) -> int:
        result, shift, b, p, end = 0, 0, self.b, self.p, self.end
        while True:
            if p >= end:
                raise ProtoError(f"varint runs past byte {end}")
            c = b[p]
            p += 1
            result |= (c & 0x7F) << shift
            if not c & 0x80:
                break
            shift += 7
            if shift > 63:
                raise ProtoError(f"varint longer than 10 bytes at {self.p}")
        self.p = p
        return result

    def svarint(self) -> int:
        """int64 field: two's complement in 64 bits."""
        v = self.varint()
        return v - (1 << 64) if v >= (1 << 63) else v

    def tag(self) -> Tuple[int, int]:
        v = self.varint()
        return v >> 3, v & 7

    def span(self) -> Tuple[int, int]:
        n = self.varint()
        s = self.p
        if s + n > self.end:
            raise ProtoError(f"length {n} at byte {s} runs past {self.end}")
        self.p = s + n
        return s, s + n

    def fixed32(self) -> bytes:
        if self.p + 4 > self.end:
            raise ProtoError("fixed32 runs past the end")
        v = bytes(self.b[self.p:self.p + 4])
        self.p += 4
        return v

    def skip(self, wire: int) -> None:
        if wire == 0:
            self.varint()
        elif wire == 1:
            self.p += 8
        elif wire == 2:
            self.span()
        elif wire == 5:
            self.p += 4
        elif wire in (3, 4):
            pass  # deprecated group markers carry no payload
        else:
            raise ProtoError(f"unknown wire type {wire} at byte {self.p - 1}")
        if self.p > self.end:
            raise ProtoError(f"field runs past byte {self.end}")


def _text(b, s: int, e: int) -> str:
    return bytes(b[s:e]).decode("utf-8", errors="replace")


def _packed_varints(r: _Reader, wire: int, signed: bool) -> List[int]:
    if wire == 0:
        return [r.svarint() if signed else r.varint()]
    if wire == 2:
        s, e = r.span()
        sub = _Reader(r.b, s, e)
        out = []
        while not sub.eof():
            out.append(sub.svarint() if signed else sub.varint())
        return out
    r.skip(wire)
    return []


def parse_tensor(b, start: int, end: int) -> TensorProto:
    """One TensorProto from b[start:end] (parseTensor, onnx-parser.js:105-160):
    dims, data type, name and the payload as little-endian bytes."""
    r = _Reader(b, start, end)
    dims: List[int] = []
    dt, name, raw = 0, "", None
    floats: List[bytes] = []
    ints32: List[int] = []
    ints64: List[int] = []
    doubles: List[bytes] = []
    while not r.eof():
        f, w = r.tag()
        if f == 1:
            dims += _packed_varints(r, w, True)
        elif f == 2 and w == 0:
            dt = r.varint()
        elif f == 4 and w == 2:
            s, e = r.span()
            floats.append(bytes(b[s:e]))
        elif f == 4 and w == 5:
            floats.append(r.fixed32())
        elif f == 5:
            ints32 += _packed_varints(r, w, True)
        elif f == 7:
            ints64 += _packed_varints(r, w, True)
        elif f == 8 and w == 2:
            s, e = r.span()
            name = _text(b, s, e)
        elif f == 9 and w == 2:
            s, e = r.span()
            raw = bytes(b[s:e])
        elif f == 10 and w == 2:
            s, e = r.span()
            doubles.append(bytes(b[s:e]))
        elif f == 10 and w == 1:
            if r.p + 8 > r.end:
                raise ProtoError("double runs past the end")
            doubles.append(bytes(b[r.p:r.p + 8]))
            r.p += 8
        else:
            r.skip(w)
    dtype = DTYPE.get(dt, f"unknown({dt})")
    data = raw
    if data is None and floats:
        data = b"".join(floats)
    elif data is None and doubles:
        data = b"".join(doubles)
    elif data is None and ints64:
        data = np.asarray(ints64, np.int64).tobytes()
    elif data is None and ints32:
        # int32_data also carries int8/16, uint8/16, bool and float16 (as bits)
        np_dt = {"int32": np.int32, "int16": np.int16, "int8": np.int8, "uint16": np.uint16,
                 "uint8": np.uint8, "bool": np.uint8, "float16": np.uint16}.get(dtype, np.int32)
        data = np.asarray(ints32, np.int64).astype(np_dt).tobytes()
    return TensorProto(dims, dtype, data, name)


def parse_attribute(b, start: int, end: int) -> Attr:
    """AttributeProto (onnx-parser.js:162-214): name, f, i, s, t, floats,
    ints, strings."""
    r = _Reader(b, start, end)
    a = Attr("")
    while not r.eof():
        f, w = r.tag()
        if f == 1 and w == 2:
            s, e = r.span()
            a.name = _text(b, s, e)
        elif f == 2 and w == 5:
            a.f = float(np.frombuffer(r.fixed32(), "<f4")[0])
        elif f == 3 and w == 0:
            a.i = r.svarint()
        elif f == 4 and w == 2:
            s, e = r.span()
            a.s = bytes(b[s:e])
        elif f == 5 and w == 2:
            s, e = r.span()
            try:
                a.t = parse_tensor(b, s, e)
            except ProtoError:
                a.t = None
        elif f == 7 and w == 2:
            s, e = r.span()
            a.floats = [float(v) for v in np.frombuffer(bytes(b[s:e]), "<f4")]
        elif f == 7 and w == 5:
            a.floats = (a.floats or []) + [float(np.frombuffer(r.fixed32(), "<f4")[0])]
        elif f == 8:
            a.ints = (a.ints or []) + _packed_varints(r, w, True)
        elif f == 9 and w == 2:
            s, e = r.span()
            a.strings = (a.strings or []) + [_text(b, s, e)]
        else:
            r.skip(w)
    return a


def parse_node(b, start: int, end: int) -> Node:
    """NodeProto (onnx-parser.js:216-249)."""
    r = _Reader(b, start, end)
    n = Node("")
    while not r.eof():
        f, w = r.tag()
        if f in (1, 2, 3, 4, 7) and w == 2:
            s, e = r.span()
            v = _text(b, s, e)
            if f == 1:
                n.inputs.append(v)
            elif f == 2:
                n.outputs.append(v)
            elif f == 3:
                n.name = v
            elif f == 4:
                n.op_type = v
            else:
                n.domain = v
        elif f == 5 and w == 2:
            s, e = r.span()
            n.attributes.append(parse_attribute(b, s, e))
        else:
            r.skip(w)
    return n


def parse_value_info(b, start: int, end: int) -> dict:
    """ValueInfoProto (onnx-parser.js:251-300): name, element type and dims
    (dim_value, or -1 for a symbolic dim)."""
    r = _Reader(b, start, end)
    vi = {"name": "", "dtype": 0, "dims": []}
    while not r.eof():
        f, w = r.tag()
        if f == 1 and w == 2:
            s, e = r.span()
            vi["name"] = _text(b, s, e)
        elif f == 2 and w == 2:
            ts, te = r.span()
            tr = _Reader(b, ts, te)
            while not tr.eof():
                f2, w2 = tr.tag()
                if f2 != 1 or w2 != 2:
                    tr.skip(w2)
                    continue
                tts, tte = tr.span()  # TypeProto.tensor_type
                ttr = _Reader(b, tts, tte)
                while not ttr.eof():
                    f3, w3 = ttr.tag()
                    if f3 == 1 and w3 == 0:
                        vi["dtype"] = ttr.varint()
                    elif f3 == 2 and w3 == 2:
                        shs, she = ttr.span()
                        shr = _Reader(b, shs, she)
                        while not shr.eof():
                            f4, w4 = shr.tag()
                            if f4 != 1 or w4 != 2:
                                shr.skip(w4)
                                continue
                            ds, de = shr.span()
                            dr, dim = _Reader(b, ds, de), -1
                            while not dr.eof():
                                f5, w5 = dr.tag()
                                if f5 == 1 and w5 == 0:
                                    dim = dr.svarint()
                                else:
                                    dr.skip(w5)
                            vi["dims"].append(dim)
                    else:
                        ttr.skip(w3)
        else:
            r.skip(w)
    return vi


@dataclass
class OnnxGraph(Graph):
    """parseONNXGraph's result: the executor Graph (nodes, inputs, outputs,
    initializers as ``tensors``) plus the op histogram, the initializer byte
    total and the parse warnings."""
    op_hist: Dict[str, int] = field(default_factory=dict)
    bytes: int = 0
    warnings: List[str] = field(default_factory=list)


def _walk_graph(b, start: int, end: int, sink: dict, warn: Callable[[str], None]) -> None:
    """GraphProto walk (parseGraph, onnx-parser.js:358-392): stops at the
    first desync and keeps what it has."""
    r = _Reader(b, start, end)
    while not r.eof():
        try:
            f, w = r.tag()
            if w == 2 and f in (1, 5, 11, 12):
                s, e = r.span()
                try:
                    if f == 5:
                        t = parse_tensor(b, s, e)
                        sink["tensors"][t.name] = t
                    elif f == 1:
                        sink["nodes"].append(parse_node(b, s, e))
                    else:
                        sink["inputs" if f == 11 else "outputs"].append(parse_value_info(b, s, e))
                except (ProtoError, IndexError) as ex:
                    warn(f"field {f} record at byte {s} skipped: {ex}")
            else:
                r.skip(w)
        except (ProtoError, IndexError) as ex:
            warn(f"graph walk halted at byte {r.p}: {ex}")
            return


def _printable(s: str) -> bool:
    return 0 < len(s) <= 512 and all(0x20 <= ord(c) <= 0x7E for c in s)


def _scan_initializers(b, start: int, end: int, tensors: dict, warn) -> int:
    """Byte-scan for initializer records (tag 0x2a) that validate
    (scanInitializers, onnx-parser.js:320-356); returns how many were added."""
    p, added, tried = start, 0, 0
    while p < end:
        p = b.find(b"\x2a", p, end)
        if p < 0:
            break
        r = _Reader(b, p + 1, end)
        try:
            n = r.varint()
        except ProtoError:
            p += 1
            continue
        if n < 8 or n > (512 << 20) or r.p + n > end:
            p += 1
            continue
        tried += 1
        try:
            t = parse_tensor(b, r.p, r.p + n)
            code = next((k for k, v in DTYPE.items() if v == t.dtype), None)
            elem = ELEM_SIZE.get(code)
            if elem and _printable(t.name) and t.data is not None and \
                    len(t.data) == int(np.prod(t.dims or [1])) * elem:
                if t.name not in tensors:
                    tensors[t.name] = t
                    added += 1
                p = r.p + n
                continue
        except (ProtoError, IndexError, ValueError):
            pass
        p += 1
    if tried:
        warn(f"scan-init: attempted {tried}, accepted {added}")
    return added


def parse_onnx_graph(data, on_progress: Optional[Callable[[str], None]] = None) -> OnnxGraph:
    """Full parse of a ModelProto (parseONNXGraph, onnx-parser.js:417-540):
    nodes, initializers, graph inputs and outputs, op histogram.  ``data``:
    bytes, bytearray or a memory map (anything else is copied to bytes)."""
    b = data if isinstance(data, (bytes, bytearray, mmap.mmap)) else bytes(data)
    progress = on_progress or (lambda _m: None)
    warnings: List[str] = []

    def warn(m):
        warnings.append(m)
        progress(f"warn: {m}")

    sink = {"tensors": {}, "nodes": [], "inputs": [], "outputs": []}
    g_start, g_end = 0, len(b)
    r = _Reader(b, 0, len(b))
    while not r.eof():
        at = r.p
        try:
            f, w = r.tag()
            if f == 7 and w == 2:
                g_start, g_end = r.span()
                _walk_graph(b, g_start, g_end, sink, warn)
            else:
                r.skip(w)
        except (ProtoError, IndexError) as ex:
            warn(f"model walk halted at byte {r.p}: {ex}; resuming at the next graph tag")
            nxt = b.find(b"\x3a", at + 1)
            if nxt < 0:
                break
            r.p = nxt
    if not sink["tensors"] and not sink["nodes"]:
        # graph-tag scan: keep the candidate with the most records, stop at a
        # strong one (> 50 tensors or nodes)
        best, p = 0, 0
        while True:
            p = b.find(b"\x3a", p)
            if p < 0:
                break
            rr = _Reader(b, p + 1, len(b))
            try:
                n = rr.varint()
            except ProtoError:
                p += 1
                continue
            if 0 < n and rr.p + n <= len(b):
                trial = {"tensors": {}, "nodes": [], "inputs": [], "outputs": []}
                _walk_graph(b, rr.p, rr.p + n, trial, lambda _m: None)
                score = len(trial["tensors"]) + len(trial["nodes"])
                if score > best:
                    sink, best = trial, score
                    g_start, g_end = rr.p, rr.p + n
                    progress(f"candidate @ byte {p}: {len(trial['tensors'])} tensors · "
                             f"{len(trial['nodes'])} nodes")
                    if len(trial["tensors"]) > 50 or len(trial["nodes"]) > 50:
                        break
            p += 1
    if len(sink["tensors"]) > 500 and len(sink["nodes"]) > 500:
        progress("scan-init: skipped (walk healthy)")
    else:
        _scan_initializers(b, g_start, g_end, sink["tensors"], warnings.append)
    nbytes = sum(len(t.data) for t in sink["tensors"].values() if t.data is not None)
    hist: Dict[str, int] = {}
    for n in sink["nodes"]:
        hist[n.op_type] = hist.get(n.op_type, 0) + 1
    progress(f"done · {len(sink['tensors'])} tensors · {len(sink['nodes'])} nodes")
    return OnnxGraph(sink["nodes"], sink["inputs"], sink["outputs"], sink["tensors"],
                     op_hist=hist, bytes=nbytes, warnings=warnings)


def parse_onnx_weights(data, on_progress=None) -> dict:
    """parseONNXWeights (onnx-parser.js:401-415): the initializers only."""
    g = parse_onnx_graph(data, on_progress)
    return {"tensors": g.tensors, "count": len(g.tensors), "bytes": g.bytes}


def load_onnx(path: str, on_progress=None) -> OnnxGraph:
    """Parse an .onnx file through a read-only memory map (the role of
    fetchAndParseONNXGraph, onnx-parser.js:543-569, for a local file)."""
    with open(path, "rb") as fh:
        size = fh.seek(0, 2)
        if size == 0:
            return parse_onnx_graph(b"", on_progress)
        with mmap.mmap(fh.fileno(), 0, access=mmap.ACCESS_READ) as mm:
            return parse_onnx_graph(mm, on_progress)
