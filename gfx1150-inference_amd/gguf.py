"""GGUF v2/v3 container parsing and writing (the file format the packed weights arrive in).

Host-side mirror of the reference's `src/gguf_parser.py` (GGUFParser :115-328,
write_synthetic_gguf :590-648, GGMLType / GGML_BLOCK_INFO / GGUFValueType :22-80,
GGUFTensorInfo :88-101): same public names, fields and layer helpers, and the same validation
(each failure is a ValueError naming the same condition).  The byte layout is the GGUF
specification's: little-endian header `GGUF`, u32 version, u64 tensor count, u64 metadata
count; metadata entries (string key, u32 type, value); tensor entries (string name, u32
n_dims, u64 dims[n_dims] with dims[0] innermost, u32 type, u64 offset relative to the data
section); the data section starts at the next multiple of `general.alignment` (default 32).

Parsing only reads the header and tables; tensor bytes stay in the file (or buffer) and are
moved to HBM by `resident.ResidentModel` through the library's parallel loader.
"""

from __future__ import annotations

import enum
import math
import struct
from dataclasses import dataclass
from typing import Any, BinaryIO, Dict, List, Optional, Tuple

GGUF_MAGIC = b"GGUF"
GGUF_DEFAULT_ALIGNMENT = 32


class GGMLType(enum.IntEnum):
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q8_1 = 9
    Q2_K = 10
    Q3_K = 11
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    Q8_K = 15


# GGML type -> (elements per block, bytes per block); the GGUF block geometry.
GGML_BLOCK_INFO: Dict[int, Tuple[int, int]] = {
    GGMLType.F32: (1, 4), GGMLType.F16: (1, 2),
    GGMLType.Q4_0: (32, 18), GGMLType.Q4_1: (32, 20), GGMLType.Q5_0: (32, 22), GGMLType.Q5_1: (32, 24),
    GGMLType.Q8_0: (32, 34), GGMLType.Q8_1: (32, 36),
    GGMLType.Q2_K: (256, 84), GGMLType.Q3_K: (256, 110), GGMLType.Q4_K: (256, 144), GGMLType.Q5_K: (256, 176),
    GGMLType.Q6_K: (256, 210), GGMLType.Q8_K: (256, 292),
}


class GGUFValueType(enum.IntEnum):
    UINT8 = 0
    INT8 = 1
    UINT16 = 2
    INT16 = 3
    UINT32 = 4
    INT32 = 5
    FLOAT32 = 6
    BOOL = 7
    STRING = 8
    ARRAY = 9
    UINT64 = 10
    INT64 = 11
    FLOAT64 = 12


# fixed-size metadata value encodings (struct codes, little-endian)
_FIXED = {
    GGUFValueType.UINT8: "B", GGUFValueType.INT8: "b", GGUFValueType.UINT16: "H", GGUFValueType.INT16: "h",
    GGUFValueType.UINT32: "I", GGUFValueType.INT32: "i", GGUFValueType.FLOAT32: "f", GGUFValueType.UINT64: "Q",
    GGUFValueType.INT64: "q", GGUFValueType.FLOAT64: "d",
}


@dataclass(frozen=True)
class GGUFTensorInfo:
    name: str
    dims: Tuple[int, ...]  # GGUF order: dims[0] is the contiguous (innermost) one
    ggml_type: GGMLType
    rel_offset: int        # from the start of the data section
    abs_offset: int        # from the start of the file
    n_elements: int
    n_bytes: int

    @property
    def shape_row_major(self) -> Tuple[int, ...]:
        """NumPy / torch shape: the GGUF dims reversed."""
        return tuple(self.dims[::-1])


def align_offset(offset: int, alignment: int = GGUF_DEFAULT_ALIGNMENT) -> int:
    return -(-offset // alignment) * alignment


class _Cursor:
    """Bounds-checked little-endian reads from a byte view."""

    def __init__(self, view: memoryview):
        self.view = view
        self.pos = 0

    def remaining(self) -> int:
        return len(self.view) - self.pos

    def take(self, fmt: str) -> Tuple[Any, ...]:
        n = struct.calcsize("<" + fmt)
        if n > self.remaining():
            raise ValueError(f"Unexpected EOF at offset {self.pos} while reading {n} bytes")
        out = struct.unpack_from("<" + fmt, self.view, self.pos)
        self.pos += n
        return out

    def string(self) -> str:
        (n,) = self.take("Q")
        if n > self.remaining():
            raise ValueError(f"Unexpected EOF while reading string of length {n} at offset {self.pos}")
        s = bytes(self.view[self.pos:self.pos + n]).decode("utf-8")
        self.pos += n
        return s

    def value(self, vtype: int) -> Any:
        if vtype in _FIXED:
            return self.take(_FIXED[vtype])[0]
        if vtype == GGUFValueType.BOOL:
            return self.take("B")[0] != 0
        if vtype == GGUFValueType.STRING:
            return self.string()
        if vtype == GGUFValueType.ARRAY:
            elem, count = self.take("IQ")
            # every element takes at least one byte, so a larger count cannot be genuine
            if count > self.remaining():
                raise ValueError(f"GGUF array count {count} exceeds remaining buffer bytes ({self.remaining()})")
            return [self.value(elem) for _ in range(count)]
        raise ValueError(f"Unsupported GGUF metadata value type: {vtype}")


class GGUFParser:
    """Parses the header, metadata and tensor table of a GGUF v2/v3 buffer (bytes, bytearray,
    memoryview or mmap).  The caller's buffer is not retained or released."""

    MAX_TENSOR_DIMS = 8
    MAX_ALIGNMENT = 65536
    MIN_KV_ENTRY_BYTES = 13      # u64 key length + u32 type + 1 value byte
    MIN_TENSOR_ENTRY_BYTES = 24  # u64 name length + u32 n_dims + u32 type + u64 offset

    def __init__(self, buf: Any):
        self.version = 0
        self.tensor_count = 0
        self.kv_count = 0
        self.metadata: Dict[str, Any] = {}
        self.tensors: Dict[str, GGUFTensorInfo] = {}
        self.alignment = GGUF_DEFAULT_ALIGNMENT
        self.data_offset = 0
        view = memoryview(buf).cast("B")
        try:
            self._parse(_Cursor(view))
        finally:
            view.release()

    def _parse(self, cur: _Cursor) -> None:
        size = len(cur.view)
        if size < 4:
            raise ValueError(f"Buffer too small for GGUF header ({size} bytes)")
        magic = bytes(cur.view[:4])
        if magic != GGUF_MAGIC:
            raise ValueError(f"Invalid GGUF magic: {magic!r} (expected b'GGUF')")
        cur.pos = 4
        self.version, self.tensor_count, self.kv_count = cur.take("IQQ")
        if self.version not in (2, 3):
            raise ValueError(f"Unsupported GGUF version: {self.version} (expected 2 or 3)")
        left = cur.remaining()
        if self.kv_count * self.MIN_KV_ENTRY_BYTES > left:
            raise ValueError(f"Corrupt GGUF header: kv_count={self.kv_count} cannot fit in the {left} bytes that remain")
        if self.tensor_count * self.MIN_TENSOR_ENTRY_BYTES > left:
            raise ValueError(
                f"Corrupt GGUF header: tensor_count={self.tensor_count} cannot fit in the {left} bytes that remain")

        for _ in range(self.kv_count):
            key = cur.string()
            (vtype,) = cur.take("I")
            self.metadata[key] = cur.value(vtype)

        align = self.metadata.get("general.alignment", GGUF_DEFAULT_ALIGNMENT)
        if isinstance(align, bool) or not isinstance(align, int):
            raise ValueError(f"Invalid general.alignment value: {align!r}")
        if not (1 <= align <= self.MAX_ALIGNMENT) or align & (align - 1):
            raise ValueError(f"Invalid general.alignment={align}: must be a power of 2 in [1, {self.MAX_ALIGNMENT}]")
        self.alignment = align

        if self.tensor_count * self.MIN_TENSOR_ENTRY_BYTES > cur.remaining():
            raise ValueError(f"Corrupt GGUF tensor table: tensor_count={self.tensor_count} cannot fit in the "
                             f"{cur.remaining()} bytes that remain")
        table = []
        names = set()
        for _ in range(self.tensor_count):
            name = cur.string()
            if name in names:
                raise ValueError(f"Duplicate tensor name in GGUF tensor table: {name!r}")
            names.add(name)
            (n_dims,) = cur.take("I")
            if not 1 <= n_dims <= self.MAX_TENSOR_DIMS:
                raise ValueError(f"Tensor '{name}' has invalid n_dims={n_dims} (must be in [1, {self.MAX_TENSOR_DIMS}])")
            dims = tuple(cur.take(f"{n_dims}Q"))
            if 0 in dims:
                raise ValueError(f"Tensor '{name}' has a zero dimension in {dims}")
            type_id, rel = cur.take("IQ")
            try:
                gtype = GGMLType(type_id)
            except ValueError:
                raise ValueError(f"Tensor '{name}' has unknown GGMLType id {type_id}") from None
            if gtype not in GGML_BLOCK_INFO:
                raise ValueError(f"Tensor '{name}' has unsupported GGMLType {gtype!r} (no block size info)")
            count = math.prod(dims)
            qk, bb = GGML_BLOCK_INFO[gtype]
            if count % qk:
                raise ValueError(f"Tensor '{name}' element count {count} is not divisible by block size {qk}")
            table.append((name, dims, gtype, rel, count, count // qk * bb))

        self.data_offset = align_offset(cur.pos, self.alignment)
        size = len(cur.view)
        if table and self.data_offset > size:
            raise ValueError(f"Truncated GGUF file: data_offset {self.data_offset} exceeds buffer size {size}")
        for name, dims, gtype, rel, count, nbytes in table:
            start = self.data_offset + rel
            if start + nbytes > size:
                raise ValueError(f"Truncated GGUF file: tensor '{name}' needs bytes [{start}, {start + nbytes}) of a "
                                 f"{size}-byte file")
            self.tensors[name] = GGUFTensorInfo(name, dims, gtype, rel, start, count, nbytes)

    # ---- layer helpers
    def get_layer_tensors(self, layer_idx: int) -> Dict[str, GGUFTensorInfo]:
        """Tensors of transformer block `layer_idx` (names starting with `blk.{layer_idx}.`)."""
        prefix = f"blk.{layer_idx}."
        return {n: t for n, t in self.tensors.items() if n.startswith(prefix)}

    def get_layer_byte_spans(self, layer_idx: int) -> List[Tuple[int, int]]:
        """(start, length) file spans covering the layer's tensors: neighbours are merged when the
        gap between them is at most one alignment unit and no other tensor lies in it."""
        mine = self.get_layer_tensors(layer_idx)
        if not mine:
            raise KeyError(f"No tensors found for layer {layer_idx}")
        others = sorted((t.abs_offset, t.abs_offset + t.n_bytes) for n, t in self.tensors.items() if n not in mine)
        spans: List[List[int]] = []
        for t in sorted(mine.values(), key=lambda t: t.abs_offset):
            lo, hi = t.abs_offset, t.abs_offset + t.n_bytes
            if spans:
                end = spans[-1][1]
                blocked = lo > end and any(a < lo and b > end for a, b in others)
                if lo - end <= self.alignment and not blocked:
                    spans[-1][1] = max(end, hi)
                    continue
            spans.append([lo, hi])
        return [(a, b - a) for a, b in spans]

    def get_layer_byte_span(self, layer_idx: int) -> Tuple[int, int]:
        """(start, length) of the hull of the layer's tensors."""
        mine = self.get_layer_tensors(layer_idx)
        if not mine:
            raise KeyError(f"No tensors found for layer {layer_idx}")
        lo = min(t.abs_offset for t in mine.values())
        hi = max(t.abs_offset + t.n_bytes for t in mine.values())
        return lo, hi - lo


def _encode_value(vtype: int, val: Any) -> bytes:
    if vtype in _FIXED:
        return struct.pack("<" + _FIXED[vtype], val)
    if vtype == GGUFValueType.BOOL:
        return b"\x01" if val else b"\x00"
    if vtype == GGUFValueType.STRING:
        raw = val.encode("utf-8")
        return struct.pack("<Q", len(raw)) + raw
    if vtype == GGUFValueType.ARRAY:
        elem, items = val
        return struct.pack("<IQ", int(elem), len(items)) + b"".join(_encode_value(elem, v) for v in items)
    raise ValueError(f"Unsupported synthetic metadata type: {vtype}")


def write_synthetic_gguf(file_obj: BinaryIO, metadata: Dict[str, Tuple[GGUFValueType, Any]],
                         tensors: List[Tuple[str, Tuple[int, ...], GGMLType, bytes]],
                         alignment: int = GGUF_DEFAULT_ALIGNMENT) -> None:
    """Writes a GGUF v3 stream: `metadata` maps key -> (value type, value) (arrays as
    (element type, items)); `tensors` are (name, GGUF dims, type, packed bytes), placed at
    `alignment`-aligned offsets of the data section in the order given."""
    head = bytearray(GGUF_MAGIC + struct.pack("<IQQ", 3, len(tensors), len(metadata)))
    for key, (vtype, val) in metadata.items():
        head += _encode_value(GGUFValueType.STRING, key) + struct.pack("<I", int(vtype)) + _encode_value(vtype, val)
    placed = []
    at = 0
    for name, dims, gtype, payload in tensors:
        at = align_offset(at, alignment)
        head += _encode_value(GGUFValueType.STRING, name)
        head += struct.pack(f"<I{len(dims)}QIQ", len(dims), *dims, int(gtype), at)
        placed.append((at, payload))
        at += len(payload)
    data_start = align_offset(len(head), alignment)
    out = bytearray(head) + bytes(data_start - len(head))
    for rel, payload in placed:
        out += bytes(data_start + rel - len(out))
        out += payload
    file_obj.write(out)
    file_obj.flush()
