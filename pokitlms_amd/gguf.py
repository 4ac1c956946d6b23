"""Minimal GGUF v3 reader and writer (the container format the reference loads:
src/gguf_reader.cpp:21-255 of the reference).

The reader memory-maps the file and returns each tensor's raw payload as a
NumPy view (row-major ``[out, in]`` rows of encoded blocks, GGUF dims
``[in, out(, n)]``), which is exactly what the HIP upload entry points take.
The writer streams tensors produced on demand, so multi-GB files never sit in
memory whole.
"""
from __future__ import annotations

import mmap
import struct
from dataclasses import dataclass, field
from typing import Callable, Iterable

import numpy as np

GGUF_MAGIC = b"GGUF"
GGUF_VERSION = 3
DEFAULT_ALIGNMENT = 32

# metadata value types
U8, I8, U16, I16, U32, I32, F32T, BOOL, STRING, ARRAY, U64, I64, F64T = range(13)

# (block elements, block bytes) of every tensor type the reference's reader
# knows (type_layout, src/gguf_reader.cpp:21-57).  A type outside this table
# is accepted when the file is parsed, with an unknown payload size, as there.
TYPE_LAYOUT = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24),
               8: (32, 34), 9: (32, 36), 10: (256, 84), 11: (256, 110), 12: (256, 144),
               13: (256, 176), 14: (256, 210), 15: (256, 292), 16: (256, 66), 17: (256, 74),
               18: (256, 98), 19: (256, 50), 20: (32, 18), 21: (256, 110), 22: (256, 82),
               23: (256, 136), 24: (1, 1), 25: (1, 2), 26: (1, 4), 27: (1, 8), 28: (1, 8),
               29: (256, 56), 30: (1, 2), 34: (256, 54), 35: (256, 66), 39: (32, 17)}

_U64_MAX = (1 << 64) - 1
# directory limits of the reference reader (src/gguf_reader.cpp:13-17)
MAX_METADATA_ENTRIES = 1_000_000
MAX_TENSORS = 10_000_000
MAX_STRING_BYTES = 16 * 1024 * 1024
MAX_ARRAY_ENTRIES = 100_000_000
MAX_ARRAY_DEPTH = 8


def payload_bytes(gtype: int, dims: Iterable[int]) -> int:
    """Bytes of a tensor's payload (tensor_payload_size, src/gguf_reader.cpp:59-80):
    ValueError for a row that is not a whole number of blocks, for sizes past
    64 bits, and for a type without a known layout."""
    dims = list(dims)
    if gtype not in TYPE_LAYOUT:
        raise ValueError(f"tensor type {gtype} has no known block layout")
    be, bb = TYPE_LAYOUT[gtype]
    if dims[0] % be:
        raise ValueError(f"first dimension {dims[0]} is not a multiple of {be}")
    n = 1
    for d in dims[1:]:
        n *= d
    total = dims[0] // be * bb * n
    if n > _U64_MAX or total > _U64_MAX:
        raise ValueError("tensor payload size overflows 64 bits")
    return total


@dataclass
class TensorInfo:
    name: str
    dims: list[int]
    gtype: int
    offset: int = 0  # relative to the data section

    @property
    def nbytes(self) -> int:
        return payload_bytes(self.gtype, self.dims)

    @property
    def known_layout(self) -> bool:
        return self.gtype in TYPE_LAYOUT


# ---- writer --------------------------------------------------------------------------

def _str(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(v) -> tuple[int, bytes]:
    if isinstance(v, bool):
        return BOOL, struct.pack("<B", 1 if v else 0)
    if isinstance(v, str):
        return STRING, _str(v)
    if isinstance(v, float):
        return F32T, struct.pack("<f", v)
    if isinstance(v, int):
        return (U32, struct.pack("<I", v)) if 0 <= v < 2**32 else (U64, struct.pack("<Q", v))
    if isinstance(v, tuple) and len(v) == 2 and v[0] == "array":
        items = v[1]
        if isinstance(items, np.ndarray):
            if items.dtype == np.int32:
                return ARRAY, struct.pack("<IQ", I32, items.size) + items.astype("<i4").tobytes()
            if items.dtype == np.uint32:
                return ARRAY, struct.pack("<IQ", U32, items.size) + items.astype("<u4").tobytes()
            raise TypeError(f"unsupported array dtype {items.dtype}")
        items = list(items)
        if not items or isinstance(items[0], str):
            return ARRAY, struct.pack("<IQ", STRING, len(items)) + b"".join(_str(s) for s in items)
        raise TypeError("unsupported array item type")
    raise TypeError(f"unsupported metadata value {type(v)}")


@dataclass
class GgufWriter:
    """Collects metadata and tensor descriptions, then streams the file.

    ``tensors`` holds (info, producer) pairs; a producer returns the tensor's
    payload as a uint8 array (called once, in file order)."""
    metadata: dict = field(default_factory=dict)
    tensors: list = field(default_factory=list)
    alignment: int = DEFAULT_ALIGNMENT

    def add_tensor(self, name: str, dims: list[int], gtype: int, producer: Callable[[], np.ndarray]):
        self.tensors.append((TensorInfo(name, list(dims), gtype), producer))

    def write(self, path: str) -> None:
        offset = 0
        for info, _ in self.tensors:
            info.offset = offset
            offset += info.nbytes
            offset += (-offset) % self.alignment
        head = bytearray()
        head += GGUF_MAGIC + struct.pack("<IQQ", GGUF_VERSION, len(self.tensors), len(self.metadata))
        for k, v in self.metadata.items():
            t, payload = _value(v)
            head += _str(k) + struct.pack("<I", t) + payload
        for info, _ in self.tensors:
            head += _str(info.name) + struct.pack("<I", len(info.dims))
            head += struct.pack(f"<{len(info.dims)}Q", *info.dims)
            head += struct.pack("<IQ", info.gtype, info.offset)
        head += b"\0" * ((-len(head)) % self.alignment)
        with open(path, "wb") as f:
            f.write(head)
            pos = 0
            for info, producer in self.tensors:
                assert pos == info.offset
                data = np.ascontiguousarray(producer(), dtype=np.uint8).reshape(-1)
                if data.size != info.nbytes:
                    raise ValueError(f"{info.name}: {data.size} bytes, expected {info.nbytes}")
                f.write(memoryview(data))
                pos += data.size
                pad = (-pos) % self.alignment
                f.write(b"\0" * pad)
                pos += pad


# ---- reader --------------------------------------------------------------------------

class GgufFile:
    """Read-only view of a GGUF v3 file: metadata dict and tensor payload views.

    Parsing applies the reference reader's checks (GgufReader,
    src/gguf_reader.cpp:173-255) and raises ValueError where it throws:
    magic and version, directory limits, truncated strings, arrays and
    booleans, unknown metadata value types, duplicate metadata keys and tensor
    names, tensor rank and zero dimensions, rows that are not whole blocks,
    ``general.alignment`` (an unsigned integer, at least 8 and a multiple of
    8), the data section's padding, and every tensor's payload offset
    (aligned, inside the file), extent (inside the file) and overlap with
    another payload.  A tensor type outside TYPE_LAYOUT is accepted, with an
    unknown size, as the reference does; ``payload`` refuses it."""

    def __init__(self, path: str):
        self._f = open(path, "rb")
        try:
            self._mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        except ValueError:  # an empty file cannot be mapped
            self._f.close()
            raise ValueError("truncated GGUF file") from None
        self.metadata: dict = {}
        self.metadata_types: dict[str, int] = {}
        self.tensors: dict[str, TensorInfo] = {}
        try:
            self._parse()
        except struct.error:
            self.close()
            raise ValueError("truncated GGUF file") from None
        except ValueError:
            self.close()
            raise

    def close(self) -> None:
        # payload views handed out keep the mapping alive; it is released with
        # the last of them
        try:
            self._mm.close()
        except BufferError:
            pass
        self._f.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _parse(self) -> None:
        mm, pos = self._mm, 0
        size = len(mm)

        def take(fmt):
            nonlocal pos
            vals = struct.unpack_from(fmt, mm, pos)  # struct.error past the end
            pos += struct.calcsize(fmt)
            return vals if len(vals) > 1 else vals[0]

        def string():
            nonlocal pos
            n = take("<Q")
            if n > MAX_STRING_BYTES or n > size - pos:
                raise ValueError("invalid or oversized GGUF string")
            s = bytes(mm[pos:pos + n]).decode("utf-8")
            pos += n
            return s

        scalar = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32T: "<f",
                  U64: "<Q", I64: "<q", F64T: "<d"}

        def value(t, depth=0):
            if t == STRING:
                return string()
            if t == BOOL:
                v = take("<B")
                if v > 1:
                    raise ValueError("invalid GGUF boolean")
                return bool(v)
            if t == ARRAY:
                if depth >= MAX_ARRAY_DEPTH:
                    raise ValueError("GGUF array nesting too deep")
                et, n = take("<I"), take("<Q")
                if n > MAX_ARRAY_ENTRIES or n > size - pos:
                    raise ValueError("invalid or oversized GGUF array")
                return [value(et, depth + 1) for _ in range(n)]
            if t not in scalar:
                raise ValueError(f"unsupported GGUF metadata value type {t}")
            return take(scalar[t])

        if bytes(mm[0:4]) != GGUF_MAGIC:
            raise ValueError("invalid GGUF magic")
        pos = 4
        version = take("<I")
        if version != GGUF_VERSION:
            raise ValueError("only GGUF version 3 is supported")
        n_tensors, n_kv = take("<QQ")
        left = size - pos
        if (n_tensors > MAX_TENSORS or n_tensors > left // 32 or n_kv > MAX_METADATA_ENTRIES
                or n_kv > left // 13):
            raise ValueError("GGUF directory exceeds implementation limits")
        for _ in range(n_kv):
            k = string()
            t = take("<I")
            v = value(t)
            if k in self.metadata:
                raise ValueError("duplicate GGUF metadata key")
            self.metadata[k] = v
            self.metadata_types[k] = t
        infos = []
        for _ in range(n_tensors):
            name = string()
            nd = take("<I")
            if nd == 0 or nd > 16:
                raise ValueError("invalid GGUF tensor rank")
            dims = list(take(f"<{nd}Q")) if nd > 1 else [take("<Q")]
            if any(d == 0 for d in dims):
                raise ValueError("zero-sized GGUF tensor dimension")
            gtype, off = take("<IQ")
            info = TensorInfo(name, dims, gtype, off)
            if info.known_layout:
                try:
                    info.nbytes
                except ValueError as e:
                    raise ValueError(f"{e}: {name}") from None
            if name in self.tensors:
                raise ValueError("duplicate GGUF tensor name")
            self.tensors[name] = info
            infos.append(info)
        align = DEFAULT_ALIGNMENT
        if "general.alignment" in self.metadata:
            a = self.metadata["general.alignment"]
            if (self.metadata_types["general.alignment"] not in (U8, U16, U32, U64) or a < 8
                    or a % 8):
                raise ValueError("invalid GGUF general.alignment")
            align = a
        pad = (-pos) % align
        if pad > size - pos:
            raise ValueError("truncated GGUF alignment padding")
        self.alignment = align
        self.data_offset = pos + pad
        span = size - self.data_offset
        for t in infos:
            if t.offset % align or t.offset > span:
                raise ValueError("invalid GGUF tensor data offset")
            if t.known_layout and t.nbytes > span - t.offset:
                raise ValueError(f"GGUF tensor payload extends beyond file: {t.name}")
        ordered = sorted(infos, key=lambda t: t.offset)
        for prev, cur in zip(ordered, ordered[1:]):
            if prev.offset == cur.offset or (prev.known_layout
                                             and prev.offset + prev.nbytes > cur.offset):
                raise ValueError("overlapping GGUF tensor payloads")

    def payload(self, name: str) -> np.ndarray:
        t = self.tensors[name]
        if not t.known_layout:
            raise ValueError(f"{name}: tensor type {t.gtype} has no known block layout")
        start = self.data_offset + t.offset
        return np.frombuffer(self._mm, dtype=np.uint8, count=t.nbytes, offset=start)
