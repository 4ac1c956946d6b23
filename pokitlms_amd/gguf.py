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

# (block elements, block bytes) of the tensor types this build reads or writes
TYPE_LAYOUT = {0: (1, 4), 1: (1, 2), 30: (1, 2), 2: (32, 18), 3: (32, 20), 8: (32, 34), 12: (256, 144),
               13: (256, 176), 14: (256, 210)}


def payload_bytes(gtype: int, dims: Iterable[int]) -> int:
    dims = list(dims)
    be, bb = TYPE_LAYOUT[gtype]
    if dims[0] % be:
        raise ValueError(f"first dimension {dims[0]} is not a multiple of {be}")
    n = 1
    for d in dims[1:]:
        n *= d
    return dims[0] // be * bb * n


@dataclass
class TensorInfo:
    name: str
    dims: list[int]
    gtype: int
    offset: int = 0  # relative to the data section

    @property
    def nbytes(self) -> int:
        return payload_bytes(self.gtype, self.dims)


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
    """Read-only view of a GGUF v3 file: metadata dict and tensor payload views."""

    def __init__(self, path: str):
        self._f = open(path, "rb")
        self._mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        self.metadata: dict = {}
        self.tensors: dict[str, TensorInfo] = {}
        self._parse()

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

        def take(fmt):
            nonlocal pos
            vals = struct.unpack_from(fmt, mm, pos)
            pos += struct.calcsize(fmt)
            return vals if len(vals) > 1 else vals[0]

        def string():
            nonlocal pos
            n = take("<Q")
            s = bytes(mm[pos:pos + n]).decode("utf-8")
            pos += n
            return s

        scalar = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32T: "<f",
                  BOOL: "<B", U64: "<Q", I64: "<q", F64T: "<d"}

        def value(t):
            if t == STRING:
                return string()
            if t == ARRAY:
                et, n = take("<I"), take("<Q")
                return [value(et) for _ in range(n)]
            v = take(scalar[t])
            return bool(v) if t == BOOL else v

        if bytes(mm[0:4]) != GGUF_MAGIC:
            raise ValueError("not a GGUF file")
        pos = 4
        version, n_tensors, n_kv = take("<IQQ")
        if version != GGUF_VERSION:
            raise ValueError(f"GGUF version {version} is not supported")
        for _ in range(n_kv):
            k = string()
            self.metadata[k] = value(take("<I"))
        infos = []
        for _ in range(n_tensors):
            name = string()
            nd = take("<I")
            dims = list(struct.unpack_from(f"<{nd}Q", mm, pos))
            pos += 8 * nd
            gtype, off = take("<IQ")
            infos.append(TensorInfo(name, dims, gtype, off))
        align = int(self.metadata.get("general.alignment", DEFAULT_ALIGNMENT))
        self.data_offset = pos + (-pos) % align
        for t in infos:
            self.tensors[t.name] = t

    def payload(self, name: str) -> np.ndarray:
        t = self.tensors[name]
        start = self.data_offset + t.offset
        if start + t.nbytes > len(self._mm):
            raise ValueError(f"{name}: payload runs past the end of the file")
        return np.frombuffer(self._mm, dtype=np.uint8, count=t.nbytes, offset=start)
