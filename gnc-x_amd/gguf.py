"""GGUF files as the reference's loader reads them (lua/gncx_gguf.lua).

Layout (little-endian), parsed by GNCXGGUF:_parse (lua/gncx_gguf.lua:223-306):
  "GGUF", u32 version, u64 tensor_count, u64 kv_count;
  kv_count x (string key, u32 value type, value);
  tensor_count x (string name, u32 n_dims, u64 dims[n_dims], u32 ggml type,
                  u64 offset relative to the data section);
  zero padding to `general.alignment` (32 when absent), then the data
  section; every tensor offset is a multiple of the alignment.
A string is u64 byte length + bytes; an array is u32 element type + u64
count + elements.  Value type codes are the table at lua/gncx_gguf.lua:14-30.
Dims are ggml order: dims[0] is the row length (in_dim), dims[1] the row count.
A tensor's byte size is elements / block_elems * block_bytes for its type
(lua/gncx_gguf.lua:46-63, 275-281).

write_gguf streams tensor data through callbacks, so multi-GB model files are
written without holding them in memory; read_gguf returns the metadata and
the absolute file offset of every tensor (`abs_file_offset` in the reference).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass
from typing import Callable, Iterable

UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_SCALAR = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f",
           BOOL: "<?", UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}

# ggml type -> (elements per block, bytes per block), lua/gncx_gguf.lua:46-63
F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 2, 8, 12, 14, 30
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24),
         Q8_0: (32, 34), 9: (32, 36), 10: (256, 84), 11: (256, 110), Q4_K: (256, 144), 13: (256, 176),
         Q6_K: (256, 210), 15: (256, 292)}
DEFAULT_ALIGNMENT = 32


def tensor_bytes(ggml_type: int, dims: Iterable[int]) -> int:
    n = 1
    for d in dims:
        n *= int(d)
    be, bb = BLOCK[ggml_type]
    return n // be * bb


def _string(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype == STRING:
        return _string(v)
    if vtype == ARRAY:
        etype, items = v
        out = [struct.pack("<IQ", etype, len(items))]
        if etype in _SCALAR:
            out.append(struct.pack("<" + _SCALAR[etype][1] * len(items), *items))
        else:
            out.extend(_value(etype, it) for it in items)
        return b"".join(out)
    return struct.pack(_SCALAR[vtype], v)


@dataclass
class TensorSpec:
    name: str
    ggml_type: int
    dims: tuple           # ggml order
    write: Callable       # write(fileobj) writes exactly tensor_bytes(ggml_type, dims) bytes


def write_gguf(path, metadata: list[tuple[str, int, object]], tensors: list[TensorSpec], version: int = 3) -> dict:
    """metadata: (key, value type, value); ARRAY values are (element type,
    list).  Returns {name: absolute file offset}."""
    align = DEFAULT_ALIGNMENT
    for k, t, v in metadata:
        if k == "general.alignment":
            align = int(v)
    head = [b"GGUF", struct.pack("<IQQ", version, len(tensors), len(metadata))]
    for k, t, v in metadata:
        head.append(_string(k) + struct.pack("<I", t) + _value(t, v))
    rel, offsets = 0, []
    for ts in tensors:
        offsets.append(rel)
        rel += (tensor_bytes(ts.ggml_type, ts.dims) + align - 1) // align * align
    for ts, off in zip(tensors, offsets):
        head.append(_string(ts.name) + struct.pack("<I", len(ts.dims)) +
                    struct.pack("<" + "Q" * len(ts.dims), *ts.dims) + struct.pack("<IQ", ts.ggml_type, off))
    header = b"".join(head)
    data0 = (len(header) + align - 1) // align * align
    abs_off = {}
    with open(path, "wb") as f:
        f.write(header)
        f.write(b"\0" * (data0 - len(header)))
        for ts, off in zip(tensors, offsets):
            assert f.tell() == data0 + off
            start = f.tell()
            ts.write(f)
            n = tensor_bytes(ts.ggml_type, ts.dims)
            if f.tell() - start != n:
                raise ValueError(f"{ts.name}: wrote {f.tell() - start} bytes, expected {n}")
            f.write(b"\0" * ((n + align - 1) // align * align - n))
            abs_off[ts.name] = data0 + off
    return abs_off


@dataclass
class TensorInfo:
    name: str
    dims: tuple
    ggml_type: int
    rel_offset: int
    abs_file_offset: int
    byte_size: int


class _Reader:
    def __init__(self, buf):
        self.b, self.p = buf, 0

    def take(self, fmt):
        v = struct.unpack_from(fmt, self.b, self.p)
        self.p += struct.calcsize(fmt)
        return v[0] if len(v) == 1 else v

    def string(self) -> str:
        n = self.take("<Q")
        s = bytes(self.b[self.p:self.p + n]).decode("utf-8")
        self.p += n
        return s

    def value(self, vtype):
        if vtype == STRING:
            return self.string()
        if vtype == ARRAY:
            etype, count = self.take("<I"), self.take("<Q")
            if etype in _SCALAR:
                items = struct.unpack_from("<" + _SCALAR[etype][1] * count, self.b, self.p)
                self.p += struct.calcsize(_SCALAR[etype][1]) * count
                return list(items)
            return [self.value(etype) for _ in range(count)]
        if vtype in _SCALAR:
            return self.take(_SCALAR[vtype])
        raise ValueError(f"unknown GGUF value type {vtype}")


def read_gguf(buf) -> tuple[dict, dict, int]:
    """(metadata, {name: TensorInfo}, data section offset) from the bytes of a
    GGUF file (a bytes object, mmap or numpy memmap)."""
    r = _Reader(memoryview(buf))
    if bytes(r.b[0:4]) != b"GGUF":
        raise ValueError("not a GGUF file (magic)")
    r.p = 4
    version = r.take("<I")
    n_tensors, n_kv = r.take("<Q"), r.take("<Q")
    meta = {"__version__": version}
    for _ in range(n_kv):
        k = r.string()
        meta[k] = r.value(r.take("<I"))
    raw = []
    for _ in range(n_tensors):
        name = r.string()
        nd = r.take("<I")
        dims = tuple(r.take("<Q") for _ in range(nd))
        raw.append((name, dims, r.take("<I"), r.take("<Q")))
    align = meta.get("general.alignment", DEFAULT_ALIGNMENT)
    if not isinstance(align, int):
        align = DEFAULT_ALIGNMENT
    data0 = (r.p + align - 1) // align * align
    tensors = {}
    for name, dims, t, off in raw:
        size = tensor_bytes(t, dims) if t in BLOCK else 0
        tensors[name] = TensorInfo(name, dims, t, off, data0 + off, size)
    return meta, tensors, data0
