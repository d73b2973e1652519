"""GGUF v3 image writer and reader.

The on-disk format the mivi-v4 loader reads (crates/mivi-model/src/gguf.rs:106-197,
loader.rs:44-415): little-endian header (magic 0x46554747, version, tensor
count, metadata count), typed metadata key/values, tensor infos
(name, n_dims, dims[] innermost first, ggml type, data offset), padding to
`general.alignment` (default 32) and the tensor data, each tensor padded to
the alignment. A weight matrix of `rows x cols` is stored with dims
`[cols, rows]` (training/export/convert_to_gguf.py:145).

Used to assemble synthetic models for tests and benchmarks and to locate
tensors inside an image.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

GGUF_MAGIC = 0x46554747
ALIGN = 32

T_UINT8, T_INT8, T_UINT16, T_INT16, T_UINT32, T_INT32, T_FLOAT32, T_BOOL, T_STRING, T_ARRAY, \
    T_UINT64, T_INT64, T_FLOAT64 = range(13)

GGML_F32, GGML_F16, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K, GGML_BF16 = 0, 1, 8, 12, 14, 30
BLOCK = {0: 1, 1: 1, 30: 1, 8: 32, 12: 256, 14: 256}
TYPE_SIZE = {0: 4, 1: 2, 30: 2, 8: 34, 12: 144, 14: 210}


def row_bytes(ggml_type: int, cols: int) -> int:
    return cols // BLOCK[ggml_type] * TYPE_SIZE[ggml_type]


def _str(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


@dataclass
class GgufWriter:
    metadata: list = field(default_factory=list)   # (key, type, payload bytes)
    tensors: list = field(default_factory=list)    # (name, dims, type, data ndarray)

    def add_u32(self, key, v):
        self.metadata.append((key, T_UINT32, struct.pack("<I", v)))

    def add_f32(self, key, v):
        self.metadata.append((key, T_FLOAT32, struct.pack("<f", v)))

    def add_string(self, key, v):
        self.metadata.append((key, T_STRING, _str(v)))

    def add_string_array(self, key, arr):
        body = struct.pack("<IQ", T_STRING, len(arr)) + b"".join(_str(s) for s in arr)
        self.metadata.append((key, T_ARRAY, body))

    def add_u32_array(self, key, arr):
        body = struct.pack("<IQ", T_UINT32, len(arr)) + b"".join(struct.pack("<I", v) for v in arr)
        self.metadata.append((key, T_ARRAY, body))

    def add_tensor(self, name: str, dims, ggml_type: int, data: np.ndarray):
        data = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        n = int(np.prod(dims))
        bs, ts = BLOCK[ggml_type], TYPE_SIZE[ggml_type]
        expect = (n + bs - 1) // bs * ts
        if data.nbytes != expect:
            raise ValueError(f"tensor {name}: {data.nbytes} bytes, expected {expect}")
        self.tensors.append((name, list(dims), ggml_type, data))

    def add_matrix(self, name: str, rows: int, cols: int, ggml_type: int, data: np.ndarray):
        self.add_tensor(name, [cols, rows], ggml_type, data)

    def add_f32_vector(self, name: str, v: np.ndarray):
        v = np.ascontiguousarray(v, np.float32)
        self.add_tensor(name, [v.size], GGML_F32, v)

    def tobytes(self) -> np.ndarray:
        head = bytearray(struct.pack("<IIQQ", GGUF_MAGIC, 3, len(self.tensors), len(self.metadata)))
        for k, t, payload in self.metadata:
            head += _str(k) + struct.pack("<I", t) + payload
        off = 0
        offsets = []
        for name, dims, t, data in self.tensors:
            head += _str(name) + struct.pack("<I", len(dims))
            head += b"".join(struct.pack("<Q", d) for d in dims)
            head += struct.pack("<IQ", t, off)
            offsets.append(off)
            off += (data.nbytes + ALIGN - 1) // ALIGN * ALIGN
        data_start = (len(head) + ALIGN - 1) // ALIGN * ALIGN
        img = np.zeros(data_start + off, np.uint8)
        img[: len(head)] = np.frombuffer(bytes(head), np.uint8)
        for (name, dims, t, data), o in zip(self.tensors, offsets):
            img[data_start + o: data_start + o + data.nbytes] = data
        return img


def read_tensor_index(img: np.ndarray) -> dict:
    """Returns {name: (ggml_type, dims, absolute byte offset, byte length)}."""
    b = memoryview(np.ascontiguousarray(img, np.uint8))
    pos = 0

    def rd(fmt):
        nonlocal pos
        v = struct.unpack_from(fmt, b, pos)
        pos += struct.calcsize(fmt)
        return v[0]

    def rstr():
        nonlocal pos
        n = rd("<Q")
        s = bytes(b[pos: pos + n]).decode()
        pos += n
        return s

    sizes = {T_UINT8: 1, T_INT8: 1, T_UINT16: 2, T_INT16: 2, T_UINT32: 4, T_INT32: 4,
             T_FLOAT32: 4, T_BOOL: 1, T_UINT64: 8, T_INT64: 8, T_FLOAT64: 8}

    def skip(t):
        nonlocal pos
        if t in sizes:
            v = bytes(b[pos: pos + sizes[t]])
            pos += sizes[t]
            return v
        if t == T_STRING:
            return rstr()
        if t == T_ARRAY:
            et = rd("<I")
            n = rd("<Q")
            return [skip(et) for _ in range(n)]
        raise ValueError(f"bad metadata type {t}")

    assert rd("<I") == GGUF_MAGIC
    rd("<I")
    nt, nm = rd("<Q"), rd("<Q")
    align = ALIGN
    for _ in range(nm):
        k = rstr()
        t = rd("<I")
        v = skip(t)
        if k == "general.alignment" and t == T_UINT32:
            align = struct.unpack("<I", v)[0]
    infos = []
    for _ in range(nt):
        name = rstr()
        nd = rd("<I")
        dims = [rd("<Q") for _ in range(nd)]
        t = rd("<I")
        off = rd("<Q")
        infos.append((name, t, dims, off))
    data_start = (pos + align - 1) // align * align
    out = {}
    for name, t, dims, off in infos:
        n = int(np.prod(dims))
        nbytes = (n + BLOCK[t] - 1) // BLOCK[t] * TYPE_SIZE[t]
        out[name] = (t, dims, data_start + off, nbytes)
    return out
