"""GGUF v3 reader and writer (this package's own; the reference depends on the third-party
`gguf` package, aneforge/_gguf.py:10-46, which is not part of this build).

GGUFView keeps the reference's accessors (meta, arch, tn, field, sc, has, get, drop_pages) and
adds `quantized(name)`, which returns Q4_0 tensors as QuantizedWeight codes instead of
dequantising them, so the Q4_0 kernels stream the file's own 4-bit codes.

Format: magic "GGUF", version 3, tensor count, metadata count, metadata key/values, tensor infos
(name, dims with dims[0] innermost, ggml type, offset), data section aligned to
general.alignment (default 32).  Dequantisers: F32, F16, BF16, Q4_0, Q8_0."""
from __future__ import annotations

import mmap as _mmap
import struct
from dataclasses import dataclass
from typing import Any

import numpy as np

GGUF_MAGIC = b"GGUF"
# ggml tensor types used here: (elements per block, bytes per block)
GGML = {"F32": 0, "F16": 1, "Q4_0": 2, "Q8_0": 8, "BF16": 30}
_BLOCK = {0: (1, 4), 1: (1, 2), 2: (32, 18), 8: (32, 34), 30: (1, 2)}
_NAMES = {v: k for k, v in GGML.items()}

# metadata value types
_U8, _I8, _U16, _I16, _U32, _I32, _F32, _BOOL, _STR, _ARR, _U64, _I64, _F64 = range(13)
_SCALAR = {_U8: "<B", _I8: "<b", _U16: "<H", _I16: "<h", _U32: "<I", _I32: "<i", _F32: "<f", _BOOL: "<?",
           _U64: "<Q", _I64: "<q", _F64: "<d"}


@dataclass
class Field:
    """A metadata entry; `parts[data[-1]][0]` is the scalar value (the gguf-py access pattern the
    reference uses, aneforge/_gguf.py:22-25)."""
    name: str
    types: list
    value: Any

    @property
    def parts(self):
        cell = np.empty(1, dtype=object)
        cell[0] = self.value
        return [cell]

    @property
    def data(self):
        return [0]


@dataclass
class TensorInfo:
    name: str
    shape: tuple          # dims in GGUF order (shape[0] innermost), as gguf-py reports them
    tensor_type: int
    offset: int           # absolute file offset of the tensor data
    nbytes: int
    data: np.ndarray      # raw view: numpy-order array for F32/F16/BF16, block bytes otherwise


def _read_str(buf, off):
    (n,) = struct.unpack_from("<Q", buf, off)
    off += 8
    return bytes(buf[off:off + n]).decode("utf-8"), off + n


def _read_value(buf, off, t):
    if t in _SCALAR:
        fmt = _SCALAR[t]
        return struct.unpack_from(fmt, buf, off)[0], off + struct.calcsize(fmt)
    if t == _STR:
        return _read_str(buf, off)
    if t == _ARR:
        (et, n) = struct.unpack_from("<IQ", buf, off)
        off += 12
        vals = []
        for _ in range(n):
            v, off = _read_value(buf, off, et)
            vals.append(v)
        return vals, off
    raise ValueError(f"GGUF: unknown metadata value type {t}")


def _nbytes(ttype, shape):
    n = int(np.prod(shape))
    per, size = _BLOCK.get(ttype, (None, None))
    if per is None:
        raise NotImplementedError(f"GGUF tensor type {ttype} is not supported by this reader")
    return n // per * size


class GGUFReader:
    """Parses a GGUF v2/v3 file over a read-only mmap."""

    def __init__(self, path: str):
        self._f = open(path, "rb")
        self._mm = _mmap.mmap(self._f.fileno(), 0, access=_mmap.ACCESS_READ)
        buf = memoryview(self._mm)
        if bytes(buf[:4]) != GGUF_MAGIC:
            raise ValueError(f"{path}: not a GGUF file")
        version, n_t, n_kv = struct.unpack_from("<IQQ", buf, 4)
        if version not in (2, 3):
            raise ValueError(f"{path}: GGUF version {version} not supported")
        off = 24
        self.fields: dict[str, Field] = {}
        for _ in range(n_kv):
            key, off = _read_str(buf, off)
            (t,) = struct.unpack_from("<I", buf, off)
            off += 4
            val, off = _read_value(buf, off, t)
            self.fields[key] = Field(key, [t], val)
        infos = []
        for _ in range(n_t):
            name, off = _read_str(buf, off)
            (nd,) = struct.unpack_from("<I", buf, off)
            off += 4
            dims = struct.unpack_from("<" + "Q" * nd, buf, off)
            off += 8 * nd
            ttype, toff = struct.unpack_from("<IQ", buf, off)
            off += 12
            infos.append((name, tuple(int(d) for d in dims), ttype, toff))
        align = int(self.fields["general.alignment"].value) if "general.alignment" in self.fields else 32
        data_start = (off + align - 1) // align * align
        self.tensors = []
        for name, dims, ttype, toff in infos:
            nb = _nbytes(ttype, dims)
            start = data_start + toff
            raw = np.frombuffer(self._mm, dtype=np.uint8, count=nb, offset=start)
            np_shape = tuple(reversed(dims))
            if ttype == 0:
                data = raw.view(np.float32).reshape(np_shape)
            elif ttype in (1, 30):
                data = raw.view(np.float16 if ttype == 1 else np.uint16).reshape(np_shape)
            else:
                per, size = _BLOCK[ttype]
                data = raw.reshape(np_shape[:-1] + (np_shape[-1] // per * size,))
            self.tensors.append(TensorInfo(name, dims, ttype, start, nb, data))
        self.data = self

    @property
    def _mmap(self):
        return self._mm


def dequantize(info: TensorInfo) -> np.ndarray:
    """-> float32 array in numpy order."""
    t = info.tensor_type
    shape = tuple(reversed(info.shape))
    if t == 0:
        return np.asarray(info.data, np.float32)
    if t == 1:
        return np.asarray(info.data).astype(np.float32)
    if t == 30:
        return (np.asarray(info.data, np.uint16).astype(np.uint32) << 16).view(np.float32)
    if t == 2:       # Q4_0: fp16 d, 16 bytes of nibbles (low = elements 0..15, high = 16..31)
        b = np.asarray(info.data).reshape(-1, 18)
        d = b[:, :2].copy().view(np.float16).astype(np.float32)
        q = b[:, 2:]
        vals = np.concatenate([q & 15, q >> 4], axis=1).astype(np.float32) - 8.0
        return (vals * d).reshape(shape)
    if t == 8:       # Q8_0: fp16 d, 32 int8 codes
        b = np.asarray(info.data).reshape(-1, 34)
        d = b[:, :2].copy().view(np.float16).astype(np.float32)
        q = b[:, 2:].copy().view(np.int8).astype(np.float32)
        return (q * d).reshape(shape)
    raise NotImplementedError(f"GGUF tensor type {_NAMES.get(t, t)} is not dequantised by this reader")


class GGUFView:
    """Accessors over one GGUF file (aneforge/_gguf.py:10-46); `arch` is the `*.block_count` prefix."""

    def __init__(self, path: str):
        self.reader = r = GGUFReader(path)
        self.meta = dict(r.fields)
        self.arch = next(k.split(".")[0] for k in self.meta if k.endswith(".block_count"))
        self.tn = {t.name: t for t in r.tensors}

    def field(self, key, default=None):
        f = self.meta.get(key)
        return f.parts[f.data[-1]][0] if f is not None else default

    def sc(self, key, default=None):
        return self.field(self.arch + "." + key, default)

    def has(self, name: str) -> bool:
        return name in self.tn

    def get(self, name: str, dtype=np.float16) -> np.ndarray:
        """Dequantise tensor `name` to `dtype` (fp16 by default)."""
        return dequantize(self.tn[name]).astype(dtype)

    def quantized(self, name: str):
        """Q4_0 tensors as QuantizedWeight codes: a 2-D tensor -> one QuantizedWeight [rows, K];
        a 3-D expert stack [E, rows, K] -> a list of E QuantizedWeights.  None for other types."""
        t = self.tn[name]
        if t.tensor_type != GGML["Q4_0"]:
            return None
        from ._engine import QuantizedWeight
        shape = tuple(reversed(t.shape))
        Kd = shape[-1]
        raw = np.asarray(t.data).reshape(-1, Kd // 32 * 18)
        if len(shape) == 2:
            return QuantizedWeight("q4_0_gguf", raw, None, (shape[0], Kd))
        E, rows = shape[0], shape[1]
        raw = raw.reshape(E, rows, -1)
        return [QuantizedWeight("q4_0_gguf", raw[e], None, (rows, Kd)) for e in range(E)]

    def drop_pages(self) -> None:
        mm = self.reader._mmap
        try:
            mm.madvise(_mmap.MADV_DONTNEED)
        except (AttributeError, OSError, ValueError):
            pass


# ----------------------------------------------------------------------------- writer
def _pack_value(v):
    if isinstance(v, bool):
        return struct.pack("<I?", _BOOL, v)
    if isinstance(v, int):
        return struct.pack("<Iq", _I64, v) if v < 0 else struct.pack("<IQ", _U64, v)
    if isinstance(v, float):
        return struct.pack("<If", _F32, v)
    if isinstance(v, str):
        b = v.encode()
        return struct.pack("<IQ", _STR, len(b)) + b
    if isinstance(v, (list, tuple)):
        if all(isinstance(x, str) for x in v):
            body = b"".join(struct.pack("<Q", len(x.encode())) + x.encode() for x in v)
            return struct.pack("<IIQ", _ARR, _STR, len(v)) + body
        return struct.pack("<IIQ", _ARR, _I32, len(v)) + struct.pack("<" + "i" * len(v), *v)
    raise TypeError(f"unsupported metadata value {v!r}")


def write_gguf(path: str, metadata: dict, tensors: dict, alignment: int = 32) -> None:
    """Write a GGUF v3 file.  tensors: name -> float array (stored F32, or F16 if fp16) or
    (ggml type name, raw block bytes [rows, bytes_per_row], numpy shape)."""
    kv = dict(metadata)
    kv.setdefault("general.alignment", alignment)
    entries = []
    for name, t in tensors.items():
        if isinstance(t, tuple):
            tname, raw, shape = t
            ttype = GGML[tname]
            data = np.ascontiguousarray(raw, np.uint8).tobytes()
        else:
            a = np.ascontiguousarray(t)
            ttype = GGML["F16"] if a.dtype == np.float16 else GGML["F32"]
            a = a.astype(np.float16 if ttype == 1 else np.float32)
            shape, data = a.shape, a.tobytes()
        dims = tuple(reversed(shape))
        if _nbytes(ttype, dims) != len(data):
            raise ValueError(f"{name}: {len(data)} bytes for shape {shape} of type {_NAMES[ttype]}")
        entries.append((name, dims, ttype, data))
    head = bytearray(GGUF_MAGIC + struct.pack("<IQQ", 3, len(entries), len(kv)))
    for k, v in kv.items():
        kb = k.encode()
        head += struct.pack("<Q", len(kb)) + kb + _pack_value(v)
    off = 0
    offsets = []
    for name, dims, ttype, data in entries:
        offsets.append(off)
        off = (off + len(data) + alignment - 1) // alignment * alignment
    for (name, dims, ttype, data), toff in zip(entries, offsets):
        nb = name.encode()
        head += struct.pack("<Q", len(nb)) + nb + struct.pack("<I", len(dims))
        head += struct.pack("<" + "Q" * len(dims), *dims) + struct.pack("<IQ", ttype, toff)
    pad = (-len(head)) % alignment
    with open(path, "wb") as f:
        f.write(head + b"\0" * pad)
        for (name, dims, ttype, data), toff in zip(entries, offsets):
            f.write(data)
            f.write(b"\0" * ((-len(data)) % alignment))
