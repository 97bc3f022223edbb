"""GGUF v3 reader and writer (this package's own; the reference depends on the third-party
`gguf` package, aneforge/_gguf.py:10-46, which is not part of this build).

GGUFView keeps the reference's accessors (meta, arch, tn, field, sc, has, get, drop_pages) and
adds `quantized(name)`, which returns Q4_0, Q4_K, Q6_K and Q8_0 tensors as QuantizedWeight codes
instead of dequantising them, so the Q4_0 / Q4_K / Q6_K / blockwise kernels stream the file's own codes.

Format: magic "GGUF", version 3, tensor count, metadata count, metadata key/values, tensor infos
(name, dims with dims[0] innermost, ggml type, offset), data section aligned to
general.alignment (default 32).

Dequantisers (the ggml block formats that llama.cpp quantisations write; the reference gets the
same float32 values from gguf.quants.dequantize and then casts to the requested dtype):
  F32, F16, BF16; Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q8_1 (32-weight blocks);
  Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K (256-weight super-blocks).
Each is evaluated in float32 in the order gguf-py uses (block scale x sub-block scale first, then
x code, then minus the block minimum), so the fp16 cast matches the reference's value exactly.
The importance-matrix "IQ" and ternary formats are not decoded (NotImplementedError names them)."""
from __future__ import annotations

import mmap as _mmap
import struct
from dataclasses import dataclass
from typing import Any

import numpy as np

GGUF_MAGIC = b"GGUF"
QK_K = 256
# ggml tensor types read here: type id, and (elements per block, bytes per block)
GGML = {"F32": 0, "F16": 1, "Q4_0": 2, "Q4_1": 3, "Q5_0": 6, "Q5_1": 7, "Q8_0": 8, "Q8_1": 9,
        "Q2_K": 10, "Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "Q8_K": 15, "BF16": 30}
_BLOCK = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 9: (32, 36),
          10: (QK_K, 84), 11: (QK_K, 110), 12: (QK_K, 144), 13: (QK_K, 176), 14: (QK_K, 210),
          15: (QK_K, 292), 30: (1, 2)}
_NAMES = {v: k for k, v in GGML.items()}
# other ggml type ids, named in errors
_UNSUPPORTED = {16: "IQ2_XXS", 17: "IQ2_XS", 18: "IQ3_XXS", 19: "IQ1_S", 20: "IQ4_NL", 21: "IQ3_S", 22: "IQ2_S",
                23: "IQ4_XS", 29: "IQ1_M", 34: "TQ1_0", 35: "TQ2_0", 39: "MXFP4"}

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
        raise NotImplementedError(f"GGUF tensor type {_UNSUPPORTED.get(ttype, ttype)} is not supported by this reader")
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


# ----------------------------------------------------------------------------- block decoders
# Each takes the blocks as uint8 [n, bytes per block] and returns float32 [n, elements per block].
def _f16(b) -> np.ndarray:
    """Little-endian fp16 fields [n, 2] -> float32 [n, 1]."""
    return np.ascontiguousarray(b).view(np.float16).astype(np.float32)


def _halves(qs) -> np.ndarray:
    """16 bytes of nibbles -> 32 codes: element j < 16 is the low nibble of byte j, element 16 + j
    the high nibble (the 32-weight ggml blocks)."""
    return np.concatenate([qs & 15, qs >> 4], axis=1)


def _lsb_bits(b) -> np.ndarray:
    """Bytes [n, m] -> bits [n, 8m]: bit i of the little-endian bit string."""
    return np.unpackbits(np.ascontiguousarray(b), axis=1, bitorder="little")


def _crumbs(qs, groups) -> np.ndarray:
    """2-bit fields of 32-byte rows: element 128h + 32s + l = (qs[32h + l] >> 2s) & 3 for each
    32-byte row h and shift s (the Q2_K / Q3_K low bits, the Q6_K high bits)."""
    n = qs.shape[0]
    sh = np.arange(0, 8, 2, dtype=np.uint8)
    return ((qs.reshape(n, groups, 1, 32) >> sh[None, None, :, None]) & 3).reshape(n, groups * 128)


def _k4_scale_min(sc):
    """The 12-byte Q4_K / Q5_K scale field -> 6-bit scale and min of each of the 8 sub-blocks:
    j < 4: scale = b[j] & 63, min = b[j + 4] & 63; j >= 4: the low 4 bits come from b[j + 4]
    (scale: low nibble, min: high nibble) and the top 2 bits from bits 6-7 of b[j - 4] (scale)
    and b[j] (min)."""
    lo, mid, hi = sc[:, 0:4], sc[:, 4:8], sc[:, 8:12]
    scale = np.concatenate([lo & 63, (hi & 15) | ((lo >> 6) << 4)], axis=1)
    mins = np.concatenate([mid & 63, (hi >> 4) | ((mid >> 6) << 4)], axis=1)
    return scale.astype(np.float32), mins.astype(np.float32)


def _q4_0(b):
    return _f16(b[:, 0:2]) * (_halves(b[:, 2:18]).astype(np.float32) - 8.0)


def _q4_1(b):
    return _f16(b[:, 0:2]) * _halves(b[:, 4:20]).astype(np.float32) + _f16(b[:, 2:4])


def _q5(b, off):
    """5-bit codes of Q5_0 / Q5_1: the nibble of _halves, bit 4 = bit j of the 32-bit field qh."""
    return (_halves(b[:, off + 4:off + 20]) | (_lsb_bits(b[:, off:off + 4]) << 4)).astype(np.float32)


def _q5_0(b):
    return _f16(b[:, 0:2]) * (_q5(b, 2) - 16.0)


def _q5_1(b):
    return _f16(b[:, 0:2]) * _q5(b, 4) + _f16(b[:, 2:4])


def _q8_0(b):
    return _f16(b[:, 0:2]) * b[:, 2:34].copy().view(np.int8).astype(np.float32)


def _q8_1(b):
    return _f16(b[:, 0:2]) * b[:, 4:36].copy().view(np.int8).astype(np.float32)


def _q2_k(b):
    """84 B: scales[16] (low nibble: scale, high: min of each 16-weight sub-block), 2-bit codes
    qs[64], fp16 d, fp16 dmin.  w = d*scale * q - dmin*min."""
    n = b.shape[0]
    sc = b[:, 0:16]
    dl = _f16(b[:, 80:82]) * (sc & 15).astype(np.float32)
    ml = _f16(b[:, 82:84]) * (sc >> 4).astype(np.float32)
    q = _crumbs(b[:, 16:80], 2).astype(np.float32).reshape(n, 16, 16)
    return (dl[:, :, None] * q - ml[:, :, None]).reshape(n, QK_K)


def _q3_k(b):
    """110 B: hmask[32], 2-bit codes qs[64], 12-byte packed signed 6-bit scales, fp16 d.
    Element e = 32i + l has high bit (hmask[l] >> i) & 1; q = low2 - (4 if that bit is clear)."""
    n = b.shape[0]
    hbit = _lsb_bits(b[:, 0:32]).reshape(n, 32, 8).transpose(0, 2, 1).reshape(n, QK_K)
    low = _crumbs(b[:, 32:96], 2).astype(np.int8)
    q = (low - ((hbit ^ 1).astype(np.int8) << 2)).astype(np.float32).reshape(n, 16, 16)
    s = b[:, 96:108]
    i = np.arange(16)
    lo4 = (s[:, i % 8] >> (4 * (i // 8)).astype(np.uint8)) & 15
    hi2 = (s[:, 8 + i % 4] >> (2 * (i // 4)).astype(np.uint8)) & 3
    scale = ((lo4 | (hi2 << 4)).astype(np.int8) - 32).astype(np.float32)
    dl = _f16(b[:, 108:110]) * scale
    return (dl[:, :, None] * q).reshape(n, QK_K)


def _k4_codes(qs):
    """128 bytes of Q4_K / Q5_K nibbles -> 256 codes: element 64c + 32h + l = (qs[32c + l] >> 4h) & 15."""
    n = qs.shape[0]
    sh = np.array([0, 4], dtype=np.uint8)
    return ((qs.reshape(n, 4, 1, 32) >> sh[None, None, :, None]) & 15).reshape(n, QK_K)


def _q4_k(b):
    """144 B: fp16 d, fp16 dmin, 12-byte scales/mins, codes[128].  w = d*scale_j * q - dmin*min_j
    over 8 sub-blocks of 32."""
    n = b.shape[0]
    scale, mins = _k4_scale_min(b[:, 4:16])
    dl = _f16(b[:, 0:2]) * scale
    ml = _f16(b[:, 2:4]) * mins
    q = _k4_codes(b[:, 16:144]).astype(np.float32).reshape(n, 8, 32)
    return (dl[:, :, None] * q - ml[:, :, None]).reshape(n, QK_K)


def _q5_k(b):
    """176 B: fp16 d, fp16 dmin, 12-byte scales/mins, qh[32], codes[128]; bit 4 of element
    32j + l is bit j of qh[l]."""
    n = b.shape[0]
    scale, mins = _k4_scale_min(b[:, 4:16])
    dl = _f16(b[:, 0:2]) * scale
    ml = _f16(b[:, 2:4]) * mins
    hbit = _lsb_bits(b[:, 16:48]).reshape(n, 32, 8).transpose(0, 2, 1).reshape(n, QK_K)
    q = (_k4_codes(b[:, 48:176]) | (hbit << 4)).astype(np.float32).reshape(n, 8, 32)
    return (dl[:, :, None] * q - ml[:, :, None]).reshape(n, QK_K)


def _q6_k(b):
    """210 B: ql[128] (low 4 bits: element 128h + 64s + l from byte 64h + l, nibble s), qh[64]
    (high 2 bits, the _crumbs layout), int8 scales[16] per 16 weights, fp16 d.  q = code - 32."""
    n = b.shape[0]
    ql = b[:, 0:128]
    sh = np.array([0, 4], dtype=np.uint8)
    low = ((ql.reshape(n, 2, 1, 64) >> sh[None, None, :, None]) & 15).reshape(n, QK_K)
    high = _crumbs(b[:, 128:192], 2)
    q = ((low | (high << 4)).astype(np.int16) - 32).astype(np.float32).reshape(n, 16, 16)
    dl = _f16(b[:, 208:210]) * b[:, 192:208].copy().view(np.int8).astype(np.float32)
    return (dl[:, :, None] * q).reshape(n, QK_K)


def _q8_k(b):
    """292 B: fp32 d, int8 codes[256], int16 block sums[16] (not needed to decode)."""
    d = np.ascontiguousarray(b[:, 0:4]).view(np.float32)
    return d * b[:, 4:260].copy().view(np.int8).astype(np.float32)


_DECODE = {2: _q4_0, 3: _q4_1, 6: _q5_0, 7: _q5_1, 8: _q8_0, 9: _q8_1,
           10: _q2_k, 11: _q3_k, 12: _q4_k, 13: _q5_k, 14: _q6_k, 15: _q8_k}


def dequantize_blocks(ttype: int, blocks) -> np.ndarray:
    """Raw blocks (uint8, any shape whose size is a whole number of blocks) -> float32 [n, per]."""
    if ttype not in _DECODE:
        raise NotImplementedError(f"GGUF tensor type {_NAMES.get(ttype, _UNSUPPORTED.get(ttype, ttype))} "
                                  "is not dequantised by this reader")
    size = _BLOCK[ttype][1]
    return _DECODE[ttype](np.asarray(blocks, np.uint8).reshape(-1, size))


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
    return dequantize_blocks(t, info.data).reshape(shape)


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
        """Tensors the kernels stream in their file encoding, as QuantizedWeight codes: Q4_0 (the
        Q4_0 kernels), Q4_K and Q6_K (their kernels, after a lossless byte repack of each super-block)
        and Q8_0 with rows of a multiple of 64 (the blockwise kernels: Q8_0's fp16(d * q) is their
        weight).  A 2-D tensor -> one QuantizedWeight [rows, K]; a 3-D expert
        stack [E, rows, K] -> a list of E.  None for other types."""
        t = self.tn[name]
        shape = tuple(reversed(t.shape))
        Kd = shape[-1]
        from ._engine import QuantizedWeight
        if t.tensor_type == GGML["Q4_0"]:
            raw = np.asarray(t.data).reshape(-1, Kd // 32 * 18)
            make = lambda r, n: QuantizedWeight("q4_0_gguf", r, None, (n, Kd))
        elif t.tensor_type == GGML["Q4_K"] and Kd % 256 == 0:
            from ._blob import q4_k_repack
            b = np.asarray(t.data).reshape(-1, Kd // 256 * 144)
            raw = q4_k_repack(b, b.shape[0], Kd)
            make = lambda r, n: QuantizedWeight("q4_k", r[0], r[1], (n, Kd))
        elif t.tensor_type == GGML["Q6_K"] and Kd % 256 == 0:
            from ._blob import q6_k_repack
            b = np.asarray(t.data).reshape(-1, Kd // 256 * 210)
            raw = q6_k_repack(b, b.shape[0], Kd)
            make = lambda r, n: QuantizedWeight("q6_k", r[0], r[1], (n, Kd))
        elif t.tensor_type == GGML["Q8_0"] and Kd % 64 == 0:
            b = np.asarray(t.data).reshape(-1, Kd // 32, 34)
            raw = (np.ascontiguousarray(b[:, :, 2:]).view(np.int8).reshape(-1, Kd),
                   np.ascontiguousarray(b[:, :, :2]).view(np.float16).reshape(-1, Kd // 32))
            make = lambda r, n: QuantizedWeight("blockwise", r[0], r[1], (n, Kd))
        else:
            return None
        if len(shape) == 2:
            return make(raw, shape[0])
        E, rows = shape[0], shape[1]
        if isinstance(raw, tuple):
            return [make((raw[0][e * rows:(e + 1) * rows], raw[1][e * rows:(e + 1) * rows]), rows) for e in range(E)]
        raw = raw.reshape(E, rows, -1)
        return [make(raw[e], rows) for e in range(E)]

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
