"""The GGUF block decoders (aneforge_amd._gguf) against the published ggml block layouts.

The reference gets these values from the third-party gguf package (gguf.quants.dequantize,
called at aneforge/_gguf.py:34-39), which is not installed here and ships no vectors.  Two
independent checks pin each decoder instead:
  * an encoder written element by element from the block layout (explicit loops and bit
    positions, nothing shared with the vectorised decoder) packs chosen codes and scales; the
    decoder must return d*scale*q (- dmin*min) for exactly those values, in float32;
  * hand-built blocks whose output has a closed form (derived by hand, written as literals or
    as a one-line expression of the element index).
A wrong nibble order, bit position, scale packing, sign or offset fails both."""
import struct

import numpy as np
import pytest

from aneforge_amd import _gguf

F32 = np.float32


def h16(x) -> bytes:
    return struct.pack("<e", float(x))


def f16v(x) -> F32:
    return F32(np.float16(x))


def bits_le(vals, nbits_each=1) -> bytes:
    """Pack a list of small fields, field i at bit i*nbits_each of a little-endian bit string."""
    acc = 0
    for i, v in enumerate(vals):
        acc |= int(v) << (i * nbits_each)
    n = (len(vals) * nbits_each + 7) // 8
    return acc.to_bytes(n, "little")


def decode(name, blob: bytes) -> np.ndarray:
    t = _gguf.GGML[name]
    return _gguf.dequantize_blocks(t, np.frombuffer(blob, np.uint8))[0]


# ----------------------------------------------------------------------------- encoders (spec, loop form)
def enc_q4_1(d, m, q):
    qs = bytes((q[j] & 15) | ((q[j + 16] & 15) << 4) for j in range(16))
    return h16(d) + h16(m) + qs


def enc_q5(q):     # q: 5-bit codes 0..31 -> (qh, qs)
    qh = bits_le([(q[j] >> 4) & 1 for j in range(32)])
    qs = bytes((q[j] & 15) | ((q[j + 16] & 15) << 4) for j in range(16))
    return qh, qs


def enc_q2_k(d, dmin, sc, mn, q):
    scales = bytes((sc[i] & 15) | ((mn[i] & 15) << 4) for i in range(16))
    qs = bytearray(64)
    for e in range(256):
        h, s, l = e // 128, (e % 128) // 32, e % 32
        qs[32 * h + l] |= (q[e] & 3) << (2 * s)
    return scales + bytes(qs) + h16(d) + h16(dmin)


def enc_q3_k(d, scale, q):   # scale: 16 signed 6-bit (-32..31); q: -4..3
    hmask = bytearray(32)
    qs = bytearray(64)
    for e in range(256):
        hbit = 1 if q[e] >= 0 else 0
        low = q[e] if q[e] >= 0 else q[e] + 4
        i, l = e // 32, e % 32
        hmask[l] |= hbit << i
        h, s, l2 = e // 128, (e % 128) // 32, e % 32
        qs[32 * h + l2] |= low << (2 * s)
    sb = bytearray(12)
    for i in range(16):
        u = scale[i] + 32
        sb[i % 8] |= (u & 15) << (4 * (i // 8))
        sb[8 + i % 4] |= ((u >> 4) & 3) << (2 * (i // 4))
    return bytes(hmask) + bytes(qs) + bytes(sb) + h16(d)


def enc_k4_scales(sc, mn):
    b = bytearray(12)
    for j in range(4):
        b[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        b[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        b[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    return bytes(b)


def enc_k4_codes(q):
    qs = bytearray(128)
    for e in range(256):
        c, half, l = e // 64, (e % 64) // 32, e % 32
        qs[32 * c + l] |= (q[e] & 15) << (4 * half)
    return bytes(qs)


def enc_q4_k(d, dmin, sc, mn, q):
    return h16(d) + h16(dmin) + enc_k4_scales(sc, mn) + enc_k4_codes(q)


def enc_q5_k(d, dmin, sc, mn, q):
    qh = bytearray(32)
    for e in range(256):
        qh[e % 32] |= ((q[e] >> 4) & 1) << (e // 32)
    return h16(d) + h16(dmin) + enc_k4_scales(sc, mn) + bytes(qh) + enc_k4_codes(q)


def enc_q6_k(d, scales, q):   # q: -32..31
    ql = bytearray(128)
    qh = bytearray(64)
    for e in range(256):
        u = q[e] + 32
        h, s, l = e // 128, (e % 128) // 64, e % 64
        ql[64 * h + l] |= (u & 15) << (4 * s)
        h2, s2, l2 = e // 128, (e % 128) // 32, e % 32
        qh[32 * h2 + l2] |= ((u >> 4) & 3) << (2 * s2)
    return bytes(ql) + bytes(qh) + struct.pack("<16b", *scales) + h16(d)


def enc_q8_k(d, q):
    sums = [sum(q[16 * i:16 * i + 16]) for i in range(16)]
    return struct.pack("<f", d) + struct.pack("<256b", *q) + struct.pack("<16h", *sums)


# ----------------------------------------------------------------------------- encoder <-> decoder
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_32_weight_blocks_match_the_layout(seed):
    rng = np.random.default_rng(seed)
    d, m = float(rng.uniform(-0.1, 0.1)), float(rng.uniform(-0.5, 0.5))
    q4 = [int(v) for v in rng.integers(0, 16, 32)]
    q5 = [int(v) for v in rng.integers(0, 32, 32)]
    q8 = [int(v) for v in rng.integers(-128, 128, 32)]
    D, M = f16v(d), f16v(m)
    np.testing.assert_array_equal(decode("Q4_1", enc_q4_1(d, m, q4)), np.array([D * F32(v) + M for v in q4], F32))
    qh, qs = enc_q5(q5)
    np.testing.assert_array_equal(decode("Q5_0", h16(d) + qh + qs), np.array([D * F32(v - 16) for v in q5], F32))
    np.testing.assert_array_equal(decode("Q5_1", h16(d) + h16(m) + qh + qs),
                                  np.array([D * F32(v) + M for v in q5], F32))
    np.testing.assert_array_equal(decode("Q8_1", h16(d) + h16(0.0) + struct.pack("<32b", *q8)),
                                  np.array([D * F32(v) for v in q8], F32))
    np.testing.assert_array_equal(decode("Q8_0", h16(d) + struct.pack("<32b", *q8)),
                                  np.array([D * F32(v) for v in q8], F32))


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_k_quant_super_blocks_match_the_layout(seed):
    rng = np.random.default_rng(100 + seed)
    d, dmin = float(rng.uniform(0.001, 0.05)), float(rng.uniform(0.001, 0.05))
    D, DM = f16v(d), f16v(dmin)
    # Q2_K: 16 sub-blocks of 16, 4-bit scale and min, 2-bit codes
    sc, mn = rng.integers(0, 16, 16), rng.integers(0, 16, 16)
    q = rng.integers(0, 4, 256)
    want = np.array([(D * F32(sc[e // 16])) * F32(q[e]) - DM * F32(mn[e // 16]) for e in range(256)], F32)
    np.testing.assert_array_equal(decode("Q2_K", enc_q2_k(d, dmin, sc, mn, q)), want)
    # Q3_K: signed 6-bit scales, codes -4..3
    s3 = [int(v) for v in rng.integers(-32, 32, 16)]
    q3 = [int(v) for v in rng.integers(-4, 4, 256)]
    want = np.array([(D * F32(s3[e // 16])) * F32(q3[e]) for e in range(256)], F32)
    np.testing.assert_array_equal(decode("Q3_K", enc_q3_k(d, s3, q3)), want)
    # Q4_K / Q5_K: 8 sub-blocks of 32, 6-bit scale and min
    sc8, mn8 = [int(v) for v in rng.integers(0, 64, 8)], [int(v) for v in rng.integers(0, 64, 8)]
    q4 = [int(v) for v in rng.integers(0, 16, 256)]
    want = np.array([(D * F32(sc8[e // 32])) * F32(q4[e]) - DM * F32(mn8[e // 32]) for e in range(256)], F32)
    np.testing.assert_array_equal(decode("Q4_K", enc_q4_k(d, dmin, sc8, mn8, q4)), want)
    q5 = [int(v) for v in rng.integers(0, 32, 256)]
    want = np.array([(D * F32(sc8[e // 32])) * F32(q5[e]) - DM * F32(mn8[e // 32]) for e in range(256)], F32)
    np.testing.assert_array_equal(decode("Q5_K", enc_q5_k(d, dmin, sc8, mn8, q5)), want)
    # Q6_K: int8 scale per 16, codes -32..31
    s6 = [int(v) for v in rng.integers(-128, 128, 16)]
    q6 = [int(v) for v in rng.integers(-32, 32, 256)]
    want = np.array([(D * F32(s6[e // 16])) * F32(q6[e]) for e in range(256)], F32)
    np.testing.assert_array_equal(decode("Q6_K", enc_q6_k(d, s6, q6)), want)
    # Q8_K: fp32 scale
    q8 = [int(v) for v in rng.integers(-128, 128, 256)]
    np.testing.assert_array_equal(decode("Q8_K", enc_q8_k(0.0123, q8)), np.array([F32(0.0123) * F32(v) for v in q8], F32))


# ----------------------------------------------------------------------------- closed-form blocks
def test_known_answer_blocks():
    e = np.arange(256)
    # Q4_K, d = 0.5, dmin = 0.25, scale_j = j + 1, min_j = 2j, every code 3:
    # w[32j + l] = 0.5 (j + 1) 3 - 0.25 (2j) = 1.5 + j
    blk = h16(0.5) + h16(0.25) + enc_k4_scales([j + 1 for j in range(8)], [2 * j for j in range(8)]) + bytes([0x33] * 128)
    np.testing.assert_array_equal(decode("Q4_K", blk), (1.5 + e // 32).astype(F32))
    # Q5_K, same scales, every code 19 (nibble 3, bit 4 set: qh all ones): w = 0.5 (j+1) 19 - 0.5 j = 9.5 + 9j
    blk = h16(0.5) + h16(0.25) + enc_k4_scales([j + 1 for j in range(8)], [2 * j for j in range(8)]) \
        + bytes([0xFF] * 32) + bytes([0x33] * 128)
    np.testing.assert_array_equal(decode("Q5_K", blk), (9.5 + 9 * (e // 32)).astype(F32))
    # Q6_K, d = 0.5, scale_i = i - 8, every code 40 (q = 8): w[16i + l] = 4 (i - 8);
    # code 40 = 0b10_1000: low nibble 8 in both ql nibbles, high bits 2 in every qh crumb
    blk = bytes([0x88] * 128) + bytes([0xAA] * 64) + struct.pack("<16b", *[i - 8 for i in range(16)]) + h16(0.5)
    np.testing.assert_array_equal(decode("Q6_K", blk), (4 * (e // 16 - 8)).astype(F32))
    # Q3_K, d = 2, every scale = -8 (stored 24 = 0b01_1000), every code -3 (hmask bit clear, low bits 1):
    # w = 2 (-8) (-3) = 48
    blk = bytes(32) + bytes([0x55] * 64) + bytes([0x88] * 8) + bytes([0x55] * 4) + h16(2.0)
    np.testing.assert_array_equal(decode("Q3_K", blk), np.full(256, 48.0, F32))
    # Q2_K, d = 1, dmin = 0.5, scale byte i = i | (15 - i) << 4, every code 2: w[16i + l] = 2i - 0.5 (15 - i)
    blk = bytes([i | ((15 - i) << 4) for i in range(16)]) + bytes([0xAA] * 64) + h16(1.0) + h16(0.5)
    np.testing.assert_array_equal(decode("Q2_K", blk), (2.5 * (e // 16) - 7.5).astype(F32))
    # Q5_0, d = 1, qh = 0xFFFF0000 (elements 16..31 have bit 4), qs bytes 0x21:
    # elements 0..15 = 1 - 16 = -15, elements 16..31 = 2 + 16 - 16 = 2
    blk = h16(1.0) + struct.pack("<I", 0xFFFF0000) + bytes([0x21] * 16)
    np.testing.assert_array_equal(decode("Q5_0", blk), np.array([-15.0] * 16 + [2.0] * 16, F32))
    # Q4_1, d = 0.5, m = -1, bytes 0xF0: elements 0..15 = -1, elements 16..31 = 0.5 * 15 - 1 = 6.5
    blk = h16(0.5) + h16(-1.0) + bytes([0xF0] * 16)
    np.testing.assert_array_equal(decode("Q4_1", blk), np.array([-1.0] * 16 + [6.5] * 16, F32))


def test_gguf_file_with_k_quant_tensors_reads_like_the_blocks(tmp_path):
    rng = np.random.default_rng(7)
    rows, K = 3, 512
    blocks = []
    for _ in range(rows * K // 256):
        sc8, mn8 = [int(v) for v in rng.integers(0, 64, 8)], [int(v) for v in rng.integers(0, 64, 8)]
        blocks.append(enc_q4_k(0.01, 0.02, sc8, mn8, [int(v) for v in rng.integers(0, 16, 256)]))
    raw = np.frombuffer(b"".join(blocks), np.uint8).reshape(rows, -1)
    p = str(tmp_path / "k.gguf")
    _gguf.write_gguf(p, {"general.architecture": "llama", "llama.block_count": 1},
                     {"w": ("Q4_K", raw, (rows, K)), "n": np.ones(K, np.float32)})
    g = _gguf.GGUFView(p)
    got = g.get("w")
    assert got.shape == (rows, K) and got.dtype == np.float16
    want = _gguf.dequantize_blocks(_gguf.GGML["Q4_K"], raw).reshape(rows, K).astype(np.float16)
    np.testing.assert_array_equal(got, want)
    q = g.quantized("w")                               # Q4_K streams as its own codes on the device
    assert q.fmt == "q4_k" and q.shape == (rows, K)
    assert np.array_equal(q.codes, raw.reshape(rows, K // 256, 144)[:, :, 16:].reshape(rows, K // 2))
    np.testing.assert_array_equal(q.dequant().astype(np.float16), want)   # the same fp16 weights as get()


def test_q6_k_tensors_stream_as_codes(tmp_path):
    rng = np.random.default_rng(8)
    rows, K = 3, 512
    blocks = [enc_q6_k(float(np.float16(rng.uniform(0.001, 0.05))), [int(v) for v in rng.integers(-128, 128, 16)],
                       [int(v) for v in rng.integers(-32, 32, 256)]) for _ in range(rows * K // 256)]
    raw = np.frombuffer(b"".join(blocks), np.uint8).reshape(rows, -1)
    p = str(tmp_path / "q6.gguf")
    _gguf.write_gguf(p, {"general.architecture": "llama", "llama.block_count": 1}, {"w": ("Q6_K", raw, (rows, K))})
    g = _gguf.GGUFView(p)
    want = _gguf.dequantize_blocks(_gguf.GGML["Q6_K"], raw).reshape(rows, K).astype(np.float16)
    np.testing.assert_array_equal(g.get("w"), want)
    q = g.quantized("w")                               # the chunked 6-bit layout, same fp16 weights
    assert q.fmt == "q6_k" and q.shape == (rows, K) and q.codes.shape == (rows, K // 2)
    np.testing.assert_array_equal(q.dequant().astype(np.float16), want)


def test_unsupported_types_are_named():
    with pytest.raises(NotImplementedError, match="IQ2_XXS"):
        _gguf._nbytes(16, (256,))
    with pytest.raises(NotImplementedError, match="IQ4_NL"):
        _gguf.dequantize_blocks(20, np.zeros(18, np.uint8))


def test_q8_0_tensors_stream_as_blockwise_codes(tmp_path):
    # Q8_0 = fp16 d + 32 int8 codes per block: the kernels' blockwise format (weight fp16(d * q))
    rng = np.random.default_rng(8)
    E, rows, K = 3, 4, 128
    d = rng.uniform(0.001, 0.01, (E * rows, K // 32)).astype(np.float16)
    q = rng.integers(-127, 128, (E * rows, K), dtype=np.int8)
    blocks = b"".join(h16(d[r, b]) + q[r, 32 * b:32 * b + 32].tobytes() for r in range(E * rows) for b in range(K // 32))
    raw = np.frombuffer(blocks, np.uint8).reshape(E * rows, -1)
    p = str(tmp_path / "q8.gguf")
    _gguf.write_gguf(p, {"general.architecture": "llama", "llama.block_count": 1},
                     {"exps": ("Q8_0", raw, (E, rows, K)), "one": ("Q8_0", raw[:rows], (rows, K)),
                      "odd": ("Q8_0", raw[:rows, :34 * 3], (rows, 96))})
    g = _gguf.GGUFView(p)
    experts = g.quantized("exps")
    assert len(experts) == E
    for e, w in enumerate(experts):
        assert w.fmt == "blockwise" and w.shape == (rows, K)
        np.testing.assert_array_equal(w.codes, q[e * rows:(e + 1) * rows])
        np.testing.assert_array_equal(w.scale, d[e * rows:(e + 1) * rows])
        want = _gguf.dequantize_blocks(_gguf.GGML["Q8_0"], raw[e * rows:(e + 1) * rows]).reshape(rows, K)
        np.testing.assert_array_equal(w.dequant(), want)
    assert g.quantized("one").fmt == "blockwise"
    assert g.quantized("odd") is None                 # K = 96: not a multiple of 64, dequantised instead


def test_q4_k_high_scale_bits_known_answer():
    # The Q4_K 12-byte scale field written out byte by byte (not through an encoder): sub-blocks 4..7
    # carry 6-bit scales and mins >= 16, whose top two bits sit in bits 6-7 of bytes 0..3 (scales) and
    # 4..7 (mins) and whose low nibbles sit in bytes 8..11 (ggml get_scale_min_k4).
    #   scales 1, 2, 3, 4, 17, 33, 50, 63; mins 5, 6, 7, 8, 48, 20, 31, 60
    field = bytes([0x41, 0x82, 0xC3, 0xC4,     # scale_j | (scale_{j+4} >> 4) << 6
                   0xC5, 0x46, 0x47, 0xC8,     # min_j | (min_{j+4} >> 4) << 6
                   0x01, 0x41, 0xF2, 0xCF])    # (scale_{j+4} & 15) | (min_{j+4} & 15) << 4
    blk = h16(1.0) + h16(0.5) + field + bytes([0x22] * 128)        # every code 2
    # w[32j + l] = 1.0 * scale_j * 2 - 0.5 * min_j
    want = np.repeat(np.array([-0.5, 1.0, 2.5, 4.0, 10.0, 56.0, 84.5, 96.0], F32), 32)
    np.testing.assert_array_equal(decode("Q4_K", blk), want)
    from oracle import ref
    np.testing.assert_array_equal(ref.dequant_q4_k(np.frombuffer(blk, np.uint8).reshape(1, 144))[0], want)
    # the device layout's unpacked header: per pair p the bytes {sc(2p), sc(2p+1), m(2p), m(2p+1)}
    from aneforge_amd import _blob
    _, hdr = _blob.q4_k_repack(np.frombuffer(blk, np.uint8).reshape(1, 144), 1, 256)
    pairs = hdr.view(np.uint32)[0, 1:5]
    got = [[int(w >> (8 * i)) & 255 for i in range(4)] for w in pairs]
    assert got == [[1, 2, 5, 6], [3, 4, 7, 8], [17, 33, 48, 20], [50, 63, 31, 60]]
