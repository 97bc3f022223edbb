"""Host-side weight codecs: the reference's `compress=` encodings (aneforge/_blob.py:20-56)
plus GGUF Q4_0, and the packing into the layouts the HIP kernels stream.

  quantize_per_row   int8 codes + fp16 per-output-row scale      (aneforge/_blob.py:20-25)
  quantize_blockwise int8 codes + fp16 scale per 32-column block (aneforge/_blob.py:46-56)
  palettize_lut4     16-entry per-tensor LUT, 4-bit indices      (aneforge/_blob.py:28-43)
  quantize_q4_0      ggml Q4_0 blocks (18 B / 32 weights) from fp weights
  q4_0_to_superblock GGUF Q4_0 bytes -> (qs, d) superblock layout (host twin of afx_q4_0_repack)
  q4_k_repack        GGUF Q4_K bytes -> (codes, header) the Q4_K kernels read (host twin of afx_q4_k_repack)
  q6_k_repack        GGUF Q6_K bytes -> (codes, side words) the Q6_K kernels read (host twin of afx_q6_k_repack)

The encodings must produce the reference's bytes, so their steps match the reference's; the
code is this package's own.  The BLOBFILE container is ANE-specific and is not rebuilt."""
from __future__ import annotations

import numpy as np

F16 = np.float16


def quantize_per_row(W: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """[OUT, IN] -> (int8 [OUT, IN], fp16 scale [OUT]).  Scale = max|row|/127 floored at 1e-8,
    computed in fp32; codes use that fp32 scale with round-half-to-even; the scale is stored fp16."""
    W32 = np.asarray(W, dtype=np.float32)
    amax = np.max(np.abs(W32), axis=1)
    scale = np.maximum(amax / np.float32(127.0), np.float32(1e-8)).astype(np.float32)
    codes = np.rint(W32 / scale[:, None])
    return np.clip(codes, -127, 127).astype(np.int8), scale.astype(F16)


def quantize_blockwise(W: np.ndarray, block_size: int = 32) -> tuple[np.ndarray, np.ndarray, int]:
    """[OUT, IN] -> (int8 [OUT, IN], fp16 scale [OUT, IN/bs], bs); bs clamps down to a divisor of IN."""
    W32 = np.asarray(W, dtype=np.float32)
    OUT, IN = W32.shape
    bs = int(block_size)
    while bs > 1 and IN % bs:
        bs -= 1
    blocks = W32.reshape(OUT, IN // bs, bs)
    scale = np.maximum(np.max(np.abs(blocks), axis=2) / np.float32(127.0), np.float32(1e-8))
    codes = np.clip(np.rint(blocks / scale[:, :, None]), -127, 127).astype(np.int8)
    return codes.reshape(OUT, IN), scale.astype(F16), bs


def palettize_lut4(W: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-tensor 16-entry codebook by 20 deterministic Lloyd iterations from quantile edges;
    indices packed two per byte, low nibble = even column.  -> (packed uint8 [OUT, ceil(IN/2)],
    fp16 codebook [16])."""
    flat = np.asarray(W, dtype=np.float32).reshape(-1)
    edges = np.quantile(flat, np.linspace(0.0, 1.0, 17))
    cb = ((edges[:-1] + edges[1:]) / 2.0).astype(np.float32)
    for _ in range(20):
        idx = np.abs(flat[:, None] - cb[None, :]).argmin(axis=1)
        for j in range(16):
            members = flat[idx == j]
            if members.size:
                cb[j] = members.mean()
    idx = np.abs(flat[:, None] - cb[None, :]).argmin(axis=1).astype(np.uint8).reshape(W.shape[0], -1)
    if idx.shape[1] % 2:
        idx = np.pad(idx, ((0, 0), (0, 1)))
    return (idx[:, 0::2] | (idx[:, 1::2] << 4)).astype(np.uint8), cb.astype(F16)


# ----------------------------------------------------------------------------- Q4_0
Q4_BLOCK, Q4_BYTES = 32, 18


def quantize_q4_0(W: np.ndarray) -> np.ndarray:
    """ggml Q4_0: per 32-block, d = (signed element of largest magnitude) / -8, code =
    min(15, trunc(x/d + 8.5)).  Returns GGUF block bytes [OUT, IN/32*18]."""
    W32 = np.asarray(W, dtype=np.float32)
    OUT, IN = W32.shape
    if IN % Q4_BLOCK:
        raise ValueError(f"Q4_0 needs IN % 32 == 0 (got {IN})")
    b = W32.reshape(OUT, IN // Q4_BLOCK, Q4_BLOCK)
    pick = np.take_along_axis(b, np.abs(b).argmax(axis=2)[:, :, None], axis=2)[:, :, 0]
    d = pick / np.float32(-8.0)
    safe = np.where(d == 0, np.float32(1.0), d)
    inv = np.where(d == 0, np.float32(0.0), np.float32(1.0) / safe).astype(np.float32)
    codes = np.clip(np.minimum(15, np.trunc(b * inv[:, :, None] + np.float32(8.5))), 0, 15).astype(np.uint8)
    out = np.empty((OUT, IN // Q4_BLOCK, Q4_BYTES), np.uint8)
    out[:, :, 0:2] = d.astype(F16)[:, :, None].view(np.uint8)
    out[:, :, 2:] = (codes[:, :, :16] & 15) | ((codes[:, :, 16:] & 15) << 4)
    return out.reshape(OUT, -1)


def q4_0_codes(blocks: np.ndarray, N: int, K: int) -> tuple[np.ndarray, np.ndarray]:
    """GGUF Q4_0 bytes -> (codes uint8 [N, K] in 0..15, d fp16 [N, K/32])."""
    b = np.asarray(blocks, np.uint8).reshape(N, K // Q4_BLOCK, Q4_BYTES)
    d = np.ascontiguousarray(b[:, :, 0:2]).view(F16).reshape(N, K // Q4_BLOCK)
    lo, hi = b[:, :, 2:] & 15, b[:, :, 2:] >> 4
    return np.concatenate([lo, hi], axis=2).reshape(N, K), d


def q4_0_to_superblock(blocks: np.ndarray, N: int, K: int) -> tuple[np.ndarray, np.ndarray]:
    """Host twin of afx_q4_0_repack: -> (qs uint8 [N, K/2], d fp16 [N, K/32]).  Word
    (row, sb, g, j) holds elements 8g..8g+7 of block 4sb+j: even elements' nibbles in bits
    0/4/8/12, odd elements' in bits 16/20/24/28."""
    if K % 128:
        raise ValueError(f"superblock layout needs K % 128 == 0 (got {K})")
    codes, d = q4_0_codes(blocks, N, K)
    c = codes.reshape(N, K // 128, 4, 4, 8).astype(np.uint32)        # [N, sb, j, g, e]
    ev, od = c[..., 0::2], c[..., 1::2]                              # [N, sb, j, g, 4]
    sh = (4 * np.arange(4, dtype=np.uint32))
    words = ((ev << sh).sum(-1) | ((od << (sh + 16)).sum(-1))).astype(np.uint32)   # [N, sb, j, g]
    words = np.ascontiguousarray(words.transpose(0, 1, 3, 2))       # [N, sb, g, j]
    return words.reshape(N, -1).view(np.uint8).reshape(N, K // 2), d


def superblock_to_q4_0(qs: np.ndarray, d: np.ndarray, N: int, K: int) -> np.ndarray:
    """Inverse of q4_0_to_superblock -> GGUF bytes [N, K/32*18]."""
    words = np.ascontiguousarray(qs).view(np.uint32).reshape(N, K // 128, 4, 4)   # [N, sb, g, j]
    words = words.transpose(0, 1, 3, 2)                                          # [N, sb, j, g]
    sh = (4 * np.arange(4, dtype=np.uint32))
    ev = (words[..., None] >> sh) & 15
    od = (words[..., None] >> (sh + 16)) & 15
    e = np.empty(words.shape + (8,), np.uint8)
    e[..., 0::2], e[..., 1::2] = ev, od
    codes = e.reshape(N, K // 32, 32)
    out = np.empty((N, K // 32, Q4_BYTES), np.uint8)
    out[:, :, 0:2] = np.asarray(d, F16).reshape(N, K // 32, 1).view(np.uint8)
    out[:, :, 2:] = (codes[:, :, :16] & 15) | ((codes[:, :, 16:] & 15) << 4)
    return out.reshape(N, -1)


# ----------------------------------------------------------------------------- row layouts
def rope_pair_order(n_heads: int, dh: int) -> np.ndarray:
    """Row permutation putting dims (i, i+dh/2) of every head next to each other, so the fused
    QKV kernel can rotate pairs held by one wavefront.  Per-row quantization is unaffected."""
    half = dh // 2
    per = np.empty(dh, np.int64)
    per[0::2], per[1::2] = np.arange(half), np.arange(half) + half
    return (np.arange(n_heads)[:, None] * dh + per[None, :]).reshape(-1)


def interleave_rows(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Rows a0, b0, a1, b1, ... (gate/up pairs for the fused SwiGLU epilogue)."""
    out = np.empty((a.shape[0] * 2,) + a.shape[1:], a.dtype)
    out[0::2], out[1::2] = a, b
    return out


def q4_k_repack(blocks: np.ndarray, N: int, K: int) -> tuple[np.ndarray, np.ndarray]:
    """Host twin of afx_q4_k_repack: GGUF Q4_K super-blocks (144 B: fp16 d, fp16 dmin, 12 bytes of
    6-bit scales and mins, 128 code bytes) -> (codes uint8 [N, K/2]: each super-block's 128 code
    bytes as they are; header int32 [N, K/256 * 5]: per super-block {d | dmin << 16} and, for each
    sub-block pair p, the bytes {sc(2p), sc(2p+1), m(2p), m(2p+1)}).  The 12-byte field: j < 4:
    sc = b[j] & 63, m = b[j+4] & 63; j >= 4: sc = (b[j+4] & 15) | (b[j-4] >> 6) << 4,
    m = (b[j+4] >> 4) | (b[j] >> 6) << 4."""
    if K % 256:
        raise ValueError(f"Q4_K rows need K % 256 == 0 (got {K})")
    b = np.ascontiguousarray(blocks, np.uint8).reshape(N, K // 256, 144)
    codes = np.ascontiguousarray(b[:, :, 16:]).reshape(N, K // 2)
    f = b[:, :, 4:16].astype(np.uint32)
    lo, mid, hi = f[..., 0:4], f[..., 4:8], f[..., 8:12]
    sc = np.concatenate([lo & 63, (hi & 15) | ((lo >> 6) << 4)], axis=-1)      # [N, nb, 8]
    mn = np.concatenate([mid & 63, (hi >> 4) | ((mid >> 6) << 4)], axis=-1)
    hdr = np.empty((N, K // 256, 5), np.uint32)
    hdr[..., 0] = np.ascontiguousarray(b[:, :, 0:4]).view(np.uint32)[..., 0]
    hdr[..., 1:] = sc[..., 0::2] | (sc[..., 1::2] << 8) | (mn[..., 0::2] << 16) | (mn[..., 1::2] << 24)
    return codes, hdr.reshape(N, -1).view(np.int32)


def q6_k_repack(blocks: np.ndarray, N: int, K: int) -> tuple[np.ndarray, np.ndarray]:
    """Host twin of afx_q6_k_repack: GGUF Q6_K super-blocks (210 B: ql[128], qh[64], int8 scales[16],
    fp16 d; element e = 128h + 32s + l has low bits nibble s >> 1 of ql[64h + 32(s & 1) + l] and high
    bits 2s..2s+1 of qh[32h + l], scale e // 16) -> (codes uint8 [N, K/2]: per 32-weight chunk, byte j
    of code dword k = low bits of elements 8k + j | 8k + 4 + j << 4; side int32 [N, K/32 * 3]: per
    chunk H0, H1 (byte j of H_p: high bits of elements 16p + j, +4, +8, +12 at bits 0, 2, 4, 6) and
    scale(0..15) | scale(16..31) << 8 | d << 16)."""
    if K % 256:
        raise ValueError(f"Q6_K rows need K % 256 == 0 (got {K})")
    b = np.ascontiguousarray(blocks, np.uint8).reshape(N, K // 256, 210)
    ql, qh = b[:, :, 0:128].astype(np.uint32), b[:, :, 128:192].astype(np.uint32)
    e = np.arange(256)
    h, s, l = e >> 7, (e >> 5) & 3, e & 31
    lo = (ql[:, :, 64 * h + 32 * (s & 1) + l] >> (4 * (s >> 1))) & 15           # [N, nb, 256]
    hi = (qh[:, :, 32 * h + l] >> (2 * s)) & 3
    lo = lo.reshape(N, K // 32, 4, 2, 4)                                        # [N, chunk, k, half, j]
    codes = (lo[:, :, :, 0, :] | (lo[:, :, :, 1, :] << 4)).astype(np.uint8).reshape(N, K // 2)
    hi = hi.reshape(N, K // 32, 2, 4, 4)                                        # [N, chunk, p, q, j]
    H = (hi[:, :, :, 0, :] | (hi[:, :, :, 1, :] << 2) | (hi[:, :, :, 2, :] << 4) | (hi[:, :, :, 3, :] << 6))
    H = (H << (8 * np.arange(4, dtype=np.uint32))).sum(-1).astype(np.uint32)   # [N, chunk, p]
    sc = b[:, :, 192:208].reshape(N, K // 32, 2).astype(np.uint32)              # two per chunk
    d = np.repeat(np.ascontiguousarray(b[:, :, 208:210]).view(np.uint16)[..., 0].astype(np.uint32), 8, axis=1)
    side = np.empty((N, K // 32, 3), np.uint32)
    side[..., 0:2] = H
    side[..., 2] = sc[..., 0] | (sc[..., 1] << 8) | (d << 16)
    return codes, side.reshape(N, -1).view(np.int32)
