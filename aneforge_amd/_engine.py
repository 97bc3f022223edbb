"""Device-resident decode engine: packed weights, per-layer executors, and the step graphs.

The reference builds a per-chunk ANE program per decode length and round-trips the hidden
state through the host for every chunk of every token (aneforge/llm.py:435-478, :584-606).
Here the whole step runs on the GPU:

  per layer:  afx_qkv_rope_kv   RMSNorm + fused [q|k|v] GEMV + RoPE + KV-cache row write
              afx_decode_attn   split-KV GQA attention over the resident cache (pos from device)
              afx_linear        o-proj GEMV + residual add (in place on h)
              afx_linear_swiglu RMSNorm + gate/up GEMV + SwiGLU
              afx_linear        down GEMV + residual add
  head:       afx_lm_head       final RMSNorm + fp16 lm_head -> fp32 logits + greedy-pick slots
  advance:    afx_decode_advance next token (prompt token, or the greedy pick with the reference's
                                 lm_head near-tie rule), pos/step, embedding

Position, step counter, prompt tokens and the generated-token history live in device memory,
so one step is captured once as a HIP graph and replayed for every token with no host sync.

Weights are packed once (compress=None -> fp16, "int8" -> per-row int8, "q4_0" -> GGUF Q4_0
in the superblock layout); the reference's other encodings ("blockwise", "int4" LUT) are
reconstructed exactly as the reference's constexpr ops would and streamed as fp16."""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from . import _blob, _cache, _hip
from . import _kernels as K

F16 = np.float16


# ----------------------------------------------------------------------------- packed weights
@dataclass
class Linear:
    """A weight [N, K] resident on the device in one of the kernel formats."""
    fmt: str                          # "int8" | "q4_0" | "fp16" | "blockwise" | "lut4" | "q4_k" | "q6_k"
    w: torch.Tensor
    scale: torch.Tensor | None
    N: int
    K: int
    bias: torch.Tensor | None = None

    @property
    def nbytes(self) -> int:
        n = self.w.numel() * self.w.element_size()
        if self.scale is not None:
            n += self.scale.numel() * self.scale.element_size()
        return n

    def __call__(self, x, y=None, residual=None, out_f32=False):
        return K.linear(self.fmt, self.w, self.scale, x, y=y, bias=self.bias, residual=residual, out_f32=out_f32)


@dataclass
class QuantizedWeight:
    """Weights that arrive already encoded (GGUF Q4_0 / Q8_0 bytes, int8 codes + row scales):
    packing keeps the codes bit-for-bit instead of round-tripping through float.
      fmt "int8":      codes int8 [N, K], scale fp16 [N]
      fmt "q4_0":      codes uint8 [N, K/2] superblock layout, scale fp16 [N, K/32]
      fmt "q4_0_gguf": codes uint8 [N, K/32*18] GGUF block bytes, scale None
      fmt "blockwise": codes int8 [N, K], scale fp16 [N, K/32] (GGUF Q8_0 blocks, K % 64 == 0)
      fmt "lut4":      codes uint8 [N, K/2] int4 indices (column 2j low nibble), scale fp16 [N, 16]:
                       each row's codebook, the palettize_lut4 codebook of its source tensor
      fmt "q4_k":      codes uint8 [N, K/2] GGUF Q4_K code bytes, scale int32 [N, K/256*5] super-block
                       headers ({d, dmin} + unpacked 6-bit scales/mins; _blob.q4_k_repack)
      fmt "q6_k":      codes uint8 [N, K/2] GGUF Q6_K low 4-bit parts by 32-weight chunk, scale int32
                       [N, K/32*3] side words (high 2-bit parts, scales, d; _blob.q6_k_repack)"""
    fmt: str
    codes: np.ndarray
    scale: np.ndarray | None
    shape: tuple

    def rows(self, idx) -> "QuantizedWeight":
        idx = np.asarray(idx)
        return QuantizedWeight(self.fmt, self.codes[idx], None if self.scale is None else self.scale[idx],
                               (len(idx), self.shape[1]))

    def to_superblock(self) -> "QuantizedWeight":
        if self.fmt != "q4_0_gguf":
            return self
        qs, d = _blob.q4_0_to_superblock(self.codes, *self.shape)
        return QuantizedWeight("q4_0", qs, d, self.shape)

    def dequant(self) -> np.ndarray:
        """Host fp32 reconstruction (exact: code * scale in fp32)."""
        N, Kd = self.shape
        if self.fmt == "int8":
            return self.codes.astype(np.float32) * self.scale.astype(np.float32)[:, None]
        if self.fmt == "blockwise":
            return (self.codes.reshape(N, Kd // 32, 32).astype(np.float32)
                    * self.scale.astype(np.float32)[:, :, None]).reshape(N, Kd)
        if self.fmt == "lut4":
            idx = np.empty((N, Kd), np.uint8)
            idx[:, 0::2], idx[:, 1::2] = self.codes & 15, self.codes >> 4
            return np.take_along_axis(self.scale.astype(np.float32), idx.astype(np.int64), axis=1)
        if self.fmt == "q6_k":
            side = np.ascontiguousarray(self.scale).view(np.uint32).reshape(N, Kd // 32, 3)
            c = self.codes.reshape(N, Kd // 32, 4, 4).astype(np.uint32)          # [N, chunk, k, j]
            lo = np.stack([c & 15, c >> 4], axis=3).reshape(N, Kd // 32, 32)     # element 8k + 4h + j
            H = (side[..., 0:2, None] >> (8 * np.arange(4, dtype=np.uint32))) & 255   # [N, chunk, p, j]
            hi = np.stack([(H >> (2 * q)) & 3 for q in range(4)], axis=3).reshape(N, Kd // 32, 32)
            sc = np.stack([side[..., 2] & 255, (side[..., 2] >> 8) & 255], -1).astype(np.uint8).view(np.int8)
            d = (side[..., 2] >> 16).astype(np.uint16).view(np.float16).astype(np.float32)
            ds = d[..., None] * sc.astype(np.float32)                            # [N, chunk, 2]
            q = (lo | (hi << 4)).astype(np.float32) - 32.0
            return (q.reshape(N, Kd // 32, 2, 16) * ds[..., None]).reshape(N, Kd)
        if self.fmt == "q4_k":
            h = np.ascontiguousarray(self.scale).view(np.uint32).reshape(N, Kd // 256, 5)
            dd = np.ascontiguousarray(h[..., 0]).view(np.float16).reshape(N, Kd // 256, 2).astype(np.float32)
            sm = ((h[..., 1:, None] >> (8 * np.arange(4, dtype=np.uint32))) & 255).astype(np.float32)  # [N,nb,p,4]
            ds = dd[..., 0, None, None] * sm[..., :2]          # [N, nb, pair, 2]: sub-blocks 2p, 2p+1
            dm = dd[..., 1, None, None] * sm[..., 2:]
            c = self.codes.reshape(N, Kd // 256, 4, 32)
            q = np.stack([c & 15, c >> 4], axis=3).astype(np.float32)      # [N, nb, pair, half, 32]
            return (ds[..., None] * q - dm[..., None]).reshape(N, Kd)
        q = self if self.fmt == "q4_0" else self.to_superblock()
        blocks = _blob.superblock_to_q4_0(q.codes, q.scale, N, Kd)
        codes, d = _blob.q4_0_codes(blocks, N, Kd)
        vals = codes.astype(np.float32) - 8.0
        return (vals.reshape(N, Kd // 32, 32) * d.astype(np.float32)[:, :, None]).reshape(N, Kd)


def _rows(W, idx):
    return W.rows(idx) if isinstance(W, QuantizedWeight) else np.asarray(W, np.float32)[np.asarray(idx)]


def _cat(parts):
    if all(isinstance(p, QuantizedWeight) for p in parts):
        ps = [p.to_superblock() for p in parts]
        if len({p.fmt for p in ps}) != 1:
            raise ValueError("cannot fuse weights of different encodings")
        sc = None if ps[0].scale is None else np.concatenate([p.scale for p in ps])
        return QuantizedWeight(ps[0].fmt, np.concatenate([p.codes for p in ps]), sc,
                               (sum(p.shape[0] for p in ps), ps[0].shape[1]))
    if any(isinstance(p, QuantizedWeight) for p in parts):
        raise ValueError("cannot fuse quantized and float weights")
    return np.concatenate([np.asarray(p, np.float32) for p in parts])


def _interleave(a, b):
    if isinstance(a, QuantizedWeight):
        a, b = a.to_superblock(), b.to_superblock()
        sc = None if a.scale is None else _blob.interleave_rows(a.scale, b.scale)
        return QuantizedWeight(a.fmt, _blob.interleave_rows(a.codes, b.codes), sc, (2 * a.shape[0], a.shape[1]))
    return _blob.interleave_rows(np.asarray(a, np.float32), np.asarray(b, np.float32))


def _shape(W):
    return W.shape if isinstance(W, QuantizedWeight) else np.asarray(W).shape


def _to_dev(a, dtype=None) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


def encode(W: np.ndarray, compress: str | None):
    """Host encoding of a float weight [N, K] -> (fmt, codes, scale) following `compress=`
    (aneforge/_compile.py:112-188: per-row int8; blockwise streams its int8 codes and 32-weight
    block scales; LUT4 is reconstructed to fp16).
    Already-encoded weights keep their codes."""
    if isinstance(W, QuantizedWeight):
        q = W.to_superblock()
        return q.fmt, q.codes, q.scale
    W = np.asarray(W, np.float32)
    if W.ndim != 2:
        raise ValueError(f"weights must be 2-D [out, in], got {W.shape}")
    if compress in (None, "fp16", "sparse"):
        return "fp16", W.astype(F16), None
    if compress in ("int8", "auto"):
        q, s = _cache.cached("quantize_per_row", _blob.quantize_per_row, W)
        return "int8", q, s
    if compress in ("q4_0", "gguf_q4_0"):
        N, Kd = W.shape
        if Kd % 128:
            raise ValueError(f"q4_0 needs in_features % 128 == 0 (got {Kd})")
        qs, d = _blob.q4_0_to_superblock(_cache.cached("quantize_q4_0", _blob.quantize_q4_0, W), N, Kd)
        return "q4_0", qs, d
    if compress == "blockwise":
        return blockwise_encoding(*_cache.cached("quantize_blockwise", _blob.quantize_blockwise, W, 32))
    if compress == "int4":
        return lut4_encoding(*_cache.cached("palettize_lut4", _blob.palettize_lut4, W), W.shape[1])
    raise ValueError(f"unknown compress={compress!r}")


def lut4_encoding(packed, cb, Kd):
    """palettize_lut4 output -> (fmt, codes, scale): the kernels' "lut4" format (the indices as
    they are, the codebook repeated per row) for K % 32 == 0, else the exact fp16 reconstruction."""
    N = packed.shape[0]
    if Kd % 32 == 0:
        return "lut4", np.ascontiguousarray(packed, np.uint8), np.tile(np.asarray(cb, F16).reshape(1, 16), (N, 1))
    idx = np.empty((N, packed.shape[1] * 2), np.uint8)
    idx[:, 0::2], idx[:, 1::2] = packed & 15, packed >> 4
    return "fp16", np.asarray(cb, np.float32)[idx[:, :Kd]].astype(F16), None


def per_tensor(W, compress):
    """A source weight about to be fused with others (q|k|v, gate|up, expert stacks): int4 is
    encoded here, per tensor, as the reference compresses each linear with its own codebook;
    the other encodings are per row or per block, so fusing before encoding is exact."""
    if compress != "int4" or isinstance(W, QuantizedWeight):
        return W
    W = np.asarray(W, np.float32)
    if W.shape[1] % 32:
        return W                                    # no lut4 kernel for this width: encoded after fusing
    packed, cb = _cache.cached("palettize_lut4", _blob.palettize_lut4, W)
    fmt, codes, scale = lut4_encoding(packed, cb, W.shape[1])
    return QuantizedWeight(fmt, codes, scale, W.shape)


def blockwise_encoding(q, s, bs):
    """quantize_blockwise output -> (fmt, codes, scale): the kernels' "blockwise" format (int8
    codes, fp16 scale [N, K/32]) for 32-weight blocks and K % 64 == 0, else the exact fp16
    reconstruction fp16(q * s) the reference's weights equal."""
    N, Kd = q.shape
    if bs == 32 and Kd % 64 == 0:
        return "blockwise", np.ascontiguousarray(q, np.int8), np.ascontiguousarray(s, F16)
    rec = (q.reshape(N, Kd // bs, bs).astype(np.float32) * s.astype(np.float32)[:, :, None]).reshape(N, Kd)
    return "fp16", rec.astype(F16), None


def pack_encoded(fmt, w, s, bias=None) -> Linear:
    N, Kd = w.shape[0], (w.shape[1] * 2 if fmt in ("q4_0", "lut4", "q4_k", "q6_k") else w.shape[1])
    return Linear(fmt, _to_dev(w), None if s is None else _to_dev(s), N, Kd,
                  None if bias is None else _to_dev(np.asarray(bias, np.float32).astype(F16)))


_GEMM_FMTS = ("int8", "fp16")                    # formats the prefill GEMM reads as packed


def prefill_gemm(eng, lin: "Linear", x, y, residual=None, epi="f16"):
    """The batched prefill's linear: afx_gemm on the packed weights (int8, fp16), or on the fp16
    expansion of the others in the engine's weight scratch (Q4_0, blockwise).  Prefill is
    compute-bound, so one expansion per matrix per prompt chunk costs little; for blockwise it
    measured faster than scaling the codes inside the GEMM (40.7 vs 48.2 ms for the 2048-token
    cfg3 prompt: the in-GEMM products lengthen its LDS-bound fragment path)."""
    if lin.fmt in _GEMM_FMTS:
        return K.gemm(lin.fmt, lin.w, lin.scale, x, y=y, bias=lin.bias, residual=residual, epi=epi)
    w16 = eng.weight_scratch(lin.N * lin.K).view(lin.N, lin.K)
    K.dequant_f16(lin.fmt, lin.w, lin.scale, lin.N, lin.K, out=w16)
    return K.gemm("fp16", w16, None, x, y=y, bias=lin.bias, residual=residual, epi=epi)


def _prefill_fmt_ok(lin: "Linear") -> bool:
    return lin.fmt in ("int8", "fp16", "q4_0", "blockwise", "lut4", "q4_k", "q6_k") and lin.K % 64 == 0 and lin.N % 16 == 0


def pack_linear(W, compress, bias=None) -> Linear:
    fmt, w, s = encode(W, compress)
    N, Kd = _shape(W)
    return Linear(fmt, _to_dev(w), None if s is None else _to_dev(s), N, Kd,
                  None if bias is None else _to_dev(np.asarray(bias, np.float32).astype(F16)))


def linear_from_q4_0_blocks(blocks, N: int, Kd: int, bias=None) -> Linear:
    """Device repack of GGUF Q4_0 bytes (kept 4-bit; the reference dequantised them on the host)."""
    b = _to_dev(np.asarray(blocks, np.uint8).reshape(N, -1))
    qs, d = K.q4_repack(b, N, Kd)
    return Linear("q4_0", qs, d, N, Kd, None if bias is None else _to_dev(np.asarray(bias, F16)))


def _gamma(g, D) -> torch.Tensor:
    g = np.asarray(g, np.float32).reshape(-1)
    if g.shape[0] != D:
        raise ValueError(f"norm weight has {g.shape[0]} entries, expected {D}")
    return _to_dev(g.astype(F16))


# ----------------------------------------------------------------------------- layer executors
class AttentionDecode:
    """Decode token mixer (aneforge/llm.py:214-237): RMSNorm -> QKV -> RoPE -> cache write ->
    GQA attention over positions [0, pos] -> o-proj + residual."""

    def __init__(self, lw: dict, cfg, ls, compress):
        if cfg.norm_type != "rms":
            raise NotImplementedError("the device decode engine implements RMSNorm decoders (norm_type='rms')")
        if cfg.rope and (cfg.rotary_dim not in (0, cfg.dh) or cfg.rope_interleaved):
            raise NotImplementedError("partial / interleaved RoPE is not fused on the device decode path yet")
        H, KV, dh, D = cfg.n_heads, cfg.n_kv_heads, cfg.dh, cfg.dim
        self.H, self.KV, self.dh, self.eps, self.rope = H, KV, dh, float(cfg.norm_eps), bool(cfg.rope)
        pq = _blob.rope_pair_order(H, dh) if self.rope else np.arange(H * dh)
        pk = _blob.rope_pair_order(KV, dh) if self.rope else np.arange(KV * dh)
        src = {k: per_tensor(lw[k], compress) for k in ("wq", "wk", "wv")}
        W = _cat([_rows(src["wq"], pq), _rows(src["wk"], pk), src["wv"]])
        bias = None
        if any(k in lw for k in ("q_bias", "k_bias", "v_bias")):
            bq = np.asarray(lw.get("q_bias", np.zeros(H * dh)), np.float32)
            bk = np.asarray(lw.get("k_bias", np.zeros(KV * dh)), np.float32)
            bv = np.asarray(lw.get("v_bias", np.zeros(KV * dh)), np.float32)
            bias = np.concatenate([bq[pq], bk[pk], bv])
        self.qkv = pack_linear(W, compress, bias)
        self.wo = pack_linear(lw["wo"], compress, lw.get("o_bias"))
        self.norm = _gamma(lw["attn_norm"], D)
        self.qk_norm = bool(ls.qk_norm)
        if self.qk_norm:
            self.q_norm, self.k_norm = _gamma(lw["q_norm"], dh), _gamma(lw["k_norm"], dh)
        self.kc = self.vc = None

    @classmethod
    def from_linears(cls, cfg, qkv: "Linear", wo: "Linear", norm: torch.Tensor, rope: bool = True):
        """Build from already-packed device weights (qkv rows in rope-pair order for q and k)."""
        self = cls.__new__(cls)
        self.H, self.KV, self.dh, self.eps, self.rope = cfg.n_heads, cfg.n_kv_heads, cfg.dh, float(cfg.norm_eps), rope
        self.qkv, self.wo, self.norm = qkv, wo, norm
        self.qk_norm = False
        self.kc = self.vc = None
        return self

    def bind(self, eng):
        shape = (eng.B, self.KV, eng.M, self.dh)
        self.kc = torch.zeros(shape, dtype=torch.float16, device="cuda")
        self.vc = torch.zeros(shape, dtype=torch.float16, device="cuda")

    def reset(self, eng):
        self.kc.zero_()
        self.vc.zero_()

    def state(self):
        return [self.kc, self.vc]

    def enqueue(self, eng):
        B, H, dh = eng.B, self.H, self.dh
        q = eng.q[:, :H * dh]
        K.qkv_rope_kv(self.qkv.fmt, self.qkv.w, self.qkv.scale, eng.h, self.norm, self.eps, self.qkv.bias,
                      H * dh, self.KV * dh, dh, eng.cos, eng.sin, eng.pos, q, self.kc, self.vc,
                      rope=self.rope and not self.qk_norm)
        if self.qk_norm:       # QK-norm sits between the projection and RoPE (Qwen3)
            K.head_norm_rope(q, H, dh, self.q_norm, self.eps, eng.cos, eng.sin, eng.pos, seq_stride=q.stride(0),
                             head_stride=dh, pos_mul=0, kv_len=eng.M, M=B, rope=self.rope)
            K.head_norm_rope(self.kc, self.KV, dh, self.k_norm, self.eps, eng.cos, eng.sin, eng.pos,
                             seq_stride=self.kc.stride(0), head_stride=self.kc.stride(1), pos_mul=dh,
                             kv_len=eng.M, M=B, rope=self.rope)
        K.decode_attn(q.view(B, H, dh), self.kc, self.vc, o=eng.a[:, :H * dh].view(B, H, dh), pos=eng.pos,
                      ws=eng.attn_ws)
        K.linear(self.wo.fmt, self.wo.w, self.wo.scale, eng.a[:, :H * dh], y=eng.h, bias=self.wo.bias,
                 residual=eng.h)

    def prefill_supported(self) -> bool:
        return self.dh == 128 and all(_prefill_fmt_ok(l) for l in (self.qkv, self.wo))

    def prefill(self, eng, X, pos0: int, bufs: dict):
        """Prompt rows X [m, D] at positions pos0.. (in place): RMSNorm -> [q|k|v] GEMM -> RoPE +
        cache rows -> causal GQA attention over the cache -> o-proj GEMM + residual."""
        m, H, KV, dh = X.shape[0], self.H, self.KV, self.dh
        hn = bufs["hn"][:m]
        K.rmsnorm(X, self.norm, self.eps, y=hn)
        qkv = bufs["qkv"][:m, :self.qkv.N]
        prefill_gemm(eng, self.qkv, hn, qkv)
        q = bufs["q"][:m, :H * dh]
        K.qkv_split_rope(qkv, H * dh, KV * dh, dh, eng.cos, eng.sin, pos0, q, self.kc[0], self.vc[0],
                         rope=self.rope and not self.qk_norm)
        if self.qk_norm:       # QK-norm sits between the projection and RoPE (Qwen3)
            pos = torch.arange(pos0, pos0 + m, dtype=torch.int32, device="cuda")
            K.head_norm_rope(q, H, dh, self.q_norm, self.eps, eng.cos, eng.sin, pos, seq_stride=q.stride(0),
                             head_stride=dh, pos_mul=0, kv_len=eng.M, M=m, rope=self.rope)
            K.head_norm_rope(self.kc[0], KV, dh, self.k_norm, self.eps, eng.cos, eng.sin, pos, seq_stride=0,
                             head_stride=self.kc.stride(1), pos_mul=dh, kv_len=eng.M, M=m, rope=self.rope)
        a = bufs["a"][:m, :H * dh]
        K.prefill_attn(q, self.kc[0], self.vc[0], a, pos0, H, KV)
        prefill_gemm(eng, self.wo, a, X, residual=X, epi="resid")

    @property
    def nbytes(self):
        return self.qkv.nbytes + self.wo.nbytes + self.norm.numel() * 2


class SwiGLUDecode:
    """SwiGLU MLP with residual (aneforge/llm.py:171-175): h + down(silu(gate(n)) * up(n)), n = rms(h)."""
    GELU = False                   # the gate's activation: silu (SwiGLU) or tanh-GELU (GeGLU)

    def __init__(self, lw: dict, cfg, ls, compress):
        D = cfg.dim
        self.F = _shape(lw["wgate"])[0]
        self.eps = float(cfg.norm_eps)
        self.gu = pack_linear(_interleave(per_tensor(lw["wgate"], compress), per_tensor(lw["wup"], compress)), compress)
        self.down = pack_linear(lw["wdown"], compress)
        self.norm = _gamma(lw["mlp_norm"], D)

    @classmethod
    def from_linears(cls, cfg, gu: "Linear", down: "Linear", norm: torch.Tensor):
        """Build from already-packed device weights (gate/up rows interleaved)."""
        self = cls.__new__(cls)
        self.F, self.eps, self.gu, self.down, self.norm = gu.N // 2, float(cfg.norm_eps), gu, down, norm
        return self

    def bind(self, eng):
        pass

    def reset(self, eng):
        pass

    def state(self):
        return []

    def enqueue(self, eng):
        act = eng.act[:, :self.F]
        K.linear_swiglu(self.gu.fmt, self.gu.w, self.gu.scale, eng.h, self.norm, self.eps, act=act, gelu=self.GELU)
        K.linear(self.down.fmt, self.down.w, self.down.scale, act, y=eng.h, residual=eng.h)

    def prefill_supported(self) -> bool:
        return all(_prefill_fmt_ok(l) for l in (self.gu, self.down))

    def prefill(self, eng, X, pos0: int, bufs: dict):
        """Prompt rows X [m, D] in place: RMSNorm -> gate/up GEMM + SwiGLU -> down GEMM + residual."""
        m = X.shape[0]
        hn = bufs["hn"][:m]
        K.rmsnorm(X, self.norm, self.eps, y=hn)
        act = bufs["act"][:m, :self.F]
        prefill_gemm(eng, self.gu, hn, act, epi="geglu" if self.GELU else "swiglu")
        prefill_gemm(eng, self.down, act, X, residual=X, epi="resid")

    @property
    def nbytes(self):
        return self.gu.nbytes + self.down.nbytes + self.norm.numel() * 2


class GeGLUDecode(SwiGLUDecode):
    """GeGLU MLP with residual, Gemma's (aneforge/llm.py:191-196): h + down(gelu_tanh(gate(n)) * up(n)),
    on the SwiGLU kernels with the tanh-GELU activation in the same epilogue."""
    GELU = True


# ----------------------------------------------------------------------------- the engine
class _Graph:
    def __init__(self, stream, fn):
        self.stream = stream
        self.exec = ctypes.c_void_p()
        with torch.cuda.stream(stream):
            _hip.call("afx_graph_begin", stream.cuda_stream)
            try:
                fn()
            finally:
                _hip.call("afx_graph_end", stream.cuda_stream, ctypes.byref(self.exec))

    def launch(self):
        _hip.call("afx_graph_launch", self.exec, self.stream.cuda_stream)

    def close(self):
        if self.exec:
            _hip.call("afx_graph_destroy", self.exec)
            self.exec = ctypes.c_void_p()


class DecodeEngine:
    """All layers + head + advance for one sequence (B=1) with a resident cache of M rows."""

    def __init__(self, cfg, layers, embed: torch.Tensor, head: Linear, final_norm: torch.Tensor, M: int,
                 rope_tables=None, head32: torch.Tensor | None = None, tie_margin: float | None = 3e-3):
        self.cfg, self.layers, self.embed, self.head, self.final_norm = cfg, layers, embed, head, final_norm
        self.M, self.B = int(M), 1
        D, H, dh = cfg.dim, cfg.n_heads, cfg.dh
        self.V = head.N
        dev = "cuda"
        self.h = torch.zeros((1, D), dtype=torch.float16, device=dev)
        self.q = torch.zeros((1, H * dh), dtype=torch.float16, device=dev)
        self.a = torch.zeros((1, H * dh), dtype=torch.float16, device=dev)
        fmax = max([getattr(m, "F", 0) for _, m in layers] + [8])
        self.act = torch.zeros((1, fmax), dtype=torch.float16, device=dev)
        self.logits = torch.zeros((1, self.V), dtype=torch.float32, device=dev)
        # lm_head greedy-pick slots, its normalised input row, and the near-tie rule's margin (a device
        # scalar, so a changed margin applies to already captured graphs); head32 holds the head in
        # fp32 when the checkpoint's values are not fp16-exact (the reference recomputes with them)
        self.slots = torch.zeros(((self.V + 7) // 8, 4), dtype=torch.float32, device=dev)
        self.hn = torch.zeros(D, dtype=torch.float16, device=dev)
        self.tie_margin = torch.zeros(1, dtype=torch.float32, device=dev)
        self.head32 = head32
        self.margin = tie_margin
        self._tie_on = tie_margin is not None and head.fmt == "fp16" and head.bias is None
        if self._tie_on:
            self.tie_margin.fill_(float(tie_margin))
        self.pos = torch.zeros(1, dtype=torch.int32, device=dev)
        self.tok = torch.zeros(1, dtype=torch.int32, device=dev)
        self.step = torch.zeros(1, dtype=torch.int32, device=dev)
        self.n_forced = torch.zeros(1, dtype=torch.int32, device=dev)
        self.hist = torch.zeros(self.M + 8, dtype=torch.int32, device=dev)
        self.forced = torch.zeros(self.M + 8, dtype=torch.int32, device=dev)
        # sampling: {temperature, top_p, top_k} and one uniform per step, both read on the device
        self.smp_params = torch.zeros(3, dtype=torch.float64, device=dev)
        self.uniforms = torch.zeros(self.M + 8, dtype=torch.float64, device=dev)
        self.smp_ws = torch.empty(K.sample_ws_elems(self.V), dtype=torch.float64, device=dev)
        if rope_tables is None:
            from .llm import rope_tables as _rt
            rope_tables = _rt(self.M, dh, cfg.rope_base, cfg.rotary_dim, cfg.rope_interleaved, cfg.rope_scaling)
        self.cos, self.sin = _to_dev(rope_tables[0]), _to_dev(rope_tables[1])
        self.attn_ws = torch.zeros(K.attn_ws_bytes(1, H, cfg.n_kv_heads, dh, self.M) // 4 + 1,
                                   dtype=torch.float32, device=dev)
        for mixer, mlp in layers:
            mixer.bind(self)
            mlp.bind(self)
        self.stream = torch.cuda.Stream()
        self._g_fwd = self._g_dec = self._g_smp = None

    # -- enqueue helpers (on the current stream) --
    def enqueue_layers(self):
        for mixer, mlp in self.layers:
            mixer.enqueue(self)
            mlp.enqueue(self)

    def enqueue_head(self):
        if self.head.fmt == "fp16" and self.head.bias is None:
            K.lm_head(self.head.w, self.h, self.final_norm, self.cfg.norm_eps, logits=self.logits, slots=self.slots,
                      hn=self.hn)
        else:
            K.linear_rms(self.head.fmt, self.head.w, self.head.scale, self.h, self.final_norm, self.cfg.norm_eps,
                         y=self.logits, bias=self.head.bias, out_f32=True)

    def set_tie_margin(self, margin: float | None):
        """The greedy near-tie margin (relative to max |logit|); None turns the recompute off."""
        was_on, self.margin = self._tie_on, margin
        self._tie_on = margin is not None and self.head.fmt == "fp16" and self.head.bias is None
        if self._tie_on:
            with torch.cuda.stream(self.stream):
                self.tie_margin.fill_(float(margin))
        if was_on != self._tie_on:                    # the captured steps change shape: capture again
            self.close()

    def enqueue_advance(self, with_logits: bool, gather: bool = True):
        """The step's token (forced, or the greedy pick) and bookkeeping; `gather` also writes the
        token's embedding row into h (otherwise enqueue_embed does it as a launch of its own)."""
        fused = with_logits and self.head.fmt == "fp16" and self.head.bias is None
        tie = fused and self._tie_on
        K.decode_advance(self.logits if with_logits else None, self.tok, self.pos, self.hist, self.step,
                         self.embed if gather else None, self.h, self.forced, self.n_forced,
                         slots=self.slots if fused else None, vocab=self.embed.shape[0],
                         tie_margin=self.tie_margin if tie else None, hn=self.hn if tie else None,
                         head16=self.head.w if tie and self.head32 is None else None,
                         head32=self.head32 if tie else None)

    def enqueue_embed(self, ids):
        """h = embed[ids[0]] (ids: a one-element int32 device tensor)."""
        K.embed(self.embed, ids, out=self.h)

    def enqueue_sample(self):
        """The step's token from the logits by the device sampler, queued as forced[step]."""
        K.sample(self.logits[0], self.smp_params, self.uniforms, step=self.step, forced=self.forced,
                 n_forced=self.n_forced, ws=self.smp_ws)

    def _graphs(self):
        if self._g_dec is None:
            self._g_fwd = _Graph(self.stream, lambda: (self.enqueue_layers(), self.enqueue_advance(False)))
            self._g_dec = _Graph(self.stream, lambda: (self.enqueue_layers(), self.enqueue_head(),
                                                      self.enqueue_advance(True)))
        return self._g_fwd, self._g_dec

    def set_sampling(self, temperature: float, top_p: float, top_k: int, uniforms, step0: int):
        """Sampling parameters and the uniforms of steps step0, step0 + 1, ... (one per token)."""
        u = np.asarray(uniforms, np.float64)
        if step0 + len(u) > self.uniforms.numel():
            raise ValueError("more sampled steps than the cache holds")
        with torch.cuda.stream(self.stream):
            self.smp_params.copy_(torch.tensor([float(temperature), float(top_p), float(top_k or 0)],
                                               dtype=torch.float64))
            if len(u):
                self.uniforms[step0:step0 + len(u)].copy_(torch.from_numpy(u))

    def run_sampled(self, n: int, graph: bool = True):
        """Enqueue n decode steps whose tokens come from the device sampler (no host sync)."""
        if graph:
            if self._g_smp is None:
                self._g_smp = _Graph(self.stream, lambda: (self.enqueue_layers(), self.enqueue_head(),
                                                          self.enqueue_sample(), self.enqueue_advance(False)))
            for _ in range(n):
                self._g_smp.launch()
        else:
            with torch.cuda.stream(self.stream):
                for _ in range(n):
                    self.enqueue_layers()
                    self.enqueue_head()
                    self.enqueue_sample()
                    self.enqueue_advance(False)

    # -- host control --
    def reset(self, prompt, pos0: int = 0, zero_state: bool = True):
        """Start a sequence: zero the resident state, queue prompt[1:] as forced tokens, h = embed[prompt[0]]."""
        prompt = [int(t) for t in prompt]
        if not prompt:
            raise ValueError("empty prompt")
        if len(prompt) + pos0 > self.M:
            raise ValueError(f"prompt of {len(prompt)} tokens does not fit the {self.M}-row cache")
        with torch.cuda.stream(self.stream):
            if zero_state:
                for mixer, mlp in self.layers:
                    mixer.reset(self)
                    mlp.reset(self)
            f = torch.tensor(prompt[1:] + [0], dtype=torch.int32)
            self.forced[:len(f)].copy_(f, non_blocking=False)
            self.n_forced.fill_(len(prompt) - 1)
            self.step.zero_()
            self.pos.fill_(pos0)
            K.embed(self.embed, torch.tensor(prompt[:1], dtype=torch.int32, device="cuda"), out=self.h)

    # -- batched prefill --
    def prefill_supported(self) -> bool:
        return all(getattr(m, "prefill_supported", lambda: False)() and getattr(p, "prefill_supported", lambda: False)()
                   for m, p in self.layers)

    def weight_scratch(self, n: int) -> torch.Tensor:
        """An fp16 buffer of at least n elements for prefill_gemm's weight expansion (reused by every
        layer in stream order)."""
        if getattr(self, "_w16", None) is None or self._w16.numel() < n:
            self._w16 = torch.empty(n, dtype=torch.float16, device="cuda")
        return self._w16[:n]

    def _prefill_buffers(self, C: int) -> dict:
        if getattr(self, "_pf", None) is None or self._pf["x"].shape[0] < C:
            cfg, dev = self.cfg, "cuda"
            nqkv = max([m.qkv.N for m, _ in self.layers] + [16])
            fmax = max([getattr(p, "F", 0) for _, p in self.layers] + [8])
            hq = cfg.n_heads * cfg.dh
            z = lambda c: torch.empty((C, c), dtype=torch.float16, device=dev)
            self._pf = {"x": z(cfg.dim), "hn": z(cfg.dim), "qkv": z(nqkv), "q": z(hq), "a": z(hq), "act": z(fmax)}
        return self._pf

    def prefill(self, prompt, chunk: int = 2048):
        """reset(prompt), then fill the cache for prompt[:-1] in one pass per layer (MFMA GEMMs and
        causal flash attention, `chunk` prompt rows at a time), leaving the engine where the
        len(prompt) - 1 forced steps of run() would: pos = step = n - 1, history = prompt[1:],
        h = embed[prompt[-1]].  Falls back to the forced steps when a layer has no batched path."""
        prompt = [int(t) for t in prompt]
        self.reset(prompt)
        n = len(prompt) - 1
        if n <= 0:
            return
        if not self.prefill_supported():
            self.run(n, 0)
            return
        C = max(1, min(int(chunk), n))
        bufs = self._prefill_buffers(C)
        with torch.cuda.stream(self.stream):
            ids = torch.tensor(prompt, dtype=torch.int32, device="cuda")
            for c0 in range(0, n, C):
                m = min(C, n - c0)
                X = bufs["x"][:m]
                K.embed(self.embed, ids[c0:c0 + m], out=X)
                for mixer, mlp in self.layers:
                    mixer.prefill(self, X, c0, bufs)
                    mlp.prefill(self, X, c0, bufs)
            self.hist[:n].copy_(ids[1:n + 1])
            self.pos.fill_(n)
            self.step.fill_(n)
            K.embed(self.embed, ids[n:n + 1], out=self.h)

    # -- speculative decoding: reposition, force, verify --
    def seek(self, pos: int, tok: int):
        """Make `tok` the pending input at position `pos`, keeping cache rows [0, pos); the next
        steps are greedy and record their tokens at hist[pos], hist[pos + 1], ..."""
        if not 0 <= pos < self.M:
            raise ValueError(f"seek: position {pos} outside the {self.M}-row cache")
        with torch.cuda.stream(self.stream):
            self.pos.fill_(pos)
            self.step.fill_(pos)
            self.n_forced.zero_()
            K.embed(self.embed, torch.tensor([int(tok)], dtype=torch.int32, device="cuda"), out=self.h)

    def force_next(self, step: int, tok: int):
        """The step with counter `step` (the pending one) emits `tok` instead of its argmax."""
        with torch.cuda.stream(self.stream):
            self.forced[step].fill_(int(tok))
            self.n_forced.fill_(step + 1)

    def verify(self, tokens, pos0: int) -> np.ndarray:
        """Greedy next token after each of `tokens`, fed at positions pos0, pos0 + 1, ...: their K/V
        rows overwrite the cache from pos0 on and row i attends to rows [0, pos0 + i].  Layers with a
        batched path run all rows at once (the prefill kernels); otherwise one forced step per row.
        Returns int64 [len(tokens)] (lowest index on ties); pos / step / h are left unspecified."""
        toks = [int(t) for t in tokens]
        n = len(toks)
        if n == 0 or pos0 < 0 or pos0 + n > self.M:
            raise ValueError(f"verify: {n} rows at position {pos0} do not fit the {self.M}-row cache")
        if getattr(self, "_vf", None) is None or self._vf["ids"].shape[0] < n:
            self._vf = {"ids": torch.empty(n, dtype=torch.int32, device="cuda"),
                        "hn": torch.empty((n, self.cfg.dim), dtype=torch.float16, device="cuda"),
                        "logits": torch.empty((n, self.V), dtype=torch.float32, device="cuda")}
        out = self._vf["ids"][:n]
        with torch.cuda.stream(self.stream):
            ids = torch.tensor(toks, dtype=torch.int32, device="cuda")
            if self.prefill_supported():
                bufs = self._prefill_buffers(n)
                X = bufs["x"][:n]
                K.embed(self.embed, ids, out=X)
                for mixer, mlp in self.layers:
                    mixer.prefill(self, X, pos0, bufs)
                    mlp.prefill(self, X, pos0, bufs)
                hn, lg = self._vf["hn"][:n], self._vf["logits"][:n]
                K.rmsnorm(X, self.final_norm, self.cfg.norm_eps, y=hn)
                K.linear(self.head.fmt, self.head.w, self.head.scale, hn, y=lg, out_f32=True)
                K.argmax(lg, out=out)
            else:
                self.pos.fill_(pos0)
                self.step.fill_(pos0)
                K.embed(self.embed, ids[:1], out=self.h)
                if n > 1:
                    self.forced[pos0:pos0 + n - 1].copy_(ids[1:])
                self.n_forced.fill_(pos0 + n - 1)
                for i in range(n):
                    self.enqueue_layers()
                    self.enqueue_head()
                    K.argmax(self.logits, out=out[i:i + 1])
                    if i + 1 < n:
                        self.enqueue_advance(False)
        self.sync()
        return out.cpu().numpy().astype(np.int64)

    def run(self, n_prefill: int, n_decode: int, graph: bool = True):
        """Enqueue n_prefill forced steps then n_decode greedy steps (no host sync)."""
        if graph:
            g_fwd, g_dec = self._graphs()
            for _ in range(n_prefill):
                g_fwd.launch()
            for _ in range(n_decode):
                g_dec.launch()
        else:
            with torch.cuda.stream(self.stream):
                for _ in range(n_prefill):
                    self.enqueue_layers()
                    self.enqueue_advance(False)
                for _ in range(n_decode):
                    self.enqueue_layers()
                    self.enqueue_head()
                    self.enqueue_advance(True)

    def sync(self):
        self.stream.synchronize()

    def history(self, start: int, count: int) -> list[int]:
        self.sync()
        return self.hist[start:start + count].cpu().tolist()

    def logits_host(self) -> np.ndarray:
        self.sync()
        return self.logits[0].cpu().numpy()

    def close(self):
        for g in (self._g_fwd, self._g_dec, self._g_smp):
            if g is not None:
                g.close()
        self._g_fwd = self._g_dec = self._g_smp = None

    @property
    def weight_bytes(self) -> int:
        return sum(m.nbytes + p.nbytes for m, p in self.layers) + self.head.nbytes
