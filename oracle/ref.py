"""CPU oracle for the quantized-decode path — TEST INFRASTRUCTURE ONLY.

This module is a numpy restatement of the reference's algorithms, used solely as the checker
by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.  The product
(aneforge_amd) never imports it, and nothing here runs on the GPU.

Every function cites the reference file:line it restates (paths relative to the
sbryngelson/ANEForge tree).  Where the reference computes in fp16 on the ANE, the oracle
computes in float64 and rounds to fp16 at the same op boundaries as the HIP kernels
(`r16`), so kernel-vs-oracle differences are accumulation-order noise only.  Passing
`exact=True` to the model-level functions disables the fp16 rounding entirely; that mode is
what the pinning tests compare against Hugging Face transformers and torch.

Pinning status (see tests/test_oracle.py):
  quantize_per_row, dequant_w8          pinned: closed form + KATs (half-even rounding)
  q4_0 pack/unpack/dequant, quantize     pinned: ggml spec KATs + brute-force loop
  dequant_q4_0_f16                      pinned: KAT (fp16 rounding of the fp32 product)
  quantize_blockwise                    pinned: closed form + reference property tests
  dequant_blockwise                     pinned: KAT (an fp16 round-half-even tie of the product)
  dequant_lut4                          pinned: KAT (hand-packed nibbles -> their codebook entries)
  dequant_q4_k(_f16), dequant_q6_k(_f16)  pinned: KATs (closed-form blocks) + element-by-element block encoders
  sample                                pinned: numpy's own RandomState.choice on the same draws, top-k /
                                        top-p support and frequency properties
  rms_norm                              pinned: torch + invariants
  rope_tables / rope / llama3 scaling    pinned: transformers' rope utilities + HF formula
  attention (sdpa / GQA decode)         pinned: torch SDPA, ctx=1 and equal-key cases
  topk_gate / moe_layer                 pinned: reference tie KAT + HF Qwen3-MoE block
  decoder step / generate               pinned: HF LlamaForCausalLM (tiny, fp32); with cfg mlp="geglu"
                                        and Gemma-baked weights, HF GemmaForCausalLM (tiny, fp64)
  gelu_tanh                             pinned: torch's gelu(approximate="tanh")
  cpu_decode_layer_f32 (timed baseline) pinned: decode_layer(exact=True) at a reduced GQA layer
  decode_rows                           pinned: n sequential decode_layer calls (dense and MoE layers)
  palettize_lut4 (aneforge_amd._blob)   pinned: vectors recorded from the reference function
                                        (tests/golden/make_lut4_vectors.py, lut4_vectors.npz)
"""
from __future__ import annotations

import numpy as np

f16 = np.float16


def r16(a, exact=False):
    """Round to fp16 (the kernels' output rounding) unless `exact`."""
    return np.asarray(a, np.float64) if exact else np.asarray(a).astype(f16).astype(np.float64)


# ----------------------------------------------------------------------------- int8 codec
def quantize_per_row(W):
    """Per-output-channel symmetric int8 (aneforge/_blob.py:20-25): scale = clip(max|W|/127,
    1e-8) in fp32, q = clip(round-half-even(W/scale), -127, 127); the scale is stored fp16
    while q used the fp32 scale.  Returns (q int8 [OUT,IN], s fp16 [OUT])."""
    W = np.asarray(W, np.float32)
    s32 = np.maximum(np.abs(W).max(axis=1, keepdims=True) / np.float32(127.0), np.float32(1e-8))
    q = np.clip(np.round(W / s32), -127, 127).astype(np.int8)
    return q, s32[:, 0].astype(f16)


def dequant_w8(q, s):
    """constexpr_affine_dequantize(axis=0, zero_point=0) (aneforge/_compile.py:171-179) taken
    in fp32: every int8 x fp16 product is exact in fp32 (<= 19 significant bits)."""
    return np.asarray(q, np.int8).astype(np.float32) * np.asarray(s, f16).astype(np.float32)[:, None]


def quantize_blockwise(W, block_size=32):
    """aneforge/_blob.py:46-56: int8 codes with one fp32->fp16 scale per [row, block]; the
    block size clamps down to a divisor of IN.  Returns (q int8 [OUT,IN], s fp16 [OUT,nb], bs)."""
    W = np.asarray(W, np.float32)
    OUT, IN = W.shape
    bs = int(block_size)
    while bs > 1 and IN % bs:
        bs -= 1
    Wb = W.reshape(OUT, IN // bs, bs)
    s = np.maximum(np.abs(Wb).max(axis=2) / np.float32(127.0), np.float32(1e-8))
    q = np.clip(np.round(Wb / s[:, :, None]), -127, 127).astype(np.int8).reshape(OUT, IN)
    return q, s.astype(f16), bs


def dequant_lut4(packed, codebooks, K):
    """The int4 palettization's reconstruction (aneforge/_blob.py:28-43 docstring): each column's
    fp16 codebook entry.  packed [N, ceil(K/2)] (column 2j in the low nibble of byte j),
    codebooks [N, 16] (one per row) or [16] (one for the tensor); returned as fp32."""
    packed = np.asarray(packed, np.uint8)
    idx = np.empty((packed.shape[0], packed.shape[1] * 2), np.int64)
    idx[:, 0::2], idx[:, 1::2] = packed & 15, packed >> 4
    cb = np.asarray(codebooks, f16).astype(np.float32)
    cb = np.broadcast_to(cb, (packed.shape[0], 16)) if cb.ndim == 1 else cb
    return np.take_along_axis(cb, idx[:, :K], axis=1)


def dequant_blockwise(q, s, bs=32):
    """The blockwise reconstruction data * scale (aneforge/_blob.py:46-56 docstring,
    constexpr_blockwise_shift_scale in aneforge/_compile.py:112-188) as fp16 weights: each
    int8 x fp16 product is exact in fp32 and rounded once to fp16."""
    q = np.asarray(q, np.int8)
    N, K = q.shape
    p = q.reshape(N, K // bs, bs).astype(np.float32) * np.asarray(s, f16).astype(np.float32)[:, :, None]
    return p.astype(f16).astype(np.float32).reshape(N, K)


# ----------------------------------------------------------------------------- Q4_0 codec
# ggml block_q4_0 (the format aneforge/_gguf.py:34-39 hands to gguf.quants.dequantize):
# 18 bytes = fp16 d, then 16 bytes qs; element i<16 = (qs[i] & 15) - 8, element i+16 =
# (qs[i] >> 4) - 8; value = element * d.
Q4_BLOCK = 32
Q4_BYTES = 18


def pack_q4_0(codes, d):
    """codes uint8 [N, K] in 0..15 (value = code - 8), d fp16 [N, K/32] -> bytes [N, K/32*18]."""
    codes = np.asarray(codes, np.uint8)
    N, K = codes.shape
    nb = K // Q4_BLOCK
    c = codes.reshape(N, nb, Q4_BLOCK)
    qs = (c[:, :, :16] & 15) | ((c[:, :, 16:] & 15) << 4)
    out = np.empty((N, nb, Q4_BYTES), np.uint8)
    out[:, :, :2] = np.asarray(d, f16).reshape(N, nb, 1).view(np.uint8).reshape(N, nb, 2)
    out[:, :, 2:] = qs
    return out.reshape(N, nb * Q4_BYTES)


def unpack_q4_0(blocks, N, K):
    """bytes [N, K/32*18] -> (codes uint8 [N, K], d fp16 [N, K/32])."""
    b = np.asarray(blocks, np.uint8).reshape(N, K // Q4_BLOCK, Q4_BYTES)
    d = b[:, :, :2].copy().view(f16).reshape(N, K // Q4_BLOCK)
    qs = b[:, :, 2:]
    codes = np.concatenate([qs & 15, qs >> 4], axis=2).reshape(N, K)
    return codes, d


def dequant_q4_0(blocks, N, K):
    """Q4_0 bytes -> fp32 weights [N, K]; (code-8)*d is exact in fp32."""
    codes, d = unpack_q4_0(blocks, N, K)
    vals = codes.astype(np.float32) - 8.0
    return (vals.reshape(N, K // Q4_BLOCK, Q4_BLOCK) * d.astype(np.float32)[:, :, None]).reshape(N, K)


def dequant_q4_0_f16(blocks, N, K):
    """The weights the reference multiplies with for a GGUF Q4_0 tensor: the ggml dequantisation
    (code-8)*d taken in fp32, then converted to float16 (GGUFView.get's default dtype,
    aneforge/_gguf.py:34-39).  Returned as fp32 holding those fp16 values."""
    return dequant_q4_0(blocks, N, K).astype(f16).astype(np.float32)


def dequant_q4_k(blocks):
    """GGUF Q4_K super-blocks uint8 [n, 144] -> fp32 weights [n, 256], the way gguf-py's Q4_K
    dequantiser evaluates ggml's block_q4_K (the reference calls it through GGUFView.get,
    aneforge/_gguf.py:34-39): fp16 d and dmin at bytes 0-3; a 12-byte field of 6-bit scales and
    mins (ggml get_scale_min_k4: sub-block j < 4 takes sc = b[j] & 63, m = b[j+4] & 63; j >= 4
    takes the low 4 bits from b[j+4] (sc low nibble, m high nibble) and the top 2 bits from bits
    6-7 of b[j-4] (sc) and b[j] (m)); 128 code bytes where byte 32c + l holds element 64c + l in
    its low nibble and 64c + 32 + l in its high nibble.  Weight = (d*sc) * q - (dmin*m), each step
    in float32."""
    b = np.asarray(blocks, np.uint8).reshape(-1, 144)
    out = np.empty((b.shape[0], 256), np.float32)
    d = b[:, 0:2].copy().view(f16).astype(np.float32)[:, 0]
    dmin = b[:, 2:4].copy().view(f16).astype(np.float32)[:, 0]
    f = b[:, 4:16].astype(np.int64)
    for j in range(8):
        if j < 4:
            sc, m = f[:, j] & 63, f[:, j + 4] & 63
        else:
            sc = (f[:, j + 4] & 15) | ((f[:, j - 4] >> 6) << 4)
            m = (f[:, j + 4] >> 4) | ((f[:, j] >> 6) << 4)
        c, h = j // 2, j % 2
        q = ((b[:, 16 + 32 * c:16 + 32 * c + 32] >> (4 * h)) & 15).astype(np.float32)
        dl = (d * sc.astype(np.float32)).astype(np.float32)
        ml = (dmin * m.astype(np.float32)).astype(np.float32)
        out[:, 32 * j:32 * j + 32] = dl[:, None] * q - ml[:, None]
    return out


def dequant_q6_k(blocks):
    """GGUF Q6_K super-blocks uint8 [n, 210] -> fp32 weights [n, 256], as gguf-py's Q6_K dequantiser
    evaluates ggml's block_q6_K (the reference calls it through GGUFView.get, aneforge/_gguf.py:34-39):
    ql[128] at byte 0, qh[64] at 128, int8 scales[16] at 192, fp16 d at 208.  ggml's loop over the
    two 128-weight halves h and l < 32: element 128h + l = (ql[64h + l] & 15) | ((qh[32h + l] >> 0) & 3)
    << 4, element + 32 = (ql[64h + 32 + l] & 15) | ((qh >> 2) & 3) << 4, element + 64 = (ql[64h + l] >> 4)
    | ((qh >> 4) & 3) << 4, element + 96 = (ql[64h + 32 + l] >> 4) | ((qh >> 6) & 3) << 4; weight =
    (d * scale[e // 16]) * (q - 32) in float32."""
    b = np.asarray(blocks, np.uint8).reshape(-1, 210)
    n = b.shape[0]
    q = np.empty((n, 256), np.int64)
    for h in range(2):
        ql, qh = b[:, 64 * h:64 * h + 64].astype(np.int64), b[:, 128 + 32 * h:128 + 32 * h + 32].astype(np.int64)
        q[:, 128 * h + 0:128 * h + 32] = (ql[:, :32] & 15) | ((qh & 3) << 4)
        q[:, 128 * h + 32:128 * h + 64] = (ql[:, 32:] & 15) | (((qh >> 2) & 3) << 4)
        q[:, 128 * h + 64:128 * h + 96] = (ql[:, :32] >> 4) | (((qh >> 4) & 3) << 4)
        q[:, 128 * h + 96:128 * h + 128] = (ql[:, 32:] >> 4) | (((qh >> 6) & 3) << 4)
    sc = b[:, 192:208].copy().view(np.int8).astype(np.float32)
    d = b[:, 208:210].copy().view(f16).astype(np.float32)[:, 0]
    dl = (d[:, None] * sc).astype(np.float32)                      # [n, 16]
    return (np.repeat(dl, 16, axis=1) * (q - 32).astype(np.float32)).astype(np.float32)


def dequant_q6_k_f16(blocks, N, K):
    """A GGUF Q6_K tensor [N, K] as the fp16 weights the reference multiplies with, as fp32 values."""
    return dequant_q6_k(blocks).reshape(N, K).astype(f16).astype(np.float32)


def dequant_q4_k_f16(blocks, N, K):
    """A GGUF Q4_K tensor [N, K] as the fp16 weights the reference multiplies with (GGUFView.get's
    fp16 cast of the float32 dequantisation), returned as fp32 holding those fp16 values."""
    return dequant_q4_k(blocks).reshape(N, K).astype(f16).astype(np.float32)


def quantize_q4_0(W):
    """ggml's reference Q4_0 quantizer (quantize_row_q4_0_ref): per block, m = the element of
    largest magnitude (signed), d = m / -8, code = min(15, trunc(x/d + 8.5)).  -> bytes."""
    W = np.asarray(W, np.float32)
    N, K = W.shape
    Wb = W.reshape(N, K // Q4_BLOCK, Q4_BLOCK)
    idx = np.abs(Wb).argmax(axis=2)
    m = np.take_along_axis(Wb, idx[:, :, None], axis=2)[:, :, 0]
    d = m / np.float32(-8.0)
    inv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, 1), np.float32(0.0)).astype(np.float32)
    codes = np.minimum(15, np.trunc(Wb * inv[:, :, None] + np.float32(8.5))).astype(np.int32)
    codes = np.clip(codes, 0, 15).astype(np.uint8).reshape(N, K)
    return pack_q4_0(codes, d.astype(f16))


# ----------------------------------------------------------------------------- linear layers
def linear(x16, Wf32, bias=None, exact=False):
    """y = x @ W^T (+ bias) in float64 from fp16 x, rounded to fp16 (aneforge/graph.py:187-195,
    aneforge/_compile.py:375-385; the kernel accumulates in fp32)."""
    y = np.asarray(x16, np.float64) @ np.asarray(Wf32, np.float64).T
    if bias is not None:
        y = y + np.asarray(bias, np.float64)
    return r16(y, exact)


# ----------------------------------------------------------------------------- norms / rope
def rms_norm(x, g, eps=1e-5, exact=False):
    """Textbook RMSNorm x / sqrt(mean(x^2) + eps) * g, as in the reference's numpy oracles
    (tests/test_moe.py:26, bench/decode_measurement.py:92-94); the device lowering
    (aneforge/_compile.py:738-755) agrees to within eps/mean(x^2)."""
    x = np.asarray(x, np.float64)
    ms = (x * x).mean(-1, keepdims=True)
    return r16(x / np.sqrt(ms + eps) * np.asarray(g, np.float64), exact)


def llama3_rope_scale(inv, s):
    """Llama-3.1 inv_freq rescaling (aneforge/llm.py:62-73)."""
    factor, lo, hi = float(s["factor"]), float(s["low_freq_factor"]), float(s["high_freq_factor"])
    old = float(s["original_max_position_embeddings"])
    low_wl, high_wl = old / lo, old / hi
    wl = 2.0 * np.pi / inv
    scaled = np.where(wl > low_wl, inv / factor, inv)
    smooth = (old / wl - lo) / (hi - lo)
    blended = (1.0 - smooth) * scaled / factor + smooth * scaled
    return np.where((wl >= high_wl) & (wl <= low_wl), blended, scaled)


def rope_tables(seq, dh, base=10000.0, rotary_dim=0, interleaved=False, scaling=None):
    """[seq, dh] cos/sin tables in float64, cast to fp16 (aneforge/llm.py:76-93)."""
    rd = rotary_dim or dh
    inv = 1.0 / (base ** (np.arange(0, rd, 2) / rd))
    if scaling and scaling.get("rope_type") == "llama3":
        inv = llama3_rope_scale(inv, scaling)
    ang = np.arange(seq)[:, None] * inv[None, :]
    if interleaved:
        c, s = np.repeat(np.cos(ang), 2, axis=1), np.repeat(np.sin(ang), 2, axis=1)
    else:
        c, s = np.cos(np.concatenate([ang, ang], -1)), np.sin(np.concatenate([ang, ang], -1))
    if rd < dh:
        c = np.concatenate([c, np.ones((seq, dh - rd))], 1)
        s = np.concatenate([s, np.zeros((seq, dh - rd))], 1)
    return c.astype(f16), s.astype(f16)


def rope(x, cos, sin, exact=False):
    """x*cos + rotate_half(x)*sin over the last axis (aneforge/llm.py:96-105, neox layout)."""
    x = np.asarray(x, np.float64)
    h = x.shape[-1] // 2
    rot = np.concatenate([-x[..., h:], x[..., :h]], -1)
    return r16(x * np.asarray(cos, np.float64) + rot * np.asarray(sin, np.float64), exact)


# ----------------------------------------------------------------------------- attention
def attention(q, K, V, scale=None, lengths=None, mask=None, exact=False):
    """softmax(q K^T * scale (+ mask)) V with fp32-or-better softmax and an fp16 result
    (aneforge/_bridges/ane_sdpa_fused.py:57-68).  GQA: query head h reads kv head h // G
    (aneforge/llm.py:205-211).  q [B, Hq, Sq, D]; K/V [B, Hkv, L, D]; `lengths[b]` limits the
    keys of batch b to [0, lengths[b]) (the -1e4 position mask of aneforge/llm.py:584-588)."""
    q = np.asarray(q, np.float64)
    K = np.asarray(K, np.float64)
    V = np.asarray(V, np.float64)
    B, Hq, Sq, D = q.shape
    Hkv = K.shape[1]
    G = Hq // Hkv
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    out = np.zeros((B, Hq, Sq, D))
    for b in range(B):
        L = K.shape[2] if lengths is None else int(lengths[b])
        for h in range(Hq):
            s = q[b, h] @ K[b, h // G, :L].T * scale           # [Sq, L]
            if mask is not None:
                s = s + np.asarray(mask, np.float64)[..., :L].reshape(-1, L)[: Sq]
            s = s - s.max(-1, keepdims=True)
            p = np.exp(s)
            p = p / p.sum(-1, keepdims=True)
            out[b, h] = p @ V[b, h // G, :L]
    return r16(out, exact)


def silu(x):
    x = np.asarray(x, np.float64)
    return x / (1.0 + np.exp(-x))


def gelu_tanh(x):
    """The tanh-approximated GELU, 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))): the reference's
    _gelu_tanh (aneforge/llm.py:185-189), Gemma's gelu_pytorch_tanh."""
    x = np.asarray(x, np.float64)
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


def glu_act(cfg):
    """The gated MLP's gate activation: silu for SwiGLU (aneforge/llm.py:171-175), tanh-GELU for the
    GeGLU of Gemma (cfg["mlp"] == "geglu", aneforge/llm.py:191-196)."""
    return gelu_tanh if cfg.get("mlp", "swiglu") == "geglu" else silu


# ----------------------------------------------------------------------------- MoE
def topk_gate(probs16, k):
    """aneforge/moe.py:21-37: k rounds of row max with the LOWEST index among exact ties;
    exactly k experts per row; returns probs masked to the chosen experts.  Bounds
    1 <= k <= E <= 2049 else ValueError (moe.py:27-28)."""
    p = np.asarray(probs16, np.float64)
    T, E = p.shape
    if not 1 <= k <= E <= 2049:
        raise ValueError(f"moe top-k: need 1 <= k <= E <= 2049; got k={k}, E={E}")
    out = np.zeros_like(p)
    for t in range(T):
        rem = p[t].copy()
        for _ in range(k):
            j = int(np.flatnonzero(rem == rem.max())[0])
            out[t, j] = p[t, j]
            rem[j] = -np.inf
    return out


def moe_route(hn16, router, k, renorm=True, exact=False):
    """Router: softmax(hn R^T) over experts (fp32+), probabilities taken at fp16 (the
    reference's fp16 tie semantics), top-k, optional renorm (aneforge/moe.py:53-56).
    Returns (gate [T, E] with zeros off the top-k, chosen index sets)."""
    lg = np.asarray(hn16, np.float64) @ np.asarray(router, np.float64).T
    p = np.exp(lg - lg.max(-1, keepdims=True))
    p = p / p.sum(-1, keepdims=True)
    if not exact:
        p = p.astype(f16).astype(np.float64)          # the reference's fp16 tie semantics
    g = topk_gate(p, k)
    if renorm:
        g = g / g.sum(1, keepdims=True)
    chosen = [sorted(np.flatnonzero(g[t]).tolist()) for t in range(g.shape[0])]
    return g, chosen


def moe_layer(h16, mlp_norm, router, Wg, Wu, Wd, k, renorm=True, eps=1e-5, exact=False):
    """MoE SwiGLU MLP with residual (aneforge/moe.py:48-63), active experts only (identical to
    the dense all-expert sum because unselected experts carry weight 0).  Wg/Wu [E, F, D] and
    Wd [E, D, F] as dequantised fp32; rounding points follow the HIP kernels:
    act = fp16(silu(fp16 g) * fp16 u), y_e = fp16(act Wd_e^T), out = fp16(h + fp16(sum g*y)).
    Each active expert's weights are taken to float64 once, for all the tokens routed to it; the
    per-token sum runs over its experts in ascending index order."""
    h = np.asarray(h16, np.float64)
    hn = rms_norm(h, mlp_norm, eps, exact)
    gate, chosen = moe_route(hn, router, k, renorm, exact)
    T, D = h.shape
    ys = {}
    for e in sorted({e for c in chosen for e in c}):
        rows = [t for t in range(T) if e in chosen[t]]
        x = hn[rows]
        g = r16(x @ np.asarray(Wg[e], np.float64).T, exact)
        u = r16(x @ np.asarray(Wu[e], np.float64).T, exact)
        a = r16(silu(g) * u, exact)
        y = r16(a @ np.asarray(Wd[e], np.float64).T, exact)
        for i, t in enumerate(rows):
            ys[t, e] = y[i]
    comb = np.zeros((T, D))
    for t in range(T):
        for e in chosen[t]:
            comb[t] += gate[t, e] * ys[t, e]
    return r16(h + r16(comb, exact), exact), gate, chosen


# ----------------------------------------------------------------------------- decoder
def decode_layer(h16, w, cfg, K, V, pos, cos_row, sin_row, exact=False, trace=None):
    """One pre-norm decoder layer for one token at position `pos` against a resident cache
    (aneforge/llm.py:214-237 `_attn_decode` + :171-175 `_swiglu`).  w holds dequantised
    fp32 weights: wq [H*dh, D], wk/wv [KV*dh, D], wo [D, H*dh], wgate/wup [F, D], wdown [D, F],
    attn_norm/mlp_norm [D], optional q_bias/k_bias/v_bias/o_bias.  K/V [KV, M, dh] are
    updated in place at row pos.  Returns the new hidden [1, D]."""
    H, KV, dh, eps = cfg["n_heads"], cfg["n_kv_heads"], cfg["dh"], cfg["norm_eps"]
    h = np.asarray(h16, np.float64).reshape(1, -1)
    xn = rms_norm(h, w["attn_norm"], eps, exact)
    q = linear(xn, w["wq"], w.get("q_bias"), exact).reshape(H, dh)
    k = linear(xn, w["wk"], w.get("k_bias"), exact).reshape(KV, dh)
    v = linear(xn, w["wv"], w.get("v_bias"), exact).reshape(KV, dh)
    if "q_norm" in w:
        q = rms_norm(q, w["q_norm"], eps, exact)
        k = rms_norm(k, w["k_norm"], eps, exact)
    if cfg.get("rope", True):
        q = rope(q, cos_row, sin_row, exact)
        k = rope(k, cos_row, sin_row, exact)
    K[:, pos] = k
    V[:, pos] = v
    a = attention(q[None, :, None, :], K[None], V[None], 1.0 / np.sqrt(dh), [pos + 1], exact=exact)
    a = a.reshape(1, H * dh)
    h1 = r16(h + linear(a, w["wo"], w.get("o_bias"), exact), exact)
    if "router" in w:                     # MoE MLP (aneforge/moe.py:48-63), experts as dequantised fp32
        out, _, _ = moe_layer(h1, w["mlp_norm"], w["router"], w["wgate_exps"], w["wup_exps"], w["wdown_exps"],
                              cfg["top_k"], cfg.get("norm_topk_prob", True), eps, exact)
        if trace is not None:
            trace.append(out.copy())
        return out
    hn = rms_norm(h1, w["mlp_norm"], eps, exact)
    g = linear(hn, w["wgate"], None, exact)
    u = linear(hn, w["wup"], None, exact)
    act = r16(glu_act(cfg)(g) * u, exact)
    out = r16(h1 + linear(act, w["wdown"], None, exact), exact)
    if trace is not None:
        trace.append(out.copy())
    return out


def decode_rows(h16, w, cfg, K, V, pos0, cos, sin, exact=False):
    """decode_layer for n consecutive tokens at positions pos0 .. pos0 + n - 1 in one pass over
    the layer's weights (teacher forcing: the n input hidden rows are given).  Row t writes cache
    row pos0 + t and attends to rows [0, pos0 + t], so the result is that of n decode_layer calls
    in order (aneforge/llm.py:214-237, :171-175).  cos/sin are the full [M, dh] tables; K/V
    [KV, M, dh] are updated in place.  Returns the new hidden rows [n, D]."""
    H, KV, dh, eps = cfg["n_heads"], cfg["n_kv_heads"], cfg["dh"], cfg["norm_eps"]
    h = np.asarray(h16, np.float64)
    n = h.shape[0]
    xn = rms_norm(h, w["attn_norm"], eps, exact)
    q = linear(xn, w["wq"], w.get("q_bias"), exact).reshape(n, H, dh)
    k = linear(xn, w["wk"], w.get("k_bias"), exact).reshape(n, KV, dh)
    v = linear(xn, w["wv"], w.get("v_bias"), exact).reshape(n, KV, dh)
    if "q_norm" in w:
        q = rms_norm(q, w["q_norm"], eps, exact)
        k = rms_norm(k, w["k_norm"], eps, exact)
    if cfg.get("rope", True):
        c = np.asarray(cos)[pos0:pos0 + n, None, :]
        s = np.asarray(sin)[pos0:pos0 + n, None, :]
        q = rope(q, c, s, exact)
        k = rope(k, c, s, exact)
    K[:, pos0:pos0 + n] = k.transpose(1, 0, 2)
    V[:, pos0:pos0 + n] = v.transpose(1, 0, 2)
    Kb = np.broadcast_to(K, (n,) + K.shape)
    Vb = np.broadcast_to(V, (n,) + V.shape)
    a = attention(q[:, :, None, :], Kb, Vb, 1.0 / np.sqrt(dh), pos0 + 1 + np.arange(n), exact=exact)
    a = a.reshape(n, H * dh)
    h1 = r16(h + linear(a, w["wo"], w.get("o_bias"), exact), exact)
    if "router" in w:
        out, _, _ = moe_layer(h1, w["mlp_norm"], w["router"], w["wgate_exps"], w["wup_exps"], w["wdown_exps"],
                              cfg["top_k"], cfg.get("norm_topk_prob", True), eps, exact)
        return out
    hn = rms_norm(h1, w["mlp_norm"], eps, exact)
    g = linear(hn, w["wgate"], None, exact)
    u = linear(hn, w["wup"], None, exact)
    act = r16(glu_act(cfg)(g) * u, exact)
    return r16(h1 + linear(act, w["wdown"], None, exact), exact)


def logits(h16, final_norm, lm_head, eps=1e-5, exact=False):
    """Final RMSNorm then the fp16 lm_head, logits kept in float64 (aneforge/llm.py:395-404).
    One row of logits per hidden row: [n, vocab]."""
    hn = rms_norm(h16, final_norm, eps, exact)
    lm = np.asarray(lm_head, np.float64)
    return np.asarray(hn, np.float64).reshape(-1, lm.shape[1]) @ lm.T


def decode_step(tok, pos, W, cfg, caches, tables, exact=False, trace=None):
    """Embedding gather -> all layers -> final norm -> lm_head logits [vocab]."""
    cos, sin = tables
    h = np.asarray(W["embed"][tok], np.float64).reshape(1, -1)
    h = r16(h, exact)
    for li, lw in enumerate(W["layers"]):
        K, V = caches[li]
        h = decode_layer(h, lw, cfg, K, V, pos, cos[pos], sin[pos], exact, trace)
    return logits(h, W["final_norm"], W["lm_head"], cfg["norm_eps"], exact)[0]


def sample(logits, temperature, top_p, top_k, u):
    """LlamaPrefill._sample (aneforge/llm.py:406-419) with np.random.choice's uniform given as u:
    argmax when temperature <= 0; else lg = logits / T in float64, the logits below the k-th largest
    set to -inf, p = exp(lg - max) / sum, the top-p nucleus (sorted descending, the prefix whose
    cumulative sum first reaches top_p, renormalised), then numpy's legacy choice(n, p=p): cdf =
    cumsum(p) / cdf[-1], the token is searchsorted(cdf, u, 'right').  Ties in the nucleus sort are
    ordered by a stable argsort (the highest index first after the reversal)."""
    if temperature <= 0.0:
        return int(np.argmax(logits))
    lg = np.asarray(logits, np.float32).astype(np.float64) / temperature
    if top_k and 0 < top_k < lg.size:
        lg[lg < np.partition(lg, -top_k)[-top_k]] = -np.inf
    p = np.exp(lg - lg.max())
    p /= p.sum()
    if 0.0 < top_p < 1.0:
        order = np.argsort(p, kind="stable")[::-1]
        cum = np.cumsum(p[order])
        keep = order[:int(np.searchsorted(cum, top_p)) + 1]
        m = np.zeros_like(p)
        m[keep] = p[keep]
        p = m / m.sum()
    cdf = np.cumsum(p)
    cdf /= cdf[-1]
    return int(np.searchsorted(cdf, u, side="right"))


def generate(prompt, n_new, W, cfg, M, exact=False, caches=None, start_pos=None):
    """Greedy token-by-token generation with a resident cache (restates the decode loop of
    aneforge/llm.py:560-633 with batched_prefill=False, and examples/gpt_multilayer_resident.py:75-101).
    Returns (tokens, list of logits per generated token)."""
    dh = cfg["dh"]
    tables = rope_tables(M, dh, cfg.get("rope_base", 10000.0), scaling=cfg.get("rope_scaling"))
    if caches is None:
        caches = [(np.zeros((cfg["n_kv_heads"], M, dh)), np.zeros((cfg["n_kv_heads"], M, dh)))
                  for _ in W["layers"]]
    p0 = 0 if start_pos is None else start_pos
    for i, tok in enumerate(prompt[:-1]):
        decode_step(tok, p0 + i, W, cfg, caches, tables, exact)
    cur, pos = prompt[-1], p0 + len(prompt) - 1
    out, all_logits = [], []
    for _ in range(n_new):
        lg = decode_step(cur, pos, W, cfg, caches, tables, exact)
        nxt = int(np.argmax(lg))
        out.append(nxt)
        all_logits.append(lg)
        cur, pos = nxt, pos + 1
    return out, all_logits


# ----------------------------------------------------------------------------- CPU baseline
def cpu_decode_layer_f32(h, w, cfg, K, V, pos, cos_row, sin_row):
    """The reference's CPU decode path in fp32 (bench/decode_measurement.py:86-132 `ref_decode`,
    extended with GQA and RoPE as in aneforge/llm.py:214-237): numpy matmuls on weights already
    dequantised to fp32, attention over the cache plus the new row, SwiGLU, residuals.  Used
    only as the timed CPU baseline; parity checks use decode_layer."""
    H, KV, dh, eps = cfg["n_heads"], cfg["n_kv_heads"], cfg["dh"], cfg["norm_eps"]
    f32 = np.float32

    def rms(x, g):
        return (x / np.sqrt((x * x).mean(-1, keepdims=True) + f32(eps))) * g

    def rot(x):
        half = x.shape[-1] // 2
        return x * cos_row + np.concatenate([-x[..., half:], x[..., :half]], -1) * sin_row

    xn = rms(h, w["attn_norm"])
    q = rot((xn @ w["wq"].T).reshape(H, dh))
    k = rot((xn @ w["wk"].T).reshape(KV, dh))
    v = (xn @ w["wv"].T).reshape(KV, dh)
    K[:, pos] = k
    V[:, pos] = v
    G = H // KV
    out = np.empty((H, dh), f32)
    for g in range(KV):
        s = (q[g * G:(g + 1) * G] @ K[g, :pos + 1].T) * f32(1.0 / np.sqrt(dh))
        s = np.exp(s - s.max(-1, keepdims=True))
        out[g * G:(g + 1) * G] = (s / s.sum(-1, keepdims=True)) @ V[g, :pos + 1]
    h = h + out.reshape(1, H * dh) @ w["wo"].T
    fn = rms(h, w["mlp_norm"])
    gg = fn @ w["wgate"].T
    return h + ((gg / (1 + np.exp(-gg))) * (fn @ w["wup"].T)) @ w["wdown"].T
