"""Seeded synthetic inputs for the benchmark configurations of the quantized-decode path
(numpy default_rng, the generator family the reference's tests use, tests/_helpers.py:10-15).

  cfg0  int8 per-channel GEMV 4096x4096, B=1
  cfg1  GGUF Q4_0 GEMV [11008x4096] / [4096x11008], B in {1, 4, 8}
  cfg2  decode attention Hq 32 / Hkv 8 / D 128, ctx in {512, 2048, 8192}, B in {1, 16}
  cfg3  32-layer Llama-style int8 decode (d 4096, 32/8 heads, FFN 11008, vocab 32000)
  cfg4  MoE layer: 8 experts, top-2, Q4_0 experts (FFN 14336), 16 tokens

Arrays are drawn in the documented order so every consumer (tests, bench) sees the same
values.  The full cfg3 model (5.7 GB of int8) is generated directly on the device by
`cfg3_device_model`, because drawing it on the host would dominate the benchmark setup."""
from __future__ import annotations

import numpy as np

F16 = np.float16


def cfg0_gemv_w8(seed: int = 0, N: int = 4096, K: int = 4096, B: int = 1):
    rng = np.random.default_rng(seed)
    q = rng.integers(-127, 128, (N, K), dtype=np.int8)
    s = (np.abs(rng.normal(0, 0.02, N)) / 127).astype(F16)
    x = rng.standard_normal((B, K)).astype(F16)
    return {"q": q, "s": s, "x": x}


def q4_blocks_from_codes(codes: np.ndarray, d: np.ndarray) -> np.ndarray:
    """codes uint8 [N, K] (0..15), d fp16 [N, K/32] -> GGUF Q4_0 bytes [N, K/32*18]."""
    N, K = codes.shape
    c = codes.reshape(N, K // 32, 32)
    out = np.empty((N, K // 32, 18), np.uint8)
    out[:, :, 0:2] = np.asarray(d, F16).reshape(N, K // 32, 1).view(np.uint8)
    out[:, :, 2:] = (c[:, :, :16] & 15) | ((c[:, :, 16:] & 15) << 4)
    return out.reshape(N, -1)


def cfg1_gemv_q4(N: int = 11008, K: int = 4096, B: int = 1, seed: int = 1):
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 16, (N, K), dtype=np.uint8)
    d = (np.abs(rng.normal(0, 0.02, (N, K // 32))) / 8).astype(F16)
    x = rng.standard_normal((B, K)).astype(F16)
    return {"blocks": q4_blocks_from_codes(codes, d), "x": x, "N": N, "K": K}


def cfg2_attn(ctx: int = 2048, B: int = 1, Hq: int = 32, Hkv: int = 8, D: int = 128, seed: int = 2):
    rng = np.random.default_rng(seed)
    K = rng.standard_normal((B, Hkv, ctx, D)).astype(F16)
    V = rng.standard_normal((B, Hkv, ctx, D)).astype(F16)
    q = rng.standard_normal((B, Hq, D)).astype(F16)
    return {"q": q, "K": K, "V": V}


CFG3 = dict(dim=4096, n_layers=32, n_heads=32, n_kv_heads=8, ffn_dim=11008, vocab=32000, norm_eps=1e-5,
            rope_base=10000.0, prefill=2048, steps=128)

CFG4 = dict(dim=4096, ffn=14336, n_experts=8, top_k=2, tokens=16)


def cfg3_layer_host(dim=4096, n_heads=32, n_kv_heads=8, ffn=11008, seed=3, layer=0):
    """One layer of the cfg3 model drawn on the host (int8 per-row codes + fp16 scales as the
    int8 GEMV config), gamma = 1.  For per-layer parity checks at the full shape."""
    rng = np.random.default_rng((seed, layer))
    dh = dim // n_heads
    shapes = {"wq": (n_heads * dh, dim), "wk": (n_kv_heads * dh, dim), "wv": (n_kv_heads * dh, dim),
              "wo": (dim, n_heads * dh), "wgate": (ffn, dim), "wup": (ffn, dim), "wdown": (dim, ffn)}
    lw = {}
    for name, (n, k) in shapes.items():
        lw[name] = (rng.integers(-127, 128, (n, k), dtype=np.int8),
                    (np.abs(rng.normal(0, 0.02, n)) / 127).astype(F16))
    lw["attn_norm"] = np.ones(dim, F16)
    lw["mlp_norm"] = np.ones(dim, F16)
    return lw


def cfg3_kv_host(layer: int, prefill: int = 2048, n_kv_heads: int = 8, dh: int = 128, seed: int = 3):
    """Layer `layer`'s prefilled cache rows [0, prefill): K then V, each N(0, 1) fp16 [KV, prefill, dh]."""
    rng = np.random.default_rng((seed, 2000 + layer))
    k = rng.standard_normal((n_kv_heads, prefill, dh)).astype(F16)
    v = rng.standard_normal((n_kv_heads, prefill, dh)).astype(F16)
    return k, v


def cfg3_embed_head_host(vocab: int = 32000, dim: int = 4096, seed: int = 3):
    """Embedding table N(0, 1) * 0.02 and lm_head N(0, 0.02), both fp16 [vocab, dim], and the
    first token id."""
    rng = np.random.default_rng((seed, 1000))
    embed = (rng.standard_normal((vocab, dim)) * 0.02).astype(F16)
    head = rng.normal(0, 0.02, (vocab, dim)).astype(F16)
    tok0 = int(rng.integers(0, vocab))
    return embed, head, tok0


def cfg4_moe(T=16, dim=4096, ffn=14336, E=8, seed=4):
    """Router fp16 N(0, 0.02), Q4_0 experts as cfg1 (gate/up [ffn, dim], down [dim, ffn]),
    hidden states N(0, 1), rms gamma = 1."""
    rng = np.random.default_rng(seed)
    router = rng.normal(0, 0.02, (E, dim)).astype(F16)

    def q4(n, k):
        codes = rng.integers(0, 16, (n, k), dtype=np.uint8)
        d = (np.abs(rng.normal(0, 0.02, (n, k // 32))) / 8).astype(F16)
        return q4_blocks_from_codes(codes, d)

    experts = [{"gate": q4(ffn, dim), "up": q4(ffn, dim), "down": q4(dim, ffn)} for _ in range(E)]
    h = rng.standard_normal((T, dim)).astype(F16)
    return {"router": router, "experts": experts, "h": h, "mlp_norm": np.ones(dim, F16)}
