"""Pins the CPU oracle (oracle/ref.py) before it is trusted as the parity checker.

Each function is checked against something that is not a retyping of its own formula:
known-answer vectors, the reference's own test vectors, brute force on tiny inputs, closed
forms / invariants chosen so a plausible slip (wrong rounding, swapped nibble order, wrong
GQA head mapping, transposed operand) fails, and independent implementations (torch SDPA,
Hugging Face transformers' Llama / Qwen3-MoE / RoPE code)."""
import numpy as np
import pytest
import torch

from oracle import ref


# ----------------------------------------------------------------------------- int8 codec
def test_quantize_per_row_known_answers():
    # row max -> +-127; 62.5 -> 62 under round-half-to-even (half-away would give 63);
    # -63.5 -> -64; zero rows floor the scale at 1e-8
    W = np.array([[1.0, 62.5 / 127, -63.5 / 127, 0.0],
                  [-2.0, 1.0, 0.5, 0.25],
                  [0.0, 0.0, 0.0, 0.0]], np.float32)
    q, s = ref.quantize_per_row(W)
    assert q.dtype == np.int8 and s.dtype == np.float16
    assert q[0].tolist() == [127, 62, -64, 0]
    assert q[1].tolist() == [-127, 64, 32, 16]         # 63.5 -> 64 (even), 31.75 -> 32, 15.875 -> 16
    assert q[2].tolist() == [0, 0, 0, 0]
    assert s[0] == np.float16(1.0 / 127) and s[1] == np.float16(2.0 / 127)
    assert s[2] == np.float16(1e-8)


def test_quantize_per_row_invariants():
    rng = np.random.default_rng(0)
    W = rng.standard_normal((64, 96)).astype(np.float32) * rng.uniform(0.01, 3, (64, 1)).astype(np.float32)
    q, s = ref.quantize_per_row(W)
    assert np.abs(q.astype(int)).max() <= 127
    assert (np.abs(q.astype(int)).max(axis=1) == 127).all()            # every row's max maps to 127
    s32 = np.abs(W).max(1) / np.float32(127)
    err = np.abs(q.astype(np.float32) * s32[:, None] - W)
    assert (err <= s32[:, None] / 2 * (1 + 1e-6)).all()                # round-to-nearest bound


def test_dequant_w8_exact_in_fp32():
    rng = np.random.default_rng(1)
    q = rng.integers(-127, 128, (8, 16)).astype(np.int8)
    s = (np.abs(rng.normal(0, 0.02, 8)) / 127).astype(np.float16)
    dq = ref.dequant_w8(q, s)
    # exact: the fp64 product rounds to the same fp32 value
    assert np.array_equal(dq, (q.astype(np.float64) * s.astype(np.float64)[:, None]).astype(np.float32))


def test_quantize_blockwise_matches_reference_properties():
    # aneforge tests/test_compress.py:417-434: relerr < 0.02 on N(0,1); codes clamp at +-127
    rng = np.random.default_rng(2)
    W = rng.standard_normal((32, 96)).astype(np.float32)
    q, s, bs = ref.quantize_blockwise(W, 32)
    assert bs == 32 and s.shape == (32, 3)
    rec = (q.reshape(32, 3, 32).astype(np.float32) * s.astype(np.float32)[:, :, None]).reshape(32, 96)
    assert np.linalg.norm(rec - W) / np.linalg.norm(W) < 0.02
    _, _, bs2 = ref.quantize_blockwise(np.ones((2, 30), np.float32), 32)
    assert bs2 == 30                                                   # clamps to a divisor of IN


def test_dequant_blockwise_known_answer():
    # 3 x fp16(0.1) = 3 x 0.0999755859375 = 0.2999267578125 = 1228.5 fp16 ulps (2^-12):
    # round-half-even -> 1228 ulps = 0.2998046875; -127 x 2^-7 = -0.9921875 exact; the second
    # block's scale (2.0) must not leak into the first block
    q = np.zeros((1, 64), np.int8)
    q[0, 0], q[0, 1], q[0, 32] = 3, -127, 5
    w = ref.dequant_blockwise(q, np.array([[0.1, 2.0]], np.float16), 32)
    assert w[0, 0] == np.float32(0.2998046875)
    assert w[0, 32] == np.float32(10.0) and w[0, 2] == 0.0 and w[0, 63] == 0.0
    w2 = ref.dequant_blockwise(q, np.array([[2.0 ** -7, 2.0]], np.float16), 32)
    assert w2[0, 1] == np.float32(-0.9921875)


# ----------------------------------------------------------------------------- Q4_0
def test_q4_0_known_answer_blocks():
    # d = 1.0, qs all 0x80 -> low nibble 0 -> -8 for elements 0..15, high nibble 8 -> 0 for 16..31
    blk = np.zeros((1, 18), np.uint8)
    blk[0, :2] = np.array([1.0], np.float16).view(np.uint8)
    blk[0, 2:] = 0x80
    w = ref.dequant_q4_0(blk, 1, 32)[0]
    assert w[:16].tolist() == [-8.0] * 16 and w[16:].tolist() == [0.0] * 16
    # qs[i] = i | (15 - i) << 4, d = 0.5: element i -> (i-8)/2, element i+16 -> (7-i)/2
    blk[0, :2] = np.array([0.5], np.float16).view(np.uint8)
    blk[0, 2:] = np.array([i | ((15 - i) << 4) for i in range(16)], np.uint8)
    w = ref.dequant_q4_0(blk, 1, 32)[0]
    assert w[:16].tolist() == [(i - 8) / 2 for i in range(16)]
    assert w[16:].tolist() == [(7 - i) / 2 for i in range(16)]


def test_q4_0_dequant_matches_bruteforce_loop():
    rng = np.random.default_rng(3)
    N, K = 3, 64
    codes = rng.integers(0, 16, (N, K)).astype(np.uint8)
    d = (np.abs(rng.normal(0, 0.02, (N, K // 32))) / 8).astype(np.float16)
    blocks = ref.pack_q4_0(codes, d)
    want = np.zeros((N, K), np.float32)
    for n in range(N):                          # byte-level walk of the ggml block layout
        raw = bytes(blocks[n])
        for b in range(K // 32):
            off = 18 * b
            dd = np.frombuffer(raw[off:off + 2], np.float16)[0]
            for i in range(16):
                byte = raw[off + 2 + i]
                want[n, 32 * b + i] = np.float32((byte & 15) - 8) * np.float32(dd)
                want[n, 32 * b + i + 16] = np.float32((byte >> 4) - 8) * np.float32(dd)
    assert np.array_equal(ref.dequant_q4_0(blocks, N, K), want)
    c2, d2 = ref.unpack_q4_0(blocks, N, K)
    assert np.array_equal(c2, codes) and np.array_equal(d2.view(np.uint16), d.view(np.uint16))


def test_quantize_q4_0_ggml_rule():
    # block = [-1, 0.5, 0, ...]: max-magnitude element -1 -> d = 1/8; codes trunc(x*8 + 8.5)
    W = np.zeros((1, 32), np.float32)
    W[0, 0], W[0, 1], W[0, 2] = -1.0, 0.5, 0.3
    blocks = ref.quantize_q4_0(W)
    codes, d = ref.unpack_q4_0(blocks, 1, 32)
    assert d[0, 0] == np.float16(0.125)
    assert codes[0, 0] == 0 and codes[0, 1] == 12 and codes[0, 2] == 10 and codes[0, 3] == 8
    rng = np.random.default_rng(4)
    W = rng.standard_normal((16, 128)).astype(np.float32)
    rec = ref.dequant_q4_0(ref.quantize_q4_0(W), 16, 128)
    blk = W.reshape(16, 4, 32)
    step = np.abs(blk).max(2, keepdims=True) / 8
    err = np.abs(rec.reshape(16, 4, 32) - blk)
    # codes span -8d..7d with d = m/-8: half a step inside the range, one step at the clipped end
    assert (err <= step * 1.0 + 1e-3).all() and np.median(err / step) < 0.3


# ----------------------------------------------------------------------------- norm / rope
def test_rms_norm_against_torch_and_invariants():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4, 64)) * 3
    g = rng.uniform(0.5, 1.5, 64)
    want = torch.nn.functional.rms_norm(torch.tensor(x), (64,), torch.tensor(g), eps=1e-5).numpy()
    assert np.allclose(ref.rms_norm(x, g, 1e-5, exact=True), want, atol=1e-12)
    y = ref.rms_norm(x * 7.0, np.ones(64), 0.0, exact=True)              # scale invariant, unit RMS
    assert np.allclose(np.sqrt((y ** 2).mean(-1)), 1.0) and np.allclose(y, ref.rms_norm(x, np.ones(64), 0.0, exact=True))


def _hf_rope(dh, base, seq, scaling=None):
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding
    rp = {"rope_type": "default", "rope_theta": base}
    if scaling:
        rp = dict(scaling, rope_theta=base)
    cfg = LlamaConfig(hidden_size=dh * 2, num_attention_heads=2, head_dim=dh, rope_parameters=rp,
                      max_position_embeddings=max(seq, 8192))
    emb = LlamaRotaryEmbedding(cfg)
    x = torch.zeros(1, seq, dh, dtype=torch.float64)
    cos, sin = emb(x, torch.arange(seq)[None])
    return cos[0].double().numpy(), sin[0].double().numpy()


@pytest.mark.parametrize("scaling", [None, {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
                                           "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}])
def test_rope_tables_match_transformers(scaling):
    cos, sin = ref.rope_tables(64, 128, 500000.0, scaling=scaling)
    hc, hs = _hf_rope(128, 500000.0, 64, scaling)
    assert np.abs(cos.astype(np.float64) - hc).max() < 1e-3 and np.abs(sin.astype(np.float64) - hs).max() < 1e-3
    if scaling:
        c0, _ = ref.rope_tables(64, 128, 500000.0)
        assert not np.allclose(c0, cos)


def test_llama3_scaling_matches_reference_closed_form():
    # aneforge tests/test_llm.py:69-85 (HF _compute_llama3_parameters math, tol 1e-12)
    sc = {"factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
          "original_max_position_embeddings": 8192, "rope_type": "llama3"}
    inv = 1.0 / (500000.0 ** (np.arange(0, 128, 2) / 128))
    f, lo, hi, old = 8.0, 1.0, 4.0, 8192.0
    wl = 2 * np.pi / inv
    il = np.where(wl > old / lo, inv / f, inv)
    smd = (1 - (old / wl - lo) / (hi - lo)) * il / f + (old / wl - lo) / (hi - lo) * il
    want = np.where(~(wl < old / hi) * ~(wl > old / lo), smd, il)
    assert np.max(np.abs(ref.llama3_rope_scale(inv, sc) - want)) < 1e-12


def test_rope_matches_transformers_apply_and_preserves_pair_norms():
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
    rng = np.random.default_rng(6)
    cos, sin = ref.rope_tables(16, 32, 10000.0)
    q = rng.standard_normal((1, 2, 16, 32))
    got = ref.rope(q, cos.astype(np.float64), sin.astype(np.float64), exact=True)
    tc, ts = torch.tensor(cos.astype(np.float64))[None], torch.tensor(sin.astype(np.float64))[None]
    want, _ = apply_rotary_pos_emb(torch.tensor(q), torch.tensor(q), tc, ts)
    assert np.allclose(got, want.numpy(), atol=1e-12)
    h = 16
    n0 = q[..., :h] ** 2 + q[..., h:] ** 2
    n1 = got[..., :h] ** 2 + got[..., h:] ** 2
    c64 = cos.astype(np.float64)[:, :h]; s64 = sin.astype(np.float64)[:, :h]
    assert np.allclose(n1, n0 * (c64 ** 2 + s64 ** 2))   # rotation preserves each (i, i+h) pair norm


# ----------------------------------------------------------------------------- attention
@pytest.mark.parametrize("B,Hq,Hkv,Sq,L,D", [(1, 1, 1, 1, 4, 8), (2, 4, 2, 1, 9, 16), (1, 8, 2, 3, 8, 16)])
def test_attention_matches_torch_sdpa(B, Hq, Hkv, Sq, L, D):
    rng = np.random.default_rng(7)
    q = rng.standard_normal((B, Hq, Sq, D))
    K = rng.standard_normal((B, Hkv, L, D))
    V = rng.standard_normal((B, Hkv, L, D))
    got = ref.attention(q, K, V, exact=True)
    G = Hq // Hkv
    Kr = torch.tensor(K).repeat_interleave(G, dim=1)                 # head h -> kv head h // G
    Vr = torch.tensor(V).repeat_interleave(G, dim=1)
    want = torch.nn.functional.scaled_dot_product_attention(torch.tensor(q), Kr, Vr).numpy()
    assert np.allclose(got, want, atol=1e-10)


def test_attention_special_cases():
    rng = np.random.default_rng(8)
    q = rng.standard_normal((1, 2, 1, 8))
    V = rng.standard_normal((1, 2, 5, 8))
    K = rng.standard_normal((1, 2, 5, 8))
    assert np.allclose(ref.attention(q, K, V, lengths=[1], exact=True)[0, :, 0], V[0, :, 0])   # ctx 1 -> V
    Ke = np.repeat(K[:, :, :1], 5, axis=2)                                                      # equal keys
    assert np.allclose(ref.attention(q, Ke, V, exact=True)[0, :, 0], V[0].mean(1))
    m = np.zeros((1, 5)); m[0, 3:] = -1e4                                                       # -1e4 mask
    assert np.allclose(ref.attention(q, K, V, mask=m, exact=True), ref.attention(q, K, V, lengths=[3], exact=True))


# ----------------------------------------------------------------------------- MoE
def test_topk_gate_reference_tie_vectors():
    # aneforge tests/test_moe.py:95-108
    rows = np.array([[0.2, 0.2, 0.2, 0.1, 0.1, 0.1, 0.05, 0.05],
                     [0.3, 0.2, 0.2, 0.2, 0.05, 0.03, 0.01, 0.01],
                     [0.1, 0.1, 0.1, 0.1, 0.1, 0.1, 0.2, 0.2],
                     [0.4, 0.3, 0.1, 0.1, 0.05, 0.03, 0.01, 0.01]], np.float16)
    got = ref.topk_gate(rows, 2)
    want = [[0, 1], [0, 1], [6, 7], [0, 1]]
    for t in range(4):
        nz = sorted(np.flatnonzero(got[t]).tolist())
        assert nz == want[t]
        assert np.allclose(got[t, nz], rows[t, nz].astype(np.float64))


@pytest.mark.parametrize("k,E", [(0, 8), (9, 8), (2, 2050)])
def test_topk_gate_rejects_unsupported_counts(k, E):
    # aneforge tests/test_moe_topk_range.py:9-15
    with pytest.raises(ValueError):
        ref.topk_gate(np.ones((1, E), np.float16), k)


def test_moe_layer_matches_hf_qwen3_moe_block():
    from transformers import Qwen3MoeConfig
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeSparseMoeBlock
    cfg = Qwen3MoeConfig(hidden_size=32, moe_intermediate_size=16, num_experts=8, num_experts_per_tok=2,
                         norm_topk_prob=True, intermediate_size=64, num_attention_heads=4, num_key_value_heads=2)
    torch.manual_seed(0)
    blk = Qwen3MoeSparseMoeBlock(cfg).double()
    for p in blk.parameters():
        torch.nn.init.normal_(p, std=0.2)
    rng = np.random.default_rng(9)
    h = rng.standard_normal((5, 32))
    hn = ref.rms_norm(h, np.ones(32), 1e-5, exact=True)
    with torch.no_grad():
        out = blk(torch.tensor(hn)[None])
    out = (out[0] if isinstance(out, tuple) else out)[0].numpy()
    sd = {k: v.detach().numpy() for k, v in blk.state_dict().items()}
    router = sd["gate.weight"]
    gu = sd["experts.gate_up_proj"]
    Wg, Wu, Wd = gu[:, :16], gu[:, 16:], sd["experts.down_proj"]
    got, _, _ = ref.moe_layer(h, np.ones(32), router, Wg, Wu, Wd, 2, True, 1e-5, exact=True)
    assert np.allclose(got - h, out, atol=1e-3 * np.abs(out).max())
    cos = float((got - h).ravel() @ out.ravel() / (np.linalg.norm(got - h) * np.linalg.norm(out)))
    assert cos > 0.9999


# ----------------------------------------------------------------------------- decoder
def _hf_tiny_llama(seed=0, **kw):
    from transformers import LlamaConfig, LlamaForCausalLM
    c = dict(hidden_size=64, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
             intermediate_size=128, vocab_size=64, rms_norm_eps=1e-5, max_position_embeddings=64)
    c.update(kw)
    torch.manual_seed(seed)
    return LlamaForCausalLM(LlamaConfig(**c)).eval().double()


def _oracle_weights(m):
    sd = {k: v.detach().numpy() for k, v in m.state_dict().items()}
    c = m.config
    W = {"embed": sd["model.embed_tokens.weight"], "final_norm": sd["model.norm.weight"],
         "lm_head": sd.get("lm_head.weight", sd["model.embed_tokens.weight"]), "layers": []}
    for L in range(c.num_hidden_layers):
        p = f"model.layers.{L}."
        W["layers"].append({"wq": sd[p + "self_attn.q_proj.weight"], "wk": sd[p + "self_attn.k_proj.weight"],
                            "wv": sd[p + "self_attn.v_proj.weight"], "wo": sd[p + "self_attn.o_proj.weight"],
                            "wgate": sd[p + "mlp.gate_proj.weight"], "wup": sd[p + "mlp.up_proj.weight"],
                            "wdown": sd[p + "mlp.down_proj.weight"], "attn_norm": sd[p + "input_layernorm.weight"],
                            "mlp_norm": sd[p + "post_attention_layernorm.weight"]})
    cfg = {"n_heads": c.num_attention_heads, "n_kv_heads": c.num_key_value_heads,
           "dh": c.hidden_size // c.num_attention_heads, "norm_eps": c.rms_norm_eps, "rope_base": 10000.0}
    return W, cfg


def test_decoder_matches_hf_llama_logits():
    m = _hf_tiny_llama()
    W, cfg = _oracle_weights(m)
    prompt = [3, 17, 5, 42, 9]
    with torch.no_grad():
        want = m(torch.tensor(prompt)[None]).logits[0].numpy()     # [S, V]
    # prefill token by token through the oracle's resident-cache decode
    toks, lg = ref.generate(prompt, 3, W, cfg, M=16, exact=True)
    cos = float(lg[0] @ want[-1] / (np.linalg.norm(lg[0]) * np.linalg.norm(want[-1])))
    assert cos > 0.99999 and int(np.argmax(lg[0])) == int(np.argmax(want[-1]))
    # greedy continuation matches HF's own greedy generate
    with torch.no_grad():
        hf = m.generate(torch.tensor(prompt)[None], max_new_tokens=3, do_sample=False)[0, len(prompt):].tolist()
    assert toks == hf


def test_decoder_gqa_mapping_is_not_interleaved():
    # a wrong kv-head mapping (h % KV instead of h // G) changes the logits: guard the pin
    m = _hf_tiny_llama(seed=1)
    W, cfg = _oracle_weights(m)
    prompt = [1, 2, 3, 4]
    with torch.no_grad():
        want = m(torch.tensor(prompt)[None]).logits[0, -1].numpy()
    _, lg = ref.generate(prompt, 1, W, cfg, M=8, exact=True)
    assert np.allclose(lg[0], want, atol=1e-5)            # HF builds inv_freq in fp32
    # swapping the two kv heads emulates the h % KV mapping for H=4, KV=2 heads 1 and 2
    dh = cfg["dh"]
    for lw in W["layers"]:
        for key in ("wk", "wv"):
            lw[key] = np.concatenate([lw[key][dh:], lw[key][:dh]])
        wq = lw["wq"].reshape(4, dh, -1)
        lw["wq"] = wq[[0, 2, 1, 3]].reshape(4 * dh, -1)
        wo = lw["wo"].reshape(lw["wo"].shape[0], 4, dh)
        lw["wo"] = wo[:, [0, 2, 1, 3]].reshape(lw["wo"].shape[0], 4 * dh)
    _, bad = ref.generate(prompt, 1, W, cfg, M=8, exact=True)
    assert np.abs(bad[0] - want).max() > 1e-3


def test_decode_rows_matches_sequential_decode_layer_and_hf():
    # teacher-forced rows through one layer at a time == the token-by-token decode, and a prefill
    # from position 0 reproduces HF's logits at every prompt position
    m = _hf_tiny_llama(seed=2)
    W, cfg = _oracle_weights(m)
    prompt = [5, 9, 2, 33, 17, 60, 1]
    n, M, dh = len(prompt), 12, cfg["dh"]
    cos, sin = ref.rope_tables(M, dh)
    with torch.no_grad():
        want = m(torch.tensor(prompt)[None]).logits[0].numpy()
    for exact in (True, False):
        seq = [(np.zeros((2, M, dh)), np.zeros((2, M, dh))) for _ in W["layers"]]
        rows = [(np.zeros((2, M, dh)), np.zeros((2, M, dh))) for _ in W["layers"]]
        H = ref.r16(np.asarray(W["embed"])[prompt], exact)
        for li, lw in enumerate(W["layers"]):
            H = ref.decode_rows(H, lw, cfg, *rows[li], 0, cos, sin, exact)
        for p, tok in enumerate(prompt):
            h = ref.r16(np.asarray(W["embed"])[tok].reshape(1, -1), exact)
            for li, lw in enumerate(W["layers"]):
                h = ref.decode_layer(h, lw, cfg, *seq[li], p, cos[p], sin[p], exact)
            tol = 1e-12 if exact else float(np.spacing(np.float16(np.abs(h).max())))
            assert np.abs(H[p] - h[0]).max() <= tol, (exact, p)
        for li in range(len(W["layers"])):
            for a, b in zip(rows[li], seq[li]):
                assert np.abs(a - b).max() <= (1e-12 if exact else 2e-3)
        if exact:
            lg = ref.logits(H, W["final_norm"], W["lm_head"], cfg["norm_eps"], exact=True)
            assert np.abs(lg - want).max() <= 1e-5 * np.abs(want).max()


def test_decode_rows_moe_layer_matches_sequential():
    rng = np.random.default_rng(12)
    D, H, KV, dh, F, E = 32, 4, 2, 8, 16, 6
    cfg = {"n_heads": H, "n_kv_heads": KV, "dh": dh, "norm_eps": 1e-5, "top_k": 2}
    R = lambda *s: rng.standard_normal(s) * 0.3
    lw = {"wq": R(H * dh, D), "wk": R(KV * dh, D), "wv": R(KV * dh, D), "wo": R(D, H * dh),
          "attn_norm": np.ones(D), "mlp_norm": rng.uniform(0.8, 1.2, D), "router": R(E, D),
          "wgate_exps": R(E, F, D), "wup_exps": R(E, F, D), "wdown_exps": R(E, D, F)}
    M, pos0, n = 10, 3, 5
    cos, sin = ref.rope_tables(M, dh)
    K0, V0 = rng.standard_normal((KV, M, dh)), rng.standard_normal((KV, M, dh))
    X = ref.r16(rng.standard_normal((n, D)))
    Kr, Vr = K0.copy(), V0.copy()
    got = ref.decode_rows(X, lw, cfg, Kr, Vr, pos0, cos, sin)
    Ks, Vs = K0.copy(), V0.copy()
    for t in range(n):
        want = ref.decode_layer(X[t:t + 1], lw, cfg, Ks, Vs, pos0 + t, cos[pos0 + t], sin[pos0 + t])
        assert np.abs(got[t] - want[0]).max() <= float(np.spacing(np.float16(np.abs(want).max()))), t
    assert np.array_equal(Kr[:, :pos0], K0[:, :pos0]) and np.abs(Kr - Ks).max() <= 2e-3


def test_q4_0_f16_dequant_matches_reference_rounding():
    # GGUFView.get converts the fp32 ggml dequantisation to float16 (aneforge/_gguf.py:34-39):
    # d = fp16(0.1) = 0.0999755859375, code 15 -> 7 * d = 0.6998291015625 (exact in fp32); the fp16
    # grid there has spacing 2^-11, so it rounds to 1433/2048 = 0.69970703125 (1434/2048 is farther)
    d = np.full((1, 1), 0.1, np.float16)
    codes = np.full((1, 32), 15, np.uint8)
    blocks = ref.pack_q4_0(codes, d)
    exact = ref.dequant_q4_0(blocks, 1, 32)
    assert exact[0, 0] == np.float32(0.6998291015625)
    r = ref.dequant_q4_0_f16(blocks, 1, 32)
    assert r[0, 0] == np.float32(1433 / 2048)
    assert np.all(r == r[0, 0])


def test_dequant_lut4_known_answer():
    # byte 0x21: column 0 -> entry 1, column 1 -> entry 2; byte 0xF0: column 2 -> 0, column 3 -> 15;
    # the second row uses its own codebook
    cb = np.stack([np.arange(16, dtype=np.float16) * np.float16(0.5), -np.arange(16, dtype=np.float16)])
    packed = np.array([[0x21, 0xF0], [0x21, 0xF0]], np.uint8)
    w = ref.dequant_lut4(packed, cb, 4)
    np.testing.assert_array_equal(w, np.array([[0.5, 1.0, 0.0, 7.5], [-1.0, -2.0, 0.0, -15.0]], np.float32))
    np.testing.assert_array_equal(ref.dequant_lut4(packed[:1], cb[0], 3), np.array([[0.5, 1.0, 0.0]], np.float32))


def test_palettize_lut4_matches_reference_vectors():
    # vectors recorded from the reference's palettize_lut4 (aneforge/_blob.py:28-43) by
    # tests/golden/make_lut4_vectors.py: packed indices and fp16 codebook must match bit for bit
    import os
    from aneforge_amd import _blob
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "lut4_vectors.npz"))
    names = sorted({k.split("__")[0] for k in z.files})
    assert len(names) == 5
    for name in names:
        W = z[f"{name}__W"]
        packed, cb = _blob.palettize_lut4(W)
        assert packed.dtype == np.uint8 and cb.dtype == np.float16, name
        np.testing.assert_array_equal(packed, z[f"{name}__packed"], err_msg=name)
        np.testing.assert_array_equal(cb.view(np.uint16), z[f"{name}__codebook"].view(np.uint16), err_msg=name)


def test_dequant_q4_k_kat_and_encoder():
    # closed form: d = 0.5, dmin = 0.25, scale_j = j + 1, min_j = 2j, every code 3
    # -> w = 0.5 (j + 1) 3 - 0.25 (2j) = 1.5 + j for the 32 elements of sub-block j
    from test_gguf_codecs import enc_q4_k
    blk = np.frombuffer(enc_q4_k(0.5, 0.25, [j + 1 for j in range(8)], [2 * j for j in range(8)], [3] * 256), np.uint8)
    e = np.arange(256)
    np.testing.assert_array_equal(ref.dequant_q4_k(blk)[0], (1.5 + e // 32).astype(np.float32))
    # element-by-element encoder: chosen 6-bit scales / mins (top bits set, so the j >= 4 packing
    # matters) and codes decode to d*sc*q - dmin*m in float32
    rng = np.random.default_rng(5)
    for _ in range(20):
        d, dmin = float(np.float16(rng.uniform(1e-3, 0.1))), float(np.float16(rng.uniform(1e-3, 0.1)))
        sc = [int(v) for v in rng.integers(0, 64, 8)]
        mn = [int(v) for v in rng.integers(0, 64, 8)]
        q = [int(v) for v in rng.integers(0, 16, 256)]
        blk = np.frombuffer(enc_q4_k(d, dmin, sc, mn, q), np.uint8)
        want = np.array([np.float32(np.float32(d) * np.float32(sc[i // 32])) * np.float32(q[i])
                         - np.float32(np.float32(dmin) * np.float32(mn[i // 32])) for i in range(256)], np.float32)
        np.testing.assert_array_equal(ref.dequant_q4_k(blk)[0], want)
    # the fp16 weights are that float32 value cast once
    assert ref.dequant_q4_k_f16(blk, 1, 256).dtype == np.float32
    np.testing.assert_array_equal(ref.dequant_q4_k_f16(blk, 1, 256)[0], want.astype(np.float16).astype(np.float32))


def test_sample_matches_numpy_choice_and_its_filters():
    # the draw: numpy's legacy RandomState.choice(n, p=p) consumes one random_sample() and returns
    # the inverse-CDF index; ref.sample given that same uniform must return the same token
    rng = np.random.default_rng(21)
    for trial in range(200):
        V = int(rng.integers(2, 400))
        logits = (rng.standard_normal(V) * rng.uniform(0.5, 4)).astype(np.float32)
        T, top_p, top_k = float(rng.uniform(0.3, 2.0)), 1.0, 0
        lg = logits.astype(np.float64) / T
        pr = np.exp(lg - lg.max()); pr /= pr.sum()
        want = np.random.RandomState(trial).choice(V, p=pr)
        u = np.random.RandomState(trial).random_sample()
        assert ref.sample(logits, T, top_p, top_k, u) == want
    logits = (rng.standard_normal(1000) * 3).astype(np.float32)
    us = (np.arange(4000) + 0.5) / 4000
    # top-k: only the k largest logits are ever drawn, top_k = 1 is argmax
    top5 = set(np.argsort(logits)[-5:].tolist())
    assert {ref.sample(logits, 1.0, 1.0, 5, u) for u in us} == top5
    assert {ref.sample(logits, 1.0, 1.0, 1, u) for u in us[::50]} == {int(np.argmax(logits))}
    # top-p: the drawn set is the smallest top set whose probability reaches top_p
    p = np.exp(logits.astype(np.float64) - logits.max()); p /= p.sum()
    srt = np.argsort(p)[::-1]
    n = int(np.argmax(np.cumsum(p[srt]) >= 0.7)) + 1
    assert {ref.sample(logits, 1.0, 0.7, 0, u) for u in us} == set(srt[:n].tolist())
    assert {ref.sample(logits, 1.0, 1e-9, 0, u) for u in us[::50]} == {int(np.argmax(logits))}
    # frequencies over a fine grid of u follow the renormalised probabilities
    keep = srt[:n]
    cnt = np.bincount([ref.sample(logits, 1.0, 0.7, 0, u) for u in us], minlength=1000)
    np.testing.assert_allclose(cnt[keep] / len(us), p[keep] / p[keep].sum(), atol=2.0 / len(us))
    assert ref.sample(logits, 0.0, 0.5, 3, 0.3) == int(np.argmax(logits))      # T <= 0: greedy


def test_dequant_q6_k_kat_and_encoder():
    # closed form: d = 0.25, scale_i = i - 8 (signed), code(e) = e % 64 -> w = 0.25 (e//16 - 8) (e%64 - 32)
    from test_gguf_codecs import enc_q6_k
    e = np.arange(256)
    blk = np.frombuffer(enc_q6_k(0.25, [i - 8 for i in range(16)], [int(v) - 32 for v in e % 64]), np.uint8)
    np.testing.assert_array_equal(ref.dequant_q6_k(blk)[0], (0.25 * (e // 16 - 8) * (e % 64 - 32)).astype(np.float32))
    # element-by-element encoder: random scales and 6-bit codes decode to (d * sc) * (q - 32) in float32
    rng = np.random.default_rng(6)
    for _ in range(20):
        d = float(np.float16(rng.uniform(1e-3, 0.05)))
        sc = [int(v) for v in rng.integers(-128, 128, 16)]
        q = [int(v) for v in rng.integers(-32, 32, 256)]
        blk = np.frombuffer(enc_q6_k(d, sc, q), np.uint8)
        want = np.array([np.float32(np.float32(d) * np.float32(sc[i // 16])) * np.float32(q[i]) for i in range(256)],
                        np.float32)
        np.testing.assert_array_equal(ref.dequant_q6_k(blk)[0], want)


def test_cpu_baseline_layer_matches_the_exact_decode_layer():
    """The timed CPU baseline (ref.cpu_decode_layer_f32, fp32 numpy) computes the same layer as the
    pinned decode_layer(exact=True): GQA 4:1 at a populated cache position, non-unit norm gains, the
    new K/V row written in place.  A wrong kv-head mapping, RoPE sign or a skipped residual moves the
    output far outside the fp32-vs-fp64 tolerance used here."""
    rng = np.random.default_rng(11)
    D, H, KV, dh, F, M, pos = 256, 8, 2, 32, 512, 96, 70
    cfg = {"n_heads": H, "n_kv_heads": KV, "dh": dh, "norm_eps": 1e-5}
    sd = lambda *s: rng.standard_normal(s) / np.sqrt(s[-1])
    w = {"wq": sd(H * dh, D), "wk": sd(KV * dh, D), "wv": sd(KV * dh, D), "wo": sd(D, H * dh),
         "wgate": sd(F, D), "wup": sd(F, D), "wdown": sd(D, F),
         "attn_norm": rng.uniform(0.5, 1.5, D), "mlp_norm": rng.uniform(0.5, 1.5, D)}
    cos, sin = ref.rope_tables(M, dh)
    h = rng.standard_normal((1, D))
    K0, V0 = rng.standard_normal((KV, M, dh)), rng.standard_normal((KV, M, dh))
    K64, V64 = K0.copy(), V0.copy()
    want = ref.decode_layer(h, w, cfg, K64, V64, pos, cos[pos], sin[pos], exact=True)
    f32 = {k: np.asarray(v, np.float32) for k, v in w.items()}
    K32, V32 = K0.astype(np.float32), V0.astype(np.float32)
    got = ref.cpu_decode_layer_f32(h.astype(np.float32), f32, cfg, K32, V32, pos,
                                   cos[pos].astype(np.float32), sin[pos].astype(np.float32))
    assert got.dtype == np.float32 and got.shape == (1, D)
    scale = np.abs(want).max()
    assert np.abs(got - want).max() <= 1e-4 * scale, np.abs(got - want).max() / scale
    assert np.abs(K32[:, pos] - K64[:, pos]).max() <= 1e-4 and np.abs(V32[:, pos] - V64[:, pos]).max() <= 1e-4
    assert np.array_equal(K32[:, :pos], K0[:, :pos].astype(np.float32))     # only row pos is written
    # a plausible slip fails: the interleaved kv-head mapping (query head j reading kv head j % KV
    # instead of j // G) is emulated by reordering the q rows and o-proj columns so that head j lands
    # where the baseline's h // G mapping gives it kv head j % KV
    perm = [j for r in range(KV) for j in range(H) if j % KV == r]
    wq, wo = f32["wq"].reshape(H, dh, D), f32["wo"].reshape(D, H, dh)
    slip = dict(f32, wq=wq[perm].reshape(H * dh, D), wo=wo[:, perm].reshape(D, H * dh))
    bad = ref.cpu_decode_layer_f32(h.astype(np.float32), slip, cfg, K0.astype(np.float32), V0.astype(np.float32),
                                   pos, cos[pos].astype(np.float32), sin[pos].astype(np.float32))
    assert np.abs(bad - want).max() > 1e-2 * scale


def test_gelu_tanh_matches_torch():
    x = np.linspace(-12, 12, 4001)
    want = torch.nn.functional.gelu(torch.from_numpy(x), approximate="tanh").numpy()
    assert np.abs(ref.gelu_tanh(x) - want).max() < 1e-14
    assert np.abs(ref.gelu_tanh(x) - ref.silu(x)).max() > 0.1          # the two gates differ


def test_decoder_geglu_matches_hf_gemma_logits():
    # the Gemma adapter's baked weights (sqrt(dim) embedding rows, (1 + w) norms) through the oracle's
    # decoder with the GeGLU gate reproduce HF GemmaForCausalLM (aneforge tests/test_llm.py:120-135)
    from transformers import GemmaConfig, GemmaForCausalLM
    from aneforge_amd import llm
    hf_cfg = GemmaConfig(hidden_size=64, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=1,
                         head_dim=16, intermediate_size=128, vocab_size=64, rms_norm_eps=1e-6,
                         max_position_embeddings=64, tie_word_embeddings=True)
    torch.manual_seed(0)
    m = GemmaForCausalLM(hf_cfg).eval().double()
    with torch.no_grad():
        for p in m.parameters():
            if p.dim() == 1:
                p.uniform_(-0.5, 0.5)                      # non-zero (1 + w) gains
            else:
                p.normal_(0.0, p.shape[1] ** -0.5)        # O(1) gate pre-activations
    prompt = [3, 17, 5, 42, 9, 60]
    with torch.no_grad():
        want = m(torch.tensor(prompt)[None]).logits[0].numpy()
        hf = m.generate(torch.tensor(prompt)[None], max_new_tokens=3, do_sample=False)[0, len(prompt):].tolist()
    sd = {k: v.detach().numpy() for k, v in m.state_dict().items()}
    cfg, W = llm._gemma_adapter(m.config, sd)
    oc = {"n_heads": 4, "n_kv_heads": 1, "dh": 16, "norm_eps": 1e-6, "rope_base": 10000.0, "mlp": "geglu"}
    toks, lg = ref.generate(prompt, 3, W, oc, M=16, exact=True)
    # GemmaRMSNorm computes in float32 (x.float(), weight.float()) even in a float64 model
    assert np.abs(lg[0] - want[-1]).max() <= 2e-4 * np.abs(want[-1]).max()
    assert toks == hf
    # the SwiGLU gate on the same weights is far off: the activation is what the test pins
    _, bad = ref.generate(prompt, 1, W, dict(oc, mlp="swiglu"), M=16, exact=True)
    assert np.abs(bad[0] - want[-1]).max() > 1e-2 * np.abs(want[-1]).max()
