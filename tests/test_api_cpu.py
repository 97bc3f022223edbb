"""Host-side logic of the API mirror (no GPU): graph construction and validation, codecs against
the oracle, the chunk planner, RoPE/theta parsing, the greedy tie-margin rule, and the GGUF
reader/writer.  Many cases restate the reference's own hardware-free tests."""
from types import SimpleNamespace

import numpy as np
import pytest

import aneforge_amd as af
from aneforge_amd import _blob, _gguf, llm
from aneforge_amd.llm import LlamaConfig, LlamaPrefill
from oracle import ref


# ----------------------------------------------------------------------------- graph
def test_graph_shapes_and_broadcast():
    x = af.input((5, 32))
    W = np.ones((16, 32), np.float32)
    assert x.linear(W).shape == (5, 16)
    assert (x @ np.ones((32, 8), np.float32)).shape == (5, 8)
    assert (x + af.input((1, 32))).shape == (5, 32)
    assert x.rms_norm(np.ones(32, np.float32)).shape == (5, 32)
    assert x.reshape(5, 4, 8).transpose([1, 0, 2]).shape == (4, 5, 8)
    assert af.concat([x, x], axis=1).shape == (5, 64)
    assert x.amax([1]).shape == (5, 1)
    with pytest.raises(ValueError):
        x.linear(np.ones((16, 31), np.float32))
    with pytest.raises(ValueError):
        x.reshape(7, 7)


def test_sdpa_validation_matches_reference_rules():
    q, k = af.input((1, 4, 1, 16)), af.input((1, 4, 8, 16))
    assert af.sdpa(q, k, k).shape == (1, 4, 1, 16)
    assert af.sdpa(af.input((1, 8, 1, 16)), af.input((1, 2, 8, 16)), af.input((1, 2, 8, 16))).shape == (1, 8, 1, 16)
    with pytest.raises(ValueError):                               # causal needs Sq == Skv
        af.sdpa(q, k, k, is_causal=True)
    with pytest.raises(ValueError):                               # batch 1 only
        af.sdpa(af.input((2, 4, 1, 16)), af.input((2, 4, 8, 16)), af.input((2, 4, 8, 16)))
    with pytest.raises(ValueError):                               # mask must be [1,1,Sq,Skv]
        af.sdpa(q, k, k, attn_mask=af.input((1, 4, 1, 8)))


@pytest.mark.parametrize("k,E", [(0, 8), (9, 8), (2, 2050)])
def test_topk_gate_rejects_unsupported_counts(k, E):
    # aneforge tests/test_moe_topk_range.py:9-15
    with pytest.raises(ValueError):
        af.moe._topk_gate(af.input((1, E)), k, E, 1)


def test_topk_gate_builds_at_largest_supported_count():
    assert af.moe._topk_gate(af.input((1, 2049)), 2, 2049, 1).shape == (1, 2049)


def test_moe_graph_builds_and_registers():
    cfg = LlamaConfig(dim=32, n_layers=1, n_heads=4, n_kv_heads=2, ffn_dim=16, vocab=16,
                      extra={"n_experts": 8, "n_experts_per_tok": 2, "norm_topk_prob": True})
    rng = np.random.default_rng(0)
    w = {"mlp_norm": np.ones(32, np.float32), "router": rng.standard_normal((8, 32)).astype(np.float32),
         "wgate_exps": rng.standard_normal((8, 16, 32)).astype(np.float32),
         "wup_exps": rng.standard_normal((8, 16, 32)).astype(np.float32),
         "wdown_exps": rng.standard_normal((8, 16, 32)).astype(np.float32)}
    assert af.moe._moe(af.input((5, 32)), w, cfg, af.LayerSpec(mlp="moe")).shape == (5, 32)
    assert "moe" in llm.DECODE_MLPS


# ----------------------------------------------------------------------------- codecs vs oracle
def test_product_codecs_equal_the_oracle():
    rng = np.random.default_rng(1)
    W = rng.standard_normal((48, 256)).astype(np.float32)
    q1, s1 = _blob.quantize_per_row(W)
    q2, s2 = ref.quantize_per_row(W)
    assert np.array_equal(q1, q2) and np.array_equal(s1.view(np.uint16), s2.view(np.uint16))
    b1, t1, n1 = _blob.quantize_blockwise(W, 32)
    b2, t2, n2 = ref.quantize_blockwise(W, 32)
    assert n1 == n2 and np.array_equal(b1, b2) and np.array_equal(t1.view(np.uint16), t2.view(np.uint16))
    assert np.array_equal(_blob.quantize_q4_0(W), ref.quantize_q4_0(W))


def test_superblock_layout_roundtrip_and_element_order():
    rng = np.random.default_rng(2)
    N, K = 5, 384
    codes = rng.integers(0, 16, (N, K)).astype(np.uint8)
    d = rng.standard_normal((N, K // 32)).astype(np.float16)
    blocks = ref.pack_q4_0(codes, d)
    qs, dd = _blob.q4_0_to_superblock(blocks, N, K)
    assert np.array_equal(_blob.superblock_to_q4_0(qs, dd, N, K), blocks)
    # word (row, sb, g, j): even elements in bits 0/4/8/12, odd in 16/20/24/28
    words = qs.view(np.uint32).reshape(N, K // 128, 4, 4)
    n, sb, g, j = 3, 2, 1, 3
    e0 = 32 * (4 * sb + j) + 8 * g
    w = int(words[n, sb, g, j])
    for t in range(4):
        assert (w >> (4 * t)) & 15 == codes[n, e0 + 2 * t]
        assert (w >> (16 + 4 * t)) & 15 == codes[n, e0 + 2 * t + 1]


def test_rope_pair_order_and_interleave():
    order = _blob.rope_pair_order(2, 8)
    assert order.tolist() == [0, 4, 1, 5, 2, 6, 3, 7, 8, 12, 9, 13, 10, 14, 11, 15]
    a, b = np.arange(6).reshape(3, 2), -np.arange(6).reshape(3, 2)
    assert _blob.interleave_rows(a, b)[1].tolist() == [0, -1]


# ----------------------------------------------------------------------------- llm host logic
def _random_model(cfg, seed=0):
    rng = np.random.default_rng(seed)
    R = lambda *s: (rng.standard_normal(s) / np.sqrt(s[-1])).astype(np.float32)
    dh = cfg.dh
    w = {"embed": R(cfg.vocab, cfg.dim), "final_norm": np.ones(cfg.dim, np.float32), "lm_head": R(cfg.vocab, cfg.dim),
         "layers": [{"wq": R(cfg.n_heads * dh, cfg.dim), "wk": R(cfg.n_kv_heads * dh, cfg.dim),
                     "wv": R(cfg.n_kv_heads * dh, cfg.dim), "wo": R(cfg.dim, cfg.n_heads * dh),
                     "wgate": R(cfg.ffn_dim, cfg.dim), "wup": R(cfg.ffn_dim, cfg.dim), "wdown": R(cfg.dim, cfg.ffn_dim),
                     "attn_norm": np.ones(cfg.dim, np.float32), "mlp_norm": np.ones(cfg.dim, np.float32)}
                    for _ in range(cfg.n_layers)]}
    return LlamaPrefill(cfg, w, ane_lm_head=False)


def test_layer_chunks_caps_layer_count():
    # aneforge tests/test_decode_chunking.py:14-27
    deep = lambda n: LlamaConfig(dim=128, n_heads=4, n_kv_heads=2, ffn_dim=256, vocab=64, n_layers=n, head_dim=32)
    m = _random_model(deep(32))
    chunks = m._layer_chunks()
    assert max(len(c) for c in chunks) <= m._chunk_max_layers
    assert [i for c in chunks for i in c] == list(range(32))
    assert _random_model(deep(8))._layer_chunks() == [range(0, 8)]


def test_rope_theta_parsing():
    # aneforge tests/test_rope_theta.py
    assert llm._rope_theta(SimpleNamespace(rope_parameters={"rope_theta": 1e6, "rope_type": "default"})) == 1e6
    assert llm._rope_theta(SimpleNamespace(rope_theta=500000.0)) == 500000.0
    assert llm._rope_theta(SimpleNamespace()) == 10000.0
    assert llm._rope_theta(SimpleNamespace(rope_parameters={"rope_type": "default"}, rope_theta=8e5)) == 8e5


def test_rope_tables_equal_oracle_bitwise():
    sc = {"factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
          "original_max_position_embeddings": 8192, "rope_type": "llama3"}
    for kw in ({}, {"scaling": sc}, {"rotary_dim": 64}, {"interleaved": True}):
        a = llm.rope_tables(50, 128, 500000.0, **kw)
        b = ref.rope_tables(50, 128, 500000.0, **kw)
        assert np.array_equal(a[0].view(np.uint16), b[0].view(np.uint16))
        assert np.array_equal(a[1].view(np.uint16), b[1].view(np.uint16))


@pytest.mark.parametrize("model_type,extra", [("gemma2", {}), ("gemma3_text", {}),
                                              ("llama", {"final_logit_softcapping": 30.0})])
def test_dense_loader_rejects_what_it_would_mis_load(model_type, extra):
    # aneforge/llm.py:776-788: the dense loader refuses configs whose semantics it would drop
    from types import SimpleNamespace
    c = SimpleNamespace(model_type=model_type, **extra)
    with pytest.raises(ValueError, match=repr(model_type)):
        llm._assert_dense_compatible(c)
    with pytest.raises(ValueError, match=repr(model_type)):
        llm.adapter_for(c)
    llm._assert_dense_compatible(SimpleNamespace(model_type="llama"))
    llm._assert_dense_compatible(SimpleNamespace(model_type="qwen2"))


def test_adapter_registry_routes_gemma_mistral_and_refuses_gpt2():
    # aneforge/llm.py:766-773: GPT-2 and Gemma have adapters of their own ahead of the dense fallback;
    # GPT-2 is refused by name here (LayerNorm, learned positions and a GELU MLP are not on this path)
    from types import SimpleNamespace
    from transformers import GPT2Config
    with pytest.raises(ValueError, match="'gpt2'"):
        llm.adapter_for(GPT2Config(n_layer=1, n_embd=32, n_head=2, vocab_size=64))(GPT2Config(), {})
    assert llm.adapter_for(SimpleNamespace(model_type="gemma")) is llm._gemma_adapter
    assert llm.adapter_for(SimpleNamespace(model_type="mistral")) is llm._mistral_adapter
    assert llm.adapter_for(SimpleNamespace(model_type="llama")) is llm._dense_adapter


def test_gemma_adapter_bakes_embed_scale_and_unit_offset_norms():
    # aneforge/llm.py:685-700 against HF's GemmaForCausalLM pieces: the scaled embedding rows are what
    # GemmaModel feeds layer 0, (1 + w) is GemmaRMSNorm's gain, the tied head keeps the raw table
    import torch
    from transformers import GemmaConfig, GemmaForCausalLM
    hf_cfg = GemmaConfig(hidden_size=64, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=1,
                         head_dim=16, intermediate_size=128, vocab_size=64, rms_norm_eps=1e-6,
                         max_position_embeddings=64, tie_word_embeddings=True)
    torch.manual_seed(0)
    m = GemmaForCausalLM(hf_cfg).eval()
    with torch.no_grad():
        for p in m.parameters():
            if p.dim() == 1:
                p.uniform_(-0.5, 0.5)                      # norms start at zero in HF: make (1 + w) visible
    sd = {k: v.detach().float().numpy() for k, v in m.state_dict().items()}
    cfg, w = llm._gemma_adapter(m.config, sd)
    assert [ls.mlp for ls in cfg.layers] == ["geglu", "geglu"] and cfg.dh == 16 and cfg.n_kv_heads == 1
    ids = torch.tensor([[3, 9, 27]])
    with torch.no_grad():
        x = m.model.embed_tokens(ids)                      # GemmaScaledWordEmbedding: table row * sqrt(dim)
        nrm = m.model.layers[0].input_layernorm(x)
    assert float(m.model.embed_tokens.embed_scale) == np.float32(np.sqrt(64))
    assert np.allclose(w["embed"][[3, 9, 27]], x[0].numpy(), rtol=1e-6, atol=1e-7)
    xn = x[0].numpy().astype(np.float64)
    mine = xn / np.sqrt((xn ** 2).mean(-1, keepdims=True) + cfg.norm_eps) * w["layers"][0]["attn_norm"]
    assert np.allclose(mine, nrm[0].numpy(), rtol=1e-5, atol=1e-6)
    assert np.array_equal(w["lm_head"], sd["model.embed_tokens.weight"])


def test_sample_greedy_and_topk():
    lg = np.array([0.1, 3.0, 2.9, -1.0])
    assert LlamaPrefill._sample(lg, 0.0, 1.0, 0) == 1
    np.random.seed(0)
    draws = {LlamaPrefill._sample(lg, 1.0, 1.0, 2) for _ in range(200)}
    assert draws <= {1, 2}


# ----------------------------------------------------------------------------- GGUF
def test_gguf_roundtrip_and_view(tmp_path):
    rng = np.random.default_rng(3)
    f32 = rng.standard_normal((3, 5)).astype(np.float32)
    f16 = rng.standard_normal((4, 64)).astype(np.float16)
    Wq = rng.standard_normal((2, 6, 128)).astype(np.float32)        # an expert stack [E, rows, K]
    q4 = np.concatenate([ref.quantize_q4_0(Wq[e]) for e in range(2)])
    q8 = np.zeros((2, 34), np.uint8)
    q8[:, :2] = np.array([[0.5], [2.0]], np.float16).view(np.uint8)
    q8[:, 2:] = np.arange(-16, 16, dtype=np.int8).view(np.uint8)
    p = str(tmp_path / "t.gguf")
    _gguf.write_gguf(p, {"general.architecture": "qwen3moe", "qwen3moe.block_count": 2,
                         "qwen3moe.rope.freq_base": 1e6, "tokenizer.ggml.tokens": ["a", "b"]},
                     {"a.weight": f32, "b.weight": f16, "blk.0.ffn_gate_exps.weight": ("Q4_0", q4, (2, 6, 128)),
                      "c.weight": ("Q8_0", q8, (2, 32))})
    g = _gguf.GGUFView(p)
    assert g.arch == "qwen3moe" and g.sc("block_count") == 2 and abs(g.sc("rope.freq_base") - 1e6) < 1
    assert g.field("tokenizer.ggml.tokens") == ["a", "b"] and g.field("missing", 7) == 7
    assert g.has("a.weight") and not g.has("z")
    assert np.array_equal(g.get("a.weight", np.float32), f32)
    assert np.array_equal(g.get("b.weight").view(np.uint16), f16.view(np.uint16))
    want = np.stack([ref.dequant_q4_0(ref.quantize_q4_0(Wq[e]), 6, 128) for e in range(2)])
    assert np.array_equal(g.get("blk.0.ffn_gate_exps.weight", np.float32), want)
    assert g.tn["blk.0.ffn_gate_exps.weight"].shape == (128, 6, 2)             # GGUF dim order
    qw = g.quantized("blk.0.ffn_gate_exps.weight")
    assert len(qw) == 2 and qw[1].shape == (6, 128)
    assert np.array_equal(qw[1].dequant(), want[1])
    c = g.get("c.weight", np.float32)
    assert c[0, 0] == -8.0 and c[1, 31] == 30.0
    assert g.quantized("a.weight") is None
    g.drop_pages()


def test_reference_import_name_resolves_to_this_build():
    # callers of the reference keep `import aneforge as af` and its module paths
    import aneforge
    import aneforge_amd
    from aneforge.llm import LlamaPrefill as LP
    from aneforge.moe import load_gguf
    import aneforge._gguf as g
    assert aneforge.compile is aneforge_amd.compile and aneforge.LlamaPrefill is aneforge_amd.LlamaPrefill
    assert LP is aneforge_amd.llm.LlamaPrefill and load_gguf is aneforge_amd.moe.load_gguf
    assert g.GGUFView is aneforge_amd.GGUFView and aneforge.sdpa is aneforge_amd.sdpa
