"""LlamaPrefill on the device vs the CPU oracle (greedy tokens, per-layer hidden states) and vs
Hugging Face (tiny random Llama).  Mirrors the reference's decode tests (tests/test_llm.py:38-101)
with tolerances tightened to the path's parity bar."""
import numpy as np
import pytest

from _util import check_f16, check_hidden, cosine, say
from oracle import ref

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def _random_weights(cfg, seed=0):
    """1/sqrt(fan-in) random weights in the reference's canonical layout (tests/_helpers.py:24-40)."""
    rng = np.random.default_rng(seed)
    dh = cfg.dh
    R = lambda *s: (rng.standard_normal(s) / np.sqrt(s[-1])).astype(np.float32)
    w = {"embed": R(cfg.vocab, cfg.dim), "final_norm": np.ones(cfg.dim, np.float32), "lm_head": R(cfg.vocab, cfg.dim),
         "layers": []}
    for _ in range(cfg.n_layers):
        w["layers"].append({"wq": R(cfg.n_heads * dh, cfg.dim), "wk": R(cfg.n_kv_heads * dh, cfg.dim),
                            "wv": R(cfg.n_kv_heads * dh, cfg.dim), "wo": R(cfg.dim, cfg.n_heads * dh),
                            "wgate": R(cfg.ffn_dim, cfg.dim), "wup": R(cfg.ffn_dim, cfg.dim),
                            "wdown": R(cfg.dim, cfg.ffn_dim),
                            "attn_norm": rng.uniform(0.8, 1.2, cfg.dim).astype(np.float32),
                            "mlp_norm": rng.uniform(0.8, 1.2, cfg.dim).astype(np.float32)})
    return w


def _effective(w, compress):
    """The weights the device actually streams, dequantised to fp32 for the oracle."""
    from aneforge_amd import _blob

    def enc(W):
        W = np.asarray(W, np.float32)
        if compress is None:
            return W.astype(np.float16).astype(np.float32)
        if compress == "int8":
            return ref.dequant_w8(*_blob.quantize_per_row(W))
        if compress == "q4_0":                       # the fp16 weights the kernels multiply with
            return ref.dequant_q4_0_f16(_blob.quantize_q4_0(W), *W.shape)
        if compress == "blockwise":
            q, sc, bs = _blob.quantize_blockwise(W, 32)
            return ref.dequant_blockwise(q, sc, bs)
        if compress == "int4":                       # one codebook per tensor, as the reference
            packed, cb = _blob.palettize_lut4(W)
            return ref.dequant_lut4(packed, cb, W.shape[1])
        raise ValueError(compress)

    out = {"embed": np.asarray(w["embed"], np.float32).astype(np.float16).astype(np.float32),
           "final_norm": np.asarray(w["final_norm"]).astype(np.float16).astype(np.float32),
           "lm_head": np.asarray(w["lm_head"]).astype(np.float16).astype(np.float32), "layers": []}
    for lw in w["layers"]:
        e = {k: enc(lw[k]) for k in ("wq", "wk", "wv", "wo", "wgate", "wup", "wdown")}
        e["attn_norm"] = np.asarray(lw["attn_norm"]).astype(np.float16).astype(np.float32)
        e["mlp_norm"] = np.asarray(lw["mlp_norm"]).astype(np.float16).astype(np.float32)
        out["layers"].append(e)
    return out


def _ocfg(cfg):
    return {"n_heads": cfg.n_heads, "n_kv_heads": cfg.n_kv_heads, "dh": cfg.dh, "norm_eps": cfg.norm_eps,
            "rope_base": cfg.rope_base}


def _assert_tokens_match(got, want, logits, what, rel_gap=2e-3):
    """Equal greedy tokens; a divergence is accepted only where the oracle's own top-2 gap is a
    near-tie (fp32-vs-fp64 accumulation order can flip it), and comparison stops there."""
    for i, (g, t) in enumerate(zip(got, want)):
        if g != t:
            lg = logits[i]
            top = np.sort(lg)[-2:]
            gap = (top[1] - top[0]) / (np.abs(lg).max() + 1e-9)
            assert gap < rel_gap and lg[g] >= top[0] - 1e-6, \
                f"{what}: token {i} differs ({g} vs {t}) with a clear oracle margin {gap:.2e}"
            return
    assert len(got) == len(want), f"{what}: {len(got)} tokens vs {len(want)}"


@pytest.mark.parametrize("compress", [None, "int8", "q4_0", "blockwise", "int4"])
def test_generate_matches_oracle(compress):
    from aneforge_amd.llm import LlamaConfig, LlamaPrefill
    say(f"LlamaPrefill.generate vs oracle compress={compress}")
    cfg = LlamaConfig(dim=256, n_layers=3, n_heads=4, n_kv_heads=2, ffn_dim=512, vocab=128)
    w = _random_weights(cfg)
    m = LlamaPrefill(cfg, w, compress=compress)
    prompt = [5, 17, 33, 2, 99]
    got = m.generate(prompt, max_new_tokens=12)
    want, lgs = ref.generate(prompt, 12, _effective(w, compress), _ocfg(cfg), M=len(prompt) + 12)
    _assert_tokens_match(got, want, lgs, f"compress={compress}")
    assert m.generate(prompt, max_new_tokens=12) == got                     # deterministic
    m.release()


def test_decode_first_token_equals_prefill_argmax():
    from aneforge_amd.llm import LlamaConfig, LlamaPrefill
    say("decode token 0 == prefill argmax; prefill logits vs oracle")
    cfg = LlamaConfig(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, ffn_dim=512, vocab=96)
    w = _random_weights(cfg, seed=1)
    m = LlamaPrefill(cfg, w, compress="int8")
    prompt = [1, 2, 3]
    lg = m.prefill(prompt)[0]
    assert m.generate(prompt, max_new_tokens=1)[0] == int(np.argmax(lg))
    _, want = ref.generate(prompt, 1, _effective(w, "int8"), _ocfg(cfg), M=len(prompt))
    assert cosine(lg, want[0]) >= 0.9999
    assert np.abs(lg - want[0]).max() <= 1e-2 * np.abs(want[0]).max() + 1e-3


def test_generate_streams_and_stops_on_eos():
    from aneforge_amd.llm import LlamaConfig, LlamaPrefill
    say("generate with on_token / eos / max_len")
    cfg = LlamaConfig(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, ffn_dim=512, vocab=64)
    m = LlamaPrefill(cfg, _random_weights(cfg, seed=2), compress="int8")
    full = m.generate([3, 4], max_new_tokens=6)
    seen = []
    eos = full[3]
    stop = full.index(eos)                                                   # first occurrence ends it
    part = m.generate([3, 4], max_new_tokens=6, on_token=seen.append, eos_id=eos)
    assert part == full[:stop + 1] and seen == full[:stop]
    assert len(m.generate([3, 4], max_new_tokens=50, max_len=6)) == 4      # cache-full stop (pos >= M-1)


@pytest.mark.parametrize("mode", ["greedy", "sampled", "host_head", "stepwise_prefill"])
def test_generate_on_stage_reports_the_reference_stages(mode):
    # aneforge/llm.py:568-628: per token `embedding` and `layers` (the halves of `step`), `step`,
    # `lm_head`, `sample`; a token-by-token prefill reports embedding / layers per prompt token.
    # The staged loop gives the same tokens as the unstaged one.
    from aneforge_amd.llm import LlamaConfig, LlamaPrefill
    say(f"generate(on_stage=...) {mode}")
    cfg = LlamaConfig(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, ffn_dim=512, vocab=128)
    m = LlamaPrefill(cfg, _random_weights(cfg, seed=5), compress="int8")
    prompt, n = [4, 9, 21, 3], 6
    kw = {"temperature": 0.9, "top_k": 20} if mode == "sampled" else {}
    if mode == "host_head":
        kw["ane_lm_head"] = False
    if mode == "stepwise_prefill":
        kw["batched_prefill"] = False
    np.random.seed(5)
    plain = m.generate(prompt, max_new_tokens=n, **kw)
    stages = []
    np.random.seed(5)
    staged = m.generate(prompt, max_new_tokens=n, on_stage=lambda name, dt: stages.append((name, dt)), **kw)
    assert staged == plain and len(plain) == n
    per_token = ["embedding", "layers", "step", "lm_head", "sample"]
    pre = ["embedding", "layers"] * (len(prompt) - 1) if mode == "stepwise_prefill" else []
    assert [s for s, _ in stages] == pre + per_token * n
    assert all(dt >= 0.0 for _, dt in stages)
    m.release()


def test_device_sampling_steps_match_oracle_and_generate_paths():
    # each sampled step: the token the device sampler queued equals the oracle's _sample on the
    # same step's logits and uniform; generate's graph loop and its per-token loop agree
    from aneforge_amd.llm import LlamaConfig, LlamaPrefill
    say("device sampling in the decode engine")
    cfg = LlamaConfig(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, ffn_dim=512, vocab=512)
    m = LlamaPrefill(cfg, _random_weights(cfg, seed=4), compress="int8")
    prompt = [7, 8, 9, 10]
    n_pre = len(prompt) - 1
    d = m._decoder(len(prompt) + 10)
    d.prefill(prompt)
    rng = np.random.default_rng(3)
    for i, (T, top_p, top_k) in enumerate([(0.9, 1.0, 0), (1.2, 0.9, 0), (0.8, 0.95, 30), (1.0, 0.5, 3),
                                            (0.7, 1.0, 50), (1.5, 0.8, 0)]):
        u = float(rng.random())
        d.set_sampling(T, top_p, top_k, [u], n_pre + i)
        d.run_sampled(1, graph=i % 2 == 0)
        tok = d.history(n_pre + i, 1)[0]
        assert tok == ref.sample(d.logits_host(), T, top_p, top_k, u), f"step {i}"
    np.random.seed(11)
    a = m.generate(prompt, max_new_tokens=8, temperature=0.8, top_p=0.9, top_k=40)
    np.random.seed(11)
    seen = []
    b = m.generate(prompt, max_new_tokens=8, temperature=0.8, top_p=0.9, top_k=40, on_token=seen.append)
    assert a == b and len(a) == 8
    m.release()


def test_per_layer_hidden_full_7b_layer_shape():
    """One cfg3 layer at its real shape (d 4096, 32/8 heads, FFN 11008, int8 codes as cfg0)
    after a 3-token prompt: per-layer hidden cosine >= 0.9999 and fp16 tolerance."""
    from aneforge_amd import _engine as E, workloads
    from aneforge_amd.llm import LlamaConfig, LlamaPrefill
    say("per-layer hidden state at the 7B layer shape")
    cfg = LlamaConfig(dim=4096, n_layers=2, n_heads=32, n_kv_heads=8, ffn_dim=11008, vocab=256)
    rng = np.random.default_rng(7)
    layers_host = [workloads.cfg3_layer_host(layer=i) for i in range(2)]
    w = {"embed": rng.standard_normal((256, 4096)).astype(np.float32),
         "final_norm": np.ones(4096, np.float32), "lm_head": (rng.standard_normal((256, 4096)) * 0.02).astype(np.float32),
         "layers": []}
    for lh in layers_host:
        lw = {k: E.QuantizedWeight("int8", v[0], v[1], v[0].shape) for k, v in lh.items() if k.startswith("w")}
        lw["attn_norm"], lw["mlp_norm"] = lh["attn_norm"], lh["mlp_norm"]
        w["layers"].append(lw)
    m = LlamaPrefill(cfg, w)
    prompt = [7, 11, 200]
    d = m._decoder(8)
    d.reset(prompt)
    d.run(len(prompt) - 1, 0)
    # oracle: same codes, fp16 rounding points of the kernels
    ow = {"embed": w["embed"].astype(np.float16).astype(np.float32), "layers": []}
    for lh in layers_host:
        e = {k: ref.dequant_w8(v[0], v[1]) for k, v in lh.items() if k.startswith("w")}
        e["attn_norm"], e["mlp_norm"] = lh["attn_norm"], lh["mlp_norm"]
        ow["layers"].append(e)
    oc = _ocfg(cfg)
    cos_t, sin_t = ref.rope_tables(8, cfg.dh)
    caches = [(np.zeros((8, 8, 128)), np.zeros((8, 8, 128))) for _ in range(2)]
    for p, tok in enumerate(prompt):
        h = ref.r16(ow["embed"][tok].reshape(1, -1))
        for li, lw in enumerate(ow["layers"]):
            h = ref.decode_layer(h, lw, oc, *caches[li], p, cos_t[p], sin_t[p])
            if p == len(prompt) - 1:
                mixer, mlp = d.layers[li]
                with torch.cuda.stream(d.stream):
                    mixer.enqueue(d)
                    mlp.enqueue(d)
                got = d.h.float().cpu().numpy()
                torch.cuda.synchronize()
                check_hidden(got, h, what=f"layer {li} hidden")
    m.release()


def test_prefill_matches_huggingface_llama():
    """Device prefill (fp16 weights) vs HF LlamaForCausalLM on a tiny random model
    (aneforge tests/test_llm.py:103-152): cosine > 0.999 and the same argmax."""
    from transformers import LlamaConfig as HF, LlamaForCausalLM
    from aneforge_amd.llm import LlamaPrefill, _dense_adapter
    say("prefill vs Hugging Face Llama")
    hf_cfg = HF(hidden_size=128, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                intermediate_size=256, vocab_size=64, rms_norm_eps=1e-5, max_position_embeddings=64)
    torch.manual_seed(0)
    hf = LlamaForCausalLM(hf_cfg).eval()
    toks = np.random.default_rng(0).integers(0, 64, 10)
    with torch.no_grad():
        want = hf(torch.tensor(toks)[None]).logits[0, -1].numpy()
    sd = {k: v.detach().float().numpy() for k, v in hf.state_dict().items()}
    cfg, weights = _dense_adapter(hf.config, sd)
    got = LlamaPrefill(cfg, weights).prefill(toks)[0]
    assert cosine(got, want) > 0.999 and int(np.argmax(got)) == int(np.argmax(want))


@pytest.mark.parametrize("compress,chunk", [("int8", 2048), ("int8", 48), (None, 2048), ("blockwise", 2048),
                                            ("q4_0", 2048), ("q4_0", 48), ("int4", 2048)])
def test_batched_prefill_matches_forced_steps_and_oracle(compress, chunk):
    """The MFMA batched prefill (head dim 128) leaves the same cache and state as the
    token-by-token forced steps, and generation from it matches the oracle."""
    from aneforge_amd.llm import LlamaConfig, LlamaPrefill
    say(f"batched prefill vs forced steps compress={compress} chunk={chunk}")
    cfg = LlamaConfig(dim=512, n_layers=2, n_heads=4, n_kv_heads=2, ffn_dim=768, vocab=128)
    w = _random_weights(cfg, seed=5)
    m = LlamaPrefill(cfg, w, compress=compress)
    prompt = [int(t) for t in np.random.default_rng(11).integers(0, cfg.vocab, 150)]
    M = len(prompt) + 8
    d = m._decoder(M)
    assert d.prefill_supported()
    d.prefill(prompt, chunk=chunk)
    d.sync()
    batched = [(mx.kc.float().cpu().numpy(), mx.vc.float().cpu().numpy()) for mx, _ in d.layers]
    st_b = (int(d.pos.item()), int(d.step.item()), d.hist[:len(prompt) - 1].cpu().tolist(), d.h.float().cpu().numpy())
    d.reset(prompt)
    d.run(len(prompt) - 1, 0)
    d.sync()
    n = len(prompt) - 1
    for li, (mx, _) in enumerate(d.layers):
        for name, got, want in (("k", batched[li][0], mx.kc.float().cpu().numpy()),
                                ("v", batched[li][1], mx.vc.float().cpu().numpy())):
            g, w_ = got[..., :n, :], want[..., :n, :]
            if li == 0:     # same fp16 inputs: the two paths differ only in accumulation order
                check_f16(g, w_, what=f"layer {li} {name} cache")
            else:           # inputs already differ by fp16 ulps (GEMM vs GEMV order, fp16 P in the
                            # flash attention); both paths are held to the oracle by the tokens below
                assert cosine(g, w_) >= 0.9999, f"layer {li} {name}: cosine {cosine(g, w_):.6f}"
                tol = 2 * float(np.spacing(np.float16(np.abs(w_).max())))
                assert np.abs(g - w_).max() <= tol, f"layer {li} {name}: max err {np.abs(g - w_).max():.3e} > {tol:.3e}"
            assert not got[..., n:, :].any(), f"layer {li} {name}: rows past the prompt written"
    assert st_b[0] == int(d.pos.item()) == n and st_b[1] == int(d.step.item()) == n
    assert st_b[2] == prompt[1:] == d.hist[:n].cpu().tolist()
    np.testing.assert_array_equal(st_b[3], d.h.float().cpu().numpy())
    got = m.generate(prompt, max_new_tokens=8)
    want, lgs = ref.generate(prompt, 8, _effective(w, compress), _ocfg(cfg), M=M)
    _assert_tokens_match(got, want, lgs, f"batched prefill compress={compress}")
    m.release()


def test_greedy_near_tie_takes_the_host_fp32_choice_in_both_loops():
    """The reference recomputes a greedy step with the host fp32 head when the device head's top-2
    logits are within lmhead_tie_margin * max|logit| (aneforge/llm.py:281, 395-404;
    tests/test_lm_head.py:186-216).  Built case: the layers add nothing (wo = wdown = 0), so h is the
    token's embedding, whose first entry is positive; the final norm keeps only that entry; lm_head
    rows 3 and 7 differ by less than an fp16 ulp, so the fp16 head ties them exactly and its plain
    argmax is 3, while the fp32 head (hn * (1 + 2^-14) > hn * 1) picks 7 at every step."""
    from aneforge_amd.llm import LlamaConfig, LlamaPrefill
    say("greedy near-tie rule: graph loop, per-token loop, host head")
    D, V = 64, 32
    cfg = LlamaConfig(dim=D, n_layers=2, n_heads=4, n_kv_heads=2, ffn_dim=128, vocab=V)
    w = _random_weights(cfg, seed=3)
    for lw in w["layers"]:
        lw["wo"][:] = 0.0
        lw["wdown"][:] = 0.0
    rng = np.random.default_rng(4)
    w["embed"] = rng.standard_normal((V, D)).astype(np.float32)
    w["embed"][:, 0] = np.abs(w["embed"][:, 0]) + 0.5
    w["final_norm"] = np.zeros(D, np.float32)
    w["final_norm"][0] = 1.0
    head = np.zeros((V, D), np.float32)
    head[:, 0] = -0.5
    head[3, 0] = 1.0
    head[7, 0] = 1.0 + 2.0 ** -14
    assert np.float16(head[7, 0]) == np.float16(head[3, 0])
    w["lm_head"] = head
    m = LlamaPrefill(cfg, w)
    prompt = [1, 2, 5]
    assert m.generate(prompt, max_new_tokens=4) == [7, 7, 7, 7]                 # graph loop
    seen = []
    assert m.generate(prompt, max_new_tokens=4, on_token=seen.append) == [7, 7, 7, 7]   # per-token loop
    assert seen == [7, 7, 7, 7]
    assert m.generate(prompt, max_new_tokens=4, ane_lm_head=False) == [7, 7, 7, 7]     # host fp32 head
    m.lmhead_tie_margin = 0.0                                                    # rule off: fp16 tie
    assert m.generate(prompt, max_new_tokens=4) == [3, 3, 3, 3]
    m.lmhead_tie_margin = 3e-3
    assert m.generate(prompt, max_new_tokens=2) == [7, 7]
    m.release()


def _hf_tiny_gemma(head_dim=16, hidden=64, heads=4, kv=1, ffn=128, vocab=64):
    from transformers import GemmaConfig, GemmaForCausalLM
    hf_cfg = GemmaConfig(hidden_size=hidden, num_hidden_layers=2, num_attention_heads=heads, num_key_value_heads=kv,
                         head_dim=head_dim, intermediate_size=ffn, vocab_size=vocab, rms_norm_eps=1e-6,
                         max_position_embeddings=256, tie_word_embeddings=True)
    torch.manual_seed(0)
    m = GemmaForCausalLM(hf_cfg).eval()
    with torch.no_grad():
        for p in m.parameters():
            if p.dim() == 1:
                p.uniform_(-0.5, 0.5)                      # non-zero (1 + w) gains
            else:
                p.normal_(0.0, p.shape[1] ** -0.5)        # O(1) gate pre-activations: GeGLU != SwiGLU
    return m


def test_prefill_matches_huggingface_gemma():
    """The Gemma adapter on the device (aneforge tests/test_llm.py:120-135): the sqrt(dim) embedding,
    (1 + w) norms and the GeGLU MLP reproduce HF GemmaForCausalLM: cosine > 0.999 and the same argmax;
    greedy generation equals the oracle's (its GeGLU decoder is pinned to HF Gemma on the CPU)."""
    from aneforge_amd.llm import LlamaPrefill, _gemma_adapter
    say("prefill + generate vs Hugging Face Gemma")
    m = _hf_tiny_gemma()
    toks = [int(t) for t in np.random.default_rng(0).integers(0, 64, 10)]
    with torch.no_grad():
        want = m(torch.tensor(toks)[None]).logits[0, -1].numpy()
    sd = {k: v.detach().float().numpy() for k, v in m.state_dict().items()}
    cfg, w = _gemma_adapter(m.config, sd)
    lp = LlamaPrefill(cfg, w)
    got = lp.prefill(toks)[0]
    assert cosine(got, want) > 0.999 and int(np.argmax(got)) == int(np.argmax(want))
    gen = lp.generate(toks, max_new_tokens=8)
    oc = dict(_ocfg(cfg), mlp="geglu")
    ow = _effective(w, None)                            # the fp16 tables and weights the device holds
    ref_toks, lgs = ref.generate(toks, 8, ow, oc, M=len(toks) + 8)
    _assert_tokens_match(gen, ref_toks, lgs, "gemma generate")
    lp.release()


@pytest.mark.parametrize("compress", [None, "int8"])
def test_gemma_batched_prefill_geglu_matches_forced_steps(compress):
    """Head dim 128, so the batched prefill runs (the GEMM's GeGLU epilogue): the same cache and the
    same greedy continuation as the token-by-token forced steps."""
    from aneforge_amd.llm import LlamaPrefill, _gemma_adapter
    say(f"gemma batched prefill (GeGLU GEMM) compress={compress}")
    m = _hf_tiny_gemma(head_dim=128, hidden=256, heads=2, kv=1, ffn=512, vocab=128)
    sd = {k: v.detach().float().numpy() for k, v in m.state_dict().items()}
    cfg, w = _gemma_adapter(m.config, sd)
    lp = LlamaPrefill(cfg, w, compress=compress)
    prompt = [int(t) for t in np.random.default_rng(12).integers(0, 128, 40)]
    d = lp._decoder(len(prompt) + 8)
    assert d.prefill_supported()
    d.prefill(prompt)
    d.sync()
    batched = [mx.kc.float().cpu().numpy()[0, :, :len(prompt) - 1] for mx, _ in d.layers]
    d.reset(prompt)
    d.run(len(prompt) - 1, 0)
    d.sync()
    stepped = [mx.kc.float().cpu().numpy()[0, :, :len(prompt) - 1] for mx, _ in d.layers]
    for li, (g_, w_) in enumerate(zip(batched, stepped)):
        if li == 0:         # same fp16 embeddings: the paths differ in accumulation order (standalone norm +
                            # GEMM vs the GEMV's fused norm), so an fp16 rounding may land one ulp apart
            check_hidden(g_, w_, what="gemma layer 0 k cache: batched prefill vs forced steps")
        else:               # inputs already differ by fp16 ulps (the GeGLU GEMM vs GEMV order)
            assert cosine(g_, w_) >= 0.9999, f"gemma layer {li}: cosine {cosine(g_, w_):.6f}"
            tol = 2 * float(np.spacing(np.float16(np.abs(w_).max())))
            assert np.abs(g_ - w_).max() <= tol, f"gemma layer {li}: max err {np.abs(g_ - w_).max():.3e} > {tol:.3e}"
    a = lp.generate(prompt, max_new_tokens=6, batched_prefill=True)
    b = lp.generate(prompt, max_new_tokens=6, batched_prefill=False)
    oc = dict(_ocfg(cfg), mlp="geglu")
    ow = _effective(w, compress)
    want, lgs = ref.generate(prompt, 6, ow, oc, M=len(prompt) + 6)
    _assert_tokens_match(a, want, lgs, "gemma batched prefill generate")
    _assert_tokens_match(b, want, lgs, "gemma stepped generate")
    lp.release()
