"""The reference's Python API on the device: af.compile (compress= encodings, fallback gate),
af.sdpa, the graph ops of the decode/MoE graphs, compile_multi + Program.share_buffer, the
sparse MoE decode executor, QK-norm decoders, and moe.load_gguf on a GGUF written by this
package.  Checked against the oracle (and Hugging Face where the reference does)."""
import math
import warnings

import numpy as np
import pytest

from _util import check_f16, check_hidden, cosine, dev, host, say
from oracle import ref

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
import aneforge_amd as af  # noqa: E402


def test_compile_int8_linear_cfg0():
    """The cfg0 call stack: af.compile(af.input((1, K)).linear(W), compress="int8")(x)."""
    say("af.compile int8 linear 4096x4096")
    rng = np.random.default_rng(0)
    W = rng.standard_normal((4096, 4096)).astype(np.float32) * 0.02
    x = rng.standard_normal((1, 4096)).astype(np.float16)
    m = af.compile(af.input((1, 4096)).linear(W), compress="int8")
    got = m(x)
    want = ref.linear(x, ref.dequant_w8(*ref.quantize_per_row(W)))
    check_f16(got, want, what="compile int8")
    assert got.dtype == np.float32 and m.n_ops == 1
    m.release()


def test_compile_many_row_linear_is_one_contraction():
    """af.compile(af.input((2048, 4096)).linear(W), compress="int8"): the reference emits one matmul for
    any M (aneforge/_compile.py:375-385); here the 2048 rows run as one MFMA GEMM that streams the weight
    once per 128-row tile, checked against the oracle and timed against the same rows as 8-row GEMV
    launches (each re-streaming the whole weight), both as captured graphs."""
    import time
    from aneforge_amd import _kernels as K
    say("af.compile int8 linear [2048 x 4096] x [4096 x 4096]: one contraction")
    rng = np.random.default_rng(5)
    M, N, Kd = 2048, 4096, 4096
    W = rng.standard_normal((N, Kd)).astype(np.float32) * 0.02
    x = rng.standard_normal((M, Kd)).astype(np.float16)
    m = af.compile(af.input((M, Kd)).linear(W), compress="int8")
    got = m(x)
    q, s = ref.quantize_per_row(W)
    rows = rng.choice(M, 96, replace=False)                       # oracle rows (float64 on the host)
    check_f16(got[rows], ref.linear(x[rows], ref.dequant_w8(q, s)), what="compile int8 M=2048")

    def best(fn, reps=5):
        fn()
        torch.cuda.synchronize()
        out = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            out.append(time.perf_counter() - t0)
        return min(out)
    t_one = best(m.execute)
    wq, ws_ = dev(q), dev(s)
    xd = m.input_view().reshape(M, Kd)
    yd = torch.empty((M, N), dtype=torch.float16, device="cuda")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for r0 in range(0, M, 8):
            K.linear("int8", wq, ws_, xd[r0:r0 + 8], y=yd[r0:r0 + 8])
    t_rows = best(g.replay)
    say(f"one contraction {t_one * 1e3:.3f} ms, 8-row launches {t_rows * 1e3:.3f} ms ({t_rows / t_one:.1f}x)")
    check_f16(host(yd)[rows], got[rows], what="8-row form")
    assert t_rows >= 10 * t_one
    m.release()


@pytest.mark.parametrize("compress", [None, "q4_0", "blockwise", "int4", "int8"])
@pytest.mark.parametrize("M", [5, 40])
def test_compile_multi_row_linear_formats(compress, M):
    """Up to 16 rows one afx_linear launch (skinny MFMA), more rows the GEMM (packed int8 / fp16, or
    the fp16 expansion of the other encodings), each with a bias, against the oracle."""
    say(f"af.compile multi-row linear compress={compress} M={M}")
    rng = np.random.default_rng(6)
    W = rng.standard_normal((256, 512)).astype(np.float32) * 0.05
    b = rng.standard_normal(256).astype(np.float32)
    x = rng.standard_normal((M, 512)).astype(np.float16)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        got = af.compile(af.input((M, 512)).linear(W, b), compress=compress, compress_atol=0.5)(x)
    if compress is None:
        Wf = W.astype(np.float16).astype(np.float32)
    elif compress == "q4_0":
        Wf = ref.dequant_q4_0_f16(ref.quantize_q4_0(W), 256, 512)
    elif compress == "blockwise":
        q, s, bs = ref.quantize_blockwise(W, 32)
        Wf = (q.reshape(256, 16, 32) * s.astype(np.float32)[:, :, None]).reshape(256, 512).astype(np.float16).astype(np.float32)
    elif compress == "int4":
        from aneforge_amd import _blob
        packed, cb = _blob.palettize_lut4(W)
        Wf = ref.dequant_lut4(packed, cb, 512)
    else:
        Wf = ref.dequant_w8(*ref.quantize_per_row(W))
    check_f16(got, ref.linear(x, Wf, b.astype(np.float16)), what=f"{compress} M={M}")


@pytest.mark.parametrize("compress", [None, "q4_0", "blockwise", "int4", "sparse", "auto"])
def test_compile_encodings(compress):
    say(f"af.compile encodings compress={compress}")
    rng = np.random.default_rng(1)
    W = rng.standard_normal((96, 256)).astype(np.float32)
    b = rng.standard_normal(96).astype(np.float32)
    x = rng.standard_normal((3, 256)).astype(np.float16)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        got = af.compile(af.input((3, 256)).linear(W, b), compress=compress, compress_atol=0.5)(x)
    if compress is None or compress == "sparse":
        Wf = W.astype(np.float16).astype(np.float32)
    elif compress == "q4_0":
        Wf = ref.dequant_q4_0_f16(ref.quantize_q4_0(W), 96, 256)
    elif compress == "blockwise":
        q, s, bs = ref.quantize_blockwise(W, 32)
        Wf = (q.reshape(96, 8, 32) * s.astype(np.float32)[:, :, None]).reshape(96, 256).astype(np.float16).astype(np.float32)
    elif compress == "auto":
        Wf = ref.dequant_w8(*ref.quantize_per_row(W))
    else:
        Wf = None
    if Wf is not None:
        check_f16(got, ref.linear(x, Wf, b.astype(np.float16)), what=str(compress))
    else:   # LUT4 codebook: only loosely pinned, compare to the float weights
        assert cosine(got, x.astype(np.float64) @ W.T.astype(np.float64) + b) > 0.95


def test_compress_fallback_warns_and_widens():
    say("compress=int4 with a tight atol falls back to int8 with a warning")
    rng = np.random.default_rng(2)
    W = rng.standard_normal((64, 128)).astype(np.float32)
    x = rng.standard_normal((1, 128)).astype(np.float16)
    with pytest.warns(af.CompressionFallbackWarning, match="rejected 1/1"):
        m = af.compile(af.input((1, 128)).linear(W), compress="int4", compress_atol=1e-6)
    check_f16(m(x), ref.linear(x, ref.dequant_w8(*ref.quantize_per_row(W))), what="int4->int8")


def test_rope_graph_matches_oracle():
    # aneforge tests/test_llm.py:29-36
    say("rope graph")
    cos, sin = af.rope_tables(8, 16)
    x = np.random.default_rng(0).standard_normal((1, 2, 8, 16)).astype(np.float16)
    got = af.compile(af.rope(af.input((1, 2, 8, 16)), cos, sin))(x)
    want = ref.rope(x.astype(np.float64), cos.astype(np.float64), sin.astype(np.float64), exact=True)
    assert cosine(got, want) > 0.9999
    assert np.abs(got - want).max() < 1e-2


@pytest.mark.parametrize("H,Hkv,Sq,Skv,D,mode", [(1, 1, 1, 4, 8, "plain"), (2, 2, 1, 8, 16, "plain"),
                                                 (2, 2, 3, 8, 16, "plain"), (4, 4, 6, 6, 64, "causal"),
                                                 (2, 2, 5, 9, 32, "mask"), (8, 2, 1, 300, 128, "plain")])
def test_sdpa(H, Hkv, Sq, Skv, D, mode):
    # aneforge tests/test_sdpa_causal.py:13-91 shapes + a GQA decode case
    say(f"af.sdpa H={H} Hkv={Hkv} Sq={Sq} Skv={Skv} D={D} {mode}")
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, H, Sq, D)).astype(np.float16)
    k = rng.standard_normal((1, Hkv, Skv, D)).astype(np.float16)
    v = rng.standard_normal((1, Hkv, Skv, D)).astype(np.float16)
    ins = [af.input((1, H, Sq, D)), af.input((1, Hkv, Skv, D)), af.input((1, Hkv, Skv, D))]
    feed = [q, k, v]
    mask = None
    if mode == "mask":
        mask = rng.standard_normal((1, 1, Sq, Skv)).astype(np.float16)
        ins.append(af.input((1, 1, Sq, Skv)))
        feed.append(mask)
    out = af.sdpa(*ins[:3], is_causal=mode == "causal", attn_mask=ins[3] if mode == "mask" else None)
    got = af.compile(out)(*feed)
    if mode == "causal":
        want = np.concatenate([ref.attention(q[:, :, s:s + 1], k, v, lengths=[s + 1]) for s in range(Sq)], axis=2)
    else:
        want = ref.attention(q, k, v, mask=None if mask is None else mask[0, 0])
    check_f16(got, want, what=f"sdpa {mode}")


@pytest.mark.parametrize("masked", [False, True])
def test_sdpa_long_query(masked):
    """The reference's query-tiled case (tests/test_sdpa_causal.py:72-91): H 4, S 1500, D 64, plain and
    with a [1, 1, S, S] additive mask, here one decode-kernel row per query (the mask row is that
    query's), against the oracle at the fp16 bar."""
    H, S, D = 4, 1500, 64
    say(f"af.sdpa long query H={H} S={S} D={D} masked={masked}")
    rng = np.random.default_rng(7)
    q, k, v = (rng.standard_normal((1, H, S, D)).astype(np.float16) for _ in range(3))
    ins = [af.input((1, H, S, D)) for _ in range(3)]
    feed = [q, k, v]
    mask = None
    if masked:
        mask = rng.standard_normal((1, 1, S, S)).astype(np.float16)
        ins.append(af.input((1, 1, S, S)))
        feed.append(mask)
    got = af.compile(af.sdpa(*ins[:3], attn_mask=ins[3] if masked else None))(*feed)
    assert tuple(np.asarray(got).shape) == (1, H, S, D)
    want = ref.attention(q, k, v, mask=None if mask is None else mask[0, 0])
    check_f16(got, want, what=f"sdpa S={S} masked={masked}")


def test_topk_gate_exact_ties_select_exactly_k():
    # aneforge tests/test_moe.py:95-108, through af.compile
    say("_topk_gate tie KAT through compile")
    rows = np.array([[0.2, 0.2, 0.2, 0.1, 0.1, 0.1, 0.05, 0.05],
                     [0.3, 0.2, 0.2, 0.2, 0.05, 0.03, 0.01, 0.01],
                     [0.1, 0.1, 0.1, 0.1, 0.1, 0.1, 0.2, 0.2],
                     [0.4, 0.3, 0.1, 0.1, 0.05, 0.03, 0.01, 0.01]], np.float16)
    got = af.compile(af.moe._topk_gate(af.input((4, 8)), 2, 8, 4))(rows)
    want = [[0, 1], [0, 1], [6, 7], [0, 1]]
    for t in range(4):
        nz = sorted(np.flatnonzero(got[t]).tolist())
        assert nz == want[t]
        assert np.allclose(got[t, nz], rows[t, nz].astype(np.float32))


def _moe_weights(E, D, F, seed=0):
    rng = np.random.default_rng(seed)
    R = lambda *s: (rng.standard_normal(s) / np.sqrt(s[-1])).astype(np.float32)
    return {"mlp_norm": np.ones(D, np.float32), "router": R(E, D), "wgate_exps": R(E, F, D), "wup_exps": R(E, F, D),
            "wdown_exps": R(E, F, D)}


def test_moe_graph_matches_reference_oracle():
    # aneforge tests/test_moe.py:48-57 (cosine > 0.99 there): held to the path's bar here, against the
    # oracle at the kernels' fp16 rounding points with the fp16 weights the layer streams
    say("_moe graph through compile")
    cfg = af.LlamaConfig(dim=32, n_layers=1, n_heads=4, n_kv_heads=2, ffn_dim=16, vocab=16,
                         extra={"n_experts": 8, "n_experts_per_tok": 2, "norm_topk_prob": True})
    w = _moe_weights(8, 32, 16)
    f16 = lambda a: np.asarray(a, np.float32).astype(np.float16).astype(np.float32)
    for T in (1, 5, 12):
        h = (np.random.default_rng(T).standard_normal((T, 32)) * 0.5).astype(np.float16)
        got = af.compile(af.moe._moe(af.input((T, 32)), w, cfg, af.LayerSpec(mlp="moe")))(h)
        want, _, _ = ref.moe_layer(h, w["mlp_norm"], f16(w["router"]), f16(w["wgate_exps"]), f16(w["wup_exps"]),
                                   f16(np.ascontiguousarray(w["wdown_exps"].transpose(0, 2, 1))), 2, True, 1e-5)
        check_hidden(got, want, what=f"moe graph T={T}")


def _bmm_reference_weights(W, compress, atol, block_size=32):
    """The weights the reference bakes for bmm_weight(W) (aneforge/_compile.py:112-188 on
    W.reshape(B, K*N), :393-399), as fp32 [B, K, N]."""
    from aneforge_amd import _blob
    B, Kd, N = W.shape
    flat = W.reshape(B, Kd * N)
    rel = lambda rec: np.linalg.norm(rec - flat) / np.linalg.norm(flat)
    if compress == "int4":
        packed, cb = _blob.palettize_lut4(flat)              # pinned by the reference's own vectors
        rec = ref.dequant_lut4(packed, cb, Kd * N)
        if rel(rec) <= atol:
            return rec.reshape(W.shape), "lut4"
        compress = "int8"
    if compress == "blockwise":
        q, s, bs = ref.quantize_blockwise(flat, block_size)
        rec = ref.dequant_blockwise(q, s, bs)
        if rel(rec) <= atol:
            return rec.reshape(W.shape), "blockwise"
        return flat.astype(np.float16).astype(np.float32).reshape(W.shape), "fp16"
    if compress == "int8":
        return ref.dequant_w8(*ref.quantize_per_row(flat)).reshape(W.shape), "int8"
    return flat.astype(np.float16).astype(np.float32).reshape(W.shape), "fp16"


@pytest.mark.parametrize("compress,atol,K,want_kind", [
    (None, 0.05, 64, "fp16"), ("int8", 0.05, 64, "int8"), ("int4", 0.3, 64, "lut4"), ("int4", 0.3, 40, "lut4"),
    ("int4", 1e-4, 64, "int8"), ("blockwise", 0.05, 64, "blockwise"), ("blockwise", 1e-5, 64, "fp16")])
def test_bmm_weight_encodings(compress, atol, K, want_kind):
    """x [B, M, K] @ W [B, K, N] through af.compile: the reference's bmm encoding precedence (int4 ->
    LUT4 or int8 with one scale per batch; blockwise -> blockwise along K*N or fp16)."""
    say(f"bmm_weight compress={compress} atol={atol} K={K}")
    rng = np.random.default_rng(30)
    B, M, N = 3, 2, 48
    W = (rng.standard_normal((B, K, N)) * np.array([0.5, 1.0, 2.0])[:, None, None]).astype(np.float32)
    x = rng.standard_normal((B, M, K)).astype(np.float16)
    Wr, kind = _bmm_reference_weights(W, compress, atol)
    assert kind == want_kind
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        got = af.compile(af.input((B, M, K)).bmm_weight(W), compress=compress, compress_atol=atol)(x)
    for b in range(B):
        check_f16(got[b], ref.linear(x[b], np.ascontiguousarray(Wr[b].T)), what=f"bmm {compress} batch {b}")


def test_compile_multi_share_buffer_keeps_state_resident():
    say("compile_multi + share_buffer resident state")
    x = af.input((1, 8))
    s = af.input((1, 8))
    y = s + x
    mm = af.compile_multi([y])
    inm = {id(t): n for t, n in mm.input_ports}
    om = dict(mm.output_ports)
    mm.prog.share_buffer(0, om[y], 0, inm[id(s)])
    mm.prog.set_input(inm[id(s)], np.zeros((1, 8), np.float16))
    mm.prog.set_input(inm[id(x)], np.full((1, 8), 0.5, np.float16))
    assert mm.prog.shared_in_place(om[y])                       # y is written into s's buffer
    assert mm.prog.output_view(om[y]).data_ptr() == mm.prog.input_view(inm[id(s)]).data_ptr()
    for _ in range(3):
        mm.prog.execute()
    assert np.allclose(mm.prog.read_output(om[y]).astype(np.float32), 1.5)
    with pytest.raises(RuntimeError):
        mm.prog.share_buffer(0, om[y], 0, inm[id(s)])      # only before the first execute


def test_share_buffer_copies_when_in_place_would_change_a_result():
    # z reads the state after y (the new state) is computed: an in-place y would hand z the new
    # value, so the program keeps s and copies y into it after each execute
    say("share_buffer hazard: copy fallback")
    x, s = af.input((1, 8)), af.input((1, 8))
    y = s + x
    z = (s * 2.0) + y
    mm = af.compile_multi([y, z])
    inm = {id(t): n for t, n in mm.input_ports}
    om = dict(mm.output_ports)
    mm.prog.share_buffer(0, om[y], 0, inm[id(s)])
    assert not mm.prog.shared_in_place(om[y])
    mm.prog.set_input(inm[id(s)], np.full((1, 8), 1.0, np.float16))
    mm.prog.set_input(inm[id(x)], np.full((1, 8), 0.5, np.float16))
    for step in range(3):
        mm.prog.execute()
        sv = 1.0 + 0.5 * step                                   # the state this execute read
        assert np.allclose(mm.prog.read_output(om[y]).astype(np.float32), sv + 0.5)
        assert np.allclose(mm.prog.read_output(om[z]).astype(np.float32), 2 * sv + sv + 0.5)


def _moe_model(E=8, k=2, D=128, F=128, layers=2, vocab=64, qk=False, seed=0, dh=32):
    rng = np.random.default_rng(seed)
    R = lambda *s: (rng.standard_normal(s) / np.sqrt(s[-1])).astype(np.float32)
    H, KV = 4, 2
    cfg = af.LlamaConfig(dim=D, n_layers=layers, n_heads=H, n_kv_heads=KV, ffn_dim=F, vocab=vocab,
                         layers=[af.LayerSpec(mlp="moe", qk_norm=qk) for _ in range(layers)],
                         extra={"n_experts": E, "n_experts_per_tok": k, "norm_topk_prob": True})
    w = {"embed": R(vocab, D), "final_norm": np.ones(D, np.float32), "lm_head": R(vocab, D), "layers": []}
    for _ in range(layers):
        lw = {"wq": R(H * dh, D), "wk": R(KV * dh, D), "wv": R(KV * dh, D), "wo": R(D, H * dh),
              "attn_norm": np.ones(D, np.float32)}
        lw.update(_moe_weights(E, D, F, seed=int(rng.integers(1 << 30))))
        if qk:
            lw["q_norm"] = rng.uniform(0.8, 1.2, dh).astype(np.float32)
            lw["k_norm"] = rng.uniform(0.8, 1.2, dh).astype(np.float32)
        w["layers"].append(lw)
    return cfg, w


def _lut4_rec(W):
    from aneforge_amd import _blob
    packed, cb = _blob.palettize_lut4(np.asarray(W, np.float32))
    return ref.dequant_lut4(packed, cb, np.asarray(W).shape[1])


def _oracle_weights(cfg, w, enc):
    ow = {"embed": w["embed"].astype(np.float16).astype(np.float32), "final_norm": w["final_norm"],
          "lm_head": w["lm_head"].astype(np.float16).astype(np.float32), "layers": []}
    for lw in w["layers"]:
        o = {k: enc(lw[k]) for k in ("wq", "wk", "wv", "wo")}
        o["attn_norm"] = lw["attn_norm"]
        if "q_norm" in lw:
            o["q_norm"], o["k_norm"] = lw["q_norm"].astype(np.float16), lw["k_norm"].astype(np.float16)
        if "router" in lw:
            o["router"] = lw["router"].astype(np.float16).astype(np.float32)
            o["mlp_norm"] = lw["mlp_norm"]
            o["wgate_exps"] = [enc(g) for g in lw["wgate_exps"]]
            o["wup_exps"] = [enc(u) for u in lw["wup_exps"]]
            o["wdown_exps"] = [enc(np.ascontiguousarray(d.T)) for d in lw["wdown_exps"]]
        ow["layers"].append(o)
    ocfg = {"n_heads": cfg.n_heads, "n_kv_heads": cfg.n_kv_heads, "dh": cfg.dh, "norm_eps": cfg.norm_eps,
            "rope_base": cfg.rope_base, "top_k": cfg.extra.get("n_experts_per_tok", 2), "norm_topk_prob": True}
    return ow, ocfg


@pytest.mark.parametrize("compress,qk", [(None, False), ("int8", True), ("q4_0", False), ("blockwise", False),
                                         ("int4", False)])
def test_moe_decoder_generate_matches_oracle(compress, qk):
    say(f"LlamaPrefill with MoE layers compress={compress} qk_norm={qk}")
    cfg, w = _moe_model(qk=qk)
    enc = {None: lambda W: np.asarray(W, np.float32).astype(np.float16).astype(np.float32),
           "int8": lambda W: ref.dequant_w8(*ref.quantize_per_row(W)),
           "blockwise": lambda W: ref.dequant_blockwise(*ref.quantize_blockwise(W, 32)),
           "int4": lambda W: _lut4_rec(W),
           "q4_0": lambda W: ref.dequant_q4_0_f16(ref.quantize_q4_0(W), *np.asarray(W).shape)}[compress]
    m = af.LlamaPrefill(cfg, w, compress=compress)
    prompt = [3, 9, 27, 1]
    got = m.generate(prompt, max_new_tokens=8)
    ow, ocfg = _oracle_weights(cfg, w, enc)
    want, lgs = ref.generate(prompt, 8, ow, ocfg, M=len(prompt) + 8)
    from test_gpu_llm import _assert_tokens_match
    _assert_tokens_match(got, want, lgs, f"moe {compress}")
    m.release()


@pytest.mark.parametrize("compress,qk", [(None, True), ("int8", False), ("int8", True)])
def test_batched_prefill_moe_and_qk_norm(compress, qk):
    """Batched prefill through MoE MLPs (grouped MFMA experts over the prompt rows) and QK-norm
    attention (per-head norm + RoPE on q and the cache rows): same state as the forced steps,
    generation as the oracle."""
    say(f"batched prefill MoE compress={compress} qk_norm={qk}")
    cfg, w = _moe_model(D=512, F=256, qk=qk, dh=128, seed=3)
    enc = {None: lambda W: np.asarray(W, np.float32).astype(np.float16).astype(np.float32),
           "int8": lambda W: ref.dequant_w8(*ref.quantize_per_row(W))}[compress]
    m = af.LlamaPrefill(cfg, w, compress=compress)
    prompt = [int(t) for t in np.random.default_rng(8).integers(0, cfg.vocab, 90)]
    M = len(prompt) + 8
    d = m._decoder(M)
    assert d.prefill_supported()
    d.prefill(prompt)
    d.sync()
    kb = [mx.kc.float().cpu().numpy() for mx, _ in d.layers]
    d.reset(prompt)
    d.run(len(prompt) - 1, 0)
    d.sync()
    n = len(prompt) - 1
    for li, (mx, _) in enumerate(d.layers):
        want_k = mx.kc.float().cpu().numpy()[..., :n, :]
        assert cosine(kb[li][..., :n, :], want_k) >= 0.9999, f"layer {li} k cache"
    got = m.generate(prompt, max_new_tokens=6)
    ow, ocfg = _oracle_weights(cfg, w, enc)
    want, lgs = ref.generate(prompt, 6, ow, ocfg, M=M)
    from test_gpu_llm import _assert_tokens_match
    _assert_tokens_match(got, want, lgs, f"batched prefill moe {compress} qk={qk}")
    m.release()


def test_qk_norm_decoder_matches_hf_qwen3():
    """Qwen3 (QK-norm) prefill on the device vs Hugging Face Qwen3ForCausalLM (tiny, random)."""
    from transformers import Qwen3Config, Qwen3ForCausalLM
    say("QK-norm decoder vs HF Qwen3")
    hc = Qwen3Config(hidden_size=128, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2, head_dim=32,
                     intermediate_size=256, vocab_size=64, rms_norm_eps=1e-6, max_position_embeddings=64)
    torch.manual_seed(0)
    hf = Qwen3ForCausalLM(hc).eval()
    for n, p in hf.named_parameters():
        if "norm" in n:
            torch.nn.init.uniform_(p, 0.8, 1.2)
    toks = np.random.default_rng(1).integers(0, 64, 9)
    with torch.no_grad():
        want = hf(torch.tensor(toks)[None]).logits[0, -1].numpy()
    sd = {k: v.detach().float().numpy() for k, v in hf.state_dict().items()}
    cfg, weights = af.llm._dense_adapter(hf.config, sd)
    assert all(ls.qk_norm for ls in cfg.layers)
    got = af.LlamaPrefill(cfg, weights).prefill(toks)[0]
    assert cosine(got, want) > 0.999 and int(np.argmax(got)) == int(np.argmax(want))


def _kq_rows(kind, rows, K, rng):
    """Random valid K-quant rows (block bytes [rows, K / 256 * block size]) with weights of about
    0.05-0.1, packed by the element-by-element encoders of test_gguf_codecs."""
    from test_gguf_codecs import enc_q4_k, enc_q5_k, enc_q6_k
    out = []
    for _ in range(rows * K // 256):
        if kind == "Q6_K":
            out.append(enc_q6_k(0.0005, [int(v) for v in rng.integers(-16, 16, 16)],
                                [int(v) for v in rng.integers(-32, 32, 256)]))
        elif kind == "Q4_K":
            sc = [int(v) for v in rng.integers(4, 9, 8)]
            out.append(enc_q4_k(0.002, 0.002, sc, [round(7.5 * s) for s in sc], [int(v) for v in rng.integers(0, 16, 256)]))
        else:
            sc = [int(v) for v in rng.integers(2, 5, 8)]
            out.append(enc_q5_k(0.002, 0.002, sc, [round(15.5 * s) for s in sc], [int(v) for v in rng.integers(0, 32, 256)]))
    return np.frombuffer(b"".join(out), np.uint8).reshape(rows, -1)


def test_load_gguf_k_quant_file(tmp_path):
    """A Q4_K_M-style Qwen3-MoE GGUF (Q4_K gate/up experts, Q6_K down experts and attention,
    fp16 elsewhere): the experts stream as their Q4_K / Q6_K codes, the attention weights are
    dequantised on the host to fp16 as the reference's GGUFView.get does (aneforge/_gguf.py:34-39),
    and the decode matches the oracle over the same fp16 weights."""
    from aneforge_amd import _gguf
    say("moe.load_gguf on a synthetic K-quant GGUF")
    E, D, F, L, dh, H, KV = 4, 256, 256, 1, 64, 4, 2
    cfg, w = _moe_model(E=E, D=D, F=F, layers=L, qk=True, seed=9, dh=dh)
    rng = np.random.default_rng(9)
    dec = lambda kind, raw, rows, K: _gguf.dequantize_blocks(_gguf.GGML[kind], raw).reshape(rows, K)
    tensors = {"token_embd.weight": w["embed"].astype(np.float16), "output_norm.weight": w["final_norm"],
               "output.weight": w["lm_head"].astype(np.float16)}
    for i, lw in enumerate(w["layers"]):
        b = f"blk.{i}."
        for key, nm, rows in (("wq", "attn_q", H * dh), ("wk", "attn_k", KV * dh), ("wv", "attn_v", KV * dh),
                              ("wo", "attn_output", D)):
            raw = _kq_rows("Q6_K", rows, 256, rng)
            tensors[b + nm + ".weight"] = ("Q6_K", raw, (rows, 256))
            lw[key] = dec("Q6_K", raw, rows, 256)
        tensors.update({b + "attn_norm.weight": lw["attn_norm"], b + "ffn_norm.weight": lw["mlp_norm"],
                        b + "ffn_gate_inp.weight": lw["router"].astype(np.float16),
                        b + "attn_q_norm.weight": lw["q_norm"], b + "attn_k_norm.weight": lw["k_norm"]})
        for key, nm in (("wgate_exps", "ffn_gate_exps"), ("wup_exps", "ffn_up_exps")):
            raws = [_kq_rows("Q4_K", F, D, rng) for _ in range(E)]
            tensors[b + nm + ".weight"] = ("Q4_K", np.concatenate(raws), (E, F, D))
            lw[key] = np.stack([dec("Q4_K", r, F, D) for r in raws])
        raws = [_kq_rows("Q6_K", D, F, rng) for _ in range(E)]               # GGUF down: [E, dim, ffn]
        tensors[b + "ffn_down_exps.weight"] = ("Q6_K", np.concatenate(raws), (E, D, F))
        lw["wdown_exps"] = np.stack([dec("Q6_K", r, D, F).T for r in raws])   # canonical [E, ffn, dim]
    meta = {"general.architecture": "qwen3moe", "qwen3moe.block_count": L, "qwen3moe.expert_count": E,
            "qwen3moe.expert_used_count": 2, "qwen3moe.embedding_length": D, "qwen3moe.attention.head_count": H,
            "qwen3moe.attention.head_count_kv": KV, "qwen3moe.attention.key_length": dh,
            "qwen3moe.rope.freq_base": 10000.0, "qwen3moe.attention.layer_norm_rms_epsilon": 1e-5}
    path = str(tmp_path / "tiny-moe-kq.gguf")
    _gguf.write_gguf(path, meta, tensors)
    m = af.moe.load_gguf(path)
    assert m.cfg.extra["n_experts"] == E and m.cfg.layers[0].qk_norm
    prompt = [5, 6, 7]
    got = m.generate(prompt, max_new_tokens=6)
    mlp = m._layers[0][1]                              # layers materialise on first use
    assert mlp.gu.fmt == "q4_k" and mlp.down.fmt == "q6_k"   # the experts stream as their K-quant codes
    enc16 = lambda W: np.asarray(W, np.float32).astype(np.float16).astype(np.float32)
    ow, ocfg = _oracle_weights(cfg, w, enc16)
    want, lgs = ref.generate(prompt, 6, ow, ocfg, M=len(prompt) + 6)
    from test_gpu_llm import _assert_tokens_match
    _assert_tokens_match(got, want, lgs, "gguf k-quants")


def _q8_0_rows(W):
    """Float rows [n, K] -> GGUF Q8_0 block bytes [n, K/32*34] (d = max|w| / 127 per block)."""
    W = np.asarray(W, np.float32)
    n, K = W.shape
    b = W.reshape(n, K // 32, 32)
    d = (np.abs(b).max(axis=2) / 127.0).astype(np.float16)
    q = np.clip(np.rint(b / np.maximum(d.astype(np.float32), 1e-8)[:, :, None]), -127, 127).astype(np.int8)
    out = np.empty((n, K // 32, 34), np.uint8)
    out[:, :, :2] = d.view(np.uint8).reshape(n, K // 32, 2)
    out[:, :, 2:] = q.view(np.uint8)
    return out.reshape(n, -1)


def test_load_gguf_q8_0_experts_stream_as_blockwise(tmp_path):
    """Q8_0 expert tensors stream as their own int8 codes + block scales (the blockwise kernels),
    and the decode matches the oracle over fp16(d * q), the reference's GGUFView.get weights."""
    from aneforge_amd import _gguf
    say("moe.load_gguf on a synthetic Q8_0-expert GGUF")
    cfg, w = _moe_model(qk=False, seed=6)
    E, D, F, L = 8, 128, 128, 2
    tensors = {"token_embd.weight": w["embed"].astype(np.float16), "output_norm.weight": w["final_norm"],
               "output.weight": w["lm_head"].astype(np.float16)}
    dq = lambda raw, n, K: _gguf.dequantize_blocks(_gguf.GGML["Q8_0"], raw).reshape(n, K)
    for i, lw in enumerate(w["layers"]):
        b = f"blk.{i}."
        tensors.update({b + "attn_q.weight": lw["wq"].astype(np.float16), b + "attn_k.weight": lw["wk"].astype(np.float16),
                        b + "attn_v.weight": lw["wv"].astype(np.float16),
                        b + "attn_output.weight": lw["wo"].astype(np.float16), b + "attn_norm.weight": lw["attn_norm"],
                        b + "ffn_norm.weight": lw["mlp_norm"], b + "ffn_gate_inp.weight": lw["router"].astype(np.float16)})
        for key, nm in (("wgate_exps", "ffn_gate_exps"), ("wup_exps", "ffn_up_exps")):
            raws = [_q8_0_rows(lw[key][e]) for e in range(E)]
            tensors[b + nm + ".weight"] = ("Q8_0", np.concatenate(raws), (E, F, D))
            lw[key] = np.stack([dq(r, F, D) for r in raws])
        raws = [_q8_0_rows(np.ascontiguousarray(lw["wdown_exps"][e].T)) for e in range(E)]
        tensors[b + "ffn_down_exps.weight"] = ("Q8_0", np.concatenate(raws), (E, D, F))
        lw["wdown_exps"] = np.stack([dq(r, D, F).T for r in raws])
    meta = {"general.architecture": "qwen3moe", "qwen3moe.block_count": L, "qwen3moe.expert_count": E,
            "qwen3moe.expert_used_count": 2, "qwen3moe.embedding_length": D, "qwen3moe.attention.head_count": 4,
            "qwen3moe.attention.head_count_kv": 2, "qwen3moe.attention.key_length": 32,
            "qwen3moe.rope.freq_base": 10000.0, "qwen3moe.attention.layer_norm_rms_epsilon": 1e-5}
    path = str(tmp_path / "tiny-moe-q8.gguf")
    _gguf.write_gguf(path, meta, tensors)
    m = af.moe.load_gguf(path)
    prompt = [5, 6, 7]
    got = m.generate(prompt, max_new_tokens=6)
    mlp = m._layers[0][1]
    assert mlp.gu.fmt == "blockwise" and mlp.down.fmt == "blockwise"
    enc16 = lambda W: np.asarray(W, np.float32).astype(np.float16).astype(np.float32)
    ow, ocfg = _oracle_weights(cfg, w, enc16)
    want, lgs = ref.generate(prompt, 6, ow, ocfg, M=len(prompt) + 6)
    from test_gpu_llm import _assert_tokens_match
    _assert_tokens_match(got, want, lgs, "gguf q8_0")


def test_load_gguf_q4_0_experts_stay_4bit(tmp_path):
    """A synthetic Qwen3-MoE GGUF (Q4_0 experts, fp16 elsewhere) written by aneforge_amd._gguf:
    load_gguf streams the file's own codes (bit-identical to the file) and decodes like the oracle."""
    from aneforge_amd import _gguf
    say("moe.load_gguf on a synthetic Q4_0 GGUF")
    cfg, w = _moe_model(qk=True, seed=5)
    E, D, F, L = 8, 128, 128, 2
    tensors = {"token_embd.weight": w["embed"].astype(np.float16), "output_norm.weight": w["final_norm"],
               "output.weight": w["lm_head"].astype(np.float16)}
    for i, lw in enumerate(w["layers"]):
        b = f"blk.{i}."
        tensors.update({b + "attn_q.weight": lw["wq"].astype(np.float16), b + "attn_k.weight": lw["wk"].astype(np.float16),
                        b + "attn_v.weight": lw["wv"].astype(np.float16),
                        b + "attn_output.weight": lw["wo"].astype(np.float16), b + "attn_norm.weight": lw["attn_norm"],
                        b + "ffn_norm.weight": lw["mlp_norm"], b + "ffn_gate_inp.weight": lw["router"].astype(np.float16),
                        b + "attn_q_norm.weight": lw["q_norm"], b + "attn_k_norm.weight": lw["k_norm"]})
        gate = np.concatenate([ref.quantize_q4_0(lw["wgate_exps"][e]) for e in range(E)])
        up = np.concatenate([ref.quantize_q4_0(lw["wup_exps"][e]) for e in range(E)])
        down = np.concatenate([ref.quantize_q4_0(np.ascontiguousarray(lw["wdown_exps"][e].T)) for e in range(E)])
        tensors[b + "ffn_gate_exps.weight"] = ("Q4_0", gate, (E, F, D))
        tensors[b + "ffn_up_exps.weight"] = ("Q4_0", up, (E, F, D))
        tensors[b + "ffn_down_exps.weight"] = ("Q4_0", down, (E, D, F))
    meta = {"general.architecture": "qwen3moe", "qwen3moe.block_count": L, "qwen3moe.expert_count": E,
            "qwen3moe.expert_used_count": 2, "qwen3moe.embedding_length": D, "qwen3moe.attention.head_count": 4,
            "qwen3moe.attention.head_count_kv": 2, "qwen3moe.attention.key_length": 32,
            "qwen3moe.rope.freq_base": 10000.0, "qwen3moe.attention.layer_norm_rms_epsilon": 1e-5}
    path = str(tmp_path / "tiny-moe.gguf")
    _gguf.write_gguf(path, meta, tensors)
    m = af.moe.load_gguf(path)
    assert m.cfg.extra["n_experts"] == E and m.cfg.layers[0].qk_norm and m.cfg.layers[0].mlp == "moe"
    prompt = [5, 6, 7]
    got = m.generate(prompt, max_new_tokens=6)
    mlp = m._layers[0][1]
    assert mlp.gu.fmt == "q4_0" and mlp.down.fmt == "q4_0"
    back = af._kernels.q4_unpack(mlp.down.w[:D], mlp.down.scale[:D], D, F)
    assert np.array_equal(back.cpu().numpy(), ref.quantize_q4_0(np.ascontiguousarray(w["layers"][0]["wdown_exps"][0].T)))
    enc16 = lambda W: np.asarray(W, np.float32).astype(np.float16).astype(np.float32)
    ow, ocfg = _oracle_weights(cfg, w, enc16)
    for i, lw in enumerate(w["layers"]):
        ow["layers"][i]["wgate_exps"] = [ref.dequant_q4_0_f16(ref.quantize_q4_0(g), F, D) for g in lw["wgate_exps"]]
        ow["layers"][i]["wup_exps"] = [ref.dequant_q4_0_f16(ref.quantize_q4_0(u), F, D) for u in lw["wup_exps"]]
        ow["layers"][i]["wdown_exps"] = [ref.dequant_q4_0_f16(ref.quantize_q4_0(np.ascontiguousarray(d.T)), D, F)
                                         for d in lw["wdown_exps"]]
    want, lgs = ref.generate(prompt, 6, ow, ocfg, M=len(prompt) + 6)
    from test_gpu_llm import _assert_tokens_match
    _assert_tokens_match(got, want, lgs, "gguf")
