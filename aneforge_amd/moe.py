"""Sparse Mixture-of-Experts for decode on one MI355X (the reference's aneforge/moe.py API).

Routing matches the reference: softmax over the router logits, top-k with the lowest expert
index winning exact fp16 ties (exactly k experts per token), optional renormalisation
(aneforge/moe.py:21-63).  The reference computes every expert densely and masks with the gate;
the device executor here (MoEDecode) computes only the experts a token routed to, which is the
same sum because unselected experts carry weight 0.  Routing, token bucketing and the expert
GEMVs all run on the device (afx_moe_*), so a MoE layer stays inside the captured step graph.

Canonical per-layer weights (as the reference): mlp_norm, router [E, dim],
wgate_exps / wup_exps [E, ffn, dim], wdown_exps [E, ffn, dim] (down stored transposed for the
batched act @ wdown); Qwen2-MoE adds wgate_sh / wup_sh / wdown_sh / shared_gate.  Expert
weights may also arrive as already-encoded QuantizedWeight stacks (GGUF Q4_0 / Q4_K / Q6_K / Q8_0 from load_gguf),
in which case their codes are streamed as they are."""
from __future__ import annotations

import numpy as np

from . import llm
from .graph import _const, concat as _concat, select
from .llm import LayerSpec, LlamaConfig

_MAX_DIM = 65536
_MAX_EXPERTS = 2049


# ----------------------------------------------------------------------------- graph builders
def _topk_gate(probs, k, E, T):
    """probs [T, E] masked to the top-k per row (0 elsewhere) without a native top-k: k rounds of
    row max, the lowest tied index chosen each round (aneforge/moe.py:21-37)."""
    if not 1 <= k <= E <= _MAX_EXPERTS:
        raise ValueError(f"moe top-k: need 1 <= k <= E <= {_MAX_EXPERTS}; got k={k}, E={E}")
    lanes = _const(np.tile(np.arange(E, dtype=np.float16), (T, 1)))
    far = _const(np.full((T, E), 4096.0, np.float16))
    gone = _const(np.full((T, E), -3.0e4, np.float16))
    on = _const(np.ones((T, E), np.float16))
    picked = _const(np.zeros((T, E), np.float16))
    rest = probs
    for _ in range(k):
        at_max = rest.greater_equal(rest.amax([1]).reshape(T, 1))
        lowest = (select(at_max, lanes, far) * -1.0).amax([1]).reshape(T, 1) * -1.0
        hit = lanes.equal(lowest)
        picked = select(hit, on, picked)
        rest = select(hit, gone, rest)
    return probs * picked


def _experts_gate(hn, wexps, E, ffn, dim, T):
    """hn @ wexps[e].T for all experts -> [T, E, ffn] (aneforge/moe.py:40-45)."""
    g = max(1, min(E, _MAX_DIM // ffn))
    parts = [hn.linear(np.asarray(wexps[s:s + g]).reshape(min(g, E - s) * ffn, dim)).reshape(T, min(g, E - s), ffn)
             for s in range(0, E, g)]
    return parts[0] if len(parts) == 1 else _concat(parts, axis=1)


def _moe(h, w, cfg, ls):
    """Graph form of the MoE SwiGLU MLP + residual (aneforge/moe.py:48-63), for af.compile."""
    e = cfg.extra
    E, k, dim = e["n_experts"], e["n_experts_per_tok"], cfg.dim
    ffn, T = np.asarray(w["wgate_exps"]).shape[1], h.shape[0]
    hn = h.rms_norm(w["mlp_norm"], cfg.norm_eps)
    gate_w = _topk_gate(hn.linear(w["router"]).softmax(-1), k, E, T)
    if e.get("norm_topk_prob", True):
        gate_w = gate_w / gate_w.sum([1]).reshape(T, 1)
    gate = _experts_gate(hn, w["wgate_exps"], E, ffn, dim, T)
    up = _experts_gate(hn, w["wup_exps"], E, ffn, dim, T)
    out = (gate.silu() * up).transpose([1, 0, 2]).bmm_weight(w["wdown_exps"])
    combined = (out * gate_w.transpose([1, 0]).reshape(E, T, 1)).sum([0]).reshape(T, dim)
    if "wgate_sh" in w:
        sh = (hn.linear(w["wgate_sh"]).silu() * hn.linear(w["wup_sh"])).linear(w["wdown_sh"])
        combined = combined + sh * hn.linear(w["shared_gate"]).sigmoid()
    return h + combined


# ----------------------------------------------------------------------------- device executor
class MoEDecode:
    """Device MoE MLP for the decode engine: RMSNorm -> router logits -> top-k + bucketing ->
    active-expert gate/up (SwiGLU) -> active-expert down -> gate-weighted combine + residual."""

    def __init__(self, lw: dict, cfg, ls, compress):
        import torch
        from . import _engine as E
        ex = cfg.extra
        self.E, self.k = int(ex["n_experts"]), int(ex["n_experts_per_tok"])
        self.renorm = bool(ex.get("norm_topk_prob", True))
        if not 1 <= self.k <= self.E <= _MAX_EXPERTS:
            raise ValueError(f"moe top-k: need 1 <= k <= E <= {_MAX_EXPERTS}; got k={self.k}, E={self.E}")
        D, eps = cfg.dim, float(cfg.norm_eps)
        self.D, self.eps = D, eps
        self.norm = E._gamma(lw["mlp_norm"], D)
        self.router = E.pack_linear(np.asarray(lw["router"], np.float32), None)
        gate, up, down = lw["wgate_exps"], lw["wup_exps"], lw["wdown_exps"]
        if compress == "int4" and not isinstance(gate, (list, tuple)):
            # one codebook per expert matrix (the reference compresses each linear separately)
            g_, u_, d_ = (np.asarray(a, np.float32) for a in (gate, up, down))
            gate = [E.per_tensor(g_[e], compress) for e in range(self.E)]
            up = [E.per_tensor(u_[e], compress) for e in range(self.E)]
            down = [E.per_tensor(np.ascontiguousarray(d_[e].T), compress) for e in range(self.E)]
        if isinstance(gate, (list, tuple)) or isinstance(down, (list, tuple)):
            # per-expert matrices: QuantizedWeight codes (GGUF Q4_0 / Q4_K / Q6_K / Q8_0), with float stacks of
            # a file's other types split per expert alongside ([F, D] gate/up, [D, F] down)
            if not isinstance(gate, (list, tuple)):
                gate, up = list(np.asarray(gate, np.float32)), list(np.asarray(up, np.float32))
            if not isinstance(down, (list, tuple)):
                d_ = np.asarray(down, np.float32)
                down = [np.ascontiguousarray(d_[e].T) for e in range(self.E)]
            F = gate[0].shape[0]
            gu = E._cat([E._interleave(g, u) for g, u in zip(gate, up)])
            dn = E._cat(list(down))                   # [E*D, F] rows
        else:
            gate, up = np.asarray(gate, np.float32), np.asarray(up, np.float32)
            F = gate.shape[1]
            gu = np.concatenate([E._interleave(gate[e], up[e]) for e in range(self.E)])
            dn = np.ascontiguousarray(np.asarray(down, np.float32).transpose(0, 2, 1)).reshape(self.E * D, F)
        self.F = F
        self.gu = E.pack_linear(gu, compress)
        self.down = E.pack_linear(dn, compress)
        self.shared = None
        if "wgate_sh" in lw:
            self.sh_gu = E.pack_linear(E._interleave(E.per_tensor(lw["wgate_sh"], compress),
                                                     E.per_tensor(lw["wup_sh"], compress)), compress)
            self.sh_down = E.pack_linear(lw["wdown_sh"], compress)
            self.sh_gate = E.pack_linear(np.asarray(lw["shared_gate"], np.float32).reshape(1, D), None)
            self.shared = True
        self._bufs = None

    def bind(self, eng):
        self._bufs = self._make_bufs(eng.B)
        self._pf = None

    def _make_bufs(self, B):
        import torch
        D, E, k, F = self.D, self.E, self.k, self.F
        dev = "cuda"
        bufs = {
            "hn": torch.empty((B, D), dtype=torch.float16, device=dev),
            "logits": torch.empty((B, E), dtype=torch.float32, device=dev),
            "gate": torch.empty((B, k), dtype=torch.float32, device=dev),
            "sel": torch.empty((B, k), dtype=torch.int32, device=dev),
            "cnt": torch.empty((E,), dtype=torch.int32, device=dev),
            "list": torch.empty((E, B), dtype=torch.int32, device=dev),
            "act": torch.empty((B * k, F), dtype=torch.float16, device=dev),
            "y": torch.empty((B * k, D), dtype=torch.float32, device=dev),
        }
        if self.shared:
            Fs = self.sh_gu.N // 2
            bufs.update({"sh_act": torch.empty((B, Fs), dtype=torch.float16, device=dev),
                         "sh_y": torch.empty((B, D), dtype=torch.float16, device=dev),
                         "sh_g": torch.empty((B, 1), dtype=torch.float16, device=dev),
                         "sh_gs": torch.empty((B, 1), dtype=torch.float16, device=dev),
                         "sh": torch.empty((B, D), dtype=torch.float16, device=dev)})
        return bufs

    def reset(self, eng):
        pass

    def state(self):
        return []

    def run(self, h, b):
        """MoE MLP + residual on h [T, D] in place, with bound buffers b (T <= buffer rows)."""
        from . import _kernels as K
        T = h.shape[0]
        K.rmsnorm(h, self.norm, self.eps, y=b["hn"][:T])
        K.linear("fp16", self.router.w, None, b["hn"][:T], y=b["logits"][:T], out_f32=True)
        K.moe_topk(b["logits"][:T], self.k, self.renorm, b["gate"][:T], b["sel"][:T], b["cnt"], b["list"])
        K.moe_gateup(self.gu.fmt, self.gu.w, self.gu.scale, b["hn"][:T], self.k, self.E, self.F, b["cnt"],
                     b["list"], act=b["act"][:T * self.k])
        K.moe_down(self.down.fmt, self.down.w, self.down.scale, b["act"][:T * self.k], T, self.k, self.E,
                   self.F, self.D, b["cnt"], b["list"], y=b["y"][:T * self.k])
        shared = None
        if self.shared:
            K.linear_swiglu(self.sh_gu.fmt, self.sh_gu.w, self.sh_gu.scale, b["hn"][:T], act=b["sh_act"][:T])
            K.linear(self.sh_down.fmt, self.sh_down.w, self.sh_down.scale, b["sh_act"][:T], y=b["sh_y"][:T])
            K.linear("fp16", self.sh_gate.w, None, b["hn"][:T], y=b["sh_g"][:T])
            K._hip.call("afx_ew_unary", K.UNARY["sigmoid"], K.P(b["sh_g"]), K.P(b["sh_gs"]), T, 0.0, 0.0, K.stream())
            shape = [T, self.D]
            K._hip.call("afx_ew_binary", K.EW["mul"], K.P(b["sh_y"]), K._ll([self.D, 1]), K.P(b["sh_gs"]),
                        K._ll([1, 0]), K.P(b["sh"]), 2, K._ii(shape), K.stream())
            shared = b["sh"][:T]
        K.moe_combine(h, b["y"][:T * self.k], b["gate"][:T], shared=shared, out=h)

    def enqueue(self, eng):
        self.run(eng.h, self._bufs)

    # batched prefill: the same layer over a chunk of prompt rows (grouped expert GEMMs on MFMA)
    def prefill_supported(self) -> bool:
        return True

    def prefill(self, eng, X, pos0: int, bufs: dict):
        T = X.shape[0]
        if self._pf is None or self._pf["hn"].shape[0] < T:
            self._pf = self._make_bufs(T)
        self.run(X, self._pf)

    @property
    def nbytes(self):
        n = self.gu.nbytes + self.down.nbytes + self.router.nbytes
        if self.shared:
            n += self.sh_gu.nbytes + self.sh_down.nbytes
        return n


llm.DECODE_MLPS["moe"] = MoEDecode


# ----------------------------------------------------------------------------- HF adapter
def _moe_adapter(c, sd) -> tuple[LlamaConfig, dict]:
    """Qwen3-MoE Hugging Face adapter (aneforge/moe.py:70-107): attention layers as usual, MoE
    layers carry the fused expert weights plus the router."""
    n, E, k = int(c.num_hidden_layers), int(c.num_experts), int(c.num_experts_per_tok)
    moe_ffn = int(c.moe_intermediate_size)
    qk = "model.layers.0.self_attn.q_norm.weight" in sd
    step = int(getattr(c, "decoder_sparse_step", 1) or 1)
    mlp_only = set(getattr(c, "mlp_only_layers", []) or [])
    is_moe = [(L not in mlp_only) and ((L + 1) % step == 0) for L in range(n)]
    specs = [LayerSpec(mixer="attention", mlp=("moe" if is_moe[L] else "swiglu"), qk_norm=qk) for L in range(n)]
    cfg = LlamaConfig(dim=c.hidden_size, n_layers=n, n_heads=c.num_attention_heads,
                      n_kv_heads=getattr(c, "num_key_value_heads", c.num_attention_heads),
                      ffn_dim=c.intermediate_size, vocab=c.vocab_size, rope_base=llm._rope_theta(c),
                      norm_eps=float(c.rms_norm_eps), head_dim=int(getattr(c, "head_dim", 0) or 0), layers=specs,
                      extra={"n_experts": E, "n_experts_per_tok": k,
                             "norm_topk_prob": bool(getattr(c, "norm_topk_prob", True))})
    w = {"embed": sd["model.embed_tokens.weight"], "final_norm": sd["model.norm.weight"],
         "lm_head": sd.get("lm_head.weight", sd["model.embed_tokens.weight"]), "layers": []}
    for L in range(n):
        p = f"model.layers.{L}."
        lw = {"wq": sd[p + "self_attn.q_proj.weight"], "wk": sd[p + "self_attn.k_proj.weight"],
              "wv": sd[p + "self_attn.v_proj.weight"], "wo": sd[p + "self_attn.o_proj.weight"],
              "attn_norm": sd[p + "input_layernorm.weight"], "mlp_norm": sd[p + "post_attention_layernorm.weight"]}
        if qk:
            lw["q_norm"] = sd[p + "self_attn.q_norm.weight"]
            lw["k_norm"] = sd[p + "self_attn.k_norm.weight"]
        if is_moe[L]:
            gu = sd[p + "mlp.experts.gate_up_proj"]
            lw["router"] = sd[p + "mlp.gate.weight"]
            lw["wgate_exps"] = np.ascontiguousarray(gu[:, :moe_ffn, :])
            lw["wup_exps"] = np.ascontiguousarray(gu[:, moe_ffn:, :])
            lw["wdown_exps"] = np.ascontiguousarray(sd[p + "mlp.experts.down_proj"].transpose(0, 2, 1))
        else:
            lw["wgate"] = sd[p + "mlp.gate_proj.weight"]
            lw["wup"] = sd[p + "mlp.up_proj.weight"]
            lw["wdown"] = sd[p + "mlp.down_proj.weight"]
        w["layers"].append(lw)
    return cfg, w


llm.ADAPTERS.append((lambda c: bool(getattr(c, "num_experts", 0)), _moe_adapter))


# ----------------------------------------------------------------------------- GGUF loader
class _LazyLayers:
    """Per-layer weights materialised on demand and dropped once packed (aneforge/moe.py:113-126)."""

    def __init__(self, materialize, n: int):
        self._mk = materialize
        self._n = n
        self._cache: dict = {}

    def __len__(self) -> int:
        return self._n

    def __getitem__(self, i: int) -> dict:
        if i not in self._cache:
            self._cache[i] = self._mk(i)
        return self._cache[i]

    def free(self, i: int) -> None:
        self._cache.pop(i, None)


def load_gguf(path: str, n_layers: int | None = None, compress: str | None = None) -> "llm.LlamaPrefill":
    """Load a Qwen-MoE GGUF (aneforge/moe.py:129-173) with this package's own GGUF reader.
    Q4_0 expert tensors stay 4-bit (streamed by the Q4_0 kernels, never dequantised); other
    tensors are dequantised to fp16 as the reference does.  Arch features (QK-norm, shared
    expert, QKV biases) are detected from the tensor names."""
    from ._gguf import GGUFView
    gg = GGUFView(path)
    sc, get, tn, arch = gg.sc, gg.get, gg.tn, gg.arch
    opt = lambda name: get(name) if gg.has(name) else None
    n_total = int(sc("block_count", 0))
    n = n_total if n_layers is None else min(n_layers, n_total)
    E, k = int(sc("expert_count", 0)), int(sc("expert_used_count", 0))
    dim = int(sc("embedding_length", 0))
    vocab = int(tn["token_embd.weight"].data.shape[0])
    heads = int(sc("attention.head_count", 0))
    moe_ffn = int(tn["blk.0.ffn_gate_exps.weight"].shape[1])
    qk = gg.has("blk.0.attn_q_norm.weight")
    shared = gg.has("blk.0.ffn_gate_shexp.weight")
    cfg = llm.LlamaConfig(
        dim=dim, n_layers=n, n_heads=heads, n_kv_heads=int(sc("attention.head_count_kv", heads)),
        ffn_dim=moe_ffn, vocab=vocab, rope_base=float(sc("rope.freq_base", 10000.0)),
        norm_eps=float(sc("attention.layer_norm_rms_epsilon", 1e-6)),
        head_dim=int(sc("attention.key_length") or dim // heads),
        layers=[llm.LayerSpec(mixer="attention", mlp="moe", qk_norm=qk) for _ in range(n)],
        extra={"n_experts": E, "n_experts_per_tok": k, "norm_topk_prob": arch != "qwen2moe"})

    def experts(name):
        """An expert stack: per-expert QuantizedWeight when the file holds Q4_0 / Q4_K / Q6_K / Q8_0 codes, else fp16."""
        q = gg.quantized(name)
        if q is not None:
            return q
        return get(name)

    def layer(L):
        b = f"blk.{L}."
        d = {"wq": get(b + "attn_q.weight"), "wk": get(b + "attn_k.weight"), "wv": get(b + "attn_v.weight"),
             "wo": get(b + "attn_output.weight"), "attn_norm": get(b + "attn_norm.weight"),
             "mlp_norm": get(b + "ffn_norm.weight"), "router": get(b + "ffn_gate_inp.weight"),
             "wgate_exps": experts(b + "ffn_gate_exps.weight"), "wup_exps": experts(b + "ffn_up_exps.weight")}
        down = experts(b + "ffn_down_exps.weight")
        # GGUF stores down as [E, dim, ffn]; the canonical float layout is [E, ffn, dim]
        d["wdown_exps"] = down if isinstance(down, list) else np.ascontiguousarray(np.asarray(down).transpose(0, 2, 1))
        for key, nm in (("q_norm", "attn_q_norm.weight"), ("k_norm", "attn_k_norm.weight"),
                        ("q_bias", "attn_q.bias"), ("k_bias", "attn_k.bias"), ("v_bias", "attn_v.bias")):
            v = opt(b + nm)
            if v is not None:
                d[key] = v
        if shared:
            d["wgate_sh"] = get(b + "ffn_gate_shexp.weight")
            d["wup_sh"] = get(b + "ffn_up_shexp.weight")
            d["wdown_sh"] = get(b + "ffn_down_shexp.weight")
            d["shared_gate"] = get(b + "ffn_gate_inp_shexp.weight").reshape(1, dim)
        gg.drop_pages()
        return d

    w = {"embed": get("token_embd.weight", np.float32), "final_norm": get("output_norm.weight"),
         "lm_head": get("output.weight", np.float32) if gg.has("output.weight") else get("token_embd.weight", np.float32),
         "layers": _LazyLayers(layer, n)}
    return llm.LlamaPrefill(cfg, w, compress=compress)
