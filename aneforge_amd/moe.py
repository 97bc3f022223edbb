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
from .graph import Tensor
from .llm import LayerSpec, LlamaConfig

_MAX_EXPERTS = 2049     # the reference carries expert indices as fp16 integers, exact up to 2048


def _check_topk(k: int, E: int) -> None:
    if not 1 <= k <= E <= _MAX_EXPERTS:
        raise ValueError(f"moe top-k: need 1 <= k <= E <= {_MAX_EXPERTS}; got k={k}, E={E}")


# ----------------------------------------------------------------------------- graph builders
def _topk_gate(probs, k, E, T):
    """The router's gate for af.compile graphs: probs [T, E] (fp16 probabilities) kept on the k
    experts each row routes to and zeroed elsewhere.  Routing contract of aneforge/moe.py:21-37:
    exactly k experts per row, chosen by k rounds of the row maximum with the lowest expert index
    winning an exact fp16 tie.  On this device that is one graph node, lowered to a single
    kernel (afx_topk_mask) rather than built from comparisons and selects."""
    _check_topk(int(k), int(E))
    if tuple(probs.shape) != (T, E):
        raise ValueError(f"moe top-k: probabilities {tuple(probs.shape)} are not [{T}, {E}]")
    return Tensor(probs.shape, "topk_mask", [probs], {"k": int(k)})


def _moe(h, w, cfg, ls):
    """af.compile form of the MoE SwiGLU MLP with its residual (aneforge/moe.py:48-63): h [T, dim]
    -> h + sum over the routed experts of gate * Wd_e(silu(Wg_e hn) * Wu_e hn) (+ the sigmoid-gated
    shared expert).  The reference evaluates every expert and masks the unselected ones with a
    zero gate; here the node lowers to the sparse device layer (MoEDecode), which computes only
    the routed experts -- the same sum, since a masked expert contributes exactly 0."""
    ex = cfg.extra
    _check_topk(int(ex["n_experts_per_tok"]), int(ex["n_experts"]))
    if len(h.shape) != 2 or h.shape[1] != cfg.dim:
        raise ValueError(f"moe: hidden states must be [T, {cfg.dim}], got {tuple(h.shape)}")
    return Tensor(h.shape, "moe_mlp", [h], {"w": w, "cfg": cfg, "ls": ls})


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
        _check_topk(self.k, self.E)
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
        from . import _kernels as K
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
            # K-split partials of the expert down projection (long expert rows)
            "ws": torch.empty(8 * B * k * D, dtype=torch.float32, device=dev),
            # the router's per-token form: arrival counter + tagged choices (zeroed once)
            "sync": K.moe_route_sync(dev),
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
        if K.moe_route_supported(h, self.router.w, self.k):
            # norm + router + top-k in one launch (the same bits as the three below)
            K.moe_route(h, self.norm, self.eps, self.router.w, self.k, self.renorm, b["hn"][:T], b["gate"][:T],
                        b["sel"][:T], b["cnt"], b["list"], sync=b["sync"])
        else:
            K.rmsnorm(h, self.norm, self.eps, y=b["hn"][:T])
            K.linear("fp16", self.router.w, None, b["hn"][:T], y=b["logits"][:T], out_f32=True)
            K.moe_topk(b["logits"][:T], self.k, self.renorm, b["gate"][:T], b["sel"][:T], b["cnt"], b["list"])
        K.moe_gateup(self.gu.fmt, self.gu.w, self.gu.scale, b["hn"][:T], self.k, self.E, self.F, b["cnt"],
                     b["list"], act=b["act"][:T * self.k])
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
        # the experts' down projection and the gate-weighted combine + residual, in place on h
        K.moe_down_combine(self.down.fmt, self.down.w, self.down.scale, b["act"][:T * self.k], T, self.k, self.E,
                           self.F, self.D, b["cnt"], b["list"], b["y"][:T * self.k], h, b["gate"][:T],
                           shared=shared, out=h, ws=b["ws"])

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
def _moe_layer_plan(c) -> list[bool]:
    """Which layers of a Qwen-MoE config carry experts: every `decoder_sparse_step`-th layer (1-based)
    that is not listed in `mlp_only_layers` (the reference's rule, aneforge/moe.py:77-79)."""
    every = int(getattr(c, "decoder_sparse_step", 1) or 1)
    dense = set(getattr(c, "mlp_only_layers", []) or [])
    return [i not in dense and (i + 1) % every == 0 for i in range(int(c.num_hidden_layers))]


def _moe_adapter(c, sd) -> tuple[LlamaConfig, dict]:
    """Hugging Face Qwen3-MoE -> (LlamaConfig, canonical weights) (aneforge/moe.py:70-107).  The dense
    decoder adapter maps the attention half and the dense MLP layers; expert layers swap their MLP
    for the router and the expert stacks, split out of the fused gate|up tensor and with down taken
    to the canonical [E, ffn, dim]."""
    plan = _moe_layer_plan(c)
    qk = "model.layers.0.self_attn.q_norm.weight" in sd
    cfg = llm._cfg_from_hf(c)
    cfg.layers = [LayerSpec(mixer="attention", mlp="moe" if on else "swiglu", qk_norm=qk) for on in plan]
    cfg.extra = {"n_experts": int(c.num_experts), "n_experts_per_tok": int(c.num_experts_per_tok),
                 "norm_topk_prob": bool(getattr(c, "norm_topk_prob", True))}
    F = int(c.moe_intermediate_size)
    w = llm._weights_from_state_dict(sd, cfg)          # expert layers have no dense MLP tensors
    for i, on in enumerate(plan):
        if not on:
            continue
        lw = w["layers"][i]
        pre = f"model.layers.{i}.mlp."
        fused = sd[pre + "experts.gate_up_proj"]                      # [E, 2F, dim]: gate rows, then up rows
        lw.update(router=sd[pre + "gate.weight"],
                  wgate_exps=np.ascontiguousarray(fused[:, :F]),
                  wup_exps=np.ascontiguousarray(fused[:, F:]),
                  wdown_exps=np.ascontiguousarray(np.swapaxes(sd[pre + "experts.down_proj"], 1, 2)))
    return cfg, w


llm.ADAPTERS.append((lambda c: bool(getattr(c, "num_experts", 0)), _moe_adapter))


# ----------------------------------------------------------------------------- GGUF loader
class _LazyLayers:
    """A sequence of per-layer weight dicts read from the file only when first indexed.  The
    decoder packs layer i onto the device and then calls free(i), so the host never holds more than
    one layer's dequantised tensors (aneforge/moe.py:113-126 plays the same role per ANE chunk)."""

    def __init__(self, read_layer, n: int):
        self._read, self._n, self._held = read_layer, n, {}

    def __len__(self) -> int:
        return self._n

    def __getitem__(self, i: int) -> dict:
        if not 0 <= i < self._n:
            raise IndexError(i)
        if i not in self._held:
            self._held[i] = self._read(i)
        return self._held[i]

    def free(self, i: int) -> None:
        self._held.pop(i, None)


# GGUF metadata -> LlamaConfig fields (key below the "<arch>." prefix, default); the key names are
# the file format's, as aneforge/moe.py:138-150 reads them.
_GGUF_HPARAMS = {
    "n_layers": ("block_count", 0), "dim": ("embedding_length", 0), "n_heads": ("attention.head_count", 0),
    "n_experts": ("expert_count", 0), "k": ("expert_used_count", 0), "rope_base": ("rope.freq_base", 10000.0),
    "norm_eps": ("attention.layer_norm_rms_epsilon", 1e-6),
}
# canonical per-layer name -> GGUF tensor below "blk.<i>.", always present
_GGUF_LAYER = {"wq": "attn_q.weight", "wk": "attn_k.weight", "wv": "attn_v.weight", "wo": "attn_output.weight",
               "attn_norm": "attn_norm.weight", "mlp_norm": "ffn_norm.weight", "router": "ffn_gate_inp.weight"}
# present only in some architectures: Qwen3 QK-norm, Qwen2 QKV biases
_GGUF_LAYER_OPTIONAL = {"q_norm": "attn_q_norm.weight", "k_norm": "attn_k_norm.weight",
                        "q_bias": "attn_q.bias", "k_bias": "attn_k.bias", "v_bias": "attn_v.bias"}
# Qwen2-MoE shared expert
_GGUF_SHARED = {"wgate_sh": "ffn_gate_shexp.weight", "wup_sh": "ffn_up_shexp.weight",
                "wdown_sh": "ffn_down_shexp.weight", "shared_gate": "ffn_gate_inp_shexp.weight"}


def load_gguf(path: str, n_layers: int | None = None, compress: str | None = None) -> "llm.LlamaPrefill":
    """A Qwen-MoE GGUF file as a LlamaPrefill (aneforge/moe.py:129-173), read by this package's own
    GGUF reader.  Expert stacks stored as Q4_0 / Q4_K / Q6_K / Q8_0 reach the device as their codes
    (the matching kernels stream them); every other tensor is dequantised as the reference does,
    embedding and lm_head to fp32, the rest to fp16.  The architecture's optional parts (QK-norm,
    QKV biases, a shared expert) are detected from the tensor names; `n_layers` keeps the first
    layers only."""
    from ._gguf import GGUFView
    gg = GGUFView(path)
    hp = {name: gg.sc(key, default) for name, (key, default) in _GGUF_HPARAMS.items()}
    n = int(hp["n_layers"]) if n_layers is None else min(int(n_layers), int(hp["n_layers"]))
    dim, heads = int(hp["dim"]), int(hp["n_heads"])
    qk = gg.has("blk.0." + _GGUF_LAYER_OPTIONAL["q_norm"])
    shared = gg.has("blk.0." + _GGUF_SHARED["wgate_sh"])
    cfg = LlamaConfig(
        dim=dim, n_layers=n, n_heads=heads, n_kv_heads=int(gg.sc("attention.head_count_kv", heads)),
        ffn_dim=int(gg.tn["blk.0.ffn_gate_exps.weight"].shape[1]),
        vocab=int(gg.tn["token_embd.weight"].data.shape[0]), rope_base=float(hp["rope_base"]),
        norm_eps=float(hp["norm_eps"]), head_dim=int(gg.sc("attention.key_length") or dim // heads),
        layers=[LayerSpec(mixer="attention", mlp="moe", qk_norm=qk) for _ in range(n)],
        # Qwen1.5 / Qwen2-MoE does not renormalise the top-k probabilities
        extra={"n_experts": int(hp["n_experts"]), "n_experts_per_tok": int(hp["k"]),
               "norm_topk_prob": gg.arch != "qwen2moe"})

    def expert_stack(name):
        codes = gg.quantized(name)
        return codes if codes is not None else gg.get(name)

    def read_layer(i: int) -> dict:
        blk = f"blk.{i}."
        lw = {key: gg.get(blk + name) for key, name in _GGUF_LAYER.items()}
        lw.update((key, gg.get(blk + name)) for key, name in _GGUF_LAYER_OPTIONAL.items() if gg.has(blk + name))
        if shared:
            lw.update((key, gg.get(blk + name)) for key, name in _GGUF_SHARED.items())
            lw["shared_gate"] = lw["shared_gate"].reshape(1, dim)
        lw["wgate_exps"] = expert_stack(blk + "ffn_gate_exps.weight")
        lw["wup_exps"] = expert_stack(blk + "ffn_up_exps.weight")
        down = expert_stack(blk + "ffn_down_exps.weight")     # [E, dim, ffn] as stored
        # code stacks stay per expert [dim, ffn]; a float stack goes to the canonical [E, ffn, dim]
        lw["wdown_exps"] = down if isinstance(down, list) else np.ascontiguousarray(np.swapaxes(down, 1, 2))
        gg.drop_pages()
        return lw

    head = "output.weight" if gg.has("output.weight") else "token_embd.weight"
    w = {"embed": gg.get("token_embd.weight", np.float32), "final_norm": gg.get("output_norm.weight"),
         "lm_head": gg.get(head, np.float32), "layers": _LazyLayers(read_layer, n)}
    return llm.LlamaPrefill(cfg, w, compress=compress)
