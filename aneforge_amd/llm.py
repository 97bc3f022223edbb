"""Config-driven decoder LMs (RMSNorm + RoPE + GQA attention + SwiGLU) on one MI355X, behind the
API of the reference's aneforge/llm.py: LlamaConfig / LayerSpec plans, the decode-layer
registries that moe.py plugs into, and LlamaPrefill.{prefill, generate, warmup, release}.

Where the reference compiles chunked ANE programs and runs one host round trip per chunk per
token (aneforge/llm.py:435-633), LlamaPrefill here packs every layer's weights onto the GPU
once and replays a captured HIP graph per token (see _engine.DecodeEngine): the KV cache,
position, prompt and generated tokens never leave the device during generation."""
from __future__ import annotations

import time
import warnings
from dataclasses import dataclass, field
from enum import Enum

import numpy as np


class ModelType(str, Enum):
    GPT2 = "gpt2"
    GEMMA = "gemma"
    GEMMA2 = "gemma2"
    GEMMA3 = "gemma3"
    GEMMA3_TEXT = "gemma3_text"
    MISTRAL = "mistral"
    LLAMA = "llama"
    QWEN = "qwen"


# Architectures whose semantics the dense Llama path would drop (Gemma-2/3 softcapping and sliding
# attention; aneforge/llm.py:30-32): rejected, never mis-loaded.  Gemma has its own adapter.
_DENSE_INCOMPATIBLE = {ModelType.GEMMA2, ModelType.GEMMA3, ModelType.GEMMA3_TEXT}


@dataclass
class LayerSpec:
    """Per-layer plan (aneforge/llm.py:35-41): registry keys of the token mixer and the MLP."""
    mixer: str = "attention"
    mlp: str = "swiglu"
    qk_norm: bool = False


@dataclass
class LlamaConfig:
    """Decoder config (aneforge/llm.py:44-59); `head_dim` defaults to dim // n_heads."""
    dim: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    ffn_dim: int
    vocab: int
    rope_base: float = 10000.0
    norm_eps: float = 1e-5
    head_dim: int = 0
    rotary_dim: int = 0
    rope_interleaved: bool = False
    rope_scaling: dict | None = None
    layers: list[LayerSpec] = field(default_factory=list)
    extra: dict = field(default_factory=dict)
    norm_type: str = "rms"
    rope: bool = True

    @property
    def dh(self) -> int:
        return self.head_dim or self.dim // self.n_heads


def _llama3_rope_scale(inv, s):
    """Llama-3.1 inv_freq rescaling (aneforge/llm.py:62-73): low frequencies divided by
    `factor`, high frequencies kept, a linear blend in between."""
    factor, lo, hi = float(s["factor"]), float(s["low_freq_factor"]), float(s["high_freq_factor"])
    old = float(s["original_max_position_embeddings"])
    wl = 2.0 * np.pi / inv
    scaled = np.where(wl > old / lo, inv / factor, inv)
    t = (old / wl - lo) / (hi - lo)
    mid = (1.0 - t) * scaled / factor + t * scaled
    return np.where((wl >= old / hi) & (wl <= old / lo), mid, scaled)


def rope_tables(seq: int, dh: int, base: float = 10000.0, rotary_dim: int = 0, interleaved: bool = False,
                scaling: dict | None = None):
    """[seq, dh] fp16 cos/sin tables computed in float64 (aneforge/llm.py:76-93): neox layout
    (frequencies repeated over the two halves) or the GPT-J pair layout; partial rotary pads
    with cos=1 / sin=0."""
    rd = rotary_dim or dh
    inv = 1.0 / (base ** (np.arange(0, rd, 2) / rd))
    if scaling and scaling.get("rope_type") == "llama3":
        inv = _llama3_rope_scale(inv, scaling)
    ang = np.outer(np.arange(seq), inv)
    full = np.repeat(ang, 2, axis=1) if interleaved else np.concatenate([ang, ang], axis=1)
    c, s = np.cos(full), np.sin(full)
    if rd < dh:
        c = np.concatenate([c, np.ones((seq, dh - rd))], axis=1)
        s = np.concatenate([s, np.zeros((seq, dh - rd))], axis=1)
    return c.astype(np.float16), s.astype(np.float16)


def rope(x, cos, sin):
    """Graph-level RoPE (aneforge/llm.py:96-105): x*cos + rotate_half(x)*sin on a Tensor [.., dh]."""
    from .graph import Tensor, _const, concat
    dh = x.shape[-1]
    half = dh // 2
    rank = len(x.shape)
    size = list(x.shape)
    size[-1] = half
    x1 = x.slice_by_size([0] * rank, size)
    b2 = [0] * rank
    b2[-1] = half
    x2 = x.slice_by_size(b2, size)
    c = cos if isinstance(cos, Tensor) else _const(cos)
    s = sin if isinstance(sin, Tensor) else _const(sin)
    return x * c + concat([x2 * -1.0, x1], axis=rank - 1) * s


# ----------------------------------------------------------------------------- registries
# Decode executors by LayerSpec key (the reference's DECODE_MIXERS / DECODE_MLPS hold graph
# builders, aneforge/llm.py:240-245; here they hold device executors with the same keys).
from . import _engine as _eng  # noqa: E402

DECODE_MIXERS: dict = {"attention": _eng.AttentionDecode}
DECODE_MLPS: dict = {"swiglu": _eng.SwiGLUDecode, "geglu": _eng.GeGLUDecode}
PREFILL_MIXERS: dict = DECODE_MIXERS
PREFILL_MLPS: dict = DECODE_MLPS


class LlamaPrefill:
    """A decoder resident on one MI355X.  `weights` is the reference's canonical dict (embed,
    final_norm, lm_head, layers=[{wq, wk, wv, wo, wgate, wup, wdown, attn_norm, mlp_norm, ...}])
    of numpy arrays; `compress` picks the weight encoding (None = fp16, "int8", "q4_0",
    "blockwise", "int4").  `ane_lm_head` keeps the reference's name: True runs the fp16 lm_head
    and the greedy argmax on the device, False computes logits on the host in fp32."""

    def __init__(self, cfg: LlamaConfig, weights: dict, compress: str | None = None, ane_lm_head: bool = True):
        self.cfg = cfg
        self.w = weights
        self.compress = compress
        self.ane_lm_head = ane_lm_head
        self._chunk_bytes = 1.6e9          # kept from the reference's chunk planner (see _layer_chunks)
        self._chunk_max_layers = 24
        self.lmhead_tie_margin = 3e-3
        self._lmT = None
        self._lmh = None                   # device lm_head (Linear) once packed
        self._lmh32 = None                 # its fp32 values when the checkpoint's are not fp16-exact
        self._lmh_off = False
        self._layers = None                # packed device layers
        self._embed = None
        self._final_norm = None
        self._dec = None                   # DecodeEngine for the current max length

    # -- planning kept for API compatibility (aneforge/llm.py:425-433) --
    _ENCODED_BYTES = {"int8": 1.0, "blockwise": 1.0, "int4": 0.5, "q4_0": 0.5}   # per weight; fp16 is 2

    def _layer_chunks(self):
        """The reference's layer grouping: consecutive layers whose weights, at this compress=
        encoding, stay under the per-program byte budget, and at most `_chunk_max_layers` a group.
        The device engine itself runs every layer in one graph; callers that plan by chunk get the
        same plan as on the reference."""
        n_layers = self.cfg.n_layers
        elems = sum(np.size(v) for v in self.w["layers"][0].values() if isinstance(v, (np.ndarray, list, tuple)))
        layer_bytes = max(1, int(elems * self._ENCODED_BYTES.get(self.compress, 2.0)))
        size = max(1, min(n_layers, self._chunk_max_layers, int(self._chunk_bytes // layer_bytes)))
        bounds = list(range(0, n_layers, size)) + [n_layers]
        return [range(lo, hi) for lo, hi in zip(bounds[:-1], bounds[1:])]

    def _spec(self, i: int) -> LayerSpec:
        if self.cfg.layers:
            return self.cfg.layers[i]
        return LayerSpec(qk_norm="q_norm" in self.w["layers"][i])

    def _check_positions(self, n: int) -> None:
        wpe = self.w.get("wpe")
        if wpe is not None and n > wpe.shape[0]:
            raise ValueError(f"sequence length {n} exceeds this model's {wpe.shape[0]} max positions")

    # -- device packing --
    def _pack(self):
        if self._layers is not None:
            return self._layers
        import torch
        if not torch.cuda.is_available():
            raise RuntimeError("LlamaPrefill needs an MI355X GPU (no CPU fallback)")
        if "wpe" in self.w:
            raise NotImplementedError("learned position embeddings (GPT-2) are not on the device decode path")
        cfg = self.cfg
        layers = []
        for i in range(cfg.n_layers):
            ls = self._spec(i)
            if ls.mixer not in DECODE_MIXERS:
                raise NotImplementedError(f"decode mixer {ls.mixer!r} is not registered")
            if ls.mlp not in DECODE_MLPS:
                raise NotImplementedError(f"decode MLP {ls.mlp!r} is not registered")
            lw = self.w["layers"][i]
            layers.append((DECODE_MIXERS[ls.mixer](lw, cfg, ls, self.compress),
                           DECODE_MLPS[ls.mlp](lw, cfg, ls, self.compress)))
            if hasattr(self.w["layers"], "free"):          # streamed weights: drop the host copy once packed
                self.w["layers"].free(i)
        self._layers = layers
        self._embed = _eng._to_dev(np.asarray(self.w["embed"], np.float32).astype(np.float16))
        self._final_norm = _eng._gamma(self.w["final_norm"], cfg.dim)
        self._lmh = _eng.pack_linear(self.w["lm_head"], None)   # the head stays fp16 (llm.py:279)
        # the near-tie recompute uses the checkpoint's own head values (aneforge/llm.py:350-355 computes
        # in fp32): when they are not all fp16-exact, an fp32 copy stays on the device for it
        lm = np.asarray(self.w["lm_head"])
        self._lmh32 = None
        if lm.dtype != np.float16 and not np.array_equal(lm.astype(np.float16).astype(lm.dtype), lm):
            self._lmh32 = _eng._to_dev(np.ascontiguousarray(lm, np.float32))
        return layers

    def _decoder(self, M: int):
        M = int(M)
        self._check_positions(M)
        if self._dec is not None and self._dec.M == M:
            if self._dec.margin != self.lmhead_tie_margin:
                self._dec.set_tie_margin(self.lmhead_tie_margin)
            return self._dec
        if self._dec is not None:
            self._dec.close()
        layers = self._pack()
        self._dec = _eng.DecodeEngine(self.cfg, layers, self._embed, self._lmh, self._final_norm, M,
                                      head32=self._lmh32, tie_margin=self.lmhead_tie_margin)
        return self._dec

    def warmup(self, max_len):
        """Pack the weights and capture the step graphs for context length `max_len`."""
        d = self._decoder(int(max_len))
        d._graphs()
        return self

    def release(self) -> None:
        """Free the device weights, caches and graphs; the next call re-packs."""
        if self._dec is not None:
            self._dec.close()
        self._dec = None
        self._layers = None
        self._embed = self._final_norm = self._lmh = self._lmh32 = None
        self._lmT = None
        try:
            import torch
            torch.cuda.empty_cache()
        except Exception:
            pass

    # -- logits --
    def _host_logits(self, hidden_row):
        lm = self._lmT
        if lm is None:
            lm = self._lmT = np.ascontiguousarray(np.asarray(self.w["lm_head"]).T, np.float32)
        return np.asarray(hidden_row, np.float32) @ lm

    def _logits(self, hidden_row, ane: bool | None = None):
        """Next-token logits for one final-normed hidden row: device fp16 head (fp32 accumulate)
        or the host fp32 head."""
        use_dev = self.ane_lm_head if ane is None else ane
        if use_dev:
            import torch
            self._pack()
            x = torch.from_numpy(np.asarray(hidden_row, np.float32).astype(np.float16).reshape(1, -1)).cuda()
            y = self._lmh(x, out_f32=True)
            torch.cuda.synchronize()
            return y[0].cpu().numpy()
        return self._host_logits(hidden_row)

    @staticmethod
    def _sample(logits, temperature, top_p, top_k):
        """Greedy when temperature <= 0, else temperature / top-k / top-p sampling
        (aneforge/llm.py:406-419)."""
        if temperature <= 0.0:
            return int(np.argmax(logits))
        lg = np.asarray(logits, np.float64) / temperature
        if top_k and 0 < top_k < lg.size:
            lg[lg < np.partition(lg, -top_k)[-top_k]] = -np.inf
        p = np.exp(lg - lg.max())
        p /= p.sum()
        if 0.0 < top_p < 1.0:
            order = np.argsort(p)[::-1]
            cum = np.cumsum(p[order])
            keep = order[:int(np.searchsorted(cum, top_p)) + 1]
            m = np.zeros_like(p)
            m[keep] = p[keep]
            p = m / m.sum()
        return int(np.random.choice(p.size, p=p))

    # -- public entry points --
    def _hidden_last(self, token_ids, M=None):
        """Run the prompt through the resident cache; returns the engine positioned after it."""
        ids = [int(t) for t in token_ids]
        d = self._decoder(M or max(len(ids), 1))
        d.prefill(ids)
        return d

    def prefill(self, token_ids):
        """Next-token logits [1, vocab] for the prompt (final norm + fp16 head on the device)."""
        ids = [int(t) for t in token_ids]
        self._check_positions(len(ids))
        d = self._hidden_last(ids, M=len(ids))
        import torch
        with torch.cuda.stream(d.stream):
            d.enqueue_layers()
            d.enqueue_head()
        return d.logits_host()[None].astype(np.float32)

    def generate(self, token_ids, max_new_tokens=40, eos_id=None, max_len=None, on_token=None,
                 temperature=0.0, top_p=1.0, top_k=0, batched_prefill=True, prefill_pad=None, on_stage=None,
                 ane_lm_head=None):
        """Autoregressive generation over the resident KV cache (aneforge/llm.py:560-633).
        Greedy decoding and temperature / top-k / top-p sampling run entirely on the device (one
        graph replay per token, one host read at the end when no eos / on_token is given); the
        sampler draws with one np.random.random_sample() per token, as the reference's
        np.random.choice does."""
        prompt = [int(t) for t in token_ids]
        if not prompt:
            raise ValueError("generate needs at least one prompt token")
        M = int(max_len or len(prompt) + max_new_tokens)
        eos = {int(eos_id)} if isinstance(eos_id, int) else {int(e) for e in (eos_id or ())}
        use_dev = self.ane_lm_head if ane_lm_head is None else bool(ane_lm_head)
        d = self._decoder(M)
        if batched_prefill:
            d.prefill(prompt)                  # batched MFMA prefill (forced steps where unsupported)
            n_run = 0
        else:
            d.reset(prompt)
            n_run = len(prompt) - 1
        n_pre = len(prompt) - 1
        n_gen = max(0, min(max_new_tokens, M - len(prompt)))
        greedy = temperature <= 0.0
        if use_dev and not eos and on_token is None and on_stage is None:
            if greedy:
                d.run(n_run, n_gen)
            else:
                # device sampling: one uniform per token from numpy's global generator, the draws
                # the reference's per-token np.random.choice makes
                d.run(n_run, 0)
                d.set_sampling(temperature, top_p, top_k, np.random.random_sample(n_gen), n_pre)
                d.run_sampled(n_gen)
            return d.history(n_pre, n_gen)
        import torch
        profiling = on_stage is not None
        if profiling and n_run:
            # token-by-token prefill, staged as the reference's step() is (aneforge/llm.py:583-597)
            for p in range(n_run):
                self._profiled_step(d, p - 1, prompt[0], on_stage)
                with torch.cuda.stream(d.stream):
                    d.enqueue_advance(False, gather=False)
        else:
            d.run(n_run, 0)
        out = []
        for i in range(n_gen):
            k = n_pre + i
            if profiling:
                # the reference's per-token stages (aneforge/llm.py:568-628): embedding and layers are
                # the two halves of `step`, then lm_head and sample; each stage is its own launches,
                # timed to the end of its device work
                t1 = time.perf_counter()
                self._profiled_step(d, k - 1, prompt[0], on_stage)
                on_stage("step", time.perf_counter() - t1)
            t1 = time.perf_counter()
            if use_dev:
                with torch.cuda.stream(d.stream):
                    if profiling:
                        d.enqueue_head()
                        d.sync()
                        on_stage("lm_head", time.perf_counter() - t1)
                        t1 = time.perf_counter()
                        if not greedy:
                            d.set_sampling(temperature, top_p, top_k, [np.random.random_sample()], k)
                            d.enqueue_sample()
                        d.enqueue_advance(greedy, gather=False)
                    elif greedy:
                        d.run(0, 1)
                    else:
                        d.set_sampling(temperature, top_p, top_k, [np.random.random_sample()], k)
                        d.run_sampled(1)
                nxt = d.history(k, 1)[0]
            else:                                    # host lm_head (ane_lm_head=False)
                if not profiling:
                    with torch.cuda.stream(d.stream):
                        d.enqueue_layers()
                    d.sync()
                hn = d.h.float().cpu().numpy()[0]
                g = np.asarray(self.w["final_norm"], np.float64)
                hn = hn / np.sqrt((hn.astype(np.float64) ** 2).mean() + self.cfg.norm_eps) * g
                logits = self._host_logits(hn.astype(np.float16).astype(np.float32))
                if profiling:
                    on_stage("lm_head", time.perf_counter() - t1)
                    t1 = time.perf_counter()
                nxt = self._sample(logits, temperature, top_p, top_k)
                with torch.cuda.stream(d.stream):
                    d.forced[k].fill_(nxt)
                    d.n_forced.fill_(k + 1)
                    d.enqueue_advance(False, gather=not profiling)
                d.sync()
            if profiling:
                on_stage("sample", time.perf_counter() - t1)
            out.append(int(nxt))
            if nxt in eos:
                break
            if on_token is not None:
                on_token(int(nxt))
        return out

    @staticmethod
    def _profiled_step(d, hist_idx: int, first_tok: int, on_stage):
        """One decode step's layers with the pending token's embedding gathered as a launch of its
        own (the token is hist[hist_idx], or first_tok before any step): emits `embedding` and
        `layers`, each timed to the end of its device work."""
        import torch
        t0 = time.perf_counter()
        with torch.cuda.stream(d.stream):
            ids = (d.hist[hist_idx:hist_idx + 1] if hist_idx >= 0
                   else torch.tensor([int(first_tok)], dtype=torch.int32, device="cuda"))
            d.enqueue_embed(ids)
        d.sync()
        on_stage("embedding", time.perf_counter() - t0)
        t0 = time.perf_counter()
        with torch.cuda.stream(d.stream):
            d.enqueue_layers()
        d.sync()
        on_stage("layers", time.perf_counter() - t0)


# ----------------------------------------------------------------------------- HF adapters
# Hugging Face Llama/Qwen parameter names below "model.layers.<i>." -> canonical per-layer keys.
_HF_LAYER = {"wq": "self_attn.q_proj.weight", "wk": "self_attn.k_proj.weight", "wv": "self_attn.v_proj.weight",
             "wo": "self_attn.o_proj.weight", "attn_norm": "input_layernorm.weight",
             "mlp_norm": "post_attention_layernorm.weight"}
# present only in some checkpoints: the dense MLP (absent on expert layers), QK-norm, projection biases
_HF_LAYER_OPTIONAL = {"wgate": "mlp.gate_proj.weight", "wup": "mlp.up_proj.weight", "wdown": "mlp.down_proj.weight",
                      "q_norm": "self_attn.q_norm.weight", "k_norm": "self_attn.k_norm.weight",
                      "q_bias": "self_attn.q_proj.bias", "k_bias": "self_attn.k_proj.bias",
                      "v_bias": "self_attn.v_proj.bias", "o_bias": "self_attn.o_proj.bias"}


def _weights_from_state_dict(sd, cfg: LlamaConfig) -> dict:
    """A Llama/Qwen Hugging Face state_dict (numpy arrays) as the canonical weight dict; a tied
    head (no lm_head.weight) reuses the embedding."""
    embed = sd["model.embed_tokens.weight"]
    layers = []
    for i in range(cfg.n_layers):
        pre = f"model.layers.{i}."
        lw = {key: sd[pre + name] for key, name in _HF_LAYER.items()}
        lw.update((key, sd[pre + name]) for key, name in _HF_LAYER_OPTIONAL.items() if pre + name in sd)
        layers.append(lw)
    return {"embed": embed, "final_norm": sd["model.norm.weight"], "lm_head": sd.get("lm_head.weight", embed),
            "layers": layers}


def _rope_theta(c) -> float:
    """RoPE base from transformers-5 `rope_parameters`, else the legacy attribute, else 1e4."""
    rp = getattr(c, "rope_parameters", None)
    if isinstance(rp, dict) and "rope_theta" in rp:
        return float(rp["rope_theta"])
    return float(getattr(c, "rope_theta", 10000.0))


def _rope_scaling(c):
    s = getattr(c, "rope_scaling", None)
    if s is None:
        rp = getattr(c, "rope_parameters", None)
        s = rp if isinstance(rp, dict) else None
    return s if isinstance(s, dict) and s.get("rope_type") == "llama3" else None


def _dense_adapter(c, sd) -> tuple[LlamaConfig, dict]:
    n = int(c.num_hidden_layers)
    qk = "model.layers.0.self_attn.q_norm.weight" in sd
    cfg = LlamaConfig(dim=c.hidden_size, n_layers=n, n_heads=c.num_attention_heads,
                      n_kv_heads=getattr(c, "num_key_value_heads", c.num_attention_heads),
                      ffn_dim=c.intermediate_size, vocab=c.vocab_size, rope_base=_rope_theta(c),
                      norm_eps=float(c.rms_norm_eps), head_dim=int(getattr(c, "head_dim", 0) or 0),
                      rope_scaling=_rope_scaling(c),
                      layers=[LayerSpec(mixer="attention", mlp="swiglu", qk_norm=qk) for _ in range(n)])
    return cfg, _weights_from_state_dict(sd, cfg)


def _mistral_adapter(c, sd) -> tuple[LlamaConfig, dict]:
    cfg, w = _dense_adapter(c, sd)
    if getattr(c, "sliding_window", None):
        cfg.extra["sliding_window"] = int(c.sliding_window)
    return cfg, w


def _cfg_from_hf(c) -> LlamaConfig:
    return LlamaConfig(dim=c.hidden_size, n_layers=c.num_hidden_layers, n_heads=c.num_attention_heads,
                       n_kv_heads=getattr(c, "num_key_value_heads", c.num_attention_heads),
                       ffn_dim=c.intermediate_size, vocab=c.vocab_size, rope_base=_rope_theta(c),
                       norm_eps=float(c.rms_norm_eps), head_dim=int(getattr(c, "head_dim", 0) or 0),
                       rope_scaling=_rope_scaling(c))


def _gemma_adapter(c, sd) -> tuple[LlamaConfig, dict]:
    """Gemma (aneforge/llm.py:685-700): a Llama-shaped decoder whose differences go into the weights at
    load time: the embedding rows scaled by sqrt(dim) (HF scales the looked-up embeddings; the tied
    head keeps the unscaled table), the RMSNorm gains in the (1 + w) convention, and the GeGLU MLP
    (`LayerSpec(mlp="geglu")`, tanh-GELU on the gate)."""
    n = int(c.num_hidden_layers)
    cfg = LlamaConfig(dim=c.hidden_size, n_layers=n, n_heads=c.num_attention_heads,
                      n_kv_heads=int(getattr(c, "num_key_value_heads", c.num_attention_heads)),
                      ffn_dim=c.intermediate_size, vocab=c.vocab_size, rope_base=_rope_theta(c),
                      norm_eps=float(c.rms_norm_eps), head_dim=int(getattr(c, "head_dim", 0) or 0),
                      layers=[LayerSpec(mixer="attention", mlp="geglu") for _ in range(n)])
    w = _weights_from_state_dict(sd, cfg)
    w["embed"] = np.asarray(w["embed"], np.float32) * np.float32(np.sqrt(c.hidden_size))
    for lw in w["layers"]:
        lw["attn_norm"] = np.asarray(lw["attn_norm"], np.float32) + 1.0
        lw["mlp_norm"] = np.asarray(lw["mlp_norm"], np.float32) + 1.0
    w["final_norm"] = np.asarray(w["final_norm"], np.float32) + 1.0
    return cfg, w


def _gpt2_adapter(c, sd):
    """GPT-2 (the reference's adapter, aneforge/llm.py:730-763) needs LayerNorm with a bias, learned
    position embeddings and a non-gated GELU MLP with biases; none of these is on this device decode
    path, so the architecture is refused by name rather than mis-loaded as a Llama."""
    raise ValueError("load_llm: 'gpt2' (LayerNorm, learned position embeddings, GELU MLP) is not on this "
                     "decode path; supported: dense Llama / Qwen / Mistral, Gemma and Qwen-MoE")


ADAPTERS: list = [
    (lambda c: getattr(c, "model_type", None) == ModelType.GPT2, _gpt2_adapter),
    (lambda c: getattr(c, "model_type", None) == ModelType.GEMMA, _gemma_adapter),
    (lambda c: getattr(c, "model_type", None) == ModelType.MISTRAL, _mistral_adapter),
]


def adapter_for(c):
    """The adapter from_pretrained uses for a Hugging Face config (first registered match, else the
    dense Llama adapter after its compatibility check)."""
    adapt = next((fn for pred, fn in ADAPTERS if pred(c)), _dense_adapter)
    if adapt is _dense_adapter:
        _assert_dense_compatible(c)
    return adapt


def _assert_dense_compatible(c) -> None:
    """A config headed for the dense Llama adapter must not carry semantics that adapter ignores: logit
    softcapping (checked first, so a Llama-shaped finetune with an unusual model_type still loads) or
    one of the architectures listed above.  The reference draws the same line (aneforge/llm.py:776-788)."""
    model_type = getattr(c, "model_type", "?")
    softcap = getattr(c, "attn_logit_softcapping", None) or getattr(c, "final_logit_softcapping", None)
    if softcap:
        raise ValueError(f"load_llm: {model_type!r} uses logit softcapping, which the dense decoder does not "
                         f"implement; loading it would give wrong logits")
    if model_type in _DENSE_INCOMPATIBLE:
        raise ValueError(f"load_llm: {model_type!r} has architecture-specific semantics the dense decoder does "
                         f"not implement (supported: dense Llama / Qwen / Mistral, Gemma and Qwen-MoE)")


def from_pretrained(name: str, compress: str | None = None, ane_lm_head: bool = True) -> LlamaPrefill:
    """Load a local Hugging Face checkpoint directory (no network access is attempted beyond
    what transformers does for a local path)."""
    import torch
    from transformers import AutoModelForCausalLM
    hf = AutoModelForCausalLM.from_pretrained(name)
    adapt = adapter_for(hf.config)
    sd = {k: v.detach().to(torch.float16).numpy() for k, v in hf.state_dict().items()}
    cfg, weights = adapt(hf.config, sd)
    return LlamaPrefill(cfg, weights, compress=compress, ane_lm_head=ane_lm_head)
