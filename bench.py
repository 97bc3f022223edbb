"""Benchmark of the quantized-decode hot path on one MI355X.

Default workload (the metric BASELINE.json names): a 32-layer 7B-shape Llama decode with all
linears int8 per-channel, fp16 lm_head, fp16 KV cache prefilled to 2048 tokens, greedy decode
at batch 1.  A "step" is one decode token (all layers + lm_head + argmax, one HIP graph).
`value` = tokens/s.  The JSON line also carries the roofline of the dominant kernel (the fused
gate/up int8 GEMV, timed live with HIP events on its launch stream over all 32 layers'
weights) and a CPU baseline (the numpy oracle on a bounded sample, run on this host).

Kernel workloads (--workload gemv_w8 | gemv_q4 | gemv_formats | attn | moe) time one configuration with
rotating weight copies inside a captured graph (working set > 2x the 256 MB MALL).
--workload copy streams a plain 1 GiB copy: the calibration run for the FETCH_SIZE /
WRITE_SIZE counters behind roofline.traffic, and a measured copy ceiling.
--workload prefill times the batched MFMA prefill of a --ctx-token prompt on the cfg3 model.
--workload sample times the device sampler per parameter set, then cfg3 decode with device sampling
against greedy decode in the same run.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload decode]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK = 8.0e12


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--workload", default="decode",
                    choices=["decode", "gemv_w8", "gemv_q4", "gemv_formats", "attn", "moe", "kernels", "copy",
                             "prefill", "sample"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--out", default=None, help="also append the JSON line to this file")
    ap.add_argument("--rows-hint", type=int, default=0)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--shape", default="11008x4096", choices=["11008x4096", "4096x11008"],
                    help="N x K of the cfg1 Q4_0 matrix for --workload gemv_q4")
    ap.add_argument("--ctx", type=int, default=2048)
    ap.add_argument("--weights", default="int8", choices=["int8", "q4_0", "blockwise", "lut4", "q4_k"],
                    help="linear weight format of the cfg3 model for --workload prefill")
    return ap.parse_args()


# ----------------------------------------------------------------------------- timing helpers
class Graph:
    """A captured kernel sequence on a private stream (afx_graph_* over hipStreamBeginCapture)."""

    def __init__(self, fn):
        import ctypes
        import torch
        from aneforge_amd import _hip
        self.stream = torch.cuda.Stream()
        self.exec = ctypes.c_void_p()
        with torch.cuda.stream(self.stream):
            _hip.call("afx_graph_begin", self.stream.cuda_stream)
            try:
                fn()
            finally:
                _hip.call("afx_graph_end", self.stream.cuda_stream, ctypes.byref(self.exec))

    def launch(self):
        from aneforge_amd import _hip
        _hip.call("afx_graph_launch", self.exec, self.stream.cuda_stream)

    def time_ms(self, reps: int) -> float:
        """Milliseconds per replay, HIP events recorded on the graph's own stream."""
        import ctypes
        from aneforge_amd import _hip
        e0, e1 = ctypes.c_void_p(), ctypes.c_void_p()
        _hip.call("afx_event_create", ctypes.byref(e0))
        _hip.call("afx_event_create", ctypes.byref(e1))
        _hip.call("afx_event_record", e0, self.stream.cuda_stream)
        for _ in range(reps):
            self.launch()
        _hip.call("afx_event_record", e1, self.stream.cuda_stream)
        ms = ctypes.c_float()
        _hip.call("afx_event_elapsed_ms", e0, e1, ctypes.byref(ms))
        _hip.call("afx_event_destroy", e0)
        _hip.call("afx_event_destroy", e1)
        return ms.value / reps

    def close(self):
        from aneforge_amd import _hip
        _hip.call("afx_graph_destroy", self.exec)


def n_copies(bytes_per_copy: int, floor: int = 4) -> int:
    """Enough independent copies to exceed 2x the 256 MB Infinity Cache."""
    return max(floor, int(np.ceil(2 * 256e6 * 1.25 / bytes_per_copy)))


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ----------------------------------------------------------------------------- kernel workloads
def bench_gemv_w8(args):
    import torch
    from aneforge_amd import _kernels as K
    N = Kd = 4096
    B = args.batch
    copies = n_copies(N * Kd)
    g = torch.Generator(device="cuda").manual_seed(0)
    ws = [torch.randint(-127, 128, (N, Kd), dtype=torch.int8, device="cuda", generator=g) for _ in range(copies)]
    ss = [(torch.rand(N, device="cuda", generator=g) * 0.02 / 127).half() for _ in range(copies)]
    x = torch.randn((B, Kd), device="cuda", generator=g).half()
    y = torch.empty((B, N), dtype=torch.float16, device="cuda")
    gr = Graph(lambda: [K.linear("int8", ws[i], ss[i], x, y=y, rows_hint=args.rows_hint) for i in range(copies)])
    for _ in range(3):
        gr.launch()
    reps = max(1, args.steps // 8)
    ms = gr.time_ms(reps) / copies
    byts = N * Kd + 2 * N + 2 * B * Kd + 2 * B * N
    return {"workload": "cfg0 int8 per-channel GEMV 4096x4096", "batch": B, "us": ms * 1e3,
            "bytes": byts, "GBps": byts / (ms * 1e-3) / 1e9, "frac": byts / (ms * 1e-3) / HBM_PEAK,
            "copies": copies}


def _format_weights(fmt, N, Kd, copies, g):
    """Random weights of one format (codes + side arrays) for a GEMV timing, `copies` distinct sets."""
    import torch
    out = []
    for _ in range(copies):
        if fmt == "fp16":
            out.append(((torch.randn((N, Kd), device="cuda", generator=g) * 0.02).half(), None))
        elif fmt in ("int8", "blockwise"):
            q = torch.randint(-127, 128, (N, Kd), dtype=torch.int8, device="cuda", generator=g)
            sh = (N, Kd // 32) if fmt == "blockwise" else (N,)
            out.append((q, (torch.rand(sh, device="cuda", generator=g) * 1e-4).half()))
        elif fmt == "q4_0":
            out.append((torch.randint(0, 256, (N, Kd // 2), dtype=torch.uint8, device="cuda", generator=g),
                        (torch.rand((N, Kd // 32), device="cuda", generator=g) * 0.005).half()))
        elif fmt == "lut4":
            out.append((torch.randint(0, 256, (N, Kd // 2), dtype=torch.uint8, device="cuda", generator=g),
                        (torch.randn((N, 16), device="cuda", generator=g) * 0.02).half()))
        elif fmt == "q4_k":
            h = torch.randint(0, 2 ** 31 - 1, (N, Kd // 256, 5), dtype=torch.int32, device="cuda", generator=g)
            h[:, :, 0] = 0x18001400                   # d = 2^-10, dmin = 2^-9
            out.append((torch.randint(0, 256, (N, Kd // 2), dtype=torch.uint8, device="cuda", generator=g),
                        h.reshape(N, -1).contiguous()))
        elif fmt == "q6_k":
            h = torch.randint(0, 2 ** 31 - 1, (N, Kd // 32, 3), dtype=torch.int32, device="cuda", generator=g)
            h[:, :, 2] = 0x1C000305                   # d = 2^-8, scales 5 and 3
            out.append((torch.randint(0, 256, (N, Kd // 2), dtype=torch.uint8, device="cuda", generator=g),
                        h.reshape(N, -1).contiguous()))
    return out


def _format_bytes(fmt, N, Kd):
    """Weight + side-array bytes of one [N, K] matrix in a kernel format."""
    return {"fp16": 2 * N * Kd, "int8": N * Kd + 2 * N, "blockwise": N * Kd + N * Kd // 16,
            "q4_0": N * Kd // 2 + N * Kd // 16, "lut4": N * Kd // 2 + 32 * N,
            "q4_k": N * Kd // 2 + N * Kd // 256 * 20, "q6_k": N * Kd // 2 + N * Kd // 32 * 12}[fmt]


def bench_gemv_formats(args):
    """Every weight format's B=1 GEMV at the 7B shapes (4096x4096, 22016x4096, 4096x11008), on
    rotating weight copies in a graph: microseconds and the format's bytes per microsecond."""
    import torch
    from aneforge_amd import _kernels as K
    g = torch.Generator(device="cuda").manual_seed(4)
    rows = []
    for N, Kd in ((4096, 4096), (22016, 4096), (4096, 11008)):
        for fmt in ("fp16", "int8", "blockwise", "q4_0", "lut4", "q4_k", "q6_k"):
            byts = _format_bytes(fmt, N, Kd)
            copies = n_copies(byts)
            ws = _format_weights(fmt, N, Kd, copies, g)
            x = torch.randn((1, Kd), device="cuda", generator=g).half()
            y = torch.empty((1, N), dtype=torch.float16, device="cuda")
            gr = Graph(lambda: [K.linear(fmt, w, sc, x, y=y) for w, sc in ws])
            for _ in range(3):
                gr.launch()
            ms = min(gr.time_ms(max(1, args.steps // 8)) for _ in range(3)) / copies
            gr.close()
            rows.append({"workload": f"GEMV {fmt} {N}x{Kd} B=1", "us": ms * 1e3, "bytes": byts,
                         "GBps": byts / (ms * 1e-3) / 1e9, "frac": byts / (ms * 1e-3) / HBM_PEAK, "copies": copies})
            del ws
            torch.cuda.empty_cache()
    return rows


def bench_gemv_q4(args, N=11008, Kd=4096):
    import torch
    from aneforge_amd import _kernels as K
    B = args.batch
    copies = n_copies(N * Kd // 2)
    g = torch.Generator(device="cuda").manual_seed(1)
    qs = [torch.randint(0, 256, (N, Kd // 2), dtype=torch.uint8, device="cuda", generator=g) for _ in range(copies)]
    ds = [(torch.rand((N, Kd // 32), device="cuda", generator=g) * 0.005).half() for _ in range(copies)]
    x = torch.randn((B, Kd), device="cuda", generator=g).half()
    y = torch.empty((B, N), dtype=torch.float16, device="cuda")
    ws = torch.empty(8 * B * N, dtype=torch.float32, device="cuda")    # K-split partials (long rows)
    gr = Graph(lambda: [K.linear("q4_0", qs[i], ds[i], x, y=y, rows_hint=args.rows_hint, ws=ws) for i in range(copies)])
    for _ in range(3):
        gr.launch()
    ms = gr.time_ms(max(1, args.steps // 8)) / copies
    byts = N * Kd // 32 * 18 + 2 * B * Kd + 2 * B * N
    return {"workload": f"cfg1 Q4_0 GEMV {N}x{Kd}", "batch": B, "us": ms * 1e3, "bytes": byts,
            "GBps": byts / (ms * 1e-3) / 1e9, "frac": byts / (ms * 1e-3) / HBM_PEAK, "copies": copies}


def bench_attn(args, ctx=None, B=None):
    import torch
    from aneforge_amd import _kernels as K
    ctx = ctx or args.ctx
    B = B or args.batch
    Hq, Hkv, D = 32, 8, 128
    per = 2 * B * Hkv * ctx * D * 2
    copies = n_copies(per, floor=2)
    g = torch.Generator(device="cuda").manual_seed(2)
    ks = [torch.randn((B, Hkv, ctx, D), device="cuda", generator=g).half() for _ in range(copies)]
    vs = [torch.randn((B, Hkv, ctx, D), device="cuda", generator=g).half() for _ in range(copies)]
    q = torch.randn((B, Hq, D), device="cuda", generator=g).half()
    o = torch.empty_like(q)
    ws = torch.zeros(K.attn_ws_bytes(B, Hq, Hkv, D, ctx) // 4 + 1, dtype=torch.float32, device="cuda")
    gr = Graph(lambda: [K.decode_attn(q, ks[i], vs[i], o=o, ctx_len=ctx, ws=ws) for i in range(copies)])
    for _ in range(3):
        gr.launch()
    ms = gr.time_ms(max(1, args.steps // 8)) / copies
    byts = per + 2 * 2 * B * Hq * D
    return {"workload": f"cfg2 decode attention ctx={ctx}", "batch": B, "us": ms * 1e3, "bytes": byts,
            "GBps": byts / (ms * 1e-3) / 1e9, "frac": byts / (ms * 1e-3) / HBM_PEAK, "copies": copies}


def bench_sample(args):
    """Device sampling: afx_sample (prep + pick launches) per parameter set at the cfg3 vocabulary and
    Qwen's 151936, N(0, 2.5^2) logits; then cfg3 decode with the sampler in the step graph against
    greedy decode in the same run."""
    import ctypes
    import torch
    from aneforge_amd import _hip, _kernels as K
    rows = []
    sets = [(0.8, 1.0, 0), (0.8, 0.9, 40), (0.7, 0.9, 0), (1.0, 0.95, 0), (0.6, 0.9, 50)]
    for V in (CFG3["vocab"], 151936):
        g = torch.Generator(device="cuda").manual_seed(7)
        lg = torch.randn(V, device="cuda", generator=g) * 2.5
        uni = torch.rand(64, dtype=torch.float64, device="cuda", generator=g)
        step = torch.zeros(1, dtype=torch.int32, device="cuda")
        out = torch.zeros(1, dtype=torch.int32, device="cuda")
        ws = torch.empty(K.sample_ws_elems(V), dtype=torch.float64, device="cuda")
        for T, top_p, top_k in sets:
            params = torch.tensor([T, top_p, float(top_k)], dtype=torch.float64, device="cuda")
            gr = Graph(lambda: [K.sample(lg, params, uni, step=step, out=out, ws=ws) for _ in range(8)])
            for _ in range(3):
                gr.launch()
            ms = gr.time_ms(8) / 8
            rows.append({"workload": f"afx_sample V={V} T={T} top_p={top_p} top_k={top_k}", "us": ms * 1e3})
    # sampled cfg3 decode against greedy, same engine and positions
    K_steps, W_steps = args.steps, args.warmup
    cfg, eng, layers = build_cfg3_engine(K_steps, W_steps)
    P = CFG3["prefill"]
    e0, e1 = ctypes.c_void_p(), ctypes.c_void_p()
    _hip.call("afx_event_create", ctypes.byref(e0))
    _hip.call("afx_event_create", ctypes.byref(e1))

    def timed(run):
        eng.reset([1], pos0=P, zero_state=False)
        run(W_steps)
        eng.sync()
        eng.reset([1], pos0=P, zero_state=False)
        eng.sync()
        _hip.call("afx_event_record", e0, eng.stream.cuda_stream)
        run(K_steps)
        _hip.call("afx_event_record", e1, eng.stream.cuda_stream)
        ms = ctypes.c_float()
        _hip.call("afx_event_elapsed_ms", e0, e1, ctypes.byref(ms))
        eng.sync()
        return K_steps / (ms.value / 1e3)

    greedy = timed(lambda n: eng.run(0, n))
    rng = np.random.default_rng(8)
    T, top_p, top_k = 0.8, 0.9, 40
    eng.set_sampling(T, top_p, top_k, rng.random(max(K_steps, W_steps) + 8), 0)
    sampled = timed(lambda n: eng.run_sampled(n))
    rows.append({"workload": f"cfg3 decode, device sampling T={T} top_p={top_p} top_k={top_k}",
                 "tokens_per_s": sampled, "greedy_tokens_per_s": greedy})
    return rows


def bench_moe(args):
    """cfg4: one MoE decode layer, 8 Q4_0 experts (gate/up 14336x4096, down 4096x14336), top-2 with
    renormalisation, 16 tokens, fp16 router ~N(0, 0.02), gamma = 1, h ~N(0, 1).  Expert codes are
    uniform nibbles written straight into the superblock layout on the device (the layout is a
    bit-preserving permutation of GGUF Q4_0), block scales |N(0, 0.02)| / 8.  Timed as a captured
    graph of the whole layer as the decode engine runs it: norm + router + top-k + bucketing in one
    launch, grouped gate/up + SwiGLU, grouped down (K-split) with the weighted combine + residual;
    algorithmic bytes = distinct active experts x 99 090 432 B
    + router + activations."""
    import torch
    from aneforge_amd import _kernels as K
    E, k, D, F, T = 8, 2, 4096, 14336, 16
    g = torch.Generator(device="cuda").manual_seed(4)
    gu_w = torch.randint(0, 256, (E * 2 * F, D // 2), dtype=torch.uint8, device="cuda", generator=g)
    gu_d = (torch.randn((E * 2 * F, D // 32), device="cuda", generator=g).abs() * (0.02 / 8)).half()
    dn_w = torch.randint(0, 256, (E * D, F // 2), dtype=torch.uint8, device="cuda", generator=g)
    dn_d = (torch.randn((E * D, F // 32), device="cuda", generator=g).abs() * (0.02 / 8)).half()
    router = (torch.randn((E, D), device="cuda", generator=g) * 0.02).half()
    gamma = torch.ones(D, dtype=torch.float16, device="cuda")
    h = torch.randn((T, D), device="cuda", generator=g).half()
    hout = torch.empty_like(h)           # the layer output goes elsewhere so every replay routes alike
    hn = torch.empty_like(h)
    logits = torch.empty((T, E), dtype=torch.float32, device="cuda")
    gate = torch.empty((T, k), dtype=torch.float32, device="cuda")
    sel = torch.empty((T, k), dtype=torch.int32, device="cuda")
    cnt = torch.empty((E,), dtype=torch.int32, device="cuda")
    lst = torch.empty((E, T), dtype=torch.int32, device="cuda")
    act = torch.empty((T * k, F), dtype=torch.float16, device="cuda")
    y = torch.empty((T * k, D), dtype=torch.float32, device="cuda")
    ws = torch.empty(8 * T * k * D, dtype=torch.float32, device="cuda")   # K-split partials of the down
    sync = K.moe_route_sync()                                              # the router's per-token form

    def layer():                          # the launches of MoEDecode.run (aneforge_amd/moe.py)
        K.moe_route(h, gamma, 1e-5, router, k, True, hn, gate, sel, cnt, lst, sync=sync)
        K.moe_gateup("q4_0", gu_w, gu_d, hn, k, E, F, cnt, lst, act=act)
        K.moe_down_combine("q4_0", dn_w, dn_d, act, T, k, E, F, D, cnt, lst, y, h, gate, out=hout, ws=ws)

    layer()
    torch.cuda.synchronize()
    active = int((cnt > 0).sum().item())
    gr = Graph(layer)
    gr.launch()
    reps = max(2, args.steps // 8)
    ms = gr.time_ms(reps)
    expert_bytes = 2 * F * (D // 32) * 18 + D * (F // 32) * 18
    byts = active * expert_bytes + E * D * 2 + 2 * T * D * 2 + 2 * D
    return {"workload": "cfg4 MoE decode layer: 8 Q4_0 experts, top-2, d4096, ffn 14336, 16 tokens",
            "active_experts": active, "us": ms * 1e3, "bytes": byts, "GBps": byts / (ms * 1e-3) / 1e9,
            "frac": byts / (ms * 1e-3) / HBM_PEAK}


def bench_copy(args):
    """A plain streaming copy of known size (1 GiB read, 1 GiB written, fp16 elements) through
    afx_copy_strided: under `rocprofv3 --pmc FETCH_SIZE` / `WRITE_SIZE` it gives the factor that
    turns those counters into HBM bytes."""
    import torch
    from aneforge_amd import _kernels as K
    n = 1 << 29
    src = torch.ones(n, dtype=torch.float16, device="cuda")
    dst = torch.empty_like(src)
    gr = Graph(lambda: K.copy_strided(src, [1], [n], dst=dst))
    for _ in range(max(1, args.warmup)):
        gr.launch()
    ms = gr.time_ms(max(1, args.steps))
    gr.close()
    return {"workload": "copy 1 GiB fp16 (afx_copy_strided)", "bytes_read": 2 * n, "bytes_written": 2 * n,
            "us": ms * 1e3, "GBps": 4 * n / (ms * 1e-3) / 1e9}


def profile_value(name: str, key: str):
    """A figure recorded in a committed profile summary (a `key: value` line), or None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", name)
    try:
        with open(path) as f:
            for line in f:
                if line.strip().startswith(key + ":"):
                    return float(line.split(":", 1)[1].split()[0])
    except OSError:
        return None
    return None


def bench_kernels(args):
    out = []
    a = argparse.Namespace(**vars(args))
    a.batch = 1
    out.append(bench_gemv_w8(a))
    for N, Kd in ((11008, 4096), (4096, 11008)):
        for B in (1, 4, 8):
            a.batch = B
            out.append(bench_gemv_q4(a, N, Kd))
    for B in (1, 16):
        for ctx in (512, 2048, 8192):
            out.append(bench_attn(a, ctx, B))
    out.append(bench_moe(a))
    return out


# ----------------------------------------------------------------------------- cfg3 decode
CFG3 = dict(dim=4096, n_layers=32, n_heads=32, n_kv_heads=8, ffn_dim=11008, vocab=32000, prefill=2048)


def cfg3_token_bytes(pos: int) -> int:
    """Algorithmic (compulsory) HBM bytes of one decode token at position `pos`: every layer's
    int8 weights + fp16 scales + fp16 norm gammas, the fp16 lm_head + final gamma, KV read of
    rows [0, pos] and the KV row write."""
    D, L, F, V, KV, dh = 4096, 32, 11008, 32000, 8, 128
    per_layer_w = (D * D + 2 * KV * dh * D + D * D + 2 * F * D + D * F)            # int8 codes
    per_layer_s = 2 * (D + 2 * KV * dh + D + 2 * F + D)                           # fp16 row scales
    per_layer_g = 2 * 2 * D                                                       # two gammas
    kv = L * 2 * KV * (pos + 1) * dh * 2 + L * 2 * KV * dh * 2                     # read + write
    return L * (per_layer_w + per_layer_s + per_layer_g) + V * D * 2 + 2 * D + kv


def build_cfg3_engine(steps: int, warmup: int, fmt: str = "int8"):
    import torch
    from aneforge_amd import _engine as E
    from aneforge_amd.llm import LlamaConfig
    c = CFG3
    cfg = LlamaConfig(dim=c["dim"], n_layers=c["n_layers"], n_heads=c["n_heads"], n_kv_heads=c["n_kv_heads"],
                      ffn_dim=c["ffn_dim"], vocab=c["vocab"])
    D, F, V = c["dim"], c["ffn_dim"], c["vocab"]
    nkv = c["n_kv_heads"] * cfg.dh
    g = torch.Generator(device="cuda").manual_seed(3)

    def i8(N, Kd):
        if fmt == "q4_0":                       # random codes in the superblock layout + block scales
            q = torch.randint(0, 256, (N, Kd // 2), dtype=torch.uint8, device="cuda", generator=g)
            d = (torch.rand((N, Kd // 32), device="cuda", generator=g) * 0.005).half()
            return E.Linear("q4_0", q, d, N, Kd)
        if fmt == "q4_k":                       # random Q4_K codes + super-block headers (d, dmin, 6-bit sc/m)
            q = torch.randint(0, 256, (N, Kd // 2), dtype=torch.uint8, device="cuda", generator=g)
            h = (torch.randint(0, 64, (N, Kd // 256, 5, 4), dtype=torch.int32, device="cuda", generator=g)
                 << (8 * torch.arange(4, dtype=torch.int32, device="cuda"))).sum(-1, dtype=torch.int32)
            h[:, :, 0] = 0x18001400                 # d = 2^-10 (fp16 0x1400), dmin = 2^-9 (0x1800)
            return E.Linear("q4_k", q, h.reshape(N, -1).contiguous(), N, Kd)
        if fmt == "lut4":                       # random indices + a codebook per row
            q = torch.randint(0, 256, (N, Kd // 2), dtype=torch.uint8, device="cuda", generator=g)
            cb = (torch.randn((N, 16), device="cuda", generator=g) * 0.02).half()
            return E.Linear("lut4", q, cb, N, Kd)
        q = torch.randint(-127, 128, (N, Kd), dtype=torch.int8, device="cuda", generator=g)
        if fmt == "blockwise":
            s = (torch.rand((N, Kd // 32), device="cuda", generator=g) * (0.02 / 127)).half()
            return E.Linear("blockwise", q, s, N, Kd)
        s = (torch.randn(N, device="cuda", generator=g).abs() * (0.02 / 127)).half()
        return E.Linear("int8", q, s, N, Kd)

    ones = torch.ones(D, dtype=torch.float16, device="cuda")
    layers = []
    for _ in range(c["n_layers"]):
        layers.append((E.AttentionDecode.from_linears(cfg, i8(D + 2 * nkv, D), i8(D, D), ones),
                       E.SwiGLUDecode.from_linears(cfg, i8(2 * F, D), i8(D, F), ones)))
    embed = (torch.randn((V, D), device="cuda", generator=g) * 0.02).half()
    head = E.Linear("fp16", (torch.randn((V, D), device="cuda", generator=g) * 0.02).half(), None, V, D)
    M = c["prefill"] + max(steps, warmup) + 8
    eng = E.DecodeEngine(cfg, layers, embed, head, ones, M)
    P = c["prefill"]
    for mixer, _ in layers:                     # resident cache prefilled with N(0, 1) rows [0, 2048)
        mixer.kc[:, :, :P].normal_(generator=g)
        mixer.vc[:, :, :P].normal_(generator=g)
    torch.cuda.synchronize()
    return cfg, eng, layers


def time_dominant_kernel(eng, layers, reps: int = 10):
    """Average duration of the fused RMSNorm + gate/up + SwiGLU int8 GEMV, one launch per layer
    (32 distinct weight sets, 2.9 GB: no cache reuse), HIP events on the launching stream."""
    from aneforge_amd import _kernels as K

    def body():
        for _, mlp in layers:
            K.linear_swiglu(mlp.gu.fmt, mlp.gu.w, mlp.gu.scale, eng.h, mlp.norm, mlp.eps, act=eng.act[:, :mlp.F])

    gr = Graph(body)
    gr.launch()
    ms = gr.time_ms(reps) / len(layers)
    gr.close()
    mlp = layers[0][1]
    N, Kd = mlp.gu.N, mlp.gu.K
    byts = N * Kd + 2 * N + 2 * Kd + 2 * Kd + 2 * (N // 2)
    return ms, byts


def cpu_baseline_decode(seconds: float = 12.0):
    """The reference CPU path (numpy fp32, oracle.ref.cpu_decode_layer_f32) on one 7B-shape
    layer + the lm_head, dequantised weights prepared outside the timed region; tokens/s is
    extrapolated to 32 layers.  Threads = what the BLAS pool actually uses."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import ref
    rng = np.random.default_rng(3)
    D, F, KV, dh, H, V, P = 4096, 11008, 8, 128, 32, 32000, 2048
    w = {}
    for name, (n, k) in {"wq": (D, D), "wk": (KV * dh, D), "wv": (KV * dh, D), "wo": (D, D),
                         "wgate": (F, D), "wup": (F, D), "wdown": (D, F)}.items():
        q = rng.integers(-127, 128, (n, k), dtype=np.int8)
        s = (np.abs(rng.normal(0, 0.02, n)) / 127).astype(np.float16)
        w[name] = ref.dequant_w8(q, s)
    w["attn_norm"] = np.ones(D, np.float32)
    w["mlp_norm"] = np.ones(D, np.float32)
    lm = (rng.standard_normal((V, D)).astype(np.float32) * np.float32(0.02))
    Kc = rng.standard_normal((KV, P + 64, dh)).astype(np.float32)
    Vc = rng.standard_normal((KV, P + 64, dh)).astype(np.float32)
    cos, sin = ref.rope_tables(P + 64, dh)
    cfg = {"n_heads": H, "n_kv_heads": KV, "dh": dh, "norm_eps": 1e-5}
    h = rng.standard_normal((1, D)).astype(np.float32)
    def sample(budget):
        t_layer, t_head, n, t_end = [], [], 0, time.perf_counter() + budget
        while time.perf_counter() < t_end or n < 2:
            t0 = time.perf_counter()
            p = P + (n % 64)
            ref.cpu_decode_layer_f32(h, w, cfg, Kc, Vc, p, cos[p].astype(np.float32), sin[p].astype(np.float32))
            t1 = time.perf_counter()
            _ = h @ lm.T
            t2 = time.perf_counter()
            t_layer.append(t1 - t0)
            t_head.append(t2 - t1)
            n += 1
        return 32 * min(t_layer) + min(t_head), n

    per_tok, n = sample(seconds)
    threads, per_tok_1, n1 = len(os.sched_getaffinity(0)), None, 0
    try:
        from threadpoolctl import threadpool_info, threadpool_limits
        threads = max([i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"] or [1])
        with threadpool_limits(limits=1, user_api="blas"):
            per_tok_1, n1 = sample(seconds / 3)
    except Exception:
        pass
    return {"value": 1.0 / per_tok, "unit": "tokens/s", "cores": int(threads), "kind": "port",
            "value_1thread": None if per_tok_1 is None else 1.0 / per_tok_1,
            "host_cores_available": len(os.sched_getaffinity(0)), "os_cpu_count": os.cpu_count(),
            "sample": f"numpy fp32 restatement of the reference CPU decode (bench/decode_measurement.py:86-132 + "
                      f"GQA/RoPE) on one 4096/11008/32-head layer at pos {P} + the 32000x4096 lm_head, min of "
                      f"{n} reps ({n1} at 1 BLAS thread), extrapolated to 32 layers"}


def bench_prefill(args):
    """Batched prefill of a --ctx-token prompt (default 2048) through the 32-layer cfg3 model
    (int8 weights): MFMA GEMMs + causal flash attention, filling the resident cache.  Timed with
    HIP events on the engine stream over `steps` prefills after `warmup`; FLOPs = 2 x linear
    weights x prompt rows + causal attention (2 x 2 x Hq x dh x sum of context lengths)."""
    import ctypes
    import torch
    from aneforge_amd import _hip
    P = int(args.ctx)
    log(f"building cfg3 engine (32 layers {args.weights}) for a {P}-token batched prefill")
    cfg, eng, layers = build_cfg3_engine(P, 0, args.weights)
    prompt = [int(t) for t in np.random.default_rng(5).integers(0, CFG3["vocab"], P + 1)]
    for _ in range(max(1, args.warmup)):
        eng.prefill(prompt)
    eng.sync()
    e0, e1 = ctypes.c_void_p(), ctypes.c_void_p()
    _hip.call("afx_event_create", ctypes.byref(e0))
    _hip.call("afx_event_create", ctypes.byref(e1))
    reps = max(1, min(args.steps, 8))
    _hip.call("afx_event_record", e0, eng.stream.cuda_stream)
    for _ in range(reps):
        eng.prefill(prompt)
    _hip.call("afx_event_record", e1, eng.stream.cuda_stream)
    ms = ctypes.c_float()
    _hip.call("afx_event_elapsed_ms", e0, e1, ctypes.byref(ms))
    torch.cuda.synchronize()
    per = ms.value / reps
    D, F, H, KV, dh = CFG3["dim"], CFG3["ffn_dim"], CFG3["n_heads"], CFG3["n_kv_heads"], 128
    lin = D * (H * dh + 2 * KV * dh) + H * dh * D + 2 * F * D + F * D
    flops = 2.0 * CFG3["n_layers"] * P * (lin + 2 * H * dh * (P + 1) / 2.0)
    return {"workload": f"cfg3 batched prefill, {P}-token prompt, 32 layers {args.weights} (MFMA GEMM + causal flash attention)",
            "prompt_tokens": P, "ms": per, "tokens_per_s": P / (per * 1e-3), "TFLOPs": flops / (per * 1e-3) / 1e12,
            "mfma_peak_TFLOPs_fp16": 2500.0}


def bench_decode(args):
    import ctypes
    import torch
    from aneforge_amd import _hip
    K_steps, W_steps = args.steps, args.warmup
    log(f"building cfg3 engine (32 layers int8, KV prefilled to {CFG3['prefill']})")
    cfg, eng, layers = build_cfg3_engine(K_steps, W_steps)
    log(f"weights resident: {eng.weight_bytes / 1e9:.3f} GB; capturing step graphs")
    P = CFG3["prefill"]
    eng.reset([1], pos0=P, zero_state=False)
    eng.run(0, W_steps)
    eng.sync()
    eng.reset([1], pos0=P, zero_state=False)     # timed steps cover positions P .. P+K-1
    eng.sync()
    torch.cuda.synchronize()
    e0, e1 = ctypes.c_void_p(), ctypes.c_void_p()
    _hip.call("afx_event_create", ctypes.byref(e0))
    _hip.call("afx_event_create", ctypes.byref(e1))
    t0 = time.perf_counter()
    _hip.call("afx_event_record", e0, eng.stream.cuda_stream)
    eng.run(0, K_steps)
    _hip.call("afx_event_record", e1, eng.stream.cuda_stream)
    ms = ctypes.c_float()
    _hip.call("afx_event_elapsed_ms", e0, e1, ctypes.byref(ms))
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_s = ms.value / 1e3
    toks = eng.history(0, K_steps)
    log(f"decoded {K_steps} tokens in {gpu_s * 1e3:.2f} ms (events), wall {wall * 1e3:.2f} ms; first tokens {toks[:8]}")
    per_tok_bytes = np.mean([cfg3_token_bytes(P + i) for i in range(K_steps)])
    tok_s = K_steps / gpu_s
    roof_tok_s = HBM_PEAK / per_tok_bytes
    k_ms, k_bytes = time_dominant_kernel(eng, layers)
    achieved = k_bytes / (k_ms * 1e-3)
    out = {
        "metric": "quantized decode GEMV GB/s (% HBM peak) + tokens/s, 7B-shape int8 decode, bs=1",
        "value": tok_s, "unit": "tokens/s", "n_gpus": 1, "steps": K_steps, "warmup": W_steps,
        "ms_per_step": gpu_s * 1e3 / K_steps, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8 weights / fp16 activations / fp32 accumulate", "data": "synthetic",
        "config": {"workload": "cfg3: 32-layer Llama-style decode, d4096, 32/8 heads, SwiGLU 11008, vocab 32000, "
                               "int8 per-channel linears, fp16 lm_head, fp16 KV prefilled to 2048, greedy bs=1",
                   "global_batch": 1, "seq_len": P + K_steps, "parallelism": "none (1 GPU)"},
        "decode": {"bytes_per_token": per_tok_bytes, "effective_GBps": per_tok_bytes * tok_s / 1e9,
                   "roofline_tokens_per_s": roof_tok_s, "frac_of_roofline": tok_s / roof_tok_s,
                   # per layer: QKV+RoPE+KV write, attention partials, split combine, o-proj, gate/up, down
                   "kernels_per_token": 6 * CFG3["n_layers"] + 2},
        "roofline": {"bound": "hbm",
                     "kernel": "gemv_row_kernel<int8, R=2, norm, SwiGLU>: fused RMSNorm + gate/up + SwiGLU (22016x4096)",
                     "achieved": achieved / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK, "avg_launch_us": k_ms * 1e3, "bytes_per_launch": k_bytes,
                     # HBM bytes per launch from the FETCH_SIZE + WRITE_SIZE counter runs, copy-calibrated
                     "traffic": profile_value("gemv_gateup_cfg3_pmc.md", "traffic_bytes_per_launch")},
    }
    if not args.no_cpu:
        log("timing the CPU baseline (bounded sample)")
        out["cpu_baseline"] = cpu_baseline_decode()
    else:
        out["cpu_baseline"] = None
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 (the multi-GPU sharding "
                                   "of the decode is designed, not built)"}))
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    if args.workload == "kernels":
        for r in bench_kernels(args):
            print(json.dumps(r), flush=True)
        return
    if args.workload == "gemv_w8":
        print(json.dumps(bench_gemv_w8(args)))
        return
    if args.workload == "gemv_formats":
        for r in bench_gemv_formats(args):
            print(json.dumps(r), flush=True)
        return
    if args.workload == "gemv_q4":
        n, kd = (int(v) for v in args.shape.split("x"))
        print(json.dumps(bench_gemv_q4(args, n, kd)))
        return
    if args.workload == "attn":
        print(json.dumps(bench_attn(args)))
        return
    if args.workload == "moe":
        print(json.dumps(bench_moe(args)))
        return
    if args.workload == "copy":
        print(json.dumps(bench_copy(args)))
        return
    if args.workload == "prefill":
        print(json.dumps(bench_prefill(args)))
        return
    if args.workload == "sample":
        for r in bench_sample(args):
            print(json.dumps(r), flush=True)
        return
    if args.workload == "decode":
        res = bench_decode(args)
        line = json.dumps(res)
        print(line, flush=True)
        if args.out:
            with open(args.out, "a") as f:
                f.write(line + "\n")
        return
    raise SystemExit(f"workload {args.workload} not built yet")


if __name__ == "__main__":
    main()
