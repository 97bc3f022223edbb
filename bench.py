"""Benchmark of the quantized-decode hot path on one MI355X.

Default workload (the metric BASELINE.json names): a 32-layer 7B-shape Llama decode with all
linears int8 per-channel, fp16 lm_head, fp16 KV cache prefilled to 2048 tokens, greedy decode
at batch 1.  A "step" is one decode token (all layers + lm_head + argmax, one HIP graph).
`value` = tokens/s.  The JSON line also carries the roofline of the dominant kernel (the fused
gate/up int8 GEMV, timed live with HIP events on its launch stream over all 32 layers'
weights) and a CPU baseline (the numpy oracle on a bounded sample, run on this host).

Kernel workloads (--workload gemv_w8 | gemv_q4 | attn | moe) time one configuration with
rotating weight copies inside a captured graph (working set > 2x the 256 MB MALL).

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
                    choices=["decode", "gemv_w8", "gemv_q4", "attn", "moe", "kernels"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--out", default=None, help="also append the JSON line to this file")
    ap.add_argument("--rows-hint", type=int, default=0)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--ctx", type=int, default=2048)
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
    gr = Graph(lambda: [K.linear("q4_0", qs[i], ds[i], x, y=y, rows_hint=args.rows_hint) for i in range(copies)])
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
    ws = torch.empty(K.attn_ws_bytes(B, Hq, Hkv, D, ctx) // 4 + 1, dtype=torch.float32, device="cuda")
    gr = Graph(lambda: [K.decode_attn(q, ks[i], vs[i], o=o, ctx_len=ctx, ws=ws) for i in range(copies)])
    for _ in range(3):
        gr.launch()
    ms = gr.time_ms(max(1, args.steps // 8)) / copies
    byts = per + 2 * 2 * B * Hq * D
    return {"workload": f"cfg2 decode attention ctx={ctx}", "batch": B, "us": ms * 1e3, "bytes": byts,
            "GBps": byts / (ms * 1e-3) / 1e9, "frac": byts / (ms * 1e-3) / HBM_PEAK, "copies": copies}


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
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 (multi-GPU sharding is "
                                   "design-only, see DESIGN.md)"}))
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
    if args.workload == "gemv_q4":
        print(json.dumps(bench_gemv_q4(args)))
        return
    if args.workload == "attn":
        print(json.dumps(bench_attn(args)))
        return
    raise SystemExit(f"workload {args.workload} not built yet")


if __name__ == "__main__":
    main()
