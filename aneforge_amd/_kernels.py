"""Tensor-level wrappers over the C ABI: device tensors (torch, used only as the allocator and
stream source) in, device tensors out.  Each wrapper validates shapes/dtypes on the host
before launching, so a bad call raises instead of reaching a kernel with wrong extents."""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import _hip

FMT = {"int8": 0, "q4_0": 1, "fp16": 2, "blockwise": 3, "lut4": 4, "q4_k": 5, "q6_k": 6}
EW = {"add": 0, "sub": 1, "mul": 2, "real_div": 3, "maximum": 4, "minimum": 5, "pow": 6,
      "greater_equal": 7, "greater": 8, "equal": 9, "less": 10, "less_equal": 11, "not_equal": 12}
UNARY = {"silu": 0, "sigmoid": 1, "relu": 2, "exp": 3, "tanh": 4, "affine": 5, "sqrt": 6, "abs": 7,
         "neg": 8, "rsqrt": 9, "gelu_tanh": 10, "log": 11, "square": 12, "inverse": 13}
REDUCE = {"reduce_sum": 0, "reduce_max": 1, "reduce_mean": 2, "reduce_min": 3, "reduce_sum_square": 4}


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _nbytes(t) -> int:
    return 0 if t is None else t.numel() * t.element_size()


def P(t) -> int | None:
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _dev(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("aneforge_amd kernels take device tensors")


def _f16(t, name):
    if t.dtype != torch.float16:
        raise TypeError(f"{name} must be float16, got {t.dtype}")


# --------------------------------------------------------------------------- linear layers
def linear(fmt: str, w, scale, x, y=None, bias=None, residual=None, out_f32=False, rows_hint=0, ws=None):
    """y[M, N] = x[M, K] @ W^T (+bias) (+residual) for a packed weight (see _blob).  ws: an optional
    fp32 device workspace; 32 * M * N bytes let long rows take the K-split MFMA path."""
    _dev(w, x, scale, bias, residual, ws)
    M, K = x.shape
    N = w.shape[0]
    if fmt in ("q4_0", "lut4", "q4_k", "q6_k") and w.shape[1] * 2 != K or fmt in ("int8", "blockwise") and w.shape[1] != K:
        raise ValueError(f"linear: weight {tuple(w.shape)} does not match K={K} for {fmt}")
    if y is None:
        y = torch.empty((M, N), dtype=torch.float32 if out_f32 else torch.float16, device=x.device)
    _hip.call("afx_linear", FMT[fmt], P(w), P(scale), P(x), x.stride(0), P(y), y.stride(0), M, N, K,
              P(bias), P(residual), int(out_f32), rows_hint, P(ws), _nbytes(ws), stream())
    return y


def linear_rms(fmt, w, scale, x, gamma, eps, y=None, bias=None, out_f32=False, rows_hint=0):
    _dev(w, x, gamma)
    M, K = x.shape
    N = w.shape[0]
    if y is None:
        y = torch.empty((M, N), dtype=torch.float32 if out_f32 else torch.float16, device=x.device)
    _hip.call("afx_linear_rms", FMT[fmt], P(w), P(scale), P(x), x.stride(0), P(gamma), float(eps), P(y),
              y.stride(0), M, N, K, P(bias), int(out_f32), rows_hint, stream())
    return y


def linear_swiglu(fmt, w, scale, x, gamma=None, eps=0.0, act=None, rows_hint=0, gelu=False):
    """act[M, F] = silu(g) * u (gelu: gelu_tanh(g) * u, GeGLU) with rows of W interleaved
    (gate_i, up_i); RMSNorm first if gamma."""
    _dev(w, x)
    M, K = x.shape
    N = w.shape[0]
    if act is None:
        act = torch.empty((M, N // 2), dtype=torch.float16, device=x.device)
    _hip.call("afx_linear_geglu" if gelu else "afx_linear_swiglu", FMT[fmt], P(w), P(scale), P(x), x.stride(0),
              P(gamma), float(eps), int(gamma is not None), P(act), act.stride(0), M, N, K, rows_hint, stream())
    return act


def qkv_rope_kv(fmt, w, scale, h, gamma, eps, bias, nq, nk, dh, cos_t, sin_t, pos, qout, kcache, vcache,
                rope=True, rows_hint=0):
    """Fused norm + [q|k|v] projection + RoPE + cache write at pos (per sequence row of h)."""
    _dev(w, h, qout, kcache, vcache, pos)
    M, K = h.shape
    if kcache.dim() != 4 or kcache.shape[1] * dh != nk or kcache.shape[3] != dh or vcache.shape != kcache.shape:
        raise ValueError(f"kcache/vcache must be [B, {nk // dh}, Mmax, {dh}], got {tuple(kcache.shape)}")
    if kcache.shape[0] < M or qout.shape[1] < nq or pos.numel() < M:
        raise ValueError("qkv_rope_kv: cache batch, q output or pos too small for M")
    if rope and (cos_t.shape[0] < kcache.shape[2] or cos_t.shape[1] != dh):
        raise ValueError("qkv_rope_kv: rope tables must cover [Mmax, dh]")
    _hip.call("afx_qkv_rope_kv", FMT[fmt], P(w), P(scale), P(h), h.stride(0), P(gamma), float(eps),
              int(gamma is not None), P(bias), nq, nk, nk, dh, P(cos_t), P(sin_t), int(rope), P(pos), P(qout),
              qout.stride(0), P(kcache), P(vcache), kcache.stride(0), kcache.stride(1), kcache.shape[2], M, K, rows_hint,
              stream())
    return qout


# --------------------------------------------------------------------------- codecs
def q4_repack(blocks, N, K):
    """GGUF Q4_0 bytes [N, K/32*18] (uint8, device) -> (qs uint8 [N, K/2], d fp16 [N, K/32])."""
    _dev(blocks)
    qs = torch.empty((N, K // 2), dtype=torch.uint8, device=blocks.device)
    d = torch.empty((N, K // 32), dtype=torch.float16, device=blocks.device)
    _hip.call("afx_q4_0_repack", P(blocks), P(qs), P(d), N, K, stream())
    return qs, d


def q4_k_repack(blocks, N, K):
    """GGUF Q4_K bytes [N, K/256*144] (uint8, device) -> (codes uint8 [N, K/2], header int32 [N, K/256*5])."""
    _dev(blocks)
    qs = torch.empty((N, K // 2), dtype=torch.uint8, device=blocks.device)
    hdr = torch.empty((N, K // 256 * 5), dtype=torch.int32, device=blocks.device)
    _hip.call("afx_q4_k_repack", P(blocks), P(qs), P(hdr), N, K, stream())
    return qs, hdr


def q6_k_repack(blocks, N, K):
    """GGUF Q6_K bytes [N, K/256*210] (uint8, device) -> (codes uint8 [N, K/2], side int32 [N, K/32*3])."""
    _dev(blocks)
    qs = torch.empty((N, K // 2), dtype=torch.uint8, device=blocks.device)
    sw = torch.empty((N, K // 32 * 3), dtype=torch.int32, device=blocks.device)
    _hip.call("afx_q6_k_repack", P(blocks), P(qs), P(sw), N, K, stream())
    return qs, sw


def q4_unpack(qs, d, N, K):
    out = torch.empty((N, K // 32 * 18), dtype=torch.uint8, device=qs.device)
    _hip.call("afx_q4_0_unpack", P(qs), P(d), P(out), N, K, stream())
    return out


def dequant_f16(fmt, w, scale, N, K, out=None):
    """Weights as fp16 [N, K] (row stride out.stride(0)): the values the kernels multiply with."""
    _dev(w, scale)
    if out is None:
        out = torch.empty((N, K), dtype=torch.float16, device=w.device)
    _hip.call("afx_dequant_f16", FMT[fmt], P(w), P(scale), P(out), out.stride(0), N, K, stream())
    return out


def dequant(fmt, w, scale, N, K):
    out = torch.empty((N, K), dtype=torch.float32, device=w.device)
    _hip.call("afx_dequant", FMT[fmt], P(w), P(scale), P(out), N, K, stream())
    return out


# --------------------------------------------------------------------------- attention
def attn_ws_bytes(B, Hq, Hkv, D, max_len, nstep_hint=0) -> int:
    n = _hip.load().afx_decode_attn_ws_bytes(B, Hq, Hkv, D, max_len, nstep_hint)
    if n == -1:
        raise ValueError(f"decode attention: unsupported head dim {D}")
    if n < 0:
        raise ValueError(f"decode attention: a {max_len}-position cache needs more than 128 splits "
                         f"at this split size (nstep {nstep_hint or 'from AFX_ATTN_NSTEP'})")
    return int(n)


def decode_attn(q, k, v, o=None, ctx_len=None, pos=None, scale=None, mask=None, causal_off=-1,
                ws=None, nstep_hint=0, q_strides=None, kv_strides=None, B=None, Hq=None):
    """q [B, Hq, D]; k/v [B, Hkv, Mmax, D]; ctx from pos[b]+1 (device) or ctx_len (host)."""
    _dev(q, k, v, pos, mask)
    if B is None:
        B, Hq, D = q.shape
    else:
        D = q.shape[-1]
    Hkv, Mmax = k.shape[1], k.shape[2]
    if k.shape[-1] != D or v.shape != k.shape:
        raise ValueError(f"decode_attn: k {tuple(k.shape)} / v {tuple(v.shape)} do not match q")
    if mask is not None and (mask.dim() != 2 or mask.shape[0] < B or mask.shape[1] < Mmax or mask.stride(1) != 1):
        raise ValueError(f"decode_attn: mask must be [B, >= {Mmax}] with unit column stride, got {tuple(mask.shape)}")
    if o is None:
        o = torch.empty_like(q)
    qbs, qhs = q_strides if q_strides else (q.stride(0), q.stride(1))
    kbs, khs = kv_strides if kv_strides else (k.stride(0), k.stride(1))
    need = attn_ws_bytes(B, Hq, Hkv, D, Mmax, nstep_hint)
    if ws is None or ws.numel() * ws.element_size() < need:
        ws = torch.empty(need // 4 + 1, dtype=torch.float32, device=q.device)
    scale = (1.0 / D ** 0.5) if scale is None else float(scale)
    _hip.call("afx_decode_attn", P(q), P(k), P(v), P(o), qbs, qhs, kbs, khs, B, Hq, Hkv, D,
              int(ctx_len if ctx_len is not None else Mmax), P(pos), Mmax, P(mask),
              mask.stride(0) if mask is not None else 0, int(causal_off), scale, P(ws),
              need, nstep_hint, stream())
    return o


# --------------------------------------------------------------------------- small ops
def rmsnorm(x, gamma, eps, y=None):
    _dev(x, gamma)
    M, D = x.shape
    if y is None:
        y = torch.empty_like(x)
    _hip.call("afx_rmsnorm", P(x), x.stride(0), P(gamma), float(eps), P(y), y.stride(0), M, D, stream())
    return y


def rope(x, cos_t, sin_t, pos0=0, rows_per_pos=None, pos_dev=None, y=None):
    """x [rows, dh] with row r at position pos0 + r // rows_per_pos (neox half-split)."""
    rows, dh = x.shape
    if y is None:
        y = torch.empty_like(x)
    _hip.call("afx_rope", P(x), P(y), rows, dh, P(cos_t), P(sin_t), P(pos_dev), int(pos0),
              int(rows_per_pos or rows), stream())
    return y


def head_norm_rope(x, heads, dh, gamma, eps, cos_t=None, sin_t=None, pos=None, seq_stride=0, head_stride=None,
                   pos_mul=0, kv_len=1 << 30, M=1, rope=True):
    """In-place per-head RMSNorm (+RoPE) on `heads` rows of length dh inside x."""
    _hip.call("afx_head_norm_rope", P(x), int(seq_stride), int(head_stride if head_stride is not None else dh),
              int(pos_mul), P(pos), int(kv_len), int(heads), int(M), int(dh), P(gamma), float(eps), P(cos_t),
              P(sin_t), int(bool(rope)), stream())
    return x


def embed(table, ids, out=None):
    M = ids.numel()
    V, D = table.shape
    if out is None:
        out = torch.empty((M, D), dtype=table.dtype, device=table.device)
    _hip.call("afx_embed", P(table), P(ids), P(out), M, D, V, stream())
    return out


def sample_ws_elems(V: int) -> int:
    """float64 elements of the afx_sample workspace for V logits (afx_sample_ws_bytes)."""
    n = _hip.load().afx_sample_ws_bytes(V)
    if n < 0:
        raise ValueError(f"sampling: bad vocabulary size {V}")
    return (int(n) + 7) // 8


def sample(logits, params, uniforms, step=None, forced=None, n_forced=None, out=None, ws=None):
    """Device sampling of the next token from fp32 logits [V] (see afx_sample).  params: float64
    [3] {temperature, top_p, top_k}; uniforms: float64, u = uniforms[step] (uniforms[0] without step);
    ws: float64 scratch of at least sample_ws_elems(V) elements (allocated when missing or short)."""
    _dev(logits, params, uniforms, step, forced, n_forced, out)
    V = logits.numel()
    if forced is None and out is None:
        out = torch.empty(1, dtype=torch.int32, device=logits.device)
    need = sample_ws_elems(V)
    if ws is None or ws.numel() < need:
        ws = torch.empty(need, dtype=torch.float64, device=logits.device)
    _hip.call("afx_sample", P(logits), V, P(params), P(uniforms), P(step), P(forced), P(n_forced), P(out),
              P(ws), ws.numel() * 8, stream())
    return out


def decode_advance(logits, tok, pos, hist, step, embed_table=None, h=None, forced=None, n_forced=None,
                   slots=None, tie_margin=None, hn=None, head16=None, head32=None, vocab=None):
    """Next token (forced prompt token, or the greedy pick with the lm_head tie rule when tie_margin
    is given) + bookkeeping + embedding gather (see afx_decode_advance).  Token ids are clamped to
    [0, vocab): the embedding table's rows, else `vocab`, else the logits' width."""
    V = logits.shape[-1] if logits is not None else 0
    D = embed_table.shape[1] if embed_table is not None else 0
    vocab = embed_table.shape[0] if embed_table is not None else (vocab if vocab is not None else V)
    if tie_margin is not None:
        D = hn.numel()
    _hip.call("afx_decode_advance", P(logits), P(slots), V, P(tie_margin), P(hn), P(head16), P(head32),
              P(forced), P(n_forced), P(tok), P(pos), P(hist), hist.numel() if hist is not None else 0, P(step),
              P(embed_table), P(h), D, vocab, stream())


def lm_head(w, x, gamma, eps, logits=None, slots=None, hn=None):
    """fp32 logits [1, N] = rms_norm(x [1, K]) @ W^T for an fp16 head, plus the greedy-pick slots
    (float32 [ceil(N/8), 4]) and, if hn is given, the fp16 normalised row (see afx_lm_head)."""
    _dev(w, x, gamma, logits, slots, hn)
    N, Kd = w.shape
    if logits is None:
        logits = torch.empty((1, N), dtype=torch.float32, device=x.device)
    if slots is None:
        slots = torch.empty(((N + 7) // 8, 4), dtype=torch.float32, device=x.device)
    _hip.call("afx_lm_head", FMT["fp16"], P(w), None, P(x), P(gamma), float(eps), P(logits), N, Kd, P(slots),
              P(hn), stream())
    return logits, slots


def argmax(x, out=None):
    M, V = x.shape
    if out is None:
        out = torch.empty((M,), dtype=torch.int32, device=x.device)
    _hip.call("afx_argmax", P(x), M, V, P(out), stream())
    return out


def fill_i32(t, v):
    _hip.call("afx_fill_i32", P(t), t.numel(), int(v), stream())


def fill_f16(t, v):
    _hip.call("afx_fill_f16", P(t), t.numel(), float(v), stream())


def _ll(vals):
    return (C.c_longlong * 5)(*[int(v) for v in vals] + [0] * (5 - len(vals)))


def _ii(vals):
    return (C.c_int * 5)(*[int(v) for v in vals] + [1] * (5 - len(vals)))


def _bstrides(t, shape):
    """Element strides of `t` broadcast to `shape` (right-aligned; size-1 dims get stride 0)."""
    st = [0] * len(shape)
    off = len(shape) - t.dim()
    for i in range(t.dim()):
        st[off + i] = 0 if t.shape[i] == 1 and shape[off + i] != 1 else t.stride(i)
    return st


def ew_binary(op, a, b, shape):
    y = torch.empty(shape, dtype=torch.float16, device=a.device)
    shape = list(shape) or [1]
    _hip.call("afx_ew_binary", EW[op], P(a), _ll(_bstrides(a, shape)), P(b), _ll(_bstrides(b, shape)), P(y),
              len(shape), _ii(shape), stream())
    return y


def ew_select(c, a, b, shape):
    y = torch.empty(shape, dtype=torch.float16, device=a.device)
    shape = list(shape) or [1]
    _hip.call("afx_ew_select", P(c), _ll(_bstrides(c, shape)), P(a), _ll(_bstrides(a, shape)), P(b),
              _ll(_bstrides(b, shape)), P(y), len(shape), _ii(shape), stream())
    return y


def ew_unary(op, x, alpha=0.0, beta=0.0):
    y = torch.empty_like(x)
    _hip.call("afx_ew_unary", UNARY[op], P(x), P(y), x.numel(), float(alpha), float(beta), stream())
    return y


def copy_strided(src, src_strides, shape, dst=None, dst_strides=None, dst_offset=0):
    """Materialise a strided view of `src` (element strides) into a contiguous tensor."""
    if dst is None:
        dst = torch.empty(shape, dtype=src.dtype, device=src.device)
    if dst_strides is None:
        dst_strides = [0] * len(shape)
        acc = 1
        for i in range(len(shape) - 1, -1, -1):
            dst_strides[i] = acc
            acc *= shape[i]
    base = dst.data_ptr() + dst_offset * dst.element_size()
    _hip.call("afx_copy_strided", P(src), _ll(src_strides), base, _ll(dst_strides), len(shape), _ii(shape),
              stream())
    return dst


def softmax_lastdim(x):
    y = torch.empty_like(x)
    cols = x.shape[-1]
    _hip.call("afx_softmax", P(x), P(y), x.numel() // cols, cols, stream())
    return y


def reduce_lastdim(op, x):
    cols = x.shape[-1]
    rows = x.numel() // cols
    y = torch.empty(tuple(x.shape[:-1]) + (1,), dtype=torch.float16, device=x.device)
    _hip.call("afx_reduce", REDUCE[op], P(x), P(y), rows, cols, stream())
    return y


def bmm(a, b):
    """a [Bt, M, K] @ b [Bt, K, N] (contiguous fp16)."""
    Bt, M, K = a.shape
    N = b.shape[-1]
    c = torch.empty((Bt, M, N), dtype=torch.float16, device=a.device)
    _hip.call("afx_bmm_f16", P(a), P(b), P(c), Bt, M, N, K, M * K if a.shape[0] > 1 else 0,
              K * N if b.shape[0] > 1 else 0, M * N, stream())
    return c


# --------------------------------------------------------------------------- MoE
def moe_topk(logits, k, renorm, gate=None, sel=None, cnt=None, lst=None):
    T, E = logits.shape
    dev = logits.device
    gate = torch.empty((T, k), dtype=torch.float32, device=dev) if gate is None else gate
    sel = torch.empty((T, k), dtype=torch.int32, device=dev) if sel is None else sel
    cnt = torch.empty((E,), dtype=torch.int32, device=dev) if cnt is None else cnt
    lst = torch.empty((E, T), dtype=torch.int32, device=dev) if lst is None else lst
    _hip.call("afx_moe_topk", P(logits), T, E, k, int(bool(renorm)), P(gate), P(sel), P(cnt), P(lst), stream())
    return gate, sel, cnt, lst


def moe_gateup(fmt, w, scale, x, k, E, F, cnt, lst, act=None, rows_hint=0):
    T, D = x.shape
    if act is None:
        act = torch.empty((T * k, F), dtype=torch.float16, device=x.device)
    _hip.call("afx_moe_gateup", FMT[fmt], P(w), P(scale), P(x), T, k, E, F, D, P(cnt), P(lst), P(act),
              rows_hint, stream())
    return act


def moe_down(fmt, w, scale, act, T, k, E, F, D, cnt, lst, y=None, rows_hint=0, ws=None):
    """ws: optional fp32 workspace; 32 * T * k * D bytes let long expert rows split K."""
    if y is None:
        y = torch.empty((T * k, D), dtype=torch.float32, device=act.device)
    _hip.call("afx_moe_down", FMT[fmt], P(w), P(scale), P(act), T, k, E, F, D, P(cnt), P(lst), P(y),
              rows_hint, P(ws), _nbytes(ws), stream())
    return y


def moe_route_supported(h, router, k):
    """Whether afx_moe_route takes this batch (one workgroup: T, E <= 16, D <= 4096, aligned rows)."""
    T, D = h.shape
    E = router.shape[0]
    return (1 <= T <= 16 and 1 <= k <= E <= 16 and D % 32 == 0 and 256 <= D <= 4096 and h.stride(0) % 8 == 0
            and h.data_ptr() % 16 == 0 and router.data_ptr() % 16 == 0)


def moe_route_sync(device="cuda"):
    """A zeroed sync buffer for moe_route's one-workgroup-per-token form (one per MoE layer state)."""
    return torch.zeros(_hip.load().afx_moe_route_sync_words(), dtype=torch.int32, device=device)


def moe_route(h, gamma, eps, router, k, renorm, hn, gate, sel, cnt, lst, logits=None, sync=None):
    """RMSNorm + router logits + top-k + bucketing in one launch (afx_moe_route); hn [T, D] out.
    With `sync` (moe_route_sync()) one workgroup per token, else one workgroup for the batch."""
    T, D = h.shape
    E = router.shape[0]
    _dev(sync)
    _hip.call("afx_moe_route", P(h), h.stride(0), P(gamma), float(eps), P(router), T, E, D, k, int(bool(renorm)),
              P(hn), hn.stride(0), P(logits), P(gate), P(sel), P(cnt), P(lst), P(sync), stream())
    return gate, sel, cnt, lst


def moe_down_combine(fmt, w, scale, act, T, k, E, F, D, cnt, lst, y, h, gate, shared=None, out=None, ws=None):
    """moe_down then moe_combine in one call, the K-split's finishing sum folded into the combine."""
    if out is None:
        out = torch.empty_like(h)
    _hip.call("afx_moe_down_combine", FMT[fmt], P(w), P(scale), P(act), T, k, E, F, D, P(cnt), P(lst), P(y),
              P(ws), _nbytes(ws), P(h), P(gate), P(shared), P(out), stream())
    return out


def moe_combine(h, y, gate, shared=None, out=None):
    T, D = h.shape
    k = gate.shape[1]
    if out is None:
        out = torch.empty_like(h)
    _hip.call("afx_moe_combine", P(h), P(y), P(gate), P(shared), P(out), T, k, D, stream())
    return out


# ----------------------------------------------------------------------------- batched prefill
GEMM_EPI = {"f16": 0, "resid": 1, "f32": 2, "swiglu": 3, "geglu": 5}


def gemm(fmt, w, scale, x, y=None, bias=None, residual=None, epi="f16"):
    """MFMA GEMM for many rows: y = epi(x @ W^T); epi "swiglu" / "geglu" writes [M, N/2]."""
    _dev(w, x)
    M, Kd = x.shape
    N = w.shape[0]
    if y is None:
        cols = N // 2 if epi in ("swiglu", "geglu") else N
        y = torch.empty((M, cols), dtype=torch.float32 if epi == "f32" else torch.float16, device=x.device)
    if epi == "resid" and residual is None:
        residual = y
    _hip.call("afx_gemm", FMT[fmt], P(w), P(scale), P(x), x.stride(0), P(y), y.stride(0), M, N, Kd, P(bias),
              P(residual), GEMM_EPI[epi], stream())
    return y


def qkv_split_rope(qkv, nq, nk, dh, cos_t, sin_t, pos0, q, kcache, vcache, rope=True):
    """Prompt projection rows -> RoPE'd q and cache rows at positions pos0 .. pos0 + M - 1."""
    M = qkv.shape[0]
    _hip.call("afx_qkv_split_rope", P(qkv), qkv.stride(0), M, nq, nk, dh, P(cos_t), P(sin_t), int(pos0), int(rope),
              P(q), q.stride(0), P(kcache), P(vcache), kcache.stride(-3), kcache.shape[-2], stream())


def prefill_attn(q, kcache, vcache, o, pos0, Hq, Hkv, scale=None):
    """Causal GQA attention of q [M, Hq*D] (query m at pos0 + m) over cache rows [0, pos0 + m]."""
    M = q.shape[0]
    D = kcache.shape[-1]
    scale = 1.0 / float(np.sqrt(D)) if scale is None else float(scale)
    _hip.call("afx_prefill_attn", P(q), q.stride(0), P(kcache), P(vcache), kcache.stride(-3), kcache.shape[-2],
              P(o), o.stride(0), M, int(pos0), Hq, Hkv, D, scale, stream())
    return o
