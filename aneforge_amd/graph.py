"""Lazy Tensor graph: the subset of the reference's front end (aneforge/graph.py:29-440,
:993-1040) that its decode and MoE graphs use.  Building a graph touches no device; `compile`
(aneforge_amd._compile) lowers it to a sequence of HIP kernel launches.

Ops: input / _const, elementwise arithmetic with numpy broadcasting, unary activations,
comparisons and select, weight matmuls (`linear`, `@` with an array, `bmm_weight`; these are
the quantizable weights of `compress=`), activation matmuls (`@` with a Tensor), reshape /
transpose / squeeze / expand_dims / slice_by_size / concat, last-axis-friendly reductions,
softmax, rms_norm, and sdpa."""
from __future__ import annotations

from typing import Any, Sequence

import numpy as np


def _check_dtype(a: np.ndarray, where: str) -> None:
    if a.dtype not in (np.float16, np.float32, np.float64):
        raise TypeError(f"aneforge: {where} has dtype {a.dtype}; weights must be floating point")


def _broadcast(sa: tuple, sb: tuple) -> tuple:
    out = []
    for x, y in zip(reversed(sa), reversed(sb)):
        if not (x == y or x == 1 or y == 1):
            raise ValueError(f"shapes {sa} and {sb} are not broadcastable")
        out.append(max(x, y))
    longer = sa if len(sa) >= len(sb) else sb
    out += list(reversed(longer[: abs(len(sa) - len(sb))]))
    return tuple(reversed(out))


class Tensor:
    """A node in the compute graph (shape, op, sources, attributes)."""

    __slots__ = ("shape", "op", "srcs", "attrs", "_name")

    def __init__(self, shape: Sequence[int], op: str, srcs: Sequence["Tensor"] = (), attrs: dict | None = None):
        self.shape = tuple(int(d) for d in shape)
        if len(self.shape) > 5:
            raise ValueError(f"tensor rank {len(self.shape)} exceeds 5 (op={op!r}, shape={self.shape})")
        self.op = op
        self.srcs = list(srcs)
        self.attrs = attrs or {}
        self._name = ""

    def __repr__(self):
        return f"Tensor({self.op}, {self.shape})"

    # -- unary --
    def relu(self): return Tensor(self.shape, "relu", [self])
    def silu(self): return Tensor(self.shape, "silu", [self])
    def sigmoid(self): return Tensor(self.shape, "sigmoid", [self])
    def tanh(self): return Tensor(self.shape, "tanh", [self])
    def exp(self): return Tensor(self.shape, "exp", [self])
    def sqrt(self): return Tensor(self.shape, "sqrt", [self])
    def abs(self): return Tensor(self.shape, "abs", [self])
    def square(self): return Tensor(self.shape, "square", [self])
    def gelu(self): return Tensor(self.shape, "gelu_tanh", [self])
    def log(self, eps: float = 0.0): return Tensor(self.shape, "log", [self], {"eps": eps})
    def rsqrt(self, eps: float = 0.0): return Tensor(self.shape, "rsqrt", [self], {"eps": eps})
    def inverse(self, eps: float = 0.0): return Tensor(self.shape, "inverse", [self], {"eps": eps})

    def clip(self, lo: float, hi: float):
        return Tensor(self.shape, "clip", [self], {"lo": float(lo), "hi": float(hi)})

    clamp = clip

    # -- binary --
    def __add__(self, o): return _binary(self, o, "add")
    def __sub__(self, o): return _binary(self, o, "sub")
    def __truediv__(self, o): return _binary(self, o, "real_div")
    def __pow__(self, o): return _binary(self, o, "pow")
    pow = __pow__

    def __mul__(self, o):
        if isinstance(o, (int, float)):
            return Tensor(self.shape, "muls", [self], {"k": float(o)})
        return _binary(self, o, "mul")
    __rmul__ = __mul__

    def adds(self, k: float):
        return Tensor(self.shape, "adds", [self], {"k": float(k)})

    def _cmp(self, o, op):
        if not isinstance(o, Tensor):
            raise TypeError(f"{op} expects a graph Tensor")
        return Tensor(_broadcast(self.shape, o.shape), op, [self, o])

    def greater(self, o): return self._cmp(o, "greater")
    def greater_equal(self, o): return self._cmp(o, "greater_equal")
    def less(self, o): return self._cmp(o, "less")
    def less_equal(self, o): return self._cmp(o, "less_equal")
    def equal(self, o): return self._cmp(o, "equal")
    def not_equal(self, o): return self._cmp(o, "not_equal")

    # -- linear algebra --
    def __matmul__(self, W):
        """`x @ W`: W a weight array [K, N] (stored transposed as [N, K], aneforge/graph.py:166-177)
        or a Tensor for an activation x activation product."""
        if isinstance(W, Tensor):
            if self.shape[-1] != W.shape[-2]:
                raise ValueError(f"matmul: {self.shape} @ {W.shape} shape mismatch")
            return Tensor(self.shape[:-1] + (W.shape[-1],), "bmm", [self, W])
        W = np.asarray(W)
        _check_dtype(W, "matmul weight")
        if W.ndim != 2 or self.shape[-1] != W.shape[0]:
            raise ValueError(f"matmul: x{self.shape} @ W{W.shape} shape mismatch")
        return Tensor(self.shape[:-1] + (W.shape[1],), "matmul", [self], {"wt": np.ascontiguousarray(W.T)})

    def bmm_weight(self, W):
        """self [B, M, K] @ W [B, K, N] with a baked quantizable W (aneforge/graph.py:179-185)."""
        W = np.asarray(W)
        _check_dtype(W, "bmm_weight")
        if W.ndim != 3 or self.shape[-1] != W.shape[-2]:
            raise ValueError(f"bmm_weight: x{self.shape} @ W{W.shape} shape mismatch")
        return Tensor(self.shape[:-1] + (W.shape[-1],), "bmm_w", [self], {"wt": np.ascontiguousarray(W)})

    def linear(self, W, bias=None):
        """x @ W.T (+ bias) with W [out, in] (aneforge/graph.py:187-195).  W may also be an
        already-encoded aneforge_amd QuantizedWeight."""
        from ._engine import QuantizedWeight
        if isinstance(W, QuantizedWeight):
            if self.shape[-1] != W.shape[1]:
                raise ValueError(f"linear: x{self.shape} W{W.shape} shape mismatch")
            attrs: dict[str, Any] = {"wt": W}
            out = W.shape[0]
        else:
            W = np.asarray(W)
            _check_dtype(W, "linear weight")
            if W.ndim != 2 or self.shape[-1] != W.shape[1]:
                raise ValueError(f"linear: x{self.shape} W{W.shape} shape mismatch")
            attrs = {"wt": np.ascontiguousarray(W)}
            out = W.shape[0]
        if bias is not None:
            attrs["bias"] = np.asarray(bias).astype(np.float32)
        return Tensor(self.shape[:-1] + (out,), "matmul", [self], attrs)

    # -- layout --
    def transpose(self, perm):
        perm = tuple(p % len(self.shape) for p in perm)
        return Tensor(tuple(self.shape[p] for p in perm), "transpose", [self], {"perm": perm})

    def reshape(self, *shape):
        if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
            shape = tuple(shape[0])
        if int(np.prod(shape)) != int(np.prod(self.shape)):
            raise ValueError(f"reshape: {self.shape} -> {shape} changes the element count")
        return Tensor(tuple(shape), "reshape", [self])

    def squeeze(self, axes):
        axes = tuple(a % len(self.shape) for a in (axes if isinstance(axes, (tuple, list)) else (axes,)))
        for a in axes:
            if self.shape[a] != 1:
                raise ValueError(f"squeeze: axis {a} has size {self.shape[a]} != 1")
        return Tensor(tuple(d for i, d in enumerate(self.shape) if i not in axes), "reshape", [self])

    def expand_dims(self, axes):
        axes = axes if isinstance(axes, (tuple, list)) else (axes,)
        rank = len(self.shape) + len(axes)
        axes = sorted(a % rank for a in axes)
        src = iter(self.shape)
        return Tensor(tuple(1 if i in axes else next(src) for i in range(rank)), "reshape", [self])

    def slice_by_size(self, begin, size):
        begin = [int(b) for b in begin]
        size = [int(s) for s in size]
        if len(begin) != len(self.shape) or len(size) != len(self.shape):
            raise ValueError(f"slice_by_size: begin/size must have rank {len(self.shape)}")
        for i, (b, s) in enumerate(zip(begin, size)):
            if b < 0 or s <= 0 or b + s > self.shape[i]:
                raise ValueError(f"slice_by_size: axis {i} window [{b}:{b + s}] out of range for {self.shape[i]}")
        return Tensor(tuple(size), "slice_by_size", [self], {"begin": begin, "size": size})

    # -- reductions / normalisation --
    def _reduce(self, op, axes):
        axes = tuple(a % len(self.shape) for a in (axes if isinstance(axes, (tuple, list)) else (axes,)))
        return Tensor(tuple(1 if i in axes else d for i, d in enumerate(self.shape)), op, [self], {"axes": axes})

    def mean(self, axes): return self._reduce("reduce_mean", axes)
    def sum(self, axes): return self._reduce("reduce_sum", axes)
    def amax(self, axes): return self._reduce("reduce_max", axes)
    def amin(self, axes): return self._reduce("reduce_min", axes)
    def sum_square(self, axes): return self._reduce("reduce_sum_square", axes)

    def softmax(self, axis: int = -1):
        return Tensor(self.shape, "softmax", [self], {"axis": axis % len(self.shape)})

    def rms_norm(self, gamma, eps: float = 1e-5):
        """RMSNorm over the last dim (aneforge/graph.py:293-301); gamma [D] baked, or a [1, D] Tensor."""
        if isinstance(gamma, Tensor):
            return self.rms_norm(np.ones(self.shape[-1], np.float32), eps) * gamma
        gamma = np.asarray(gamma)
        _check_dtype(gamma, "rms_norm gamma")
        if gamma.shape != (self.shape[-1],):
            raise ValueError(f"rms_norm expects gamma [{self.shape[-1]}], got {gamma.shape}")
        return Tensor(self.shape, "rms_norm", [self], {"gamma": gamma.astype(np.float32), "eps": float(eps)})


_input_counter = [0]


def input(shape: Sequence[int], dtype: str = "fp16", max_abs: float | None = None) -> Tensor:
    """A graph input placeholder, fed to the compiled Model in creation order."""
    if dtype != "fp16":
        raise ValueError("aneforge_amd inputs are fp16")
    t = Tensor(tuple(shape), "input")
    t.attrs["idx"] = _input_counter[0]
    if max_abs is not None:
        t.attrs["max_abs"] = float(max_abs)
    _input_counter[0] += 1
    return t


def _const(v) -> Tensor:
    v = np.asarray(v, np.float16)
    return Tensor(v.shape, "const_array", [], {"value": v})


def _binary(a: Tensor, b, kind: str) -> Tensor:
    if not isinstance(b, Tensor):
        b = _const(b)
    return Tensor(_broadcast(a.shape, b.shape), kind, [a, b])


def maximum(a: Tensor, b) -> Tensor:
    return _binary(a, b, "maximum")


def minimum(a: Tensor, b) -> Tensor:
    return _binary(a, b, "minimum")


def concat(ts: Sequence[Tensor], axis: int) -> Tensor:
    ts = list(ts)
    ax = axis % len(ts[0].shape)
    for t in ts:
        if len(t.shape) != len(ts[0].shape) or any(t.shape[i] != ts[0].shape[i] for i in range(len(t.shape)) if i != ax):
            raise ValueError("concat: shapes differ off the concat axis")
    shape = list(ts[0].shape)
    shape[ax] = sum(t.shape[ax] for t in ts)
    return Tensor(tuple(shape), "concat", ts, {"axis": ax})


def select(cond: Tensor, a, b) -> Tensor:
    """Elementwise cond ? a : b (broadcasting)."""
    a = a if isinstance(a, Tensor) else _const(a)
    b = b if isinstance(b, Tensor) else _const(b)
    return Tensor(_broadcast(_broadcast(cond.shape, a.shape), b.shape), "select", [cond, a, b])


def sdpa(q: Tensor, k: Tensor, v: Tensor, scale: float | None = None, is_causal: bool = False,
         attn_mask: Tensor | None = None) -> Tensor:
    """softmax(q k^T * scale (+ mask)) v for q [1, H, Sq, D], k/v [1, Hkv, Skv, D]
    (aneforge/graph.py:993-1040).  Validation follows the reference; grouped-query k/v
    (H a multiple of Hkv) is accepted in addition.  The device kernel is split-KV decode
    attention for every regime, so there is no native/decomposed switch."""
    if not (len(q.shape) == 4 == len(k.shape) == len(v.shape)):
        raise ValueError(f"af.sdpa expects 4D q,k,v of [1,H,S,D]; got {q.shape}, {k.shape}, {v.shape}")
    if k.shape != v.shape:
        raise ValueError(f"af.sdpa: k,v must share shape; got {k.shape}, {v.shape}")
    if q.shape[3] != k.shape[3] or q.shape[1] % k.shape[1]:
        raise ValueError(f"af.sdpa: q,k must share D and H must be a multiple of the kv heads; got {q.shape}, {k.shape}")
    if q.shape[0] != 1 or k.shape[0] != 1:
        raise ValueError(f"af.sdpa: batch must be 1; got {q.shape[0]}/{k.shape[0]}")
    if is_causal and q.shape[2] != k.shape[2]:
        raise ValueError("af.sdpa: is_causal requires equal q/k seq; pass an attn_mask for decode")
    if attn_mask is not None:
        if is_causal:
            raise ValueError("af.sdpa: pass either is_causal or an explicit attn_mask, not both")
        if tuple(attn_mask.shape) != (1, 1, q.shape[2], k.shape[2]):
            raise ValueError(f"af.sdpa: attn_mask must be [1,1,Sq,Skv]={[1, 1, q.shape[2], k.shape[2]]}; "
                             f"got {list(attn_mask.shape)}")
    sc = scale if scale is not None else 1.0 / q.shape[-1] ** 0.5
    srcs = [q, k, v] + ([attn_mask] if attn_mask is not None else [])
    return Tensor(q.shape, "sdpa", srcs, {"scale": float(sc), "causal": bool(is_causal),
                                          "masked": attn_mask is not None})
