"""Shared helpers for the parity tests (plain module, not a test file)."""
from __future__ import annotations

import sys

import numpy as np

RTOL, ATOL, MIN_COS = 1e-2, 1e-3, 0.9999     # the fp16 parity bar of the path


def say(msg: str) -> None:
    """Name the case before a GPU step, so a failure log identifies it."""
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def cosine(a, b) -> float:
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-30))


def check_f16(got, want, rtol=RTOL, atol=ATOL, min_cos=MIN_COS, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    bad = ~np.isclose(got, want, rtol=rtol, atol=atol)
    c = cosine(got, want)
    assert not bad.any(), (f"{what}: {int(bad.sum())}/{bad.size} outside rtol={rtol} atol={atol}; "
                           f"max abs err {np.abs(got - want).max():.3e}; cos {c:.6f}")
    assert c >= min_cos, f"{what}: cosine {c:.6f} < {min_cos}"


def check_hidden(got, want, what=""):
    """Residual-stream hidden states are sums of fp16-rounded terms: where h + f(h) cancels, a
    one-ulp difference in an operand (ulp of the operand's magnitude) survives the subtraction.
    The absolute tolerance is therefore one fp16 ulp of the layer's largest |value| (at least
    1e-3), on top of rtol 1e-2 and cosine >= 0.9999."""
    want = np.asarray(want, np.float64)
    ulp = float(np.spacing(np.float16(np.abs(want).max())))
    check_f16(got, want, atol=max(ATOL, ulp), what=what)


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()
