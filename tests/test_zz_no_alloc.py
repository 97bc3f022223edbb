"""afx_decode_attn_noalloc (split partials in the library's own device array, no workspace and no
allocation) against afx_decode_attn with a caller workspace, through the C ABI: identical outputs
on two calls in a row, the second with a smaller input, and both within the fp16 bar of the
oracle's attention (aneforge/_bridges/ane_sdpa_fused.py:57-68)."""
import numpy as np
import pytest
import torch

from _util import check_f16, dev, host, say
from oracle import ref

pytestmark = pytest.mark.gpu


def _call(name, q, k, v, o, B, Hq, Hkv, D, ctx, ws=None):
    from aneforge_amd import _hip, _kernels as K
    P = lambda t: None if t is None else t.data_ptr()
    Mmax = k.shape[2]
    args = [P(q), P(k), P(v), P(o), q.stride(0), q.stride(1), k.stride(0), k.stride(1), B, Hq, Hkv, D, ctx,
            None, Mmax, None, 0, -1, 1.0 / D ** 0.5]
    if ws is not None:
        args += [P(ws), ws.numel() * ws.element_size()]
    _hip.call(name, *args, 0, K.stream())
    return o


def _inputs(B, Hq, Hkv, D, Mmax, seed):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, Hq, D)).astype(np.float16)
    kc = rng.standard_normal((B, Hkv, Mmax, D)).astype(np.float16)
    vc = rng.standard_normal((B, Hkv, Mmax, D)).astype(np.float16)
    return q, kc, vc


def test_noalloc_first_call_inside_a_graph_capture():
    """The process's first noalloc call (which resolves the scratch array's device address) made while
    torch captures a graph: the replays equal the workspace entry point, bit for bit, at a shape whose
    B * Hkv is not a multiple of 8 (the three-dimensional grids)."""
    from aneforge_amd import _kernels as K
    B, Hq, Hkv, D, ctx, Mmax = 3, 16, 2, 128, 700, 768
    say(f"decode attention noalloc: first call under graph capture, B={B} Hq={Hq} Hkv={Hkv} ctx={ctx}")
    q, kc, vc = _inputs(B, Hq, Hkv, D, Mmax, 690)
    qd, kd, vd = dev(q), dev(kc), dev(vc)
    o = torch.empty_like(qd)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _call("afx_decode_attn_noalloc", qd, kd, vd, o, B, Hq, Hkv, D, ctx)
    ws = torch.empty(K.attn_ws_bytes(B, Hq, Hkv, D, Mmax) // 4 + 1, dtype=torch.float32, device="cuda")
    want_ws = host(_call("afx_decode_attn", qd, kd, vd, torch.empty_like(qd), B, Hq, Hkv, D, ctx, ws=ws))
    for r in range(3):                                     # eager work and a sync between the replays
        o.fill_(7.0)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(o).view(np.uint16), want_ws.view(np.uint16)), f"replay {r} differs"
    want = ref.attention(q[:, :, None, :], kc[:, :, :ctx], vc[:, :, :ctx])[:, :, 0]
    check_f16(host(o), want, what="noalloc under capture vs oracle")


@pytest.mark.parametrize("cases", [[(2, 32, 8, 2048, 2048), (1, 32, 8, 300, 512)],
                                   [(16, 32, 8, 512, 512), (3, 32, 8, 77, 100)],
                                   [(3, 16, 2, 1000, 1024), (1, 8, 1, 64, 64)]])
def test_noalloc_matches_workspace_entry_point(cases):
    from aneforge_amd import _kernels as K
    D = 128
    for i, (B, Hq, Hkv, ctx, Mmax) in enumerate(cases):
        say(f"decode attention noalloc call {i}: B={B} Hq={Hq} Hkv={Hkv} ctx={ctx} Mmax={Mmax}")
        q, kc, vc = _inputs(B, Hq, Hkv, D, Mmax, 700 + i)
        qd, kd, vd = dev(q), dev(kc), dev(vc)
        ws = torch.empty(K.attn_ws_bytes(B, Hq, Hkv, D, Mmax) // 4 + 1, dtype=torch.float32, device="cuda")
        want_ws = host(_call("afx_decode_attn", qd, kd, vd, torch.empty_like(qd), B, Hq, Hkv, D, ctx, ws=ws))
        got = host(_call("afx_decode_attn_noalloc", qd, kd, vd, torch.full_like(qd, 7.0), B, Hq, Hkv, D, ctx))
        assert np.array_equal(got.view(np.uint16), want_ws.view(np.uint16)), f"call {i}: outputs differ"
        want = ref.attention(q[:, :, None, :], kc[:, :, :ctx], vc[:, :, :ctx])[:, :, 0]
        check_f16(got, want, what=f"noalloc call {i} vs oracle")
