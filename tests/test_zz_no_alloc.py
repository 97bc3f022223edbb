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


@pytest.mark.parametrize("cases", [[(2, 2048, 2048), (1, 300, 512)], [(16, 512, 512), (3, 77, 100)]])
def test_noalloc_matches_workspace_entry_point(cases):
    from aneforge_amd import _kernels as K
    Hq, Hkv, D = 32, 8, 128
    for i, (B, ctx, Mmax) in enumerate(cases):
        say(f"decode attention noalloc call {i}: B={B} ctx={ctx} Mmax={Mmax}")
        rng = np.random.default_rng(700 + i)
        q = rng.standard_normal((B, Hq, D)).astype(np.float16)
        kc = rng.standard_normal((B, Hkv, Mmax, D)).astype(np.float16)
        vc = rng.standard_normal((B, Hkv, Mmax, D)).astype(np.float16)
        qd, kd, vd = dev(q), dev(kc), dev(vc)
        ws = torch.empty(K.attn_ws_bytes(B, Hq, Hkv, D, Mmax) // 4 + 1, dtype=torch.float32, device="cuda")
        want_ws = host(_call("afx_decode_attn", qd, kd, vd, torch.empty_like(qd), B, Hq, Hkv, D, ctx, ws=ws))
        got = host(_call("afx_decode_attn_noalloc", qd, kd, vd, torch.full_like(qd, 7.0), B, Hq, Hkv, D, ctx))
        assert np.array_equal(got.view(np.uint16), want_ws.view(np.uint16)), f"call {i}: outputs differ"
        want = ref.attention(q[:, :, None, :], kc[:, :, :ctx], vc[:, :, :ctx])[:, :, 0]
        check_f16(got, want, what=f"noalloc call {i} vs oracle")
