"""Parity of the batched-prefill kernels (MFMA GEMM, q/cache split with RoPE, causal GQA flash
attention) against the oracle, at sizes the oracle finishes in seconds."""
from __future__ import annotations

import numpy as np
import pytest

from _util import check_f16, check_hidden, dev, host, say
from oracle import ref

pytestmark = pytest.mark.gpu


def _weights(fmt, N, K, rng):
    import torch
    if fmt == "int8":
        q = rng.integers(-127, 128, (N, K), dtype=np.int8)
        s = (np.abs(rng.normal(0, 0.02, N)) / 127).astype(np.float16)
        return dev(q), dev(s), ref.dequant_w8(q, s)
    if fmt == "blockwise":
        q = rng.integers(-127, 128, (N, K), dtype=np.int8)
        s = (np.abs(rng.normal(0, 0.02, (N, K // 32))) / 127 + 1e-5).astype(np.float16)
        return dev(q), dev(s), ref.dequant_blockwise(q, s)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float16)
    return dev(w), None, w.astype(np.float32)


@pytest.mark.parametrize("fmt", ["int8", "fp16", "blockwise"])
@pytest.mark.parametrize("M,N,K", [(1, 256, 128), (70, 384, 320), (300, 256, 640)])
@pytest.mark.parametrize("epi", ["f16", "resid", "f32", "swiglu"])
def test_gemm_matches_oracle(fmt, M, N, K, epi):
    import torch
    from aneforge_amd import _kernels as Kn
    rng = np.random.default_rng(M * 1000 + N + K)
    w, s, Wf = _weights(fmt, N, K, rng)
    x = rng.standard_normal((M, K)).astype(np.float16)
    bias = (rng.standard_normal(N) * 0.1).astype(np.float16) if epi in ("f16", "f32") else None
    say(f"gemm {fmt} M={M} N={N} K={K} epi={epi}")
    want_lin = np.asarray(x, np.float64) @ np.asarray(Wf, np.float64).T
    if bias is not None:
        want_lin = want_lin + bias.astype(np.float64)
    if epi == "resid":
        r = rng.standard_normal((M, N)).astype(np.float16)
        y = dev(r)
        Kn.gemm(fmt, w, s, dev(x), y=y, residual=y, epi="resid")
        want = ref.r16(r.astype(np.float64) + ref.r16(want_lin))
        check_hidden(host(y), want, what=f"gemm {fmt} resid")
        return
    got = Kn.gemm(fmt, w, s, dev(x), bias=None if bias is None else dev(bias), epi=epi)
    if epi == "swiglu":
        g, u = ref.r16(want_lin[:, 0::2]), ref.r16(want_lin[:, 1::2])
        check_f16(host(got), ref.r16(ref.silu(g) * u), what=f"gemm {fmt} swiglu")
    elif epi == "f32":
        check_f16(host(got), want_lin, what=f"gemm {fmt} f32")
    else:
        check_f16(host(got), ref.r16(want_lin), what=f"gemm {fmt} f16")


def test_gemm_rejects_bad_shapes():
    import torch
    from aneforge_amd import _kernels as Kn
    w = torch.zeros((256, 100), dtype=torch.float16, device="cuda")
    x = torch.zeros((4, 100), dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="K % 64"):
        Kn.gemm("fp16", w, None, x)


@pytest.mark.parametrize("M,pos0,H,KV,dh", [(1, 0, 2, 1, 64), (5, 3, 2, 1, 64), (40, 17, 2, 1, 64),
                                            (33, 20, 4, 2, 128), (7, 0, 3, 1, 8)])
def test_qkv_split_rope_matches_oracle(M, pos0, H, KV, dh):
    """The split against the oracle; 8 packed rows per thread (default) and one pair per thread
    (AFX_QKV_SPLIT_VEC=0) write the same bits."""
    import torch
    from aneforge_amd import _blob
    from aneforge_amd import _kernels as Kn
    Mmax = 64
    rng = np.random.default_rng(M + 31 * pos0)
    nq, nk = H * dh, KV * dh
    nat = rng.standard_normal((M, nq + 2 * nk)).astype(np.float16)     # natural [q | k | v]
    pq, pk = _blob.rope_pair_order(H, dh), _blob.rope_pair_order(KV, dh)
    packed = np.concatenate([nat[:, :nq][:, pq], nat[:, nq:nq + nk][:, pk], nat[:, nq + nk:]], 1)
    cos, sin = ref.rope_tables(Mmax, dh)
    outs = []
    old = _env("AFX_QKV_SPLIT_VEC", None)
    try:
        for vec in (None, 0):
            _env("AFX_QKV_SPLIT_VEC", vec)
            q = torch.zeros((M, nq), dtype=torch.float16, device="cuda")
            kc = torch.zeros((KV, Mmax, dh), dtype=torch.float16, device="cuda")
            vc = torch.zeros((KV, Mmax, dh), dtype=torch.float16, device="cuda")
            say(f"qkv_split_rope M={M} pos0={pos0} H={H} KV={KV} dh={dh} vec={vec}")
            Kn.qkv_split_rope(dev(packed), nq, nk, dh, dev(cos), dev(sin), pos0, q, kc, vc)
            outs.append((host(q), host(kc), host(vc)))
    finally:
        _env("AFX_QKV_SPLIT_VEC", old)
    for a, b in zip(outs[0], outs[1]):
        np.testing.assert_array_equal(a, b)
    p = np.arange(pos0, pos0 + M)
    want_q = ref.rope(nat[:, :nq].reshape(M, H, dh), cos[p][:, None], sin[p][:, None]).reshape(M, nq)
    want_k = ref.rope(nat[:, nq:nq + nk].reshape(M, KV, dh), cos[p][:, None], sin[p][:, None])
    got_q, got_k, got_v = outs[0]
    check_f16(got_q, want_q, what="q")
    check_f16(got_k[:, pos0:pos0 + M].transpose(1, 0, 2), want_k, what="k rows")
    np.testing.assert_array_equal(got_v[:, pos0:pos0 + M].transpose(1, 0, 2),
                                  nat[:, nq + nk:].reshape(M, KV, dh))
    assert not got_k[:, :pos0].any() and not got_k[:, pos0 + M:].any()     # other rows untouched


@pytest.mark.parametrize("M,pos0,Hq,Hkv", [(1, 0, 4, 2), (70, 37, 4, 2), (130, 0, 8, 2), (64, 190, 2, 2)])
def test_prefill_attention_matches_oracle(M, pos0, Hq, Hkv):
    import torch
    from aneforge_amd import _kernels as Kn
    D, Mmax = 128, 256
    rng = np.random.default_rng(M + pos0 + Hq)
    L = pos0 + M
    Kc = np.zeros((Hkv, Mmax, D), np.float16)
    Vc = np.zeros((Hkv, Mmax, D), np.float16)
    Kc[:, :L] = rng.standard_normal((Hkv, L, D)).astype(np.float16)
    Vc[:, :L] = rng.standard_normal((Hkv, L, D)).astype(np.float16)
    q = rng.standard_normal((M, Hq * D)).astype(np.float16)
    o = torch.zeros((M, Hq * D), dtype=torch.float16, device="cuda")
    say(f"prefill_attn M={M} pos0={pos0} Hq={Hq} Hkv={Hkv}")
    Kn.prefill_attn(dev(q), dev(Kc), dev(Vc), o, pos0, Hq, Hkv)
    mask = np.where(np.arange(L)[None, :] <= pos0 + np.arange(M)[:, None], 0.0, -np.inf)
    want = ref.attention(q.reshape(M, Hq, D).transpose(1, 0, 2)[None], Kc[None, :, :L], Vc[None, :, :L], mask=mask)
    check_f16(host(o), want[0].transpose(1, 0, 2).reshape(M, Hq * D), what="prefill attention")


def _env(name, value):
    """Set (or clear, value None) one of the kernel-form environment switches; returns the old value."""
    import os
    old = os.environ.get(name)
    if value is None:
        os.environ.pop(name, None)
    else:
        os.environ[name] = str(value)
    return old


@pytest.mark.parametrize("M,pos0,Hq,Hkv,Mmax", [(300, 0, 16, 8, 320), (257, 40, 8, 8, 300), (130, 0, 8, 2, 256),
                                                (1, 5, 4, 2, 64), (640, 100, 16, 8, 800)])
def test_prefill_attention_forms(M, pos0, Hq, Hkv, Mmax):
    """Every prefill-attention form against the oracle: single-buffered (1), pipelined (2, the same
    arithmetic: bit-identical to 1), transposed scores (3) with both tile orders and both V stagings, and 3
    with each tile's keys split over two halves of the workgroup (4: a single-block tile whose first
    half is empty, and queries that see no key of the second half), on grids with several workgroup
    rounds, the XCD mapping (Hkv = 8) and without it (Hkv = 2); 5 is form 4 with the second half one
    phase behind (bit-identical to 4)."""
    import torch
    from aneforge_amd import _kernels as Kn
    D = 128
    rng = np.random.default_rng(M * 7 + pos0 + Hq + Hkv)
    L = pos0 + M
    Kc = np.zeros((Hkv, Mmax, D), np.float16)
    Vc = np.zeros((Hkv, Mmax, D), np.float16)
    Kc[:, :L] = rng.standard_normal((Hkv, L, D)).astype(np.float16)
    Vc[:, :L] = rng.standard_normal((Hkv, L, D)).astype(np.float16)
    q = rng.standard_normal((M, Hq * D)).astype(np.float16)
    mask = np.where(np.arange(L)[None, :] <= pos0 + np.arange(M)[:, None], 0.0, -np.inf)
    want = ref.attention(q.reshape(M, Hq, D).transpose(1, 0, 2)[None], Kc[None, :, :L], Vc[None, :, :L], mask=mask)
    want = want[0].transpose(1, 0, 2).reshape(M, Hq * D)
    outs = {}
    old_f, old_o = _env("AFX_PREFILL_ATTN_FORM", None), _env("AFX_PREFILL_ATTN_ORDER", None)
    old_v = _env("AFX_PREFILL_ATTN_VTR", None)
    try:
        for form, order, vtr in ((1, None, None), (2, None, None), (3, 0, None), (3, 1, None), (3, 1, 0),
                                 (4, None, None), (4, None, 0), (5, None, None), (5, None, 0)):
            _env("AFX_PREFILL_ATTN_FORM", form)
            _env("AFX_PREFILL_ATTN_ORDER", order)
            _env("AFX_PREFILL_ATTN_VTR", vtr)
            say(f"prefill_attn form={form} order={order} vtr={vtr} M={M} pos0={pos0} Hq={Hq} Hkv={Hkv}")
            o = torch.zeros((M, Hq * D), dtype=torch.float16, device="cuda")
            Kn.prefill_attn(dev(q), dev(Kc), dev(Vc), o, pos0, Hq, Hkv)
            outs[(form, order, vtr)] = host(o)
            check_f16(outs[(form, order, vtr)], want, what=f"prefill attention form {form} order {order} vtr {vtr}")
    finally:
        _env("AFX_PREFILL_ATTN_FORM", old_f)
        _env("AFX_PREFILL_ATTN_ORDER", old_o)
        _env("AFX_PREFILL_ATTN_VTR", old_v)
    np.testing.assert_array_equal(outs[(1, None, None)], outs[(2, None, None)])
    np.testing.assert_array_equal(outs[(3, 0, None)], outs[(3, 1, None)])
    # the V operand's staging layout (row-major + transposing reads, or V^T) changes no arithmetic
    np.testing.assert_array_equal(outs[(3, 1, None)], outs[(3, 1, 0)])
    np.testing.assert_array_equal(outs[(4, None, None)], outs[(4, None, 0)])
    # form 5 reorders form 4's phases across the two halves, not its arithmetic
    np.testing.assert_array_equal(outs[(5, None, None)], outs[(4, None, None)])
    np.testing.assert_array_equal(outs[(5, None, 0)], outs[(4, None, None)])


@pytest.mark.parametrize("fmt", ["int8", "fp16", "blockwise"])
@pytest.mark.parametrize("M,N,K", [(300, 2304, 256), (1000, 1280, 512), (2048, 4096, 128)])
def test_gemm_tile_orders_bit_identical(fmt, M, N, K):
    """The grouped tile order (default), other group sizes and the contiguous order (AFX_GEMM_GN=0),
    and every kernel form (AFX_GEMM_WL: 0 the 2 x 2 layout, 2 the 1 x 4 layout, 3 the 1 x 4 layout
    with the second half-step's fragments read during the first's products, 4 form 3's loop over
    eight wavefronts in 2 x 4, 6 form 4 with the barrier in the middle of the K step)
    compute every output tile the same way: bit-identical, and to the oracle's bar."""
    import torch
    from aneforge_amd import _kernels as Kn
    rng = np.random.default_rng(M + N + K)
    w, s, Wf = _weights(fmt, N, K, rng)
    x = rng.standard_normal((M, K)).astype(np.float16)
    want = ref.r16(np.asarray(x, np.float64) @ np.asarray(Wf, np.float64).T)
    outs = []
    old, old_wl = _env("AFX_GEMM_GN", None), _env("AFX_GEMM_WL", None)
    try:
        for gn, wl in ((None, None), (0, None), (3, None), (16, None), (None, 0), (None, 2), (None, 3), (None, 4),
                       (None, 6)):
            _env("AFX_GEMM_GN", gn)
            _env("AFX_GEMM_WL", wl)
            say(f"gemm tile order GN={gn} WL={wl} {fmt} M={M} N={N} K={K}")
            outs.append(host(Kn.gemm(fmt, w, s, dev(x), epi="f16")))
    finally:
        _env("AFX_GEMM_GN", old)
        _env("AFX_GEMM_WL", old_wl)
    check_f16(outs[0], want, what=f"gemm {fmt} grouped order")
    for o in outs[1:]:
        np.testing.assert_array_equal(o, outs[0])


@pytest.mark.parametrize("fmt", ["int8", "fp16"])
@pytest.mark.parametrize("M,N,K", [(2048, 6144, 64), (600, 4096, 128), (333, 400, 192)])
@pytest.mark.parametrize("epi", ["resid", "swiglu", "f32"])
def test_gemm_epilogues_every_form(fmt, M, N, K, epi):
    """Each epilogue under every kernel form, at a grid whose default is form 3 (768 int8 tiles: three
    workgroups per CU), one whose default is form 6 (160 tiles), and ragged rows and columns (333 x 400:
    partial tiles in both directions): bit-identical across the forms, and the default to the oracle's
    bar."""
    import torch
    from aneforge_amd import _kernels as Kn
    rng = np.random.default_rng(M + N + K + len(epi))
    w, s, Wf = _weights(fmt, N, K, rng)
    x = rng.standard_normal((M, K)).astype(np.float16)
    lin = np.asarray(x, np.float64) @ np.asarray(Wf, np.float64).T
    r = rng.standard_normal((M, N)).astype(np.float16) if epi == "resid" else None
    outs = []
    old = _env("AFX_GEMM_WL", None)
    try:
        for wl in (None, 0, 2, 3, 4, 6):
            _env("AFX_GEMM_WL", wl)
            say(f"gemm epilogue {epi} WL={wl} {fmt} M={M} N={N} K={K}")
            if epi == "resid":
                y = dev(r)
                Kn.gemm(fmt, w, s, dev(x), y=y, residual=y, epi="resid")
                outs.append(host(y))
            else:
                outs.append(host(Kn.gemm(fmt, w, s, dev(x), epi=epi)))
    finally:
        _env("AFX_GEMM_WL", old)
    for o in outs[1:]:
        np.testing.assert_array_equal(o, outs[0])
    if epi == "resid":
        check_hidden(outs[0], ref.r16(r.astype(np.float64) + ref.r16(lin)), what=f"gemm {fmt} resid")
    elif epi == "swiglu":
        g, u = ref.r16(lin[:, 0::2]), ref.r16(lin[:, 1::2])
        check_f16(outs[0], ref.r16(ref.silu(g) * u), what=f"gemm {fmt} swiglu")
    else:
        check_f16(outs[0], lin, what=f"gemm {fmt} f32")
