"""Seeded randomized parity sweep of the skinny MFMA paths against the CPU oracle (oracle/ref.py).

Dense linears of 4..16 rows (plain, bias + residual, fp32 out and SwiGLU epilogues) and MoE gate/up +
down launches (1..39 experts, some never routed, up to 24 tokens) over int8, blockwise, fp16 and Q4_0
weights, at random shapes the kernels accept.  Covers both skinny MFMA kernels (persistent and
tile-per-workgroup) and the vector fallback for short K.  Bar: rtol 1e-2 / atol 1e-3, cosine >= 0.9999;
residual-stream outputs take one fp16 ulp of their largest value as atol; the SwiGLU epilogue is
checked against the device's own linear (it rounds the same fp32 sums to fp16 first)."""
import numpy as np
import pytest

from _util import ATOL, RTOL, cosine, dev, host, say
from oracle import ref

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

KS = {"int8": 64, "fp16": 32, "blockwise": 64, "q4_0": 128}     # k per MFMA step of each format


def _bad(got, want, hidden=False):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    atol = max(ATOL, float(np.abs(want).max()) * 2.0 ** -10) if hidden else ATOL
    n = int((~np.isclose(got, want, rtol=RTOL, atol=atol)).sum())
    return n if n or cosine(got, want) >= 0.9999 else got.size


def _weights(rng, fmt, N, Kd):
    from aneforge_amd import _blob
    if fmt == "int8":
        q = rng.integers(-127, 128, (N, Kd), dtype=np.int8)
        s = (np.abs(rng.normal(0, 0.02, N)) / 127).astype(np.float16)
        return q, s, ref.dequant_w8(q, s)
    if fmt == "fp16":
        w = (rng.standard_normal((N, Kd)) * 0.02).astype(np.float16)
        return w, None, w.astype(np.float32)
    if fmt == "blockwise":
        q = rng.integers(-127, 128, (N, Kd), dtype=np.int8)
        s = (np.abs(rng.normal(0, 0.02, (N, Kd // 32))) / 127 + 1e-5).astype(np.float16)
        return q, s, ref.dequant_blockwise(q, s)
    blocks = ref.quantize_q4_0((rng.standard_normal((N, Kd)) * 0.05).astype(np.float32))
    qs, d = _blob.q4_0_to_superblock(blocks, N, Kd)
    return qs, d, ref.dequant_q4_0_f16(blocks, N, Kd)


@pytest.mark.parametrize("seed", [101, 102])
def test_dense_skinny_sweep(seed):
    from aneforge_amd import _kernels as K
    rng = np.random.default_rng(seed)
    for trial in range(10):
        fmt = list(KS)[trial % 4]
        Kd = int(rng.integers(8, 70)) * KS[fmt]
        N = int(rng.integers(1, 2600)) * 4
        N = min(N, max(4, (20_000_000 // Kd) // 4 * 4))
        M = int(rng.integers(4, 17))
        say(f"sweep {seed}/{trial}: dense {fmt} M={M} N={N} K={Kd}")
        w, s, W = _weights(rng, fmt, N, Kd)
        wd, sd = dev(w), (dev(s) if s is not None else None)
        x = rng.standard_normal((M, Kd)).astype(np.float16)
        b = (rng.standard_normal(N) * 0.1).astype(np.float16)
        r = rng.standard_normal((M, N)).astype(np.float16)
        y = host(K.linear(fmt, wd, sd, dev(x)))
        assert _bad(y, ref.linear(x, W)) == 0, "plain"
        got = host(K.linear(fmt, wd, sd, dev(x), bias=dev(b), residual=dev(r)))
        assert _bad(got, ref.r16(r.astype(np.float64) + ref.linear(x, W, b)), hidden=True) == 0, "bias + residual"
        assert _bad(host(K.linear(fmt, wd, sd, dev(x), out_f32=True)), ref.linear(x, W, exact=True)) == 0, "fp32 out"
        yd = y.astype(np.float32)
        act = host(K.linear_swiglu(fmt, wd, sd, dev(x)))
        assert _bad(act, ref.r16(ref.silu(yd[:, 0::2]) * yd[:, 1::2])) == 0, "swiglu"


@pytest.mark.parametrize("seed", [201, 202])
def test_moe_skinny_sweep(seed):
    from aneforge_amd import _blob, _kernels as K
    rng = np.random.default_rng(seed)
    for trial in range(4):
        fmt = ["int8", "q4_0", "blockwise", "q4_0"][trial]
        E = int(rng.integers(1, 40))
        T = int(rng.integers(1, 25))
        D = int(rng.integers(2, 33)) * 128
        F = int(rng.integers(1, 40)) * 128
        routed = rng.choice(E, int(rng.integers(1, E + 1)), replace=False)
        k = int(rng.integers(1, min(len(routed), 4) + 1))
        pick = [rng.choice(routed, k, replace=False) for _ in range(T)]
        say(f"sweep {seed}/{trial}: moe {fmt} E={E} k={k} T={T} D={D} F={F}")
        cnt = np.zeros(E, np.int32)
        lst = np.zeros((E, T), np.int32)
        for t in range(T):
            for sl, e in enumerate(pick[t]):
                lst[e, cnt[e]] = t * k + sl
                cnt[e] += 1
        used = sorted({int(e) for p in pick for e in p})
        ws, ss, wdn, sdn, G, U, Dn = [], [], [], [], {}, {}, {}
        for e in range(E):
            if e in used:
                qg, sg, G[e] = _weights(rng, fmt, F, D)
                qu, su, U[e] = _weights(rng, fmt, F, D)
                qd, sdd, Dn[e] = _weights(rng, fmt, D, F)
            else:                                      # never routed: zero codes of the right shape
                zg, zs, _ = _weights(rng, fmt, 2, D)
                zd, zds, _ = _weights(rng, fmt, 2, F)
                qg = qu = np.zeros((F,) + zg.shape[1:], zg.dtype)
                sg = su = np.zeros((F,) + zs.shape[1:], zs.dtype)
                qd, sdd = np.zeros((D,) + zd.shape[1:], zd.dtype), np.zeros((D,) + zds.shape[1:], zds.dtype)
            ws.append(_blob.interleave_rows(qg, qu)); ss.append(_blob.interleave_rows(sg, su))
            wdn.append(qd); sdn.append(sdd)
        x = rng.standard_normal((T, D)).astype(np.float16)
        act = K.moe_gateup(fmt, dev(np.stack(ws)), dev(np.stack(ss)), dev(x), k, E, F, dev(cnt), dev(lst))
        y = host(K.moe_down(fmt, dev(np.stack(wdn)), dev(np.stack(sdn)), act, T, k, E, F, D, dev(cnt), dev(lst)))
        a = host(act)
        for t in range(T):
            for sl, e in enumerate(pick[t]):
                ent = t * k + sl
                g, u = ref.linear(x[t:t + 1], G[e]), ref.linear(x[t:t + 1], U[e])
                assert _bad(a[ent:ent + 1], ref.r16(ref.silu(g) * u)) == 0, f"gate/up token {t} expert {e}"
                assert _bad(y[ent:ent + 1], ref.linear(a[ent:ent + 1], Dn[e], exact=True)) == 0, f"down token {t} expert {e}"


@pytest.mark.parametrize("fmt", ["int8", "q4_0", "blockwise"])
def test_dense_split_k(fmt):
    """Long rows (K = 11008, 14336: the cfg1 down projection and longer) with a workspace take the
    K-split persistent kernel (partials in the workspace, a finishing launch for the epilogue);
    without one they take the tile kernel.  Both meet the oracle bar, for every epilogue."""
    from aneforge_amd import _kernels as K
    rng = np.random.default_rng(301)
    for Kd in (11008, 14336):
        N = 1044                       # a partial last tile of 16 rows
        w, s, W = _weights(rng, fmt, N, Kd)
        wd, sd = dev(w), dev(s)
        for M in (4, 8, 13, 16):
            say(f"split-K: dense {fmt} M={M} N={N} K={Kd}")
            x = rng.standard_normal((M, Kd)).astype(np.float16)
            b = (rng.standard_normal(N) * 0.1).astype(np.float16)
            r = rng.standard_normal((M, N)).astype(np.float16)
            ws = torch.full((8 * M * N,), float("nan"), dtype=torch.float32, device="cuda")   # stale contents
            want = ref.linear(x, W)
            assert _bad(host(K.linear(fmt, wd, sd, dev(x), ws=ws)), want) == 0, "plain, split"
            assert _bad(host(K.linear(fmt, wd, sd, dev(x))), want) == 0, "plain, no workspace"
            got = host(K.linear(fmt, wd, sd, dev(x), bias=dev(b), residual=dev(r), ws=ws))
            assert _bad(got, ref.r16(r.astype(np.float64) + ref.linear(x, W, b)), hidden=True) == 0, "bias + residual"
            got = host(K.linear(fmt, wd, sd, dev(x), out_f32=True, ws=ws))
            assert _bad(got, ref.linear(x, W, exact=True)) == 0, "fp32 out"
            small = torch.empty(2 * M * N - 1, dtype=torch.float32, device="cuda")   # too small to split
            assert _bad(host(K.linear(fmt, wd, sd, dev(x), ws=small)), want) == 0, "workspace too small"


@pytest.mark.parametrize("fmt", ["int8", "q4_0"])
def test_moe_down_split_k(fmt):
    """The expert down projection over long expert rows (F = 14336, the cfg4 experts) with a
    workspace: K-split units (expert, slice, tile); experts left unrouted; T up to 16 tokens."""
    from aneforge_amd import _kernels as K
    rng = np.random.default_rng(302)
    E, F, D = 6, 14336, 512
    wdn, sdn, Dn = [], [], []
    for e in range(E):
        q, s_, W = _weights(rng, fmt, D, F)
        wdn.append(q); sdn.append(s_); Dn.append(W)
    wd, sd = dev(np.stack(wdn)), dev(np.stack(sdn))
    for T, k in ((1, 2), (4, 2), (16, 2), (9, 3)):
        say(f"split-K: moe down {fmt} E={E} k={k} T={T} D={D} F={F}")
        pick = [rng.choice(E - 1, k, replace=False) for _ in range(T)]     # expert E-1 never routed
        cnt = np.zeros(E, np.int32)
        lst = np.zeros((E, T), np.int32)
        for t in range(T):
            for sl, e in enumerate(pick[t]):
                lst[e, cnt[e]] = t * k + sl
                cnt[e] += 1
        a = (rng.standard_normal((T * k, F)) * 0.5).astype(np.float16)
        ws = torch.full((8 * T * k * D,), float("nan"), dtype=torch.float32, device="cuda")
        for w_ in (ws, None):
            y = host(K.moe_down(fmt, wd, sd, dev(a), T, k, E, F, D, dev(cnt), dev(lst), ws=w_))
            for t in range(T):
                for sl, e in enumerate(pick[t]):
                    ent = t * k + sl
                    assert _bad(y[ent:ent + 1], ref.linear(a[ent:ent + 1], Dn[e], exact=True)) == 0, \
                        f"token {t} expert {e} workspace={w_ is not None}"


@pytest.mark.parametrize("seed", [301, 302])
def test_prefill_gemm_sweep(seed):
    """The prefill GEMM at random shapes: ragged row and column tiles, odd numbers of 64-deep K steps
    (the K loop runs two steps per iteration), activations read through a row stride wider than K,
    every epilogue, int8 / blockwise / fp16 weights, against the oracle's float64 product."""
    from aneforge_amd import _kernels as K
    rng = np.random.default_rng(seed)
    epis = ["f16", "resid", "f32", "swiglu", "geglu"]
    for trial in range(15):
        fmt = ["int8", "blockwise", "fp16"][trial % 3]
        epi = epis[trial % 5]
        M = int(rng.integers(1, 600))
        N = int(rng.integers(1, 48)) * 16 * (2 if epi in ("swiglu", "geglu") else 1)
        Kd = int(rng.integers(1, 24)) * 64
        pad = int(rng.integers(0, 3)) * 8
        say(f"sweep {seed}/{trial}: prefill gemm {fmt} {epi} M={M} N={N} K={Kd} ldx={Kd + pad}")
        w, s, W = _weights(rng, fmt, N, Kd)
        xbuf = rng.standard_normal((M, Kd + pad)).astype(np.float16)
        x = xbuf[:, :Kd]
        xd = dev(xbuf)[:, :Kd]                         # a row stride of K + pad
        lin = np.asarray(x, np.float64) @ np.asarray(W, np.float64).T
        wd, sd = dev(w), (dev(s) if s is not None else None)
        if epi == "resid":
            r = rng.standard_normal((M, N)).astype(np.float16)
            y = dev(r)
            K.gemm(fmt, wd, sd, xd, y=y, residual=y, epi="resid")
            assert _bad(host(y), ref.r16(r.astype(np.float64) + ref.r16(lin)), hidden=True) == 0, "resid"
            continue
        got = host(K.gemm(fmt, wd, sd, xd, epi=epi))
        if epi in ("swiglu", "geglu"):
            g, u = ref.r16(lin[:, 0::2]), ref.r16(lin[:, 1::2])
            act = ref.silu(g) if epi == "swiglu" else ref.gelu_tanh(g)
            assert _bad(got, ref.r16(act * u)) == 0, epi
        elif epi == "f32":
            assert _bad(got, lin) == 0, "f32"
        else:
            assert _bad(got, ref.r16(lin)) == 0, "f16"


@pytest.mark.parametrize("seed", [401, 402])
def test_sampling_sweep(seed):
    """Device sampling against the oracle's restatement of the reference's _sample, token for token, at
    random vocabularies (1 .. 300000), logit spreads (nearly flat to very sharp), masked (-inf) and
    rounded (tied) logits, and random temperature / top-k / top-p, so the candidate window takes every
    size: none, in LDS, in the workspace, and past it (the whole-vocabulary selection)."""
    from aneforge_amd import _kernels as K
    rng = np.random.default_rng(seed)
    for trial in range(24):
        V = int(np.exp(rng.uniform(0, np.log(300000)))) + 1
        sd = float(np.exp(rng.uniform(np.log(0.01), np.log(8.0))))
        logits = (rng.standard_normal(V) * sd).astype(np.float32)
        if rng.random() < 0.3:
            logits = (np.round(logits / (sd / 4)) * (sd / 4)).astype(np.float32)
        if rng.random() < 0.3 and V > 2:
            logits[rng.random(V) < rng.uniform(0.0, 0.5)] = -np.inf
            logits[int(rng.integers(0, V))] = 0.0                # at least one finite logit
        T = 0.0 if rng.random() < 0.1 else float(np.exp(rng.uniform(np.log(0.05), np.log(3.0))))
        top_p = 1.0 if rng.random() < 0.3 else float(rng.uniform(0.01, 0.999))
        top_k = 0 if rng.random() < 0.4 else int(np.exp(rng.uniform(0, np.log(V + 6))))
        us = rng.random(4)
        say(f"sweep {seed}/{trial}: sample V={V} sd={sd:.3g} T={T:.3g} top_p={top_p:.3g} top_k={top_k}")
        lg = dev(logits)
        params = torch.tensor([T, top_p, float(top_k)], dtype=torch.float64, device="cuda")
        uni = torch.from_numpy(us).cuda()
        ws = torch.empty(K.sample_ws_elems(V), dtype=torch.float64, device="cuda")
        for j, u in enumerate(us):
            step = torch.tensor([j], dtype=torch.int32, device="cuda")
            got = int(host(K.sample(lg, params, uni, step=step, ws=ws))[0])
            want = ref.sample(logits, T, top_p, top_k, float(u))
            assert got == want, f"V={V} T={T} top_p={top_p} top_k={top_k} u={u}: {got} vs {want}"
