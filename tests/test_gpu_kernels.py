"""Parity of each HIP kernel against the CPU oracle (oracle/ref.py), through the C ABI.

Integer unpack/dequant is checked bit-for-bit; fp16 outputs within rtol 1e-2 / atol 1e-3
with cosine >= 0.9999.  Shapes cover the benchmark configurations (full size) plus ragged
sizes that exercise the tails (rows not a multiple of the tile, K not a multiple of the
wavefront's slab, partial attention splits)."""
import numpy as np
import pytest

from _util import MIN_COS, check_f16, check_hidden, cosine, dev, host, say
from oracle import ref

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def K():
    from aneforge_amd import _kernels
    return _kernels


# ----------------------------------------------------------------------------- codecs
def test_dequant_int8_bit_exact(K):
    say("dequant int8 [300, 4096]")
    rng = np.random.default_rng(10)
    q = rng.integers(-128, 128, (300, 4096), dtype=np.int8)          # includes -128 (beyond the codec)
    s = (np.abs(rng.normal(0, 0.02, 300)) / 127).astype(np.float16)
    got = host(K.dequant("int8", dev(q), dev(s), 300, 4096))
    want = ref.dequant_w8(q, s)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("N,Kd", [(1, 128), (37, 384), (4096, 11008)])
def test_q4_0_repack_roundtrip_and_dequant_bit_exact(K, N, Kd):
    say(f"q4_0 repack/unpack/dequant N={N} K={Kd}")
    from aneforge_amd import _blob, workloads
    rng = np.random.default_rng(11)
    codes = rng.integers(0, 16, (N, Kd), dtype=np.uint8)
    d = (np.abs(rng.normal(0, 0.02, (N, Kd // 32))) / 8).astype(np.float16)
    blocks = workloads.q4_blocks_from_codes(codes, d)
    qs, dd = K.q4_repack(dev(blocks), N, Kd)
    hq, hd = _blob.q4_0_to_superblock(blocks, N, Kd)
    assert np.array_equal(host(qs), hq) and np.array_equal(host(dd).view(np.uint16), hd.view(np.uint16))
    back = host(K.q4_unpack(qs, dd, N, Kd))
    assert np.array_equal(back, blocks)
    got = host(K.dequant("q4_0", qs, dd, N, Kd))
    want = ref.dequant_q4_0(blocks, N, Kd)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ----------------------------------------------------------------------------- linear layers
def _w8(N, Kd, seed):
    rng = np.random.default_rng(seed)
    q = rng.integers(-127, 128, (N, Kd), dtype=np.int8)
    s = (np.abs(rng.normal(0, 0.02, N)) / 127).astype(np.float16)
    return q, s


@pytest.mark.parametrize("M,N,Kd", [(1, 4096, 4096), (1, 1000, 1024), (3, 777, 4112), (8, 256, 11008),
                                    (5, 6144, 4096), (2, 22016, 4096), (1, 4096, 11008),
                                    (12, 777, 4112), (20, 1000, 1024)])   # > 8 rows: vector in 8s / MFMA
def test_linear_int8(K, M, N, Kd):
    say(f"linear int8 M={M} N={N} K={Kd}")
    q, s = _w8(N, Kd, 20 + M)
    x = np.random.default_rng(21).standard_normal((M, Kd)).astype(np.float16)
    got = host(K.linear("int8", dev(q), dev(s), dev(x)))
    want = ref.linear(x, ref.dequant_w8(q, s))
    check_f16(got, want, what="int8 linear")


def _bw(N, Kd, seed):
    rng = np.random.default_rng(seed)
    q = rng.integers(-127, 128, (N, Kd), dtype=np.int8)
    s = (np.abs(rng.normal(0, 0.02, (N, Kd // 32))) / 127 + 1e-5).astype(np.float16)
    return q, s


def test_dequant_blockwise_bit_exact(K):
    say("dequant blockwise [300, 4096]")
    q, s = _bw(300, 4096, 12)
    got = host(K.dequant("blockwise", dev(q), dev(s), 300, 4096))
    assert np.array_equal(got.view(np.uint32), ref.dequant_blockwise(q, s).view(np.uint32))


def _l4(N, Kd, seed):
    rng = np.random.default_rng(seed)
    packed = rng.integers(0, 256, (N, Kd // 2), dtype=np.uint8)
    cb = (rng.standard_normal((N, 16)) * 0.05).astype(np.float16)      # a different codebook per row
    return packed, cb


@pytest.mark.parametrize("M,N,Kd", [(1, 4096, 4096), (1, 4096, 11008), (3, 1000, 1024), (1, 777, 4128),
                                    (6, 777, 4128), (12, 256, 11008)])
def test_linear_lut4(K, M, N, Kd):
    # fast path (M = 1, K 4096 / 11008), generic path with a ragged last unit (K = 4128), 8-row chunks
    say(f"linear lut4 M={M} N={N} K={Kd}")
    packed, cb = _l4(N, Kd, 70 + M)
    x = np.random.default_rng(71).standard_normal((M, Kd)).astype(np.float16)
    got = host(K.linear("lut4", dev(packed), dev(cb), dev(x)))
    check_f16(got, ref.linear(x, ref.dequant_lut4(packed, cb, Kd)), what="lut4 linear")


def _q4k(N, Kd, seed):
    # random GGUF Q4_K super-blocks: sane fp16 d / dmin, random 6-bit scale and min bytes (all bits,
    # so the j >= 4 packing is exercised) and random codes
    rng = np.random.default_rng(seed)
    nb = N * Kd // 256
    b = rng.integers(0, 256, (nb, 144), dtype=np.uint8)
    b[:, 0:2] = (np.abs(rng.standard_normal(nb)) * 0.002 + 1e-4).astype(np.float16).view(np.uint8).reshape(nb, 2)
    b[:, 2:4] = (np.abs(rng.standard_normal(nb)) * 0.004 + 1e-4).astype(np.float16).view(np.uint8).reshape(nb, 2)
    return b.reshape(N, Kd // 256 * 144)


@pytest.mark.parametrize("N,Kd", [(3, 256), (257, 4096), (64, 11008)])
def test_q4_k_repack_and_dequant_bit_exact(K, N, Kd):
    say(f"q4_k repack + dequant N={N} K={Kd}")
    from aneforge_amd import _blob
    blocks = _q4k(N, Kd, 15 + N)
    qs, hdr = K.q4_k_repack(dev(blocks), N, Kd)
    hq, hh = _blob.q4_k_repack(blocks, N, Kd)                # the device repack equals its host twin
    assert np.array_equal(host(qs), hq) and np.array_equal(host(hdr), hh)
    want = ref.dequant_q4_k_f16(blocks, N, Kd)               # gguf-py's float32 steps, then fp16
    got = host(K.dequant("q4_k", qs, hdr, N, Kd))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    out = torch.full((N, Kd + 64), 7.0, dtype=torch.float16, device="cuda")
    K.dequant_f16("q4_k", qs, hdr, N, Kd, out=out[:, :Kd])
    got16 = host(out)
    assert np.array_equal(got16[:, :Kd].view(np.uint16), want.astype(np.float16).view(np.uint16))
    assert (got16[:, Kd:] == 7.0).all()


@pytest.mark.parametrize("M,N,Kd", [(1, 4096, 4096), (1, 4096, 11008), (1, 22016, 4096), (3, 1000, 1024),
                                    (1, 777, 4352), (5, 777, 4352), (12, 256, 11008)])
def test_linear_q4_k(K, M, N, Kd):
    # fast path (M = 1, K 4096 / 11008), generic path with a ragged last unit (K = 4352 = 17 super-blocks),
    # 8-row chunks (M = 12)
    say(f"linear q4_k M={M} N={N} K={Kd}")
    blocks = _q4k(N, Kd, 80 + M)
    qs, hdr = K.q4_k_repack(dev(blocks), N, Kd)
    x = np.random.default_rng(81).standard_normal((M, Kd)).astype(np.float16)
    got = host(K.linear("q4_k", qs, hdr, dev(x)))
    check_f16(got, ref.linear(x, ref.dequant_q4_k_f16(blocks, N, Kd)), what="q4_k linear")


def _q6k(N, Kd, seed):
    # random GGUF Q6_K super-blocks: random ql / qh / int8 scales, a sane fp16 d
    rng = np.random.default_rng(seed)
    nb = N * Kd // 256
    b = rng.integers(0, 256, (nb, 210), dtype=np.uint8)
    b[:, 208:210] = (np.abs(rng.standard_normal(nb)) * 0.0005 + 1e-5).astype(np.float16).view(np.uint8).reshape(nb, 2)
    return b.reshape(N, Kd // 256 * 210)


@pytest.mark.parametrize("N,Kd", [(3, 256), (257, 4096), (64, 11008)])
def test_q6_k_repack_and_dequant_bit_exact(K, N, Kd):
    say(f"q6_k repack + dequant N={N} K={Kd}")
    from aneforge_amd import _blob
    blocks = _q6k(N, Kd, 25 + N)
    qs, sw = K.q6_k_repack(dev(blocks), N, Kd)
    hq, hs = _blob.q6_k_repack(blocks, N, Kd)                # the device repack equals its host twin
    assert np.array_equal(host(qs), hq) and np.array_equal(host(sw), hs)
    want = ref.dequant_q6_k_f16(blocks, N, Kd)               # gguf-py's float32 steps, then fp16
    got = host(K.dequant("q6_k", qs, sw, N, Kd))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    out = torch.full((N, Kd + 64), 7.0, dtype=torch.float16, device="cuda")
    K.dequant_f16("q6_k", qs, sw, N, Kd, out=out[:, :Kd])
    got16 = host(out)
    assert np.array_equal(got16[:, :Kd].view(np.uint16), want.astype(np.float16).view(np.uint16))
    assert (got16[:, Kd:] == 7.0).all()


@pytest.mark.parametrize("M,N,Kd", [(1, 4096, 4096), (1, 4096, 11008), (1, 22016, 4096), (3, 1000, 1024),
                                    (1, 777, 4352), (5, 777, 4352), (12, 256, 11008)])
def test_linear_q6_k(K, M, N, Kd):
    say(f"linear q6_k M={M} N={N} K={Kd}")
    blocks = _q6k(N, Kd, 90 + M)
    qs, sw = K.q6_k_repack(dev(blocks), N, Kd)
    x = np.random.default_rng(91).standard_normal((M, Kd)).astype(np.float16)
    got = host(K.linear("q6_k", qs, sw, dev(x)))
    check_f16(got, ref.linear(x, ref.dequant_q6_k_f16(blocks, N, Kd)), what="q6_k linear")


@pytest.mark.parametrize("fmt", ["int8", "q4_0", "blockwise", "lut4"])
def test_dequant_f16_bit_exact(K, fmt):
    # the fp16 weights the batched prefill expands a matrix to (rows of a wider scratch buffer)
    say(f"dequant_f16 {fmt} [72, 1024]")
    from aneforge_amd import _blob
    N, Kd = 72, 1024
    rng = np.random.default_rng(13)
    if fmt == "int8":
        q, s = _w8(N, Kd, 14)
        want = (q.astype(np.float32) * s.astype(np.float32)[:, None]).astype(np.float16)
    elif fmt == "blockwise":
        q, s = _bw(N, Kd, 14)
        want = ref.dequant_blockwise(q, s).astype(np.float16)
    elif fmt == "lut4":
        q, s = _l4(N, Kd, 14)
        want = ref.dequant_lut4(q, s, Kd).astype(np.float16)
    else:
        blocks = ref.quantize_q4_0(rng.standard_normal((N, Kd)).astype(np.float32) * 0.05)
        q, s = _blob.q4_0_to_superblock(blocks, N, Kd)
        want = ref.dequant_q4_0_f16(blocks, N, Kd).astype(np.float16)
    out = torch.full((N, Kd + 64), 7.0, dtype=torch.float16, device="cuda")
    K.dequant_f16(fmt, dev(q), dev(s), N, Kd, out=out[:, :Kd])
    got = host(out)
    assert np.array_equal(got[:, :Kd].view(np.uint16), want.view(np.uint16))
    assert (got[:, Kd:] == 7.0).all()                    # the padding columns are untouched


@pytest.mark.parametrize("M,N,Kd", [(1, 4096, 4096), (1, 4096, 11008), (3, 1000, 1024), (1, 777, 4160),
                                    (6, 777, 4160), (8, 1024, 4096), (20, 1000, 1024), (12, 778, 1088)])
def test_linear_blockwise(K, M, N, Kd):
    # fast path (M = 1, K 4096 / 11008), generic vector path, MFMA (M >= 4, N % 4 == 0), 8-row chunks
    say(f"linear blockwise M={M} N={N} K={Kd}")
    q, s = _bw(N, Kd, 60 + M)
    x = np.random.default_rng(61).standard_normal((M, Kd)).astype(np.float16)
    got = host(K.linear("blockwise", dev(q), dev(s), dev(x)))
    check_f16(got, ref.linear(x, ref.dequant_blockwise(q, s)), what="blockwise linear")


def test_linear_int8_cfg0_seeded(K):
    say("linear int8 cfg0 (seeded 4096x4096)")
    from aneforge_amd import workloads
    c = workloads.cfg0_gemv_w8()
    got = host(K.linear("int8", dev(c["q"]), dev(c["s"]), dev(c["x"])))
    check_f16(got, ref.linear(c["x"], ref.dequant_w8(c["q"], c["s"])), what="cfg0")


def test_linear_int8_bias_residual_inplace(K):
    say("linear int8 + bias + residual in place")
    q, s = _w8(512, 1024, 22)
    rng = np.random.default_rng(23)
    x = rng.standard_normal((2, 1024)).astype(np.float16)
    b = rng.standard_normal(512).astype(np.float16)
    r = rng.standard_normal((2, 512)).astype(np.float16)
    rd = dev(r)
    K.linear("int8", dev(q), dev(s), dev(x), y=rd, bias=dev(b), residual=rd)
    want = ref.r16(r.astype(np.float64) + ref.linear(x, ref.dequant_w8(q, s), b))
    check_f16(host(rd), want, what="bias+residual")


@pytest.mark.parametrize("M,N,Kd", [(4, 100, 512), (6, 4096, 4096), (8, 1004, 11008), (5, 22016, 4096)])
def test_linear_int8_mfma_rows_and_tails(K, M, N, Kd):
    # 4..8 activation rows take the MFMA path; N % 16 != 0 exercises the partial last tile
    say(f"linear int8 MFMA M={M} N={N} K={Kd}")
    q, s = _w8(N, Kd, 40 + M)
    x = np.random.default_rng(41 + M).standard_normal((M, Kd)).astype(np.float16)
    got = host(K.linear("int8", dev(q), dev(s), dev(x)))
    check_f16(got, ref.linear(x, ref.dequant_w8(q, s)), what="int8 linear (MFMA)")


def test_linear_mfma_bias_residual_and_fp16(K):
    say("MFMA path: bias + residual in place (int8), fp16 weights")
    rng = np.random.default_rng(42)
    q, s = _w8(260, 1024, 43)
    x = rng.standard_normal((5, 1024)).astype(np.float16)
    b = rng.standard_normal(260).astype(np.float16)
    r = rng.standard_normal((5, 260)).astype(np.float16)
    rd = dev(r)
    K.linear("int8", dev(q), dev(s), dev(x), y=rd, bias=dev(b), residual=rd)
    want = ref.r16(r.astype(np.float64) + ref.linear(x, ref.dequant_w8(q, s), b))
    check_hidden(host(rd), want, what="MFMA bias+residual")
    w = (rng.standard_normal((512, 2048)) * 0.02).astype(np.float16)
    x2 = rng.standard_normal((7, 2048)).astype(np.float16)
    got = host(K.linear("fp16", dev(w), None, dev(x2)))
    check_f16(got, ref.linear(x2, w.astype(np.float32)), what="fp16 MFMA")


@pytest.mark.parametrize("fmt,M,N,Kd", [("int8", 16, 4100, 4096), ("q4_0", 16, 4100, 4096), ("blockwise", 9, 4100, 4096),
                                         ("fp16", 12, 4100, 2048), ("q4_0", 4, 11008, 2048), ("int8", 13, 8200, 1024),
                                         ("q4_0", 5, 25000, 4096)])
def test_linear_mfma_persistent_tiles_and_epilogues(K, fmt, M, N, Kd):
    # dense linears of <= 16 rows whose K fits one batch per wavefront run on the persistent
    # MFMA kernel (one workgroup per CU walking the 16-row tiles): N = 4100 gives workgroup 0 a
    # second, ragged tile; N = 25000 (Q4_0, >= 6 tiles per workgroup) keeps three tiles of weights
    # in flight; plain, bias + residual, fp32 and SwiGLU epilogues
    say(f"linear MFMA persistent fmt={fmt} M={M} N={N} K={Kd}")
    from aneforge_amd import _blob
    rng = np.random.default_rng(N + M + Kd)
    if fmt == "int8":
        q, s = _w8(N, Kd, 90 + M)
        w, sc, W = dev(q), dev(s), ref.dequant_w8(q, s)
    elif fmt == "blockwise":
        q, s = _bw(N, Kd, 91 + M)
        w, sc, W = dev(q), dev(s), ref.dequant_blockwise(q, s)
    elif fmt == "fp16":
        W16 = (rng.standard_normal((N, Kd)) * 0.02).astype(np.float16)
        w, sc, W = dev(W16), None, W16.astype(np.float32)
    else:
        blocks = ref.quantize_q4_0((rng.standard_normal((N, Kd)) * 0.05).astype(np.float32))
        qs, d = _blob.q4_0_to_superblock(blocks, N, Kd)
        # the MFMA operand is the fp16 weight fp16((code - 8) * d), as GGUFView.get hands it over
        w, sc, W = dev(qs), dev(d), ref.dequant_q4_0_f16(blocks, N, Kd)
    x = rng.standard_normal((M, Kd)).astype(np.float16)
    b = (rng.standard_normal(N) * 0.1).astype(np.float16)
    r = rng.standard_normal((M, N)).astype(np.float16)
    y = host(K.linear(fmt, w, sc, dev(x)))
    check_f16(y, ref.linear(x, W), what=f"{fmt} persistent MFMA")
    got = host(K.linear(fmt, w, sc, dev(x), bias=dev(b), residual=dev(r)))
    check_hidden(got, ref.r16(r.astype(np.float64) + ref.linear(x, W, b)), what=f"{fmt} bias+residual")
    got32 = host(K.linear(fmt, w, sc, dev(x), out_f32=True))
    check_f16(got32, ref.linear(x, W, exact=True), what=f"{fmt} fp32 out")
    # interleaved gate/up rows: the epilogue rounds gate and up to fp16 before silu(g) * u
    act = host(K.linear_swiglu(fmt, w, sc, dev(x)))
    yd = y.astype(np.float32)
    check_f16(act, ref.r16(ref.silu(yd[:, 0::2]) * yd[:, 1::2]), what=f"{fmt} swiglu epilogue")


@pytest.mark.parametrize("M,N,Kd", [(1, 11008, 4096), (1, 4096, 11008), (4, 11008, 4096), (4, 4096, 11008),
                                    (8, 11008, 4096), (8, 4096, 11008), (3, 100, 384)])
def test_linear_q4_0_cfg1(K, M, N, Kd):
    say(f"linear q4_0 M={M} N={N} K={Kd}")
    from aneforge_amd import workloads
    c = workloads.cfg1_gemv_q4(N, Kd, M)
    qs, d = K.q4_repack(dev(c["blocks"]), N, Kd)
    got = host(K.linear("q4_0", qs, d, dev(c["x"])))
    want = ref.linear(c["x"], ref.dequant_q4_0_f16(c["blocks"], N, Kd))
    check_f16(got, want, what="q4_0 linear")


@pytest.mark.parametrize("M,N,Kd", [(1, 32000, 4096), (2, 1000, 520)])
def test_linear_f16_logits(K, M, N, Kd):
    say(f"linear fp16 -> fp32 M={M} N={N} K={Kd}")
    rng = np.random.default_rng(24)
    w = rng.normal(0, 0.02, (N, Kd)).astype(np.float16)
    x = rng.standard_normal((M, Kd)).astype(np.float16)
    got = host(K.linear("fp16", dev(w), None, dev(x), out_f32=True))
    want = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.abs(got - want).max() < 1e-4 * max(1.0, np.abs(want).max())


@pytest.mark.parametrize("fmt", ["int8", "q4_0", "fp16"])
def test_linear_rms_prologue(K, fmt):
    say(f"linear + rmsnorm prologue fmt={fmt}")
    rng = np.random.default_rng(25)
    M, N, Kd = 3, 1536, 4096
    h = (rng.standard_normal((M, Kd)) * 2).astype(np.float16)
    g = rng.uniform(0.5, 1.5, Kd).astype(np.float16)
    if fmt == "int8":
        q, s = _w8(N, Kd, 26)
        wd, sd, Wf = dev(q), dev(s), ref.dequant_w8(q, s)
    elif fmt == "q4_0":
        from aneforge_amd import workloads
        c = workloads.cfg1_gemv_q4(N, Kd, 1, seed=26)
        wd, sd = K.q4_repack(dev(c["blocks"]), N, Kd)
        Wf = ref.dequant_q4_0_f16(c["blocks"], N, Kd)
    else:
        Wf16 = rng.normal(0, 0.02, (N, Kd)).astype(np.float16)
        wd, sd, Wf = dev(Wf16), None, Wf16.astype(np.float32)
    got = host(K.linear_rms(fmt, wd, sd, dev(h), dev(g), 1e-5))
    want = ref.linear(ref.rms_norm(h, g, 1e-5), Wf)
    check_f16(got, want, what=f"rms+{fmt}")


@pytest.mark.parametrize("Kd", [4096, 4000, 2048])
def test_linear_int8_norm_row_kernel_positive_mean(K, Kd):
    """One activation row through the int8 norm-prologue row kernel (plain and SwiGLU), whose dot
    products run on the codes offset by +1152 and subtract 1152 * sum(x) per row: a row with a large
    positive mean makes that correction as large as it gets, and K = 4000 / 2048 leave part or all of
    the last units past K (their x must add nothing)."""
    from aneforge_amd import _blob
    say(f"int8 norm row kernel, positive-mean row, K={Kd}")
    rng = np.random.default_rng(31)
    N = 1536
    h = rng.uniform(0.5, 1.5, (1, Kd)).astype(np.float16)
    g = rng.uniform(0.5, 1.5, Kd).astype(np.float16)
    hn = ref.rms_norm(h, g, 1e-5)
    q, s = _w8(N, Kd, 32)
    got = host(K.linear_rms("int8", dev(q), dev(s), dev(h), dev(g), 1e-5))
    check_f16(got, ref.linear(hn, ref.dequant_w8(q, s)), what=f"rms int8 K={Kd}")
    qg, sg = _w8(N // 2, Kd, 33)
    qu, su = _w8(N // 2, Kd, 34)
    act = host(K.linear_swiglu("int8", dev(_blob.interleave_rows(qg, qu)), dev(_blob.interleave_rows(sg, su)), dev(h),
                               gamma=dev(g), eps=1e-5))
    gg = ref.linear(hn, ref.dequant_w8(qg, sg))
    uu = ref.linear(hn, ref.dequant_w8(qu, su))
    check_f16(act, ref.r16(ref.silu(gg) * uu), what=f"rms swiglu int8 K={Kd}")


def test_linear_swiglu(K):
    say("linear swiglu (gate/up interleaved) with norm")
    from aneforge_amd import _blob
    rng = np.random.default_rng(27)
    M, F, Kd = 2, 1376, 4096
    qg, sg = _w8(F, Kd, 28)
    qu, su = _w8(F, Kd, 29)
    h = rng.standard_normal((M, Kd)).astype(np.float16)
    g = np.ones(Kd, np.float16)
    w = _blob.interleave_rows(qg, qu)
    s = _blob.interleave_rows(sg, su)
    got = host(K.linear_swiglu("int8", dev(w), dev(s), dev(h), dev(g), 1e-5))
    hn = ref.rms_norm(h, g, 1e-5)
    gg = ref.linear(hn, ref.dequant_w8(qg, sg))
    uu = ref.linear(hn, ref.dequant_w8(qu, su))
    check_f16(got, ref.r16(ref.silu(gg) * uu), what="swiglu")


@pytest.mark.parametrize("M,norm,path", [(1, True, "vector"), (3, True, "vector"), (6, False, "mfma"),
                                         (70, False, "gemm")])
def test_linear_geglu(K, M, norm, path):
    """Gemma's GeGLU front half, act = gelu_tanh(g) * u (aneforge/llm.py:185-196), on each kernel family
    that carries the gated epilogue: the vector GEMV (with the RMSNorm prologue), the skinny MFMA
    (4+ rows, no norm) and the prefill GEMM."""
    say(f"linear geglu M={M} norm={norm} path={path}")
    from aneforge_amd import _blob
    rng = np.random.default_rng(31)
    F, Kd = 1024, 4096
    qg, sg = _w8(F, Kd, 32)
    qu, su = _w8(F, Kd, 33)
    h = rng.standard_normal((M, Kd)).astype(np.float16)
    g = rng.uniform(0.5, 1.5, Kd).astype(np.float16)
    w = dev(_blob.interleave_rows(qg, qu))
    s = dev(_blob.interleave_rows(sg, su))
    if path == "gemm":
        got = host(K.gemm("int8", w, s, dev(h), epi="geglu"))
        hn = h
    else:
        got = host(K.linear_swiglu("int8", w, s, dev(h), dev(g) if norm else None, 1e-5, gelu=True))
        hn = ref.rms_norm(h, g, 1e-5) if norm else h
    gg = ref.linear(hn, ref.dequant_w8(qg, sg))
    uu = ref.linear(hn, ref.dequant_w8(qu, su))
    assert np.abs(gg).max() > 2.0                       # gate values reach where gelu and silu differ
    check_f16(got, ref.r16(ref.gelu_tanh(gg) * uu), what=f"geglu {path}")
    assert np.abs(got - ref.r16(ref.silu(gg) * uu)).max() > 0.05


@pytest.mark.parametrize("M,H,KV,dh,pos", [(1, 32, 8, 128, 2048), (2, 4, 2, 64, 5), (10, 4, 2, 64, 5)])
def test_qkv_rope_kv_fused(K, M, H, KV, dh, pos):
    say(f"fused qkv+rope+kv write M={M} H={H} KV={KV} dh={dh} pos={pos}")
    from aneforge_amd import _blob
    rng = np.random.default_rng(30)
    D = H * dh if H * dh >= 1024 else 1024
    Mmax = pos + M + 3
    qq, sq = _w8(H * dh, D, 31)
    qk, sk = _w8(KV * dh, D, 32)
    qv, sv = _w8(KV * dh, D, 33)
    bias = rng.standard_normal(H * dh + 2 * KV * dh).astype(np.float16) * 0.1
    permq, permk = _blob.rope_pair_order(H, dh), _blob.rope_pair_order(KV, dh)
    w = np.concatenate([qq[permq], qk[permk], qv])
    s = np.concatenate([sq[permq], sk[permk], sv])
    bb = np.concatenate([bias[:H * dh][permq], bias[H * dh:H * dh + KV * dh][permk], bias[H * dh + KV * dh:]])
    h = rng.standard_normal((M, D)).astype(np.float16)
    g = rng.uniform(0.8, 1.2, D).astype(np.float16)
    cos, sin = ref.rope_tables(Mmax, dh)
    kc = torch.zeros((M, KV, Mmax, dh), dtype=torch.float16, device="cuda")
    vc = torch.zeros_like(kc)
    posd = torch.tensor([pos + m for m in range(M)], dtype=torch.int32, device="cuda")
    qout = torch.empty((M, H * dh), dtype=torch.float16, device="cuda")
    K.qkv_rope_kv("int8", dev(w), dev(s), dev(h), dev(g), 1e-5, dev(bb), H * dh, KV * dh, dh, dev(cos), dev(sin),
                  posd, qout, kc, vc)
    hq, hk, hv = host(qout), host(kc), host(vc)
    for m in range(M):
        p = pos + m
        xn = ref.rms_norm(h[m:m + 1], g, 1e-5)
        qr = ref.rope(ref.linear(xn, ref.dequant_w8(qq, sq), bias[:H * dh]).reshape(H, dh), cos[p], sin[p])
        kr = ref.rope(ref.linear(xn, ref.dequant_w8(qk, sk), bias[H * dh:H * dh + KV * dh]).reshape(KV, dh),
                      cos[p], sin[p])
        vr = ref.linear(xn, ref.dequant_w8(qv, sv), bias[H * dh + KV * dh:]).reshape(KV, dh)
        check_f16(hq[m].reshape(H, dh), qr, what="q")
        check_f16(hk[m, :, p], kr, what="k cache row")
        check_f16(hv[m, :, p], vr, what="v cache row")
        assert not hk[m, :, :p].any() and not hk[m, :, p + 1:].any()    # nothing else written


# ----------------------------------------------------------------------------- attention
@pytest.mark.parametrize("B,ctx", [(1, 512), (1, 2048), (1, 8192), (16, 512), (16, 2048), (16, 8192)])
def test_decode_attn_cfg2(K, B, ctx):
    say(f"decode attention cfg2 B={B} ctx={ctx}")
    from aneforge_amd import workloads
    c = workloads.cfg2_attn(ctx, B)
    got = host(K.decode_attn(dev(c["q"]), dev(c["K"]), dev(c["V"]), ctx_len=ctx))
    # every sequence: the XCD placement maps each (split, kv head, sequence) from a 1-D block index
    for b in range(B):
        want = ref.attention(c["q"][b:b + 1, :, None, :], c["K"][b:b + 1], c["V"][b:b + 1])[0, :, 0]
        check_f16(got[b], want, what=f"attn b={b}")


@pytest.mark.parametrize("Hq,Hkv,D,Mmax", [(4, 4, 64, 37), (8, 2, 128, 300), (16, 2, 64, 1000), (8, 1, 128, 5),
                                           (4, 2, 32, 50), (4, 4, 256, 20)])
def test_decode_attn_device_positions(K, Hq, Hkv, D, Mmax):
    say(f"decode attention pos-driven Hq={Hq} Hkv={Hkv} D={D} Mmax={Mmax}")
    rng = np.random.default_rng(40)
    B = 3
    q = rng.standard_normal((B, Hq, D)).astype(np.float16)
    Kc = rng.standard_normal((B, Hkv, Mmax, D)).astype(np.float16)
    Vc = rng.standard_normal((B, Hkv, Mmax, D)).astype(np.float16)
    pos = np.array([0, Mmax // 2, Mmax - 1], np.int32)
    got = host(K.decode_attn(dev(q), dev(Kc), dev(Vc), pos=dev(pos)))
    want = ref.attention(q[:, :, None, :], Kc, Vc, lengths=pos + 1)[:, :, 0]
    check_f16(got, want, what="attn pos")


@pytest.mark.parametrize("nstep", [2, 3, 4, 5, 6, 8, 16])
def test_decode_attn_every_split_size_at_the_7b_cache_bound(K, nstep):
    """Each instantiated chunk (16 * nstep positions) at the cfg3 engine's cache bound (2184 rows, 32/8
    heads, dh 128), positions from the device: a partly filled last split, the final row, and ctx 1.
    (16-position chunks would need 137 > 128 splits here.)"""
    say(f"decode attention 7B cache bound nstep={nstep}")
    rng = np.random.default_rng(41)
    B, Hq, Hkv, D, Mmax = 3, 32, 8, 128, 2184
    q = rng.standard_normal((B, Hq, D)).astype(np.float16)
    Kc = rng.standard_normal((B, Hkv, Mmax, D)).astype(np.float16)
    Vc = rng.standard_normal((B, Hkv, Mmax, D)).astype(np.float16)
    pos = np.array([2048, Mmax - 1, 0], np.int32)
    got = host(K.decode_attn(dev(q), dev(Kc), dev(Vc), pos=dev(pos), nstep_hint=nstep))
    want = ref.attention(q[:, :, None, :], Kc, Vc, lengths=pos + 1)[:, :, 0]
    check_f16(got, want, what=f"attn nstep={nstep}")


def test_decode_attn_workspace_reuse_and_graph_replay(K):
    say("decode attention: one workspace reused across calls and graph replays")
    import bench
    from aneforge_amd import workloads
    outs = []
    for ctx in (300, 2048):
        c = workloads.cfg2_attn(ctx, 2, seed=ctx)
        q, k, v = dev(c["q"]), dev(c["K"]), dev(c["V"])
        ws = torch.zeros(K.attn_ws_bytes(2, 32, 8, 128, ctx) // 4 + 1, dtype=torch.float32, device="cuda")
        want = ref.attention(c["q"][:, :, None, :], c["K"], c["V"])[:, :, 0]
        for _ in range(3):                                   # eager reuse of one workspace
            check_f16(host(K.decode_attn(q, k, v, ctx_len=ctx, ws=ws)), want, what=f"eager ctx={ctx}")
        o = torch.empty_like(q)
        g = bench.Graph(lambda: K.decode_attn(q, k, v, o=o, ctx_len=ctx, ws=ws))
        for _ in range(3):
            o.zero_()
            g.launch()
            g.stream.synchronize()
            check_f16(host(o), want, what=f"replay ctx={ctx}")
        g.close()


def test_decode_attn_mask_and_causal(K):
    say("decode attention additive mask + causal alignment")
    rng = np.random.default_rng(41)
    Sq, Skv, H, D = 6, 6, 2, 64
    q = rng.standard_normal((1, H, Sq, D)).astype(np.float16)
    k = rng.standard_normal((1, H, Skv, D)).astype(np.float16)
    v = rng.standard_normal((1, H, Skv, D)).astype(np.float16)
    qd = dev(q)
    # queries as the batch axis sharing one KV (af.sdpa layout [1, H, S, D])
    o = torch.empty_like(qd)
    K.decode_attn(qd, dev(k), dev(v), o=o, ctx_len=Skv, causal_off=0, q_strides=(D, Sq * D),
                  kv_strides=(0, Skv * D), B=Sq, Hq=H)
    want = np.stack([ref.attention(q[:, :, s:s + 1], k, v, lengths=[s + 1])[0, :, 0] for s in range(Sq)], 1)
    check_f16(host(o)[0], want, what="causal")
    m = rng.standard_normal((Sq, Skv)).astype(np.float16)
    o2 = torch.empty_like(qd)
    K.decode_attn(qd, dev(k), dev(v), o=o2, ctx_len=Skv, mask=dev(m), q_strides=(D, Sq * D),
                  kv_strides=(0, Skv * D), B=Sq, Hq=H)
    want2 = np.stack([ref.attention(q[:, :, s:s + 1], k, v, mask=m[s:s + 1])[0, :, 0] for s in range(Sq)], 1)
    check_f16(host(o2)[0], want2, what="mask")


@pytest.mark.parametrize("fmt,M,N,Kd", [("int8", 8, 300, 4096), ("q4_0", 16, 52, 4480), ("q6_k", 9, 466, 5632),
                                         ("int8", 3, 128, 11008), ("fp16", 5, 64, 16000)])
def test_norm_prologue_linears_split_rows_to_fit_lds(K, fmt, M, N, Kd):
    # RMSNorm-prologue linears stage M normalised rows in 64 KB of LDS; larger M * K runs in row groups
    say(f"rms linear + swiglu {fmt} M={M} N={N} K={Kd}")
    from aneforge_amd import _blob
    rng = np.random.default_rng(M * 1000 + N)
    if fmt == "int8":
        q, s = _w8(N, Kd, 33)
        w, sc, W = dev(q), dev(s), ref.dequant_w8(q, s)
    elif fmt == "fp16":
        W16 = (rng.standard_normal((N, Kd)) * 0.02).astype(np.float16)
        w, sc, W = dev(W16), None, W16.astype(np.float32)
    elif fmt == "q4_0":
        blocks = ref.quantize_q4_0((rng.standard_normal((N, Kd)) * 0.05).astype(np.float32))
        qs, d = _blob.q4_0_to_superblock(blocks, N, Kd)
        w, sc, W = dev(qs), dev(d), ref.dequant_q4_0_f16(blocks, N, Kd)
    else:
        blocks = _q6k(N, Kd, 7)
        w, sc = K.q6_k_repack(dev(blocks), N, Kd)
        W = ref.dequant_q6_k_f16(blocks, N, Kd)
    x = rng.standard_normal((M, Kd)).astype(np.float16)
    g = rng.uniform(0.5, 1.5, Kd).astype(np.float16)
    hn = ref.rms_norm(x, g, 1e-5)
    yd = host(K.linear_rms(fmt, w, sc, dev(x), dev(g), 1e-5)).astype(np.float32)
    check_f16(yd, ref.linear(hn, W), what="rms linear")
    # The SwiGLU epilogue rounds the same fp32 accumulators to fp16 before silu(g) * u. Where one
    # factor is small beside K terms of this size, accumulation-order noise inside the linear's own
    # tolerance is >1% of it, so the epilogue is pinned against the device linear checked above and
    # the whole against the oracle's product by cosine.
    act = host(K.linear_swiglu(fmt, w, sc, dev(x), gamma=dev(g), eps=1e-5))
    check_f16(act, ref.r16(ref.silu(yd[:, 0::2]) * yd[:, 1::2]), what="rms swiglu epilogue")
    yy = ref.linear(hn, W).astype(np.float16).astype(np.float32)
    assert cosine(act, ref.silu(yy[:, 0::2]) * yy[:, 1::2]) >= MIN_COS


# ----------------------------------------------------------------------------- sampling
@pytest.mark.parametrize("V,grid,sd", [(32000, 0.0, 2.5), (1000, 0.25, 2.5), (151936, 0.0, 2.5), (32000, 0.0, 0.05),
                                       (262144, 0.0, 2.5), (151936, 0.0, 0.01)])
def test_sample_matches_oracle(K, V, grid, sd):
    # temperature / top-k / top-p / the inverse-CDF draw against the oracle's restatement of the
    # reference's _sample; grid > 0 rounds the logits so ties are common (top-k and nucleus edges).
    # The window of candidate logits takes every size: sd = 0.05 makes the distribution nearly flat,
    # so a top-p nucleus holds most of the vocabulary (a window above the pick kernel's LDS cap, read
    # from the workspace); at V = 262144 a top-k of 7000 and T = 2 top-p edges land there too; and
    # sd = 0.01 at V = 151936 puts every logit in one bin (above the workspace window: the selection
    # runs over the whole vocabulary)
    say(f"device sampling V={V} ties={grid > 0} sd={sd}")
    rng = np.random.default_rng(V)
    logits = (rng.standard_normal(V) * sd).astype(np.float32)
    if grid:
        logits = (np.round(logits / grid) * grid).astype(np.float32)
    lg = dev(logits)
    ws = torch.empty(V, dtype=torch.float64, device="cuda")
    us = np.concatenate([[0.0, 0.5, 1.0 - 1e-12], rng.random(21)])
    for T, top_p, top_k in [(0.0, 1.0, 0), (1.0, 1.0, 0), (0.7, 1.0, 0), (0.8, 1.0, 40), (1.0, 0.9, 0),
                            (0.8, 0.9, 40), (1.3, 0.5, 5), (1.0, 0.999, 0), (0.6, 0.95, 1), (2.0, 0.3, V + 5),
                            (2.0, 0.95, 0), (0.9, 1.0, 7000)]:
        params = torch.tensor([T, top_p, float(top_k)], dtype=torch.float64, device="cuda")
        uni = torch.from_numpy(us).cuda()
        for j, u in enumerate(us):
            step = torch.tensor([j], dtype=torch.int32, device="cuda")
            got = int(host(K.sample(lg, params, uni, step=step, ws=ws))[0])
            want = ref.sample(logits, T, top_p, top_k, float(u))
            assert got == want, f"T={T} top_p={top_p} top_k={top_k} u={u}: {got} vs {want}"


@pytest.mark.parametrize("V", [1, 8, 2049, 40000])
def test_sample_edge_cases_match_oracle(K, V):
    """Masked (-inf) logits, a vocabulary one past a 2048-logit chunk, a single logit, ties, a nucleus
    holding only the maximum (top_p 1e-9), top_k = 1, a very sharp (T = 0.05) and a nearly flat
    (T = 10) distribution, each token for token against the oracle's _sample."""
    say(f"device sampling edge cases V={V}")
    rng = np.random.default_rng(100 + V)
    logits = (rng.standard_normal(V) * 2.0).astype(np.float32)
    if V >= 8:
        logits[rng.random(V) < 0.1] = -np.inf                      # banned tokens
        logits[3] = logits[5] = np.float32(np.max(logits[np.isfinite(logits)]) + 0.5)   # a tie at the top
    lg = dev(logits)
    ws = torch.empty(K.sample_ws_elems(V), dtype=torch.float64, device="cuda")
    us = np.concatenate([[0.0, 0.5, 1.0 - 1e-12], rng.random(9)])
    uni = torch.from_numpy(us).cuda()
    for T, top_p, top_k in [(0.5, 1.0, 0), (1.0, 0.9, 0), (1.0, 1e-9, 0), (0.05, 0.9, 5), (10.0, 0.95, 0),
                            (1.0, 0.5, 1), (0.8, 0.9, 3)]:
        params = torch.tensor([T, top_p, float(top_k)], dtype=torch.float64, device="cuda")
        for j, u in enumerate(us):
            step = torch.tensor([j], dtype=torch.int32, device="cuda")
            got = int(host(K.sample(lg, params, uni, step=step, ws=ws))[0])
            want = ref.sample(logits, T, top_p, top_k, float(u))
            assert got == want, f"V={V} T={T} top_p={top_p} top_k={top_k} u={u}: {got} vs {want}"


# ----------------------------------------------------------------------------- small ops
def test_rmsnorm_rope_embed_argmax(K):
    say("rmsnorm / rope / embed / argmax")
    rng = np.random.default_rng(50)
    x = rng.standard_normal((3, 4096)).astype(np.float16)
    g = rng.uniform(0.5, 1.5, 4096).astype(np.float16)
    check_f16(host(K.rmsnorm(dev(x), dev(g), 1e-5)), ref.rms_norm(x, g, 1e-5), what="rmsnorm")
    cos, sin = ref.rope_tables(40, 128)
    xr = rng.standard_normal((8, 128)).astype(np.float16)
    got = host(K.rope(dev(xr), dev(cos), dev(sin), pos0=30, rows_per_pos=4))
    want = np.concatenate([ref.rope(xr[:4], cos[30], sin[30]), ref.rope(xr[4:], cos[31], sin[31])])
    check_f16(got, want, what="rope")
    table = rng.standard_normal((100, 64)).astype(np.float16)
    ids = np.array([5, 99, 0], np.int32)
    assert np.array_equal(host(K.embed(dev(table), dev(ids))), table[ids])
    lg = rng.standard_normal((2, 32000)).astype(np.float32)
    lg[1, 7] = lg[1, 9] = 100.0                                   # tie -> lowest index
    assert host(K.argmax(dev(lg))).tolist() == [int(np.argmax(lg[0])), 7]


@pytest.mark.parametrize("V,D", [(32000, 4096), (1000, 4088), (1000, 4104), (300, 8)])
def test_decode_advance_greedy_and_forced(K, V, D):
    """A forced step, then a greedy one, with the embedding row gathered into h, at row widths that
    do and do not fill the workgroup's 16-byte pieces evenly (4088, 4104, 8)."""
    say(f"decode advance (argmax / forced + hist + pos + embed) V={V} D={D}")
    rng = np.random.default_rng(51)
    lg = rng.standard_normal(V).astype(np.float32)
    table = rng.standard_normal((V, D)).astype(np.float16)
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    pos = torch.tensor([10], dtype=torch.int32, device="cuda")
    step = torch.tensor([2], dtype=torch.int32, device="cuda")
    hist = torch.full((8,), -1, dtype=torch.int32, device="cuda")
    h = torch.zeros((1, D), dtype=torch.float16, device="cuda")
    forced = torch.tensor([7, 8, 9], dtype=torch.int32, device="cuda")
    nf = torch.tensor([3], dtype=torch.int32, device="cuda")
    tb = dev(table)
    K.decode_advance(dev(lg), tok, pos, hist, step, tb, h, forced, nf)     # step 2 < 3: forced[2]
    assert host(tok)[0] == 9 and host(pos)[0] == 11 and host(step)[0] == 3 and host(hist)[2] == 9
    assert np.array_equal(host(h)[0], table[9])
    K.decode_advance(dev(lg), tok, pos, hist, step, tb, h, forced, nf)     # step 3: greedy
    t = int(np.argmax(lg))
    assert host(tok)[0] == t and host(pos)[0] == 12 and host(step)[0] == 4 and host(hist)[3] == t
    assert np.array_equal(host(h)[0], table[t])


@pytest.mark.parametrize("N,Kd", [(32000, 4096), (77, 64), (1000, 256)])
def test_lm_head_logits_slots_and_normalised_row(K, N, Kd):
    """afx_lm_head (the fused K = 4096 head and the generic path): the same logits as the plain
    RMSNorm linear, slots that summarise each 8 rows (largest, its lowest row, second largest,
    largest magnitude), and the fp16 normalised row the products used."""
    say(f"lm_head slots N={N} K={Kd}")
    rng = np.random.default_rng(52)
    W = (rng.standard_normal((N, Kd)) * 0.02).astype(np.float16)
    W[5] = W[3]                                                     # an exact tie inside slot 0
    x = rng.standard_normal((1, Kd)).astype(np.float16)
    g = rng.uniform(0.5, 1.5, Kd).astype(np.float16)
    hn = torch.zeros(Kd, dtype=torch.float16, device="cuda")
    lg, slots = K.lm_head(dev(W), dev(x), dev(g), 1e-5, hn=hn)
    lg, slots = host(lg)[0], host(slots)
    plain = host(K.linear_rms("fp16", dev(W), None, dev(x), dev(g), 1e-5, out_f32=True))[0]
    assert np.array_equal(lg, plain)
    check_f16(lg, ref.linear(ref.rms_norm(x, g, 1e-5), W.astype(np.float32), exact=True)[0], what="head logits")
    for s in range((N + 7) // 8):
        r = lg[8 * s:8 * s + 8]
        i1 = int(np.argmax(r))
        top2 = np.sort(r)[-2] if r.size > 1 else -np.inf
        want = (r[i1], 8 * s + i1, top2, np.abs(r).max())
        got = (slots[s, 0], int(slots[s, 1:2].view(np.int32)[0]), slots[s, 2], slots[s, 3])
        assert got == want, f"slot {s}: {got} vs {want}"
    assert slots[0, 0] != lg[3] or slots[0, 2] == slots[0, 0]       # the tie shows as a zero gap
    hn = host(hn).astype(np.float64)
    want = ref.rms_norm(x, g, 1e-5)[0]
    assert np.abs(hn - want).max() <= np.spacing(np.float16(np.abs(want).max()))
    # the logits are the products of exactly this row
    assert np.allclose(lg, W.astype(np.float64) @ hn, rtol=1e-5, atol=1e-5)


def test_decode_advance_near_tie_recomputes_exactly(K):
    """The reference's greedy near-tie rule (aneforge/llm.py:395-404) on the device: two logits closer
    than margin * max|logit| are recomputed exactly from the head's input row and the head's fp32 rows,
    and the exact winner is taken; a clear gap, or no margin, keeps the plain argmax."""
    say("decode advance near-tie recompute")
    rng = np.random.default_rng(53)
    V, D = 4096, 256
    hn = rng.uniform(0.1, 1.0, D).astype(np.float16)
    W32 = (rng.standard_normal((V, D)) * 0.01).astype(np.float32)
    W32[100] = (np.abs(W32[100]) + 0.05).astype(np.float16).astype(np.float32)   # fp16-exact, >= 2^-5
    W32[900] = W32[100] + 2.0 ** -18        # under half an fp16 ulp: the fp16 rows tie, the fp32 rows do not
    W16 = W32.astype(np.float16)
    assert np.array_equal(W16[100], W16[900])
    lg = (W16.astype(np.float64) @ hn.astype(np.float64)).astype(np.float32)
    lg[900] = lg[100]                                               # the fp16 head's exact tie
    ref_host = W32.astype(np.float64) @ hn.astype(np.float64)
    assert int(np.argmax(ref_host)) == 900 and int(np.argmax(lg)) == 100

    table = rng.standard_normal((V, D)).astype(np.float16)        # embedding rows: h follows the pick
    tb = dev(table)

    def step_once(logits, margin, head32=True):
        tok = torch.zeros(1, dtype=torch.int32, device="cuda")
        pos = torch.zeros(1, dtype=torch.int32, device="cuda")
        stp = torch.zeros(1, dtype=torch.int32, device="cuda")
        hist = torch.zeros(4, dtype=torch.int32, device="cuda")
        h = torch.zeros((1, D), dtype=torch.float16, device="cuda")
        m = None if margin is None else torch.tensor([margin], dtype=torch.float32, device="cuda")
        K.decode_advance(dev(logits[None]), tok, pos, hist, stp, tb, h, tie_margin=m, hn=dev(hn),
                         head16=None if head32 else dev(W16), head32=dev(W32) if head32 else None)
        t = int(host(tok)[0])
        assert np.array_equal(host(h)[0], table[t])
        return t

    assert step_once(lg, 3e-3) == 900                               # near tie: exact recompute
    assert step_once(lg, None) == 100                               # no rule: lowest index
    assert step_once(lg, 3e-3, head32=False) == 100                 # fp16 rows tie exactly: lowest index
    clear = lg.copy()
    clear[100] += 1.0
    assert step_once(clear, 3e-3) == 100                            # a clear gap: no recompute
    # the same rule when the pick comes from the lm_head's slot summaries
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    h = torch.zeros((1, D), dtype=torch.float16, device="cuda")
    K.decode_advance(dev(lg[None]), tok, torch.zeros(1, dtype=torch.int32, device="cuda"),
                     torch.zeros(4, dtype=torch.int32, device="cuda"), torch.zeros(1, dtype=torch.int32, device="cuda"),
                     tb, h, slots=dev(_host_slots(lg)), tie_margin=torch.tensor([3e-3], dtype=torch.float32, device="cuda"),
                     hn=dev(hn), head32=dev(W32))
    assert int(host(tok)[0]) == 900
    assert np.array_equal(host(h)[0], table[900])                   # not the top-1's row (100)


def _host_slots(lg):
    """The lm_head's greedy-pick summaries of 8 logits each (largest, its lowest index as int32
    bits, second largest, largest magnitude), built on the host."""
    V = lg.size
    ns = (V + 7) // 8
    r = np.full(ns * 8, -np.inf, np.float32)
    r[:V] = lg
    r = r.reshape(ns, 8)
    i1 = r.argmax(1)
    rows = np.arange(ns)
    r2 = r.copy()
    r2[rows, i1] = -np.inf
    out = np.zeros((ns, 4), np.float32)
    out[:, 0] = r[rows, i1]
    out[:, 1] = (8 * rows + i1).astype(np.int32).view(np.float32)
    out[:, 2] = r2.max(1)
    out[:, 3] = np.abs(np.where(np.isfinite(r), r, 0.0)).max(1)
    return out


@pytest.mark.parametrize("V", [32000, 152064, 77, 8])
def test_decode_advance_from_slots_is_the_argmax(K, V):
    """The greedy pick from slot summaries (one float4 per 8 logits, several load rounds of the
    workgroup for a 152k vocabulary) is np.argmax of the logits: the lowest index on a tie across
    slots and inside one, and the step bookkeeping and embedding gather follow it."""
    say(f"decode advance from slots V={V}")
    rng = np.random.default_rng(54 + V)
    D = 64
    table = rng.standard_normal((V, D)).astype(np.float16)
    tb = dev(table)
    cases = [rng.standard_normal(V).astype(np.float32)]
    tie = rng.standard_normal(V).astype(np.float32)
    hi = sorted(rng.choice(V, size=min(V, 3), replace=False).tolist())
    tie[hi] = tie.max() + 1.0                                       # tie across slots: the lowest index
    cases.append(tie)
    last = rng.standard_normal(V).astype(np.float32)
    last[V - 1] = last.max() + 0.5                                  # the maximum in the last (ragged) slot
    cases.append(last)
    for lg in cases:
        tok = torch.zeros(1, dtype=torch.int32, device="cuda")
        pos = torch.tensor([5], dtype=torch.int32, device="cuda")
        step = torch.tensor([1], dtype=torch.int32, device="cuda")
        hist = torch.full((4,), -1, dtype=torch.int32, device="cuda")
        h = torch.zeros((1, D), dtype=torch.float16, device="cuda")
        K.decode_advance(dev(lg[None]), tok, pos, hist, step, tb, h, slots=dev(_host_slots(lg)))
        want = int(np.argmax(lg))
        assert int(host(tok)[0]) == want and host(hist)[1] == want
        assert host(pos)[0] == 6 and host(step)[0] == 2
        assert np.array_equal(host(h)[0], table[want])


# ----------------------------------------------------------------------------- MoE
def test_moe_topk_reference_ties(K):
    say("moe top-k tie vectors")
    rows = np.array([[0.2, 0.2, 0.2, 0.1, 0.1, 0.1, 0.05, 0.05],
                     [0.3, 0.2, 0.2, 0.2, 0.05, 0.03, 0.01, 0.01],
                     [0.1, 0.1, 0.1, 0.1, 0.1, 0.1, 0.2, 0.2],
                     [0.4, 0.3, 0.1, 0.1, 0.05, 0.03, 0.01, 0.01]], np.float16)
    # logits whose softmax reproduces the rows exactly up to fp16 rounding: log(p)
    lg = np.log(rows.astype(np.float64)).astype(np.float32)
    gate, sel, cnt, lst = K.moe_topk(dev(lg), 2, renorm=False)
    sel = host(sel)
    want = [[0, 1], [0, 1], [6, 7], [0, 1]]
    assert [sorted(r) for r in sel.tolist()] == want
    cnt = host(cnt)
    assert cnt.tolist() == [3, 3, 0, 0, 0, 0, 1, 1]
    lst = host(lst)
    assert lst[0, :3].tolist() == [0, 2, 6] and lst[6, 0] == 4 and lst[7, 0] == 5


@pytest.mark.parametrize("fmt", ["q4_0", "int8"])
def test_moe_layer_sparse_dispatch(K, fmt):
    say(f"moe layer E=8 k=2 T=16 D=512 F=768 fmt={fmt}")
    from aneforge_amd import _blob
    rng = np.random.default_rng(60)
    E, k, T, D, F = 8, 2, 16, 512, 768
    router = rng.normal(0, 0.2, (E, D)).astype(np.float16)
    h = rng.standard_normal((T, D)).astype(np.float16)
    g = np.ones(D, np.float16)
    Wg = rng.normal(0, 0.05, (E, F, D)).astype(np.float32)
    Wu = rng.normal(0, 0.05, (E, F, D)).astype(np.float32)
    Wd = rng.normal(0, 0.05, (E, D, F)).astype(np.float32)
    if fmt == "q4_0":
        gu, dn, Gf, Uf, Df = [], [], [], [], []
        for e in range(E):
            bg, bu, bd = _blob.quantize_q4_0(Wg[e]), _blob.quantize_q4_0(Wu[e]), _blob.quantize_q4_0(Wd[e])
            # the reference streams these experts as fp16-converted dequantised weights
            Gf.append(ref.dequant_q4_0_f16(bg, F, D)); Uf.append(ref.dequant_q4_0_f16(bu, F, D))
            Df.append(ref.dequant_q4_0_f16(bd, D, F))
            qg, dg = _blob.q4_0_to_superblock(bg, F, D)
            qu, du = _blob.q4_0_to_superblock(bu, F, D)
            gu.append((_blob.interleave_rows(qg, qu), _blob.interleave_rows(dg, du)))
            dn.append(_blob.q4_0_to_superblock(bd, D, F))
        wgu = np.stack([a for a, _ in gu]); sgu = np.stack([b for _, b in gu])
        wdn = np.stack([a for a, _ in dn]); sdn = np.stack([b for _, b in dn])
    else:
        gu, dn, Gf, Uf, Df = [], [], [], [], []
        for e in range(E):
            qg, sg = _blob.quantize_per_row(Wg[e]); qu, su = _blob.quantize_per_row(Wu[e]); qd, sd = _blob.quantize_per_row(Wd[e])
            Gf.append(ref.dequant_w8(qg, sg)); Uf.append(ref.dequant_w8(qu, su)); Df.append(ref.dequant_w8(qd, sd))
            gu.append((_blob.interleave_rows(qg, qu), _blob.interleave_rows(sg, su)))
            dn.append((qd, sd))
        wgu = np.stack([a for a, _ in gu]); sgu = np.stack([b for _, b in gu])
        wdn = np.stack([a for a, _ in dn]); sdn = np.stack([b for _, b in dn])
    hd = dev(h)
    hn = K.rmsnorm(hd, dev(g), 1e-5)
    logits = K.linear("fp16", dev(router), None, hn, out_f32=True) if T <= 8 else torch.cat(
        [K.linear("fp16", dev(router), None, hn[i:i + 8], out_f32=True) for i in range(0, T, 8)])
    gate, sel, cnt, lst = K.moe_topk(logits, k, renorm=True)
    act = K.moe_gateup(fmt, dev(wgu), dev(sgu), hn, k, E, F, cnt, lst)
    y = K.moe_down(fmt, dev(wdn), dev(sdn), act, T, k, E, F, D, cnt, lst)
    out = host(K.moe_combine(hd, y, gate))
    want, wgate, chosen = ref.moe_layer(h, g, router, Gf, Uf, Df, k, True, 1e-5)
    assert [sorted(r) for r in host(sel).tolist()] == chosen
    check_hidden(out, want, what="moe")           # residual-stream output: fp16-ulp atol


@pytest.mark.parametrize("T,E,D,k", [(1, 8, 4096, 2), (5, 4, 256, 1), (16, 8, 4096, 2), (16, 16, 2048, 4),
                                     (9, 16, 4096, 16), (3, 1, 512, 1)])
def test_moe_route_is_norm_router_topk_bit_for_bit(K, T, E, D, k):
    # the one-launch router against the three launches it replaces: hn identical to afx_rmsnorm's,
    # the logits to afx_linear's from 4 rows up (its MFMA path; below 4 rows it sums on the vector
    # kernels, in another order), gate, sel and the buckets to afx_moe_topk's on the same logits
    # (D 2048 takes the 16-wavefront K split, 4096 the 8-wavefront one, 256 / 512 the shortest);
    # two duplicated router rows give exact logit ties for the tie rule
    say(f"moe route T={T} E={E} D={D} k={k}")
    rng = np.random.default_rng(1000 + T * E + k)
    router = rng.normal(0, 0.05, (E, D)).astype(np.float16)
    if E >= 4:
        router[3] = router[1]
    h = (rng.standard_normal((T, D)) * 2).astype(np.float16)
    g = (1 + 0.1 * rng.standard_normal(D)).astype(np.float16)
    hd, gd, rd = dev(h), dev(g), dev(router)
    hn_ref = K.rmsnorm(hd, gd, 1e-5)
    lg_ref = K.linear("fp16", rd, None, hn_ref, out_f32=True)
    assert K.moe_route_supported(hd, rd, k)
    hn = torch.empty_like(hd)
    lg = torch.empty((T, E), dtype=torch.float32, device="cuda")
    gate = torch.empty((T, k), dtype=torch.float32, device="cuda")
    sel = torch.empty((T, k), dtype=torch.int32, device="cuda")
    cnt = torch.empty((E,), dtype=torch.int32, device="cuda")
    lst = torch.empty((E, T), dtype=torch.int32, device="cuda")
    K.moe_route(hd, gd, 1e-5, rd, k, True, hn, gate, sel, cnt, lst, logits=lg)
    assert np.array_equal(host(hn).view(np.uint16), host(hn_ref).view(np.uint16)), "hn"
    if T >= 4:
        assert np.array_equal(host(lg).view(np.uint32), host(lg_ref).view(np.uint32)), "logits"
    else:
        np.testing.assert_allclose(host(lg), host(lg_ref), rtol=1e-5, atol=1e-6)
    gate_ref, sel_ref, cnt_ref, lst_ref = K.moe_topk(lg, k, renorm=True)
    assert np.array_equal(host(gate).view(np.uint32), host(gate_ref).view(np.uint32)), "gate"
    assert np.array_equal(host(sel), host(sel_ref)), "sel"
    c = host(cnt)
    assert np.array_equal(c, host(cnt_ref)), "cnt"
    lr, lw = host(lst), host(lst_ref)
    for e in range(E):
        assert np.array_equal(lr[e, :c[e]], lw[e, :c[e]]), f"list of expert {e}"
    # one workgroup per token (the sync buffer): the same bits, on repeated calls that share the buffer
    # (a smaller batch in between re-aligns its counter) and as graph replays
    sync = K.moe_route_sync()
    outs = [torch.full_like(t, -7) for t in (hn, lg, gate, sel, cnt, lst)]

    def per_token(rows):
        K.moe_route(hd[:rows], gd, 1e-5, rd, k, True, outs[0][:rows], outs[2][:rows], outs[3][:rows], outs[4],
                    outs[5], logits=outs[1][:rows], sync=sync)

    def same(what):
        torch.cuda.synchronize()
        for name, a, b in zip(("hn", "logits", "gate", "sel", "cnt"), outs[:5], (hn, lg, gate, sel, cnt)):
            assert np.array_equal(host(a).view(np.uint8), host(b).view(np.uint8)), f"{what}: {name}"
        lp = host(outs[5])
        for e in range(E):
            assert np.array_equal(lp[e, :c[e]], lr[e, :c[e]]), f"{what}: list of expert {e}"
    per_token(T)
    same("per-token call 1")
    per_token(max(1, T - 2))
    for t_ in outs:
        t_.fill_(-7)
    per_token(T)
    same("per-token call 3 (after a smaller batch)")
    gph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gph):
        per_token(T)
    for rep in range(3):
        for t_ in outs:
            t_.fill_(-7)
        gph.replay()
        same(f"per-token graph replay {rep}")
    assert int(host(sync)[0]) % 16 == 0


@pytest.mark.parametrize("fmt,F,shared", [("q4_0", 14336, False), ("q4_0", 768, True), ("int8", 11008, True)])
def test_moe_down_combine_is_down_then_combine_bit_for_bit(K, fmt, F, shared):
    # F = 14336 / 11008 cut the expert rows into K slices whose finishing sum the fused combine does;
    # F = 768 writes y directly; with a shared expert output added last
    say(f"moe down+combine fmt={fmt} F={F} shared={shared}")
    from aneforge_amd import _blob
    rng = np.random.default_rng(F + len(fmt))
    E, k, T, D = 8, 2, 16, 512
    Wd = rng.normal(0, 0.05, (E, D, F)).astype(np.float32)
    if fmt == "q4_0":
        dn = [_blob.q4_0_to_superblock(_blob.quantize_q4_0(Wd[e]), D, F) for e in range(E)]
    else:
        dn = [_blob.quantize_per_row(Wd[e]) for e in range(E)]
    wdn, sdn = dev(np.stack([a for a, _ in dn])), dev(np.stack([b for _, b in dn]))
    lg = dev(rng.standard_normal((T, E)).astype(np.float32))
    gate, sel, cnt, lst = K.moe_topk(lg, k, renorm=True)
    act = dev((rng.standard_normal((T * k, F)) * 0.5).astype(np.float16))
    h = dev(rng.standard_normal((T, D)).astype(np.float16))
    sh = dev(rng.standard_normal((T, D)).astype(np.float16)) if shared else None
    ws = torch.empty(8 * T * k * D, dtype=torch.float32, device="cuda")
    y = K.moe_down(fmt, wdn, sdn, act, T, k, E, F, D, cnt, lst, ws=ws)
    want = host(K.moe_combine(h, y, gate, shared=sh))
    y2 = torch.empty((T * k, D), dtype=torch.float32, device="cuda")
    got = host(K.moe_down_combine(fmt, wdn, sdn, act, T, k, E, F, D, cnt, lst, y2, h, gate, shared=sh, ws=ws))
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    # in place on h, as the decode engine calls it
    h2 = h.clone()
    K.moe_down_combine(fmt, wdn, sdn, act, T, k, E, F, D, cnt, lst, y2, h2, gate, shared=sh, out=h2, ws=ws)
    assert np.array_equal(host(h2).view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("fmt", ["q4_0", "int8"])
def test_moe_gateup_units_cross_experts_and_skip_empty_ones(K, fmt):
    # 12 tokens top-2 over 5 experts, expert 2 routed no token; 2100 intermediate rows (263
    # tiles per expert): with at most 16 tokens per expert the persistent MFMA kernel gives each
    # workgroup a contiguous range of the active experts' tiles, and the ranges cross experts
    say(f"moe gate/up E=5 (one empty) k=2 T=12 D=1024 F=2100 fmt={fmt}")
    from aneforge_amd import _blob
    rng = np.random.default_rng(75)
    E, k, T, D, F = 5, 2, 12, 1024, 2100
    x = rng.standard_normal((T, D)).astype(np.float16)
    Wg = rng.normal(0, 0.05, (E, F, D)).astype(np.float32)
    Wu = rng.normal(0, 0.05, (E, F, D)).astype(np.float32)
    ws, ss, Gf, Uf = [], [], [], []
    for e in range(E):
        if fmt == "q4_0":
            bg, bu = _blob.quantize_q4_0(Wg[e]), _blob.quantize_q4_0(Wu[e])
            Gf.append(ref.dequant_q4_0_f16(bg, F, D)); Uf.append(ref.dequant_q4_0_f16(bu, F, D))
            qg, dg = _blob.q4_0_to_superblock(bg, F, D)
            qu, du = _blob.q4_0_to_superblock(bu, F, D)
        else:
            qg, dg = _blob.quantize_per_row(Wg[e]); qu, du = _blob.quantize_per_row(Wu[e])
            Gf.append(ref.dequant_w8(qg, dg)); Uf.append(ref.dequant_w8(qu, du))
        ws.append(_blob.interleave_rows(qg, qu)); ss.append(_blob.interleave_rows(dg, du))
    active = [0, 1, 3, 4]
    pick = [rng.choice(active, 2, replace=False) for _ in range(T)]
    cnt = np.zeros(E, np.int32)
    lst = np.zeros((E, T), np.int32)
    for t in range(T):
        for slot, e in enumerate(pick[t]):
            lst[e, cnt[e]] = t * k + slot
            cnt[e] += 1
    assert cnt[2] == 0 and cnt.max() <= 16
    act = host(K.moe_gateup(fmt, dev(np.stack(ws)), dev(np.stack(ss)), dev(x), k, E, F, dev(cnt), dev(lst)))
    for t in range(T):
        for slot, e in enumerate(pick[t]):
            g = ref.linear(x[t:t + 1], Gf[e])
            u = ref.linear(x[t:t + 1], Uf[e])
            check_f16(act[t * k + slot:t * k + slot + 1], ref.r16(ref.silu(g) * u), what=f"token {t} expert {e}")


def test_moe_gateup_many_experts_few_active(K):
    # 600 experts, 24 of them routed: the persistent MFMA kernel compacts the active experts
    # into LDS over several rounds of the whole workgroup (512 threads per round)
    say("moe gate/up E=600 (24 active) k=2 T=12 D=1024 F=64 int8")
    rng = np.random.default_rng(76)
    E, k, T, D, F = 600, 2, 12, 1024, 64
    q = rng.integers(-127, 128, (E, 2 * F, D), dtype=np.int8)                 # gate/up rows interleaved
    s = (np.abs(rng.normal(0, 0.02, (E, 2 * F))) / 127).astype(np.float16)
    x = rng.standard_normal((T, D)).astype(np.float16)
    active = rng.choice(E, 24, replace=False)
    pick = [rng.choice(active, 2, replace=False) for _ in range(T)]
    cnt = np.zeros(E, np.int32)
    lst = np.zeros((E, T), np.int32)
    for t in range(T):
        for slot, e in enumerate(pick[t]):
            lst[e, cnt[e]] = t * k + slot
            cnt[e] += 1
    act = host(K.moe_gateup("int8", dev(q), dev(s), dev(x), k, E, F, dev(cnt), dev(lst)))
    for t in range(T):
        for slot, e in enumerate(pick[t]):
            W = ref.dequant_w8(q[e], s[e])
            g, u = ref.linear(x[t:t + 1], W[0::2]), ref.linear(x[t:t + 1], W[1::2])
            check_f16(act[t * k + slot:t * k + slot + 1], ref.r16(ref.silu(g) * u), what=f"token {t} expert {e}")


def test_moe_topk_largest_expert_count_with_ties(K):
    # E = 2049 (the reference's upper bound) and k = 64: probabilities on power-of-two levels with
    # many exact ties, so the lowest-index rule decides most picks
    say("moe top-k E=2049 k=64 with ties")
    rng = np.random.default_rng(70)
    T, E, k = 3, 2049, 64
    levels = rng.integers(1, 12, (T, E))
    lg = np.log(2.0 ** -levels.astype(np.float64)).astype(np.float32)
    gate, sel, cnt, lst = K.moe_topk(dev(lg), k, renorm=False)
    p = np.exp(lg.astype(np.float64) - lg.max(1, keepdims=True).astype(np.float64))
    p16 = (p / p.sum(1, keepdims=True)).astype(np.float16)
    want = ref.topk_gate(p16, k)
    got_sel = host(sel)
    for t in range(T):
        assert sorted(got_sel[t].tolist()) == np.flatnonzero(want[t]).tolist(), f"token {t}"
    np.testing.assert_allclose(host(gate), np.take_along_axis(want, got_sel.astype(np.int64), 1), rtol=1e-3)
    c = host(cnt)
    assert c.sum() == T * k and c.max() <= T


@pytest.mark.parametrize("fmt", ["int8", "q4_0"])
def test_moe_expert_with_more_than_16_tokens(K, fmt):
    # 40 tokens, 2 experts, top-1: an expert receives > 16 tokens, so the MFMA kernel runs
    # several token groups over the same weights
    say(f"moe E=2 k=1 T=40 D=F=1024 fmt={fmt}")
    from aneforge_amd import _blob
    rng = np.random.default_rng(71)
    E, k, T, D, F = 2, 1, 40, 1024, 1024
    router = rng.normal(0, 0.2, (E, D)).astype(np.float16)
    h = rng.standard_normal((T, D)).astype(np.float16)
    g = np.ones(D, np.float16)
    Wg = rng.normal(0, 0.05, (E, F, D)).astype(np.float32)
    Wu = rng.normal(0, 0.05, (E, F, D)).astype(np.float32)
    Wd = rng.normal(0, 0.05, (E, D, F)).astype(np.float32)
    gu, dn, Gf, Uf, Df = [], [], [], [], []
    for e in range(E):
        if fmt == "q4_0":
            bg, bu, bd = _blob.quantize_q4_0(Wg[e]), _blob.quantize_q4_0(Wu[e]), _blob.quantize_q4_0(Wd[e])
            Gf.append(ref.dequant_q4_0_f16(bg, F, D)); Uf.append(ref.dequant_q4_0_f16(bu, F, D))
            Df.append(ref.dequant_q4_0_f16(bd, D, F))
            qg, dg = _blob.q4_0_to_superblock(bg, F, D)
            qu, du = _blob.q4_0_to_superblock(bu, F, D)
            gu.append((_blob.interleave_rows(qg, qu), _blob.interleave_rows(dg, du)))
            dn.append(_blob.q4_0_to_superblock(bd, D, F))
        else:
            qg, sg = _blob.quantize_per_row(Wg[e]); qu, su = _blob.quantize_per_row(Wu[e]); qd, sd = _blob.quantize_per_row(Wd[e])
            Gf.append(ref.dequant_w8(qg, sg)); Uf.append(ref.dequant_w8(qu, su)); Df.append(ref.dequant_w8(qd, sd))
            gu.append((_blob.interleave_rows(qg, qu), _blob.interleave_rows(sg, su)))
            dn.append((qd, sd))
    wgu = np.stack([a for a, _ in gu]); sgu = np.stack([b for _, b in gu])
    wdn = np.stack([a for a, _ in dn]); sdn = np.stack([b for _, b in dn])
    hd = dev(h)
    hn = K.rmsnorm(hd, dev(g), 1e-5)
    logits = torch.cat([K.linear("fp16", dev(router), None, hn[i:i + 8], out_f32=True) for i in range(0, T, 8)])
    gate, sel, cnt, lst = K.moe_topk(logits, k, renorm=True)
    assert host(cnt).max() > 16
    act = K.moe_gateup(fmt, dev(wgu), dev(sgu), hn, k, E, F, cnt, lst)
    y = K.moe_down(fmt, dev(wdn), dev(sdn), act, T, k, E, F, D, cnt, lst)
    out = host(K.moe_combine(hd, y, gate))
    want, _, chosen = ref.moe_layer(h, g, router, Gf, Uf, Df, k, True, 1e-5)
    assert [sorted(r) for r in host(sel).tolist()] == chosen
    check_hidden(out, want, what="moe >16 tokens")
