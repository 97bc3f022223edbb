"""The C-ABI library loads and exports exactly what include/aneforge_hip.h declares, and the
ctypes table agrees with the header (no compute calls; runs without a GPU)."""
import re
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "aneforge_hip.h"


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?[\w\s\*]*?\b(afx_\w+)\s*\(", text, flags=re.M)


def test_header_declares_the_binding_table():
    from aneforge_amd import _hip
    decl = _declared()
    assert len(decl) == len(set(decl))
    assert sorted(decl) == sorted(_hip.exported_symbols())


def test_library_exports_every_declared_symbol():
    from aneforge_amd import _hip
    lib = _hip.load()
    for name in _declared():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(_hip.lib_path())], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (afx_\w+)", out))
    assert set(_declared()) <= exported
    assert lib.afx_abi_version() == 2


def test_argument_counts_match_header():
    from aneforge_amd import _hip
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    for name, (_, args) in _hip.SIGNATURES.items():
        m = re.search(rf"\b{name}\s*\(([^)]*)\)", text)
        assert m, name
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(params) == len(args), f"{name}: header {len(params)} args, ctypes {len(args)}"


def test_errors_surface_as_runtime_error_without_a_gpu():
    # argument validation happens on the host before any launch
    import pytest
    from aneforge_amd import _hip
    with pytest.raises(RuntimeError, match="unknown weight format"):
        _hip.call("afx_linear", 7, None, None, None, 8, None, 8, 1, 8, 8, None, None, 0, 0, None, 0, None)
    with pytest.raises(RuntimeError, match="need 1 <= k <= E"):
        # non-null dummy addresses: validation rejects k before anything is dereferenced
        _hip.call("afx_moe_topk", 256, 1, 8, 9, 1, 256, 256, 256, 256, None)
    assert "k <= E" in _hip.last_error()


def test_attention_workspace_sizes_and_their_errors_without_a_gpu():
    # the workspace query is host arithmetic: a head dim outside {8..256} and a cache too long for the
    # requested split size are told apart
    import pytest
    from aneforge_amd import _kernels as K
    n = K.attn_ws_bytes(1, 32, 8, 128, 2048)
    assert n > 0 and n % 4 == 0
    assert K.attn_ws_bytes(16, 32, 8, 128, 8192) > n
    with pytest.raises(ValueError, match="head dim"):
        K.attn_ws_bytes(1, 32, 8, 100, 2048)
    with pytest.raises(ValueError, match="128 splits"):
        K.attn_ws_bytes(1, 32, 8, 128, 8192, nstep_hint=1)
    # the split size: fewest dispatch rounds over 256 CUs times the chunk.  ctx 2048: 64-position
    # chunks, 32 splits x 8 kv heads = one round; the 7B engine's 2184-row cache: 80-position chunks
    # (28 splits, 224 workgroups) rather than 64 (35 splits, 280 workgroups, a second round); B=16 at
    # ctx 8192 ties every chunk of 4..16 steps and takes 8 steps (128 positions, 64 splits), not 16
    part = lambda nsp: 32 * nsp * (128 + 2) * 4
    assert n == part(32)
    assert K.attn_ws_bytes(1, 32, 8, 128, 2184) == part(28)
    assert K.attn_ws_bytes(1, 32, 8, 128, 2184, nstep_hint=4) == part(36)   # 35 splits, padded to 4
    assert K.attn_ws_bytes(16, 32, 8, 128, 8192) == 16 * part(64)


def test_sampler_workspace_size_and_its_check_without_a_gpu():
    # fp64 terms for V logits (padded to 256 bytes), a 64-byte header (largest key, total mass,
    # window), then per 2048-logit chunk: its sum (fp64), 256 suffix masses (fp64), 256 suffix counts
    # (u32), its window offset (u32, one more) and its largest key (u32); and a 65536-logit window
    # (key, index, fp64 term)
    import pytest
    from aneforge_amd import _hip, _kernels as K
    lib = _hip.load()
    for V in (1, 8, 2048, 2049, 32000, 151936):
        nb = -(-V // 2048)
        assert lib.afx_sample_ws_bytes(V) == (-(-V * 8 // 256) * 256 + 64 + nb * (8 + 256 * 8 + 256 * 4)
                                              + (nb + 1) * 4 + 65536 * (8 + 4 + 4) + nb * 4)
    assert lib.afx_sample_ws_bytes(0) == -1
    assert K.sample_ws_elems(32000) * 8 >= lib.afx_sample_ws_bytes(32000)
    # a workspace of V doubles (the old contract) is now too small: rejected before any launch
    with pytest.raises(RuntimeError, match="afx_sample_ws_bytes"):
        _hip.call("afx_sample", 256, 32000, 256, 256, None, None, None, 256, 256, 32000 * 8, None)


def test_noalloc_attention_rejects_shapes_beyond_its_scratch_without_a_gpu():
    # the size check is host arithmetic before any device call: 64 sequences of 32 heads at 8192
    # positions (16-step chunks: 32 splits) need 34 MB of split partials, more than the 32 MiB array
    import pytest
    from aneforge_amd import _hip
    with pytest.raises(RuntimeError, match="scratch array"):
        _hip.call("afx_decode_attn_noalloc", 256, 256, 256, 256, 32 * 128, 128, 8 * 8192 * 128, 8192 * 128,
                  64, 32, 8, 128, 8192, None, 8192, None, 0, -1, 0.088, 16, None)
    with pytest.raises(RuntimeError, match="head dim"):
        _hip.call("afx_decode_attn_noalloc", 256, 256, 256, 256, 32 * 100, 100, 8 * 64 * 100, 64 * 100,
                  1, 32, 8, 100, 64, None, 64, None, 0, -1, 0.1, 0, None)


def test_fused_moe_router_rejects_batches_beyond_one_workgroup_without_a_gpu():
    # the shape checks are host arithmetic before any launch (non-null dummy addresses)
    import pytest
    from aneforge_amd import _hip
    with pytest.raises(RuntimeError, match="T <= 16"):
        _hip.call("afx_moe_route", 256, 4096, 256, 1e-5, 256, 17, 8, 4096, 2, 1, 256, 4096, None, 256, 256, 256,
                  256, None, None)
    with pytest.raises(RuntimeError, match="multiple of 32"):
        _hip.call("afx_moe_route", 256, 8192, 256, 1e-5, 256, 4, 8, 8192, 2, 1, 256, 8192, None, 256, 256, 256,
                  256, None, None)
