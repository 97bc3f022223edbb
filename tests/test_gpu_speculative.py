"""Speculative decoding (aneforge/speculative.py:131-165; the reference's tests/test_speculative.py):
greedy, so it emits target.generate's tokens for any draft, and an identical draft is accepted in
bulk (far fewer target passes than tokens)."""
import numpy as np
import pytest

from _util import say
from oracle import ref

pytestmark = pytest.mark.gpu


def _model(cfg, seed, compress=None):
    from aneforge_amd.llm import LlamaPrefill
    from test_gpu_llm import _random_weights
    return LlamaPrefill(cfg, _random_weights(cfg, seed=seed), compress=compress)


def test_spec_generate_matches_greedy_row_by_row_verify():
    # head dim 16 has no batched path: the target verifies with forced decode steps, the same
    # kernels generate() uses, so the tokens must be identical
    from aneforge_amd.llm import LlamaConfig
    from aneforge_amd.speculative import spec_generate
    say("spec_generate vs generate, dh=16 (row-by-row verify)")
    cfg = LlamaConfig(dim=64, n_layers=2, n_heads=4, n_kv_heads=2, ffn_dim=128, vocab=48)
    tgt, drf = _model(cfg, 0), _model(cfg, 1)              # a different draft exercises rejection
    prompt = [1, 2, 3, 4]
    g = tgt.generate(list(prompt), max_new_tokens=12, max_len=40)
    s = spec_generate(tgt, drf, prompt, max_new_tokens=12, max_len=40, n_draft=3)
    assert g == s, f"spec != greedy:\n  greedy {g}\n  spec   {s}"


@pytest.mark.parametrize("compress", [None, "int8"])
def test_spec_generate_batched_verify_matches_oracle(compress):
    # head dim 128: the target verifies n_draft + 1 rows with the prefill kernels
    from aneforge_amd.llm import LlamaConfig
    from aneforge_amd.speculative import spec_generate
    from test_gpu_llm import _assert_tokens_match, _effective, _ocfg, _random_weights
    say(f"spec_generate with batched verify, dh=128 compress={compress}")
    cfg = LlamaConfig(dim=256, n_layers=2, n_heads=2, n_kv_heads=1, ffn_dim=512, vocab=128)
    w = _random_weights(cfg, seed=3)
    from aneforge_amd.llm import LlamaPrefill
    tgt = LlamaPrefill(cfg, w, compress=compress)
    assert tgt._decoder(64).prefill_supported()
    drf = _model(LlamaConfig(dim=256, n_layers=1, n_heads=2, n_kv_heads=1, ffn_dim=256, vocab=128), 4, compress)
    prompt = [5, 17, 33, 2, 99]
    s = spec_generate(tgt, drf, prompt, max_new_tokens=16, max_len=64, n_draft=4)
    want, lgs = ref.generate(prompt, 16, _effective(w, compress), _ocfg(cfg), M=len(prompt) + 16)
    _assert_tokens_match(s, want, lgs, f"spec compress={compress}")
    g = tgt.generate(prompt, max_new_tokens=16, max_len=64)
    _assert_tokens_match(g, want, lgs, f"greedy compress={compress}")


@pytest.mark.parametrize("dim,heads", [(64, 4), (256, 2)])
def test_identical_draft_is_accepted_in_bulk(monkeypatch, dim, heads):
    from aneforge_amd import speculative as sp
    from aneforge_amd.llm import LlamaConfig
    say(f"spec_generate with draft == target, dim={dim}")
    cfg = LlamaConfig(dim=dim, n_layers=2, n_heads=heads, n_kv_heads=heads // 2 or 1, ffn_dim=2 * dim, vocab=48)
    tgt, drf = _model(cfg, 0), _model(cfg, 0)
    calls = {"n": 0}
    real = sp._verify

    def counting(*a, **k):
        calls["n"] += 1
        return real(*a, **k)

    monkeypatch.setattr(sp, "_verify", counting)
    out = sp.spec_generate(tgt, drf, [1, 2, 3, 4], max_new_tokens=16, max_len=48, n_draft=3)
    g = tgt.generate([1, 2, 3, 4], max_new_tokens=16, max_len=48)
    assert len(out) == 16
    if dim == 64:
        assert out == g
    assert calls["n"] < len(out) // 2, f"{calls['n']} target passes for {len(out)} tokens"


def test_spec_generate_eos_and_streaming():
    from aneforge_amd.llm import LlamaConfig
    from aneforge_amd.speculative import spec_generate
    say("spec_generate eos + on_token")
    cfg = LlamaConfig(dim=64, n_layers=2, n_heads=4, n_kv_heads=2, ffn_dim=128, vocab=48)
    tgt, drf = _model(cfg, 0), _model(cfg, 1)
    full = tgt.generate([1, 2, 3, 4], max_new_tokens=10, max_len=40)
    eos = full[5]
    seen = []
    s = spec_generate(tgt, drf, [1, 2, 3, 4], max_new_tokens=10, max_len=40, n_draft=3, eos_id=eos,
                      on_token=seen.append)
    stop = full.index(eos)
    assert s == full[:stop + 1] and seen == full[:stop]
    with pytest.raises(ValueError):
        spec_generate(tgt, drf, [], max_new_tokens=4)
