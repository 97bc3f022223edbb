"""Greedy speculative decoding (aneforge/speculative.py:131-165): a small draft model proposes
`n_draft` tokens, the target checks all of them in one pass over its resident KV cache, and the
matching prefix plus one correction is emitted.  The result equals target.generate(...) token for
token (greedy); only the number of target passes changes.

Here both models run on the device: the draft proposes with its greedy step graph (no host
round trip between proposals), and the target verifies the `n_draft + 1` rows with the batched
prefill kernels (MFMA GEMMs and causal flash attention from position p over the cache), or with
one forced decode step per row for layers that have no batched path.  Rejected cache rows are
simply overwritten by the next pass, as in the reference."""
from __future__ import annotations

__all__ = ["spec_generate"]


def _verify(target_engine, toks, pos0):
    """Target greedy next tokens after each of `toks` fed at positions pos0.. (one pass)."""
    return target_engine.verify(toks, pos0)


def spec_generate(target, draft, token_ids, max_new_tokens=40, eos_id=None, max_len=None, n_draft=4,
                  on_token=None):
    """Greedy speculative decoding with the reference's signature and result: `draft` proposes
    `n_draft` tokens, `target` verifies them in one pass, the matching prefix + 1 correction is
    emitted.  Both models share the tokenizer / vocab."""
    prompt = [int(t) for t in token_ids]
    if not prompt:
        raise ValueError("spec_generate needs at least one prompt token")
    if int(n_draft) < 1:
        raise ValueError(f"n_draft must be >= 1, got {n_draft}")
    n_draft = int(n_draft)
    M = int(max_len or len(prompt) + max_new_tokens)
    Kq = n_draft + 1
    P = len(prompt)
    if target.cfg.vocab != draft.cfg.vocab:
        raise ValueError(f"target and draft vocabularies differ ({target.cfg.vocab} vs {draft.cfg.vocab})")
    if P + 1 > M:
        raise ValueError(f"a {P}-token prompt leaves no room in max_len={M}")
    dt = target._decoder(M)
    dd = draft.warmup(M)._dec
    # target: cache rows for prompt[:-1], then the first token from the last prompt row
    dt.prefill(prompt)
    cur = int(_verify(dt, [prompt[-1]], P - 1)[0])
    out = [cur]
    if on_token is not None and cur != eos_id:
        on_token(cur)
    if cur == eos_id or max_new_tokens <= 1:
        return out[:max_new_tokens]
    # draft: cache rows for the whole prompt, then `cur` pending at position P
    dd.prefill(prompt)
    dd.force_next(P - 1, cur)
    dd.run(1, 0)
    p = P                                       # position of `cur`
    while len(out) < max_new_tokens and p + Kq < M:
        dd.run(0, n_draft)                      # greedy proposals from `cur`, recorded at hist[p..]
        drafts = dd.history(p, n_draft)
        am = _verify(dt, [cur] + drafts, p)
        a = 0
        while a < n_draft and int(am[a]) == drafts[a]:
            a += 1
        emit = drafts[:a] + [int(am[a])]
        for t in emit:
            if len(out) >= max_new_tokens:
                break
            out.append(t)
            if on_token is not None and t != eos_id:
                on_token(t)
            if t == eos_id:
                return out
        cur = emit[-1]
        # the draft cache holds [cur, drafts[:a]] at p..p+a when a < n_draft; when every proposal
        # was accepted, the last proposal still has to be fed at p + n_draft
        if a < n_draft:
            dd.seek(p + a + 1, cur)
        else:
            dd.seek(p + n_draft, drafts[-1])
            dd.force_next(p + n_draft, cur)
            dd.run(1, 0)
        p += a + 1
    return out[:max_new_tokens]
