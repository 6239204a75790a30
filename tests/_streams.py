"""Stream checks against the oracle (a helper of the GPU parity tests).

A decoded stream is checked decision by decision.  The oracle runs one all-row forward
over the prompt followed by the codes the HIP path produced (teacher forcing): its row i
holds the logits that predict codes[i] from the prompt and codes[:i].  Those rows equal
the oracle's own prefill + step logits along that prefix (the oracle's prefill/step
self-consistency is bit-exact, tests/test_oracle_model.py), so replaying the oracle's
sampler on them (sampler.rs:191-284; seen set from codes[:i], STOP masked while fewer
than min_codes codes exist, sampler.rs:372-376; the RNG state carried from decision to
decision, one draw per sampled decision) gives the reference's decision at every step of
the stream, not only up to a first divergence.

A decision may differ from the oracle's only where the oracle's own decision changes
under a logit perturbation no larger than eps, a bound on the HIP-vs-oracle logit
difference the same test measures on decode steps at these contexts: the HIP token must
be what the oracle's sampler picks from some perturbed copy of the oracle's logits
(perturbations aimed at the token: raising it, moving the cumulative probability at its
rank either way, or swapping it with a neighbour in the sampler's order).
"""
import numpy as np

import ito


def oracle_rows(M, prompt, codes, kv_bf16, max_seq=2048):
    """[len(codes)][mel_vocab]: row i = the oracle's logits predicting codes[i]."""
    codes = np.ascontiguousarray(codes, np.int32)
    emb = M.sequence_embedding(prompt.text_tokens, prompt.conds, prompt.lang_id, codes[:-1])
    row0 = emb.shape[0] - len(codes)  # the START_MEL row
    return M.forward_rows(M.kv(max_seq, kv_bf16=kv_bf16), emb, row0)


def _decide(row, seen, params, state, mask_stop, stop):
    x = np.array(row, dtype=np.float32, copy=True)
    if mask_stop:
        x[stop] = -np.inf
    return ito.sample_next_token(x, seen, params, state)


def _penalised_order(row, seen_words, params, stop, mask_stop):
    """Token ids by descending penalised logit (sampler.rs:138-157 applied in numpy), the
    order the sampler's top-k list takes; used only to aim perturbations, the decision
    itself is always the oracle's."""
    x = np.array(row, dtype=np.float64, copy=True)
    if mask_stop:
        x[stop] = -np.inf
    p = float(params.repetition_penalty)
    ids = np.nonzero(np.unpackbits(seen_words.view(np.uint8), bitorder="little"))[0]
    ids = ids[ids < len(x)]
    x[ids] = np.where(x[ids] < 0, x[ids] * p, x[ids] / p)
    return np.argsort(-x, kind="stable")


def _patterns(row, seen, params, stop, mask_stop, tok):
    """Sign patterns that move the sampler's decision toward tok: raise tok, raise or lower
    the candidates ranked before and after it so that the cumulative probability at tok's
    place moves in either direction, and swap tok with a neighbour in the order."""
    n = len(row)
    order = _penalised_order(row, seen, params, stop, mask_stop)
    k = n if params.top_k == 0 else min(int(params.top_k), n)
    rank = int(np.nonzero(order == tok)[0][0])
    top = order[: max(k, rank + 1)]
    pats = []
    s = np.zeros(n, np.float32)
    s[tok] = 1
    pats.append(s)
    s = -np.ones(n, np.float32)
    s[tok] = 1
    pats.append(s)
    for before in (1.0, -1.0):
        s = np.zeros(n, np.float32)
        s[top[:rank]] = before
        s[top[rank:]] = -before
        s[tok] = 1
        pats.append(s)
    # order swaps with the neighbours: the draw falls at the same cumulative position, but
    # the slot there changes owner when two near-equal candidates trade places
    for j in (rank - 2, rank - 1, rank + 1, rank + 2):
        if 0 <= j < len(top) and top[j] != tok:
            for sg in (1.0, -1.0):
                s = np.zeros(n, np.float32)
                s[tok] = sg
                s[top[j]] = -sg
                pats.append(s)
    return pats


def min_perturbation(row, seen, params, state, mask_stop, stop, tok, limit=0.5):
    """The smallest eps (to within a factor 1.25) for which one of the aimed sign patterns,
    scaled by eps, makes the oracle's sampler pick tok from the same seen set and RNG
    state; inf if none does up to limit.  The decision is not monotone in eps (a large
    swap carries tok past its neighbours), so eps is scanned upward on a geometric grid."""
    base = np.asarray(row, dtype=np.float32)
    pats = _patterns(row, seen, params, stop, mask_stop, tok)
    e = 1e-7
    while e <= limit:
        for s in pats:
            t, _ = _decide(base + np.float32(e) * s, seen, params, state, mask_stop, stop)
            if t == tok:
                return e
        e *= 1.25
    return np.inf


def replay_stream(rows, codes, params, state, min_codes, stop, eps, report=None):
    """Replays every decision of a stream on the oracle rows.  Returns (mismatched steps,
    unexplained steps, RNG state after the last decision); a mismatch is explained when a
    perturbation of at most eps per logit turns the oracle's decision into the stream's.
    report(step, eps_needed) is called for every mismatch."""
    seen = ito.seen_init(stop - 1)
    mism, unexplained = [], []
    for i, tok in enumerate(np.asarray(codes).tolist()):
        mask = i < min_codes
        t, nxt = _decide(rows[i], seen, params, state, mask, stop)
        if t != tok:
            mism.append(i)
            need = min_perturbation(rows[i], seen, params, state, mask, stop, tok)
            if report:
                report(i, need)
            if not need <= eps:
                unexplained.append(i)
        state = nxt
        ito.lib.ito_seen_insert(ito._p(seen), int(tok))
    return mism, unexplained, state


def step_checkpoint(g, kv, prompt, codes, rows, c, n_steps):
    """HIP prefill_after with codes[:c] as prior codes, then n_steps decode steps with the
    next codes at their positions (code i sits at Mel position i + 2, gpt.rs:618-625).
    Returns the max |logit difference| to the oracle rows of each call and the key count
    of the last step."""
    a = g.prefill_after(prompt.text_tokens, prompt.conds, prompt.lang_id, np.asarray(codes[:c], np.int32), kv)
    errs = [float(np.abs(a - rows[c]).max())]
    for i in range(n_steps):
        a = g.step(kv, int(codes[c + i]), c + i + 2)
        errs.append(float(np.abs(a - rows[c + i + 1]).max()))
    return errs, kv.valid_len()
