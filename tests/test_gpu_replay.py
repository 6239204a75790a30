"""Teacher-forced replay on the HIP path against the oracle, through the C ABI:
Gpt::teacher_forced / code_log_probs / alignment_attention (gpt.rs:756-915) and the
batched all-row forward.  Log-probabilities are log_softmax of the oracle's all-row logits
(gpt.rs:846-848) picked at the codes; attention maps are the oracle's probes averaged over
the alignment heads (gpt.rs:849-851)."""
import sys

import numpy as np
import pytest

import ito
import itts_hip as H
from itts_hip import synth

pytestmark = pytest.mark.gpu

TIGHT = 2e-4     # logits / log-probs (fp32 on both sides, different summation order)
PROB_TOL = 2e-5  # attention probabilities


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def log_softmax_pick(logits, codes):
    x = logits.astype(np.float64)
    x = x - x.max(1, keepdims=True)
    lp = x - np.log(np.exp(x).sum(1, keepdims=True))
    return lp[np.arange(len(codes)), codes]


@pytest.fixture(scope="module")
def tiny():
    say("[gpu] tiny decoder for replay")
    W = synth.make_weights(synth.SMALL_CONFIG, seed=5, init="rich")
    g = H.Gpt(W)
    g.set_alignment_heads([(1, 2), (3, 0)])
    yield W, g, ito.Model(W)
    g.close()


def _oracle_replay(M, W, pr, fed, n_layers, probes, row0):
    emb = M.sequence_embedding(pr.text_tokens, pr.conds, pr.lang_id, fed)
    return M.replay(M.kv(2048, kv_bf16=False), emb, n_layers=n_layers, probes=probes, row0=row0)


@pytest.mark.parametrize("n_text,n_codes", [(10, 1), (12, 40), (60, 200)])
def test_teacher_forced_matches_oracle(tiny, n_text, n_codes):
    W, g, M = tiny
    say(f"[gpu] teacher_forced n_text={n_text} n_codes={n_codes}")
    pr = synth.make_prompt(W.cfg, 3, n_text, seed=n_codes)
    codes = np.random.default_rng(n_codes).integers(0, W.cfg["mel_vocab"] - 2, n_codes).astype(np.int32)
    kv = g.kv_cache(1024)
    lp, att = g.teacher_forced(pr.text_tokens, pr.conds, pr.lang_id, codes, kv)
    assert kv.valid_len() == 0
    text_lo, text_hi = 3, 3 + n_text + 2
    lg, maps = _oracle_replay(M, W, pr, codes[:-1], W.cfg["n_layer"],
                              [(1, 2, text_hi, text_lo, text_hi), (3, 0, text_hi, text_lo, text_hi)], text_hi)
    ref_lp = log_softmax_pick(lg, codes)
    assert np.abs(lp - ref_lp).max() < TIGHT
    ref_att = (maps[0] + maps[1]) / 2
    assert att.shape == ref_att.shape == (n_codes, n_text + 2)
    assert np.abs(att - ref_att).max() < PROB_TOL
    # code_log_probs is the same replay without the attention export
    lp2 = g.code_log_probs(pr.text_tokens, pr.conds, pr.lang_id, codes, kv)
    assert np.array_equal(lp, lp2)


def test_code_log_probs_consistent_with_prefill(tiny):
    """log_probs[i] = log_softmax(prefill_after(codes[:i]) logits)[codes[i]] on the HIP path."""
    W, g, M = tiny
    pr = synth.make_prompt(W.cfg, 3, 9, seed=4)
    codes = np.array([7, 300, 12, 999, 5], np.int32)
    lp = g.code_log_probs(pr.text_tokens, pr.conds, pr.lang_id, codes, g.kv_cache(256))
    for i in range(len(codes)):
        lg = g.prefill_after(pr.text_tokens, pr.conds, pr.lang_id, codes[:i], g.kv_cache(256, H.ITTS_F32))
        assert abs(log_softmax_pick(lg[None], codes[i:i + 1])[0] - lp[i]) < TIGHT


@pytest.mark.parametrize("n_prior", [0, 7])
def test_alignment_attention_matches_oracle(tiny, n_prior):
    W, g, M = tiny
    say(f"[gpu] alignment_attention n_prior={n_prior}")
    pr = synth.make_prompt(W.cfg, 3, 15, seed=9)
    rng = np.random.default_rng(n_prior)
    prior = rng.integers(0, 1000, n_prior).astype(np.int32)
    codes = rng.integers(0, 1000, 25).astype(np.int32)
    kv = g.kv_cache(512)
    att = g.alignment_attention(pr.text_tokens, pr.conds, pr.lang_id, prior, codes, kv)
    text_lo, text_hi = 3, 3 + 15 + 2
    q0 = text_hi + n_prior
    fed = np.concatenate([prior, codes[:-1]]).astype(np.int32)
    _, maps = _oracle_replay(M, W, pr, fed, 4, [(1, 2, q0, text_lo, text_hi), (3, 0, q0, text_lo, text_hi)], None)
    assert att.shape == (25, 17)
    assert np.abs(att - (maps[0] + maps[1]) / 2).max() < PROB_TOL


def test_forward_logits_batch_matches_oracle(tiny):
    W, g, M = tiny
    say("[gpu] forward_logits batch of 3")
    prompts, refs = [], []
    for b, (n_text, n_prior, lang) in enumerate([(20, 0, 1), (5, 30, 3), (33, 4, 0)]):
        pr = synth.make_prompt(W.cfg, 3, n_text, seed=50 + b)
        prior = np.random.default_rng(b).integers(0, 1000, n_prior).astype(np.int32)
        prompts.append(H.CodePrompt(pr.text_tokens, pr.conds, lang, prior))
        emb = M.sequence_embedding(pr.text_tokens, pr.conds, lang, prior)
        refs.append(M.forward_rows(M.kv(2048, kv_bf16=False), emb, 0))
    got = g.forward_logits(prompts)
    ref = np.concatenate(refs)
    assert got.shape == ref.shape
    assert np.abs(got - ref).max() < TIGHT


def test_replay_validation(tiny):
    W, g, M = tiny
    pr = synth.make_prompt(W.cfg, 3, 8, seed=6)
    kv = g.kv_cache(64)
    with pytest.raises(H.ValidationError) as e:
        g.teacher_forced(pr.text_tokens, pr.conds, pr.lang_id, [], kv)
    assert e.value.message.startswith("codes")
    with pytest.raises(H.ValidationError):
        g.teacher_forced(pr.text_tokens, pr.conds, pr.lang_id, [W.cfg["mel_vocab"]], kv)
    with pytest.raises(H.CapacityError):
        g.code_log_probs(pr.text_tokens, pr.conds, pr.lang_id, np.zeros(60, np.int32), kv)
    with pytest.raises(H.ValidationError):
        g.set_alignment_heads([(4, 10)])     # the small model has 4 layers
    g2 = H.Gpt(W)                             # default heads (4, 10), (5, 10) need 6 layers
    try:
        with pytest.raises(H.ValidationError) as e:
            g2.teacher_forced(pr.text_tokens, pr.conds, pr.lang_id, [1, 2], g2.kv_cache(64))
        assert e.value.message.startswith("alignment_heads")
        lp = g2.code_log_probs(pr.text_tokens, pr.conds, pr.lang_id, [1, 2], g2.kv_cache(64))
        assert lp.shape == (2,)
    finally:
        g2.close()


@pytest.mark.parametrize("kvt", [H.ITTS_BF16, H.ITTS_F32])
def test_long_prefill_flash_attention_matches_oracle(tiny, kvt):
    """Prompts above 384 rows take the MFMA flash attention in prefill (cache K/V read as
    bf16 or fp32): logits and the cache match the oracle, and decode continues from it."""
    W, g, M = tiny
    say(f"[gpu] long prefill (flash attention) kv={kvt}")
    pr = synth.make_prompt(W.cfg, 3, 100, seed=77)
    prior = np.random.default_rng(7).integers(0, 1000, 450).astype(np.int32)
    kv = g.kv_cache(1024, kvt)
    okv = M.kv(1024, kv_bf16=kvt == H.ITTS_BF16)
    a = g.prefill_after(pr.text_tokens, pr.conds, pr.lang_id, prior, kv)
    b = M.prefill_after(okv, pr.text_tokens, pr.conds, pr.lang_id, prior)
    assert kv.valid_len() == okv.valid_len() == 3 + 100 + 3 + 450
    tol = TIGHT if kvt == H.ITTS_F32 else 2e-3
    assert np.abs(a - b).max() < tol
    for t in (5, 17):
        a = g.step(kv, t, 452 + t)
        b = M.step(okv, t, 452 + t)
        assert np.abs(a - b).max() < tol
