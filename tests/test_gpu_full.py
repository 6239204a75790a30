"""Parity at the decoder's real shape, through the C ABI: 24 layers, d_model 1280, 20
heads x 64, FFN 5120, 8194 Mel ids, int8 MLX-affine group-64 weights with fp16 params,
seeded spec init (N(0, 0.02) linears, N(0, 0.02) tables).  The HIP path (prefill GEMMs,
persistent or multi-kernel decode step, device sampler) is checked against the oracle on
the same inputs: logits within the workload's 2e-2 max-abs bar, and greedy ids (repetition
penalty 10, STOP masked) identical over the decode as the reference's greedy-codes test
asks (sampler.rs:487-536) - exactly with fp32 caches, and wherever the decision margin
exceeds the numeric noise with bf16 caches."""
import sys

import numpy as np
import pytest

import ito
import itts_hip as H
from itts_hip import synth

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-2


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def full(full_model):
    return full_model


@pytest.mark.parametrize("n_cond,n_text", [(32, 64), (32, 200), (32, 500)])
def test_full_prefill_logits(full, n_cond, n_text):
    W, g, M = full
    say(f"[gpu] full prefill {n_cond}+{n_text}")
    pr = synth.make_prompt(W.cfg, n_cond, n_text, seed=n_text)
    kv = g.kv_cache(2048)
    a = g.prefill(pr.text_tokens, pr.conds, pr.lang_id, kv)
    b = M.prefill_after(M.kv(2048), pr.text_tokens, pr.conds, pr.lang_id)
    err = float(np.abs(a - b).max())
    say(f"[gpu]   max |logit diff| = {err:.3g} (logit range {float(np.abs(b).max()):.3g})")
    assert err < LOGIT_TOL
    kv32 = g.kv_cache(2048, H.ITTS_F32)
    a32 = g.prefill(pr.text_tokens, pr.conds, pr.lang_id, kv32)
    b32 = M.prefill_after(M.kv(2048, kv_bf16=False), pr.text_tokens, pr.conds, pr.lang_id)
    err32 = float(np.abs(a32 - b32).max())
    say(f"[gpu]   fp32 KV: max |logit diff| = {err32:.3g}")
    assert err32 < 1e-4     # what fp32 caches on both sides achieve; guards regressions
    assert int(np.argmax(a)) == int(np.argmax(b))


def _penalised(logits, seen, p=10.0):
    x = logits.copy()
    for t in seen:
        x[t] = x[t] * p if x[t] < 0 else x[t] / p
    x[8193] = -np.inf                      # STOP masked (min_codes)
    return x


def test_full_greedy_codes_identical_f32_kv(full):
    """With the reference's fp32 KV cache, greedy ids over 48 steps are identical."""
    W, g, M = full
    say("[gpu] full greedy decode, fp32 KV")
    pr = synth.make_prompt(W.cfg, 32, 64, seed=5)
    n = 48
    p = H.SamplingParams(greedy=True, repetition_penalty=10.0, max_mel_tokens=n)
    kv = g.kv_cache(2048, H.ITTS_F32)
    codes = H.generate_codes_after(g, H.CodePrompt(pr.text_tokens, pr.conds, pr.lang_id, None, n), kv,
                                   p, H.SamplerRng(0))
    ref, _, _ = M.generate_codes_after(M.kv(2048, kv_bf16=False), pr.text_tokens, pr.conds, pr.lang_id, p,
                                       0, min_codes=n)
    assert len(codes) == n
    assert codes.tolist() == ref.tolist()


@pytest.mark.parametrize("path", [H.ITTS_DECODE_AUTO, H.ITTS_DECODE_MULTI])
def test_full_greedy_bf16_kv(full, path):
    """bf16 KV (the workload's cache): both sides round K/V to bf16, so an element whose
    fp32 value differs in the last bits can round to the neighbouring bf16 value; logits
    then differ by more than the fp32 paths do.  Teacher-forced on the oracle's ids, every
    step's logits stay within the bar, and the greedy pick (penalty 10) agrees at every
    step whose oracle top-2 margin exceeds 4x the largest logit difference seen; the
    free-running decode is identical up to the first step inside that margin."""
    W, g, M = full
    say(f"[gpu] full greedy decode, bf16 KV, path {path}")
    g.set_decode_path(path)
    try:
        pr = synth.make_prompt(W.cfg, 32, 64, seed=5)
        n = 48
        p = H.SamplingParams(greedy=True, repetition_penalty=10.0, max_mel_tokens=n)
        ref, _, _ = M.generate_codes_after(M.kv(2048), pr.text_tokens, pr.conds, pr.lang_id, p, 0, min_codes=n)
        ref = ref.tolist()
        kv, okv = g.kv_cache(2048), M.kv(2048)
        a = g.prefill(pr.text_tokens, pr.conds, pr.lang_id, kv)
        b = M.prefill_after(okv, pr.text_tokens, pr.conds, pr.lang_id)
        seen, steps = {1, 8192}, []
        for s in range(n):
            pa, pb = _penalised(a, seen), _penalised(b, seen)
            top = np.sort(pb)[-2:]
            steps.append((float(np.abs(a - b).max()), float(top[1] - top[0]), int(np.argmax(pa)), int(np.argmax(pb))))
            seen.add(ref[s])
            if s + 1 < n:
                a, b = g.step(kv, ref[s], s + 2), M.step(okv, ref[s], s + 2)
        err = max(e for e, _, _, _ in steps)
        margin = 4 * err
        ties = [i for i, (_, gap, _, _) in enumerate(steps) if gap <= margin]
        say(f"[gpu]   max |logit diff| {err:.3g}; steps inside the margin: {ties}")
        assert err < LOGIT_TOL
        for i, (_, gap, ia, ib) in enumerate(steps):
            assert ib == ref[i]
            if gap > margin:
                assert ia == ib, (i, gap, margin)
        kv = g.kv_cache(2048)
        codes = H.generate_codes_after(g, H.CodePrompt(pr.text_tokens, pr.conds, pr.lang_id, None, n), kv,
                                       p, H.SamplerRng(0)).tolist()
        upto = ties[0] if ties else n
        assert codes[:upto] == ref[:upto]
    finally:
        g.set_decode_path(H.ITTS_DECODE_AUTO)


def test_full_step_logits(full):
    """Teacher-forced steps after a prefill: every step's logits within the bar."""
    W, g, M = full
    say("[gpu] full prefill + 16 steps")
    pr = synth.make_prompt(W.cfg, 32, 64, seed=9)
    kv = g.kv_cache(2048)
    okv = M.kv(2048)
    g.prefill(pr.text_tokens, pr.conds, pr.lang_id, kv)
    M.prefill_after(okv, pr.text_tokens, pr.conds, pr.lang_id)
    rng = np.random.default_rng(3)
    worst = 0.0
    for i, t in enumerate(rng.integers(0, 8192, 16)):
        a = g.step(kv, int(t), i + 2)
        b = M.step(okv, int(t), i + 2)
        worst = max(worst, float(np.abs(a - b).max()))
    say(f"[gpu]   worst max |logit diff| over 16 steps = {worst:.3g}")
    assert worst < LOGIT_TOL


def test_full_teacher_forced(full):
    """teacher_forced at the real shape with the reference's alignment heads (4, 10), (5, 10):
    log-probabilities of 48 codes and the averaged text attention against the oracle."""
    W, g, M = full
    say("[gpu] full teacher_forced, 48 codes")
    pr = synth.make_prompt(W.cfg, 32, 64, seed=12)
    codes = np.random.default_rng(12).integers(0, 8192, 48).astype(np.int32)
    lp, att = g.teacher_forced(pr.text_tokens, pr.conds, pr.lang_id, codes, g.kv_cache(2048))
    text_lo, text_hi = 32, 32 + 64 + 2
    emb = M.sequence_embedding(pr.text_tokens, pr.conds, pr.lang_id, codes[:-1])
    lg, maps = M.replay(M.kv(2048, kv_bf16=False), emb,
                        probes=[(4, 10, text_hi, text_lo, text_hi), (5, 10, text_hi, text_lo, text_hi)], row0=text_hi)
    x = lg.astype(np.float64)
    x -= x.max(1, keepdims=True)
    ref = (x - np.log(np.exp(x).sum(1, keepdims=True)))[np.arange(48), codes]
    err_lp = float(np.abs(lp - ref).max())
    err_att = float(np.abs(att - (maps[0] + maps[1]) / 2).max())
    say(f"[gpu]   max |log p diff| {err_lp:.3g}, max |attention diff| {err_att:.3g}")
    assert err_lp < LOGIT_TOL and err_lp < 1e-4
    assert err_att < 1e-4


def test_full_forward_logits_batch(full):
    """The batched all-row forward (two prompts of 32 + 100 text ids, one with prior codes)
    against the oracle's per-prompt all-row logits."""
    W, g, M = full
    say("[gpu] full forward_logits, batch of 2")
    prompts, refs = [], []
    for b in range(2):
        pr = synth.make_prompt(W.cfg, 32, 100, seed=40 + b)
        prior = np.arange(b * 20, dtype=np.int32)
        prompts.append(H.CodePrompt(pr.text_tokens, pr.conds, pr.lang_id, prior))
        emb = M.sequence_embedding(pr.text_tokens, pr.conds, pr.lang_id, prior)
        refs.append(M.forward_rows(M.kv(2048, kv_bf16=False), emb, 0))
    got = g.forward_logits(prompts)
    ref = np.concatenate(refs)
    err = float(np.abs(got - ref).max())
    say(f"[gpu]   rows {got.shape[0]}, max |logit diff| {err:.3g}")
    assert got.shape == ref.shape and err < 1e-4


def test_full_generate_batch(full):
    """Four sequences decoded together at the real shape (fp32 caches): per sequence, the
    greedy ids (penalty 10) equal the oracle's for that sequence alone."""
    W, g, M = full
    say("[gpu] full generate_codes_batch, 4 sequences")
    prompts, refs = [], []
    lengths = [24, 32, 16, 28]
    for b in range(4):
        pr = synth.make_prompt(W.cfg, 32, 40 + 20 * b, seed=60 + b)
        p = H.SamplingParams(greedy=True, repetition_penalty=10.0, max_mel_tokens=lengths[b])
        prompts.append((H.CodePrompt(pr.text_tokens, pr.conds, pr.lang_id, None, lengths[b]), p))
        ref, _, _ = M.generate_codes_after(M.kv(2048, kv_bf16=False), pr.text_tokens, pr.conds, pr.lang_id, p, 0,
                                           min_codes=lengths[b])
        refs.append(ref.tolist())
    caches = [g.kv_cache(2048, H.ITTS_F32) for _ in range(4)]
    got = H.generate_codes_batch(g, [c for c, _ in prompts], caches, [p for _, p in prompts],
                                 [H.SamplerRng(0) for _ in range(4)])
    for b in range(4):
        assert got[b].tolist() == refs[b], b


@pytest.mark.parametrize("path", [H.ITTS_DECODE_AUTO, H.ITTS_DECODE_MULTI])
def test_full_int4_steps(full_int4, path):
    """4-bit weights at the real shape (persistent step by default, or the multi-kernel
    step): prefill of 32 + 128 text ids and 16 teacher-forced steps against the oracle."""
    say(f"[gpu] full int4 decoder, path {path}")
    W, g, M = full_int4
    try:
        g.set_decode_path(path)
        pr = synth.make_prompt(W.cfg, 32, 128, seed=3)
        kv = g.kv_cache(2048)
        assert kv.decode_path() == (H.ITTS_DECODE_PERSISTENT if path == H.ITTS_DECODE_AUTO else H.ITTS_DECODE_MULTI)
        okv = M.kv(2048)
        worst = float(np.abs(g.prefill(pr.text_tokens, pr.conds, pr.lang_id, kv) -
                             M.prefill_after(okv, pr.text_tokens, pr.conds, pr.lang_id)).max())
        for i, t in enumerate(np.random.default_rng(4).integers(0, 8192, 16)):
            worst = max(worst, float(np.abs(g.step(kv, int(t), i + 2) - M.step(okv, int(t), i + 2)).max()))
        say(f"[gpu]   worst max |logit diff| {worst:.3g}")
        assert worst < LOGIT_TOL and worst < 2e-3
    finally:
        g.set_decode_path(H.ITTS_DECODE_AUTO)
