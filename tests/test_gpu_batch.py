"""Batched decode (several independent sequences stepped together) on the HIP path,
through the C ABI, against the oracle run on each sequence alone: Gpt::step per sequence
(gpt.rs:706-754) and generate_codes_after per sequence (sampler.rs:340-392) with its own
prompt, sampling parameters, RNG, min_codes and length."""
import sys

import numpy as np
import pytest

import ito
import itts_hip as H
from itts_hip import synth

pytestmark = pytest.mark.gpu

TIGHT = 2e-4


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def small():
    say("[gpu] small decoder for batched decode")
    W = synth.make_weights(synth.SMALL_CONFIG, seed=8, init="rich")
    g = H.Gpt(W)
    yield W, g, ito.Model(W)
    g.close()


def _prompts(W, specs, seed0):
    out = []
    for i, (n_text, n_prior, lang) in enumerate(specs):
        pr = synth.make_prompt(W.cfg, 3, n_text, seed=seed0 + i)
        prior = np.random.default_rng(seed0 + i).integers(0, 1000, n_prior).astype(np.int32)
        out.append((pr, prior, lang))
    return out


@pytest.mark.parametrize("kvt", [H.ITTS_BF16, H.ITTS_F32])
def test_step_batch_ten_sequences(small, kvt):
    """More than 8 rows: the tiled products (LayerNorm row kernels, the QKV epilogue's
    per-sequence K/V scatter read from the sequence descriptors) instead of the few-row
    ones, each sequence against the oracle stepping it alone."""
    W, g, M = small
    say(f"[gpu] step_batch of 10 kv={kvt}")
    specs = [(4 + 7 * i, (5 * i) % 13, i % 4) for i in range(10)]
    ps = _prompts(W, specs, 40)
    caches, okvs = [], []
    for pr, prior, lang in ps:
        kv = g.kv_cache(256, kvt)
        okv = M.kv(256, kv_bf16=kvt == H.ITTS_BF16)
        g.prefill_after(pr.text_tokens, pr.conds, lang, prior, kv, logits=False)
        M.prefill_after(okv, pr.text_tokens, pr.conds, lang, prior)
        caches.append(kv)
        okvs.append(okv)
    rng = np.random.default_rng(3)
    for step in range(3):
        toks = rng.integers(0, 1000, len(ps)).astype(np.int32)
        pos = np.array([len(prior) + 2 + step for _, prior, _ in ps], np.int32)
        got = H.step_batch(g, caches, toks, pos)
        for b, okv in enumerate(okvs):
            ref = M.step(okv, int(toks[b]), int(pos[b]))
            assert np.abs(got[b] - ref).max() < TIGHT, (step, b)
            assert caches[b].valid_len() == okv.valid_len()
    for l in range(W.cfg["n_layer"]):
        for b in (0, 9):
            assert np.allclose(caches[b].read(l, 1), okvs[b].read(l, 1), rtol=1e-2, atol=1e-4)


@pytest.mark.parametrize("kvt", [H.ITTS_BF16, H.ITTS_F32])
def test_step_batch_matches_oracle_per_sequence(small, kvt):
    W, g, M = small
    say(f"[gpu] step_batch kv={kvt}")
    specs = [(12, 0, 1), (40, 9, 3), (5, 60, 0)]
    ps = _prompts(W, specs, 10)
    caches, okvs = [], []
    for pr, prior, lang in ps:
        kv = g.kv_cache(512, kvt)
        okv = M.kv(512, kv_bf16=kvt == H.ITTS_BF16)
        g.prefill_after(pr.text_tokens, pr.conds, lang, prior, kv, logits=False)
        M.prefill_after(okv, pr.text_tokens, pr.conds, lang, prior)
        caches.append(kv)
        okvs.append(okv)
    rng = np.random.default_rng(0)
    for step in range(6):
        toks = rng.integers(0, 1000, len(ps)).astype(np.int32)
        pos = np.array([len(prior) + 2 + step for _, prior, _ in ps], np.int32)
        got = H.step_batch(g, caches, toks, pos)
        for b, okv in enumerate(okvs):
            ref = M.step(okv, int(toks[b]), int(pos[b]))
            assert np.abs(got[b] - ref).max() < TIGHT, (step, b)
            assert caches[b].valid_len() == okv.valid_len()


@pytest.mark.parametrize("greedy", [True, False])
def test_generate_batch_equals_per_sequence(small, greedy):
    W, g, M = small
    say(f"[gpu] generate_codes_batch greedy={greedy}")
    specs = [(12, 0, 1), (30, 5, 2), (7, 0, 0), (50, 20, 4)]
    ps = _prompts(W, specs, 30)
    params = [H.SamplingParams(greedy=greedy, temperature=0.8, top_k=[30, 5, 80, 1][i], top_p=0.8,
                               repetition_penalty=10.0, max_mel_tokens=[60, 25, 90, 40][i]) for i in range(4)]
    min_codes = [60, 0, 90, 10]
    seeds = [11, 22, 33, 44]
    prompts = [H.CodePrompt(pr.text_tokens, pr.conds, lang, prior, mc)
               for (pr, prior, lang), mc in zip(ps, min_codes)]
    caches = [g.kv_cache(512) for _ in ps]
    rngs = [H.SamplerRng(s) for s in seeds]
    got = H.generate_codes_batch(g, prompts, caches, params, rngs)
    for b, ((pr, prior, lang), p) in enumerate(zip(ps, params)):
        ref, st, _ = M.generate_codes_after(M.kv(512), pr.text_tokens, pr.conds, lang, p,
                                            ito.lib.ito_rng_init(seeds[b]), prior=prior, min_codes=min_codes[b])
        if not greedy and got[b].tolist() != ref.tolist():
            _assert_order_flip(W, g, M, pr, prior, lang, p, min_codes[b], got[b].tolist(), ref.tolist())
            continue
        assert got[b].tolist() == ref.tolist(), b
        assert rngs[b].state.value == st
        assert caches[b].valid_len() == 3 + specs[b][0] + 3 + len(prior) + len(ref) - 1


def _assert_order_flip(W, g, M, pr, prior, lang, p, min_codes, codes, ref):
    """A sampled stream that parts from the oracle's at step i is the same decision only if
    the two picks are nearly equal candidates whose order the logit difference can swap:
    replayed on the common prefix, |z_oracle[c] - z_oracle[r]| <= 2 max|z_hip - z_oracle| for
    the penalised, temperature-scaled (and STOP-masked) logits z."""
    i = next(k for k in range(min(len(codes), len(ref))) if codes[k] != ref[k])
    V = W.cfg["mel_vocab"]
    kv, okv = g.kv_cache(512), M.kv(512)
    a = g.prefill_after(pr.text_tokens, pr.conds, lang, prior, kv)
    b = M.prefill_after(okv, pr.text_tokens, pr.conds, lang, prior)
    for s in range(i):
        a, b = g.step(kv, ref[s], len(prior) + 2 + s), M.step(okv, ref[s], len(prior) + 2 + s)
    seen = {1, V - 2} | set(ref[:i])

    def z(x):
        x = x.astype(np.float64).copy()
        for t in seen:
            x[t] = x[t] * p.repetition_penalty if x[t] < 0 else x[t] / p.repetition_penalty
        if i < min_codes:
            x[V - 1] = -np.inf
        return x / p.temperature

    za, zb = z(a), z(b)
    fin = np.isfinite(za) & np.isfinite(zb)
    err = float(np.abs(za - zb)[fin].max())
    say(f"[gpu]   streams part at step {i}: {codes[i]} vs {ref[i]}, |dz| {abs(zb[codes[i]] - zb[ref[i]]):.3g}, "
        f"max|z diff| {err:.3g}")
    assert abs(zb[codes[i]] - zb[ref[i]]) <= 2 * err + 1e-7
    assert codes[:i] == ref[:i]


def test_batch_validation(small):
    W, g, M = small
    kv1, kv2, kv3 = g.kv_cache(64), g.kv_cache(64), g.kv_cache(128)
    with pytest.raises(H.ValidationError):
        H.step_batch(g, [kv1, kv1], [1, 2], [2, 2])           # the same cache twice
    with pytest.raises(H.ValidationError):
        H.step_batch(g, [kv1, kv3], [1, 2], [2, 2])           # capacities differ
    with pytest.raises(H.ValidationError):
        H.step_batch(g, [kv1, kv2], [1, W.cfg["mel_vocab"]], [2, 2])
    g2 = H.Gpt(W)
    try:
        with pytest.raises(H.ValidationError):
            H.step_batch(g, [kv1, g2.kv_cache(64)], [1, 2], [2, 2])
    finally:
        g2.close()
