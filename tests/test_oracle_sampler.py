"""Pins the oracle sampler (sampler.rs:19-284) with the reference's own known answers,
its proptest invariant, the published SplitMix64 vectors and the distribution the
top-k / top-p / temperature algorithm fixes."""
import ctypes as C
import math

import numpy as np
import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

import ito
from itts_hip import SamplingParams


def params(**kw):
    return SamplingParams(**kw)


def test_reference_repetition_penalty_known_answer():
    # sampler.rs:430-454: penalty 2 on seen {1, 8192, 10, 20}
    seen = ito.seen_init()
    ito.lib.ito_seen_insert(ito._p(seen), 10)
    ito.lib.ito_seen_insert(ito._p(seen), 20)
    logits = np.zeros(32, np.float32)
    logits[1], logits[10], logits[20], logits[25] = 2.0, 4.0, -3.0, 4.0
    ito.lib.ito_apply_repetition_penalty(ito._p(seen), ito._p(logits), 32, 2.0)
    assert abs(logits[1] - 1.0) < 1e-6
    assert abs(logits[10] - 2.0) < 1e-6
    assert abs(logits[20] - (-6.0)) < 1e-6
    assert abs(logits[25] - 4.0) < 1e-6


def test_reference_doctest_returns_42():
    # sampler.rs:176-189: all -10 except [42] = 25, default params, seed 7 -> 42
    logits = np.full(8194, -10.0, np.float32)
    logits[42] = 25.0
    tok, _ = ito.sample_next_token(logits, ito.seen_init(), params(), ito.lib.ito_rng_init(7))
    assert tok == 42


def test_seen_initial_tokens():
    # sampler.rs:101-115: {1, 8192}
    w = ito.seen_init()
    bits = [i for i in range(129 * 64) if (int(w[i // 64]) >> (i % 64)) & 1]
    assert bits == [1, 8192]


def test_splitmix64_published_vector():
    # SplitMix64 (Steele, Lea & Flood 2014) from state 1234567 (Vigna's reference
    # splitmix64.c); SamplerRng::new(seed) starts from seed ^ 0x9E3779B97F4A7C15.
    s = C.c_uint64(ito.lib.ito_rng_init(1234567 ^ 0x9E3779B97F4A7C15))
    got = [ito.lib.ito_rng_next_u64(C.byref(s)) for _ in range(5)]
    assert got == [6457827717110365317, 3203168211198807973, 9817491932198370423,
                   4593380528125082431, 16408922859458223821]


def test_next_f32_is_top_24_bits():
    s = C.c_uint64(ito.lib.ito_rng_init(42))
    s2 = C.c_uint64(s.value)
    for _ in range(1000):
        u = ito.lib.ito_rng_next_u64(C.byref(s2))
        f = ito.lib.ito_rng_next_f32(C.byref(s))
        assert f == (u >> 40) / 2.0 ** 24
        assert 0.0 <= f < 1.0


def any_f32_logits(data_seed: int, mix: int, n: int = 8194) -> np.ndarray:
    """8194 logits drawn from every f32 bit pattern (NaN, +-inf, subnormals included),
    as prop::num::f32::ANY does, mixed with ordinary values."""
    g = np.random.default_rng(data_seed)
    raw = g.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32).view(np.float32)
    if mix == 0:
        return raw
    normal = (g.standard_normal(n) * 3).astype(np.float32)
    pick = g.random(n) < (0.01 if mix == 1 else 0.5)
    return np.where(pick, raw, normal).astype(np.float32)


@settings(max_examples=300, deadline=None)
@given(
    data_seed=st.integers(0, 2**32 - 1),
    mix=st.integers(0, 2),
    temp=st.floats(float(np.float32(0.05)), 2.0, width=32),
    top_p=st.floats(float(np.float32(0.05)), 1.0, width=32),
    top_k=st.integers(1, 500),
    rep=st.floats(1.0, 2.5, width=32),
    greedy=st.booleans(),
    seed=st.integers(0, 2**64 - 1),
)
def test_proptest_always_returns_valid_mel_token_id(data_seed, mix, temp, top_p, top_k, rep, greedy,
                                                     seed):
    # sampler.rs:456-485
    logits = any_f32_logits(data_seed, mix)
    p = params(greedy=greedy, temperature=temp, top_p=top_p, top_k=top_k, repetition_penalty=rep,
               max_mel_tokens=32)
    tok, _ = ito.sample_next_token(logits, ito.seen_init(), p, ito.lib.ito_rng_init(seed))
    assert 0 <= tok < 8194


def test_greedy_ties_pick_lowest_index_and_ignore_nonfinite():
    lg = np.array([1.0, 5.0, np.inf, 5.0, np.nan, 3.0], np.float32)
    seen = np.zeros(129, np.uint64)
    tok, st_ = ito.sample_next_token(lg, seen, params(greedy=True, repetition_penalty=1.0), 99)
    assert tok == 1 and st_ == 99  # greedy draws nothing
    lg = np.array([-np.inf, np.nan, np.inf], np.float32)
    tok, _ = ito.sample_next_token(lg, seen, params(greedy=True, repetition_penalty=1.0), 99)
    assert tok == 0


def test_greedy_applies_penalty_first():
    # D7: the reference's greedy mode still applies the repetition penalty
    lg = np.zeros(8194, np.float32)
    lg[100], lg[200] = 5.0, 4.0
    seen = ito.seen_init()
    ito.lib.ito_seen_insert(ito._p(seen), 100)
    tok, _ = ito.sample_next_token(lg, seen, params(greedy=True, repetition_penalty=10.0), 0)
    assert tok == 200


def _nucleus(v, temp, k, top_p):
    """Distribution fixed by sampler.rs:210-283 (in float64): top-k by value, softmax,
    keep while the cumulative probability before the i-th is <= top_p."""
    s = v.astype(np.float64) / temp
    order = np.argsort(-s, kind="stable")[:k]
    p = np.exp(s[order] - s[order[0]])
    p /= p.sum()
    cum = np.concatenate([[0.0], np.cumsum(p)[:-1]])
    keep = (cum <= top_p) | (np.arange(len(p)) == 0)
    order, p = order[keep], p[keep]
    return order, p / p.sum()


@pytest.mark.parametrize("temp,k,top_p", [(0.8, 30, 0.8), (1.0, 5, 1.0), (0.5, 0, 0.9), (2.0, 3, 0.5)])
def test_draw_frequencies_follow_the_nucleus_distribution(temp, k, top_p):
    rng = np.random.default_rng(3)
    base = (rng.standard_normal(64) * 1.5).astype(np.float32)
    kk = 64 if k == 0 else k
    ids, probs = _nucleus(base, temp, kk, top_p)
    counts = np.zeros(64)
    n = 20000
    state = ito.lib.ito_rng_init(1)
    seen = np.zeros(129, np.uint64)
    p = params(temperature=temp, top_k=k, top_p=top_p, repetition_penalty=1.0)
    for _ in range(n):
        tok, state = ito.sample_next_token(base.copy(), seen, p, state)
        counts[tok] += 1
    assert set(np.nonzero(counts)[0]) <= set(ids.tolist())
    freq = counts[ids] / n
    # 5-sigma binomial band
    assert np.all(np.abs(freq - probs) <= 5 * np.sqrt(probs * (1 - probs) / n) + 1e-9)


def test_top_k_one_is_argmax_of_scaled_values():
    rng = np.random.default_rng(4)
    for s in range(50):
        lg = rng.standard_normal(8194).astype(np.float32)
        tok, _ = ito.sample_next_token(lg.copy(), np.zeros(129, np.uint64),
                                       params(top_k=1, repetition_penalty=1.0), s)
        assert tok == int(np.argmax(lg))


def test_sampling_validation_ranges():
    ok = ito.sampling(params())
    assert ito.lib.ito_sampling_validate(C.byref(ok)) == 0
    for kw in [dict(temperature=0.01), dict(temperature=2.5), dict(top_p=0.0), dict(top_p=1.5),
               dict(top_k=9000), dict(repetition_penalty=0.5), dict(repetition_penalty=60.0),
               dict(max_mel_tokens=0), dict(max_mel_tokens=1816), dict(temperature=math.nan)]:
        bad = ito.sampling(params(**kw))
        assert ito.lib.ito_sampling_validate(C.byref(bad)) == ito.ITO_E_VALIDATION, kw
