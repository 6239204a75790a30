"""itts_sample_next_token_noalloc (the sampler entry point that allocates no device
memory) against itts_sample_next_token, through the C ABI: token, penalised logits and
RNG state bit for bit, over two calls in a row (the second with fewer logits, so stale
staging contents past n would show), greedy and sampled; sizes past the staging area are
rejected."""
import sys

import numpy as np
import pytest

import itts_hip as H
from itts_hip import synth

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def gpt():
    say("[gpu] no-alloc sampler: tiny decoder handle")
    g = H.Gpt(synth.make_weights(synth.TINY_CONFIG, seed=41))
    yield g
    g.close()


def _case(n, seed):
    rng = np.random.default_rng(seed)
    logits = (rng.standard_normal(n) * 3).astype(np.float32)
    seen = H.SeenTokenBitSet()
    for t in rng.integers(0, n, 40):
        seen.insert(int(t))
    return logits, seen


CALLS = [
    (8194, dict(greedy=False, temperature=0.8, top_k=30, top_p=0.8, repetition_penalty=10.0)),
    (300, dict(greedy=False, temperature=1.3, top_k=500, top_p=0.95, repetition_penalty=2.0)),
    (9216, dict(greedy=True, repetition_penalty=10.0)),
    (17, dict(greedy=False, temperature=0.5, top_k=0, top_p=1.0, repetition_penalty=1.0)),
]


@pytest.mark.parametrize("first,second", [(0, 1), (2, 3), (0, 3)])
def test_noalloc_matches_allocating_entry(gpt, first, second):
    say(f"[gpu] no-alloc sampler calls n={CALLS[first][0]} then n={CALLS[second][0]}")
    state_a = H.SamplerRng(7)
    state_b = H.SamplerRng(7)
    for i, k in enumerate((first, second)):
        n, samp = CALLS[k]
        logits, seen = _case(n, 100 * first + 10 * second + i)
        params = H.SamplingParams(**samp)
        la, lb = logits.copy(), logits.copy()
        ta = H.sample_next_token(gpt, la, seen, params, state_a)
        tb = H.sample_next_token_noalloc(gpt, lb, seen, params, state_b)
        assert ta == tb
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
        assert state_a.state.value == state_b.state.value


def test_noalloc_rejects_oversize(gpt):
    logits = np.zeros(9217, np.float32)
    with pytest.raises(H.ValidationError, match="staging area"):
        H.sample_next_token_noalloc(gpt, logits, H.SeenTokenBitSet(), H.SamplingParams(), H.SamplerRng(0))
