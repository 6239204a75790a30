"""The stream checker of the GPU parity tests (tests/_streams.py), on the CPU.

The oracle's own generation replayed on its teacher-forced all-row logits must reproduce
every decision and the final RNG state (this also pins all-row logits == prefill + step
logits along a sampled stream); a planted wrong token must be reported, and reported as
unexplained when no logit perturbation is allowed."""
import numpy as np
import pytest

import ito
import itts_hip as H
from itts_hip import synth
from _streams import oracle_rows, replay_stream


@pytest.mark.parametrize("kv_bf16", [True, False])
@pytest.mark.parametrize("greedy", [True, False])
def test_oracle_stream_replays_exactly(tiny_weights, kv_bf16, greedy):
    W = tiny_weights
    M = ito.Model(W)
    pr = synth.make_prompt(W.cfg, 3, 12, seed=8)
    n = 120
    samp = dict(greedy=True) if greedy else dict(greedy=False, temperature=0.8, top_k=30, top_p=0.8)
    sp = H.SamplingParams(max_mel_tokens=n, repetition_penalty=10.0, **samp)
    st0 = H.SamplerRng(77).state.value
    stop = W.cfg["mel_vocab"] - 1
    codes, st_end, _ = M.generate_codes_after(M.kv(256, kv_bf16=kv_bf16), pr.text_tokens, pr.conds, pr.lang_id,
                                              sp, st0, min_codes=n)
    assert len(codes) == n
    rows = oracle_rows(M, pr, codes, kv_bf16, max_seq=256)
    mism, unexplained, st = replay_stream(rows, codes, sp, st0, n, stop, 0.0)
    assert mism == [] and unexplained == []
    assert st == st_end
    # a planted wrong decision is caught: the first code replaced by a token the oracle
    # gives a much lower logit
    bad = codes.copy()
    bad[0] = int(np.argmin(rows[0][:stop]))
    mism, unexplained, _ = replay_stream(rows, bad, sp, st0, n, stop, 0.0)
    assert mism[:1] == [0] and unexplained[:1] == [0]
    mism, unexplained, _ = replay_stream(rows, bad, sp, st0, n, stop, 1e-3)
    assert unexplained[:1] == [0]
