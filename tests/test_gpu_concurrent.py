"""Two decoders stepping at the same time from two host threads.

Each decoder owns its stream, and a persistent decode step assumes its blocks hold the
whole chip; the library chains persistent launches of different decoders so that one
never starts while another runs.  Both decoders must produce, concurrently, exactly what
they produce alone (the step is deterministic), and agree with the oracle."""
import sys
import threading

import numpy as np
import pytest

import ito
import itts_hip as H
from itts_hip import synth

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _run(g, pr, toks, out, key):
    kv = g.kv_cache(256)
    assert kv.decode_path() == H.ITTS_DECODE_PERSISTENT
    rows = [g.prefill(pr.text_tokens, pr.conds, pr.lang_id, kv)]
    for i, t in enumerate(toks):
        rows.append(g.step(kv, int(t), i + 2))
    out[key] = np.stack(rows)


def test_two_decoders_concurrent_steps():
    say("[gpu] two tiny decoders, 60 persistent steps each, concurrently")
    Ws = [synth.make_weights(synth.TINY_CONFIG, seed=s, init="rich") for s in (31, 32)]
    gs = [H.Gpt(W) for W in Ws]
    try:
        prs = [synth.make_prompt(W.cfg, 3, 15, seed=s) for W, s in zip(Ws, (1, 2))]
        toks = [np.random.default_rng(s).integers(0, 256, 60) for s in (3, 4)]
        alone = {}
        for i in range(2):
            _run(gs[i], prs[i], toks[i], alone, i)
        together, errors = {}, []

        def worker(i):
            try:
                _run(gs[i], prs[i], toks[i], together, i)
            except Exception as e:  # reported below
                errors.append(e)

        ts = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
        for t in ts:
            t.start()
        for t in ts:
            t.join(timeout=120)
        assert not errors, errors
        for i in range(2):
            assert np.array_equal(alone[i], together[i]), i
            M = ito.Model(Ws[i])
            okv = M.kv(256)
            ref = [M.prefill_after(okv, prs[i].text_tokens, prs[i].conds, prs[i].lang_id)]
            for j, t in enumerate(toks[i]):
                ref.append(M.step(okv, int(t), j + 2))
            err = float(np.abs(together[i] - np.stack(ref)).max())
            say(f"[gpu]   decoder {i}: max |logit diff| vs oracle {err:.3g}")
            assert err < 2e-4
    finally:
        for g in gs:
            g.close()
