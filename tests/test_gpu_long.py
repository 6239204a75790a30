"""Parity at the workloads' sizes and long contexts, at the decoder's real shape (24 layers,
d_model 1280, 20 heads x 64, FFN 5120, 8194 Mel ids, MLX-affine group-64 weights), through
the C ABI.  Reference: Gpt::prefill_after / step (gpt.rs:636-754), sample_next_token and
generate_codes_after (sampler.rs:191-392), the greedy-codes test (sampler.rs:487-536).

For each workload a whole HIP generation is checked decision by decision against the
oracle's sampler on the oracle's teacher-forced logits (tests/_streams.py), and HIP decode
steps taken at contexts where the persistent step's attention runs its second and third
key passes (more than 864 and 1728 keys with 12 key splits of 72 key slots) are compared
with the oracle's logits, within the workload's 2e-2 bar:

- long utterance: 32 cond + 200 text, 1500 sampled steps (T 0.8, top-k 30, top-p 0.8,
  penalty 10, STOP masked), bf16 and fp32 caches, contexts to 1734 keys;
- long greedy: 32 cond + 200 text, 1500 greedy steps (penalty 10) on the reference's fp32
  cache, id for id against the oracle's free-running decode;
- 4-bit weights: 32 + 128 text, 1500 greedy steps, contexts to 1662 keys;
- short: 32 + 64 text, 128 greedy steps: identical ids with fp32 caches;
- batch 8: text lengths U[20,200], decode lengths U[200,1200], sampled, bf16 caches,
  every sequence's stream, and batched steps near each sequence's end;
- prefill-heavy: 4 x (32 + 512) rows, the logits of every row.
"""
import os
import sys

import numpy as np
import pytest

import ito
import itts_hip as H
from itts_hip import synth
from _streams import oracle_rows, replay_stream, step_checkpoint

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-2
STOP = 8193
SAMPLED = dict(greedy=False, temperature=0.8, top_k=30, top_p=0.8, repetition_penalty=10.0)
GREEDY = dict(greedy=True, repetition_penalty=10.0)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _generate(g, pr, n, samp, dtype, seed):
    sp = H.SamplingParams(max_mel_tokens=n, **samp)
    rng = H.SamplerRng(seed)
    st0 = rng.state.value
    kv = g.kv_cache(2048, dtype)
    codes = H.generate_codes_after(g, H.CodePrompt(pr.text_tokens, pr.conds, pr.lang_id, None, n), kv, sp, rng)
    assert len(codes) == n
    return sp, st0, rng.state.value, codes, kv


def _checkpoints(g, dtype, pr, codes, rows, cps, n_steps=3):
    worst, keys = 0.0, []
    for c in cps:
        kv = g.kv_cache(2048, dtype)
        errs, L = step_checkpoint(g, kv, pr, codes, rows, c, n_steps)
        say(f"[gpu]   prior {c}: steps to {L} keys, max |logit diff| prefill {errs[0]:.3g}, steps {max(errs[1:]):.3g}")
        worst = max(worst, max(errs))
        keys.append(L)
    return worst, keys


def _dump(name, **arrays):
    """Keeps a test's HIP streams for offline analysis when ITTS_TEST_DUMP names a folder."""
    d = os.environ.get("ITTS_TEST_DUMP")
    if d:
        os.makedirs(d, exist_ok=True)
        np.savez(os.path.join(d, name + ".npz"), **arrays)


def _check_stream(rows, codes, sp, st0, st_end, eps, max_mism):
    need = {}
    mism, unexplained, st = replay_stream(rows, codes, sp, st0, len(codes), STOP, eps,
                                          report=lambda i, e: need.__setitem__(i, e))
    say(f"[gpu]   stream of {len(codes)}: {len(mism)} decisions differ, unexplained {unexplained} (eps {eps:.3g}); "
        f"perturbation each needs: {', '.join(f'{i}: {e:.2g}' for i, e in list(need.items())[:16])}")
    assert st == st_end, "RNG state after the stream differs (a different number of draws)"
    assert not unexplained
    assert len(mism) <= max_mism


@pytest.mark.parametrize("kv_dtype", [H.ITTS_BF16, H.ITTS_F32], ids=["bf16", "f32"])
def test_long_utterance(full_model, kv_dtype):
    """Config 2 end to end: the 1500-step sampled stream and steps at 876-1734 keys."""
    W, g, M = full_model
    say(f"[gpu] long utterance 32+200, 1500 sampled steps, kv {'bf16' if kv_dtype == H.ITTS_BF16 else 'f32'}")
    pr = synth.make_prompt(W.cfg, 32, 200, seed=2)
    sp, st0, st_end, codes, kv = _generate(g, pr, 1500, SAMPLED, kv_dtype, 1234)
    say(f"[gpu]   decode path {kv.decode_path()}, cache {kv.valid_len()} rows; oracle rows ...")
    assert kv.decode_path() == H.ITTS_DECODE_PERSISTENT
    rows = oracle_rows(M, pr, codes, kv_bf16=kv_dtype == H.ITTS_BF16)
    _dump(f"long_{kv_dtype}", codes=codes, st0=st0, st_end=st_end)
    worst, keys = _checkpoints(g, kv_dtype, pr, codes, rows, (640, 1065, 1496))
    assert keys[0] > 12 * 72 and keys[-1] > 2 * 12 * 72
    assert worst < LOGIT_TOL
    assert worst < (5e-3 if kv_dtype == H.ITTS_BF16 else 1e-4)
    _check_stream(rows, codes, sp, st0, st_end, eps=4 * worst, max_mism=15 if kv_dtype == H.ITTS_BF16 else 2)


@pytest.mark.parametrize("kv_dtype", [H.ITTS_BF16, H.ITTS_F32], ids=["bf16", "f32"])
def test_long_utterance_multi_kernel_steps(full_model, kv_dtype):
    """The multi-kernel decode step at the same long contexts."""
    W, g, M = full_model
    say(f"[gpu] long contexts, multi-kernel step, kv {'bf16' if kv_dtype == H.ITTS_BF16 else 'f32'}")
    pr = synth.make_prompt(W.cfg, 32, 200, seed=2)
    codes = np.random.default_rng(21).integers(0, 8192, 1500).astype(np.int32)
    rows = oracle_rows(M, pr, codes, kv_bf16=kv_dtype == H.ITTS_BF16)
    g.set_decode_path(H.ITTS_DECODE_MULTI)
    try:
        worst, _ = _checkpoints(g, kv_dtype, pr, codes, rows, (640, 1496))
    finally:
        g.set_decode_path(H.ITTS_DECODE_AUTO)
    assert worst < LOGIT_TOL and worst < (5e-3 if kv_dtype == H.ITTS_BF16 else 1e-4)


def test_int4_long(full_int4):
    """Config 5: 4-bit weights, 1500 greedy steps (penalty 10), contexts to 1662 keys."""
    W, g, M = full_int4
    say("[gpu] int4 32+128, 1500 greedy steps, bf16")
    pr = synth.make_prompt(W.cfg, 32, 128, seed=3)
    sp, st0, st_end, codes, kv = _generate(g, pr, 1500, GREEDY, H.ITTS_BF16, 0)
    assert kv.decode_path() == H.ITTS_DECODE_PERSISTENT
    rows = oracle_rows(M, pr, codes, kv_bf16=True)
    _dump("int4", codes=codes)
    worst, keys = _checkpoints(g, H.ITTS_BF16, pr, codes, rows, (712, 1137, 1496))
    assert keys[0] > 12 * 72 and keys[-1] == 163 + 1499
    assert worst < LOGIT_TOL and worst < 5e-3
    _check_stream(rows, codes, sp, st0, st_end, eps=4 * worst, max_mism=15)


@pytest.mark.parametrize("path", [H.ITTS_DECODE_AUTO, H.ITTS_DECODE_MULTI], ids=["persistent", "multi"])
def test_short_greedy_identical_f32(full_model, path):
    """Config 1 with the reference's fp32 cache, on the persistent step (what AUTO picks)
    and on the multi-kernel step: all 128 greedy ids identical to the oracle's decisions
    (and so to its free-running decode)."""
    W, g, M = full_model
    say(f"[gpu] short 32+64, 128 greedy steps, f32, path {path}")
    pr = synth.make_prompt(W.cfg, 32, 64, seed=5)
    g.set_decode_path(path)
    try:
        sp, st0, st_end, codes, kv = _generate(g, pr, 128, GREEDY, H.ITTS_F32, 0)
        assert kv.decode_path() == (H.ITTS_DECODE_PERSISTENT if path == H.ITTS_DECODE_AUTO else H.ITTS_DECODE_MULTI)
    finally:
        g.set_decode_path(H.ITTS_DECODE_AUTO)
    rows = oracle_rows(M, pr, codes, kv_bf16=False)
    mism, _, _ = replay_stream(rows, codes, sp, st0, 128, STOP, 0.0)
    say(f"[gpu]   decode path {kv.decode_path()}; differing decisions {mism}")
    assert mism == []
    ref, _, _ = M.generate_codes_after(M.kv(2048, kv_bf16=False), pr.text_tokens, pr.conds, pr.lang_id, sp, st0,
                                       min_codes=128)
    assert codes.tolist() == ref.tolist()


def _margin(row, seen_codes, params):
    """Top-2 margin of the penalised logits the greedy pick sees (sampler.rs:138-157,
    STOP masked): the perturbation that would swap the two best ids."""
    x = np.array(row, dtype=np.float64, copy=True)
    x[STOP] = -np.inf
    p = float(params.repetition_penalty)
    seen = np.unique(np.concatenate([np.asarray(seen_codes, np.int64), [1, 8192]]))
    seen = seen[seen < len(x)]
    x[seen] = np.where(x[seen] < 0, x[seen] * p, x[seen] / p)
    top = np.sort(x)[-2:]
    return float(top[1] - top[0])


def test_long_greedy_identical_f32(full_model):
    """The long prompt (32 cond + 200 text) with 1500 greedy steps (penalty 10, STOP
    masked) on the reference's fp32 cache (gpt.rs:117,185-186), compared id for id with the
    oracle's free-running generate_codes_after (the CP-11 semantics of sampler.rs:487-536
    over the whole decode).  Should the ids part, the first departing step must be a
    near-tie: its top-2 margin within 4x the logit difference the persistent step shows
    at that context."""
    W, g, M = full_model
    say("[gpu] long 32+200, 1500 greedy steps, f32 cache, id for id against the oracle")
    pr = synth.make_prompt(W.cfg, 32, 200, seed=2)
    sp, st0, st_end, codes, kv = _generate(g, pr, 1500, GREEDY, H.ITTS_F32, 0)
    assert kv.decode_path() == H.ITTS_DECODE_PERSISTENT
    ref, _, _ = M.generate_codes_after(M.kv(2048, kv_bf16=False), pr.text_tokens, pr.conds, pr.lang_id, sp, st0,
                                       min_codes=1500)
    assert len(ref) == 1500
    diff = np.nonzero(codes != ref)[0]
    if len(diff) == 0:
        say("[gpu]   1500 greedy ids identical to the oracle's free-running decode")
        return
    i = int(diff[0])
    okv = M.kv(2048, kv_bf16=False)
    row = M.prefill_after(okv, pr.text_tokens, pr.conds, pr.lang_id, np.asarray(ref[:i], np.int32))
    # the persistent step's logits there (code j sits at Mel position j + 2, gpt.rs:618-625)
    hkv = g.kv_cache(2048, H.ITTS_F32)
    if i == 0:
        hrow = g.prefill(pr.text_tokens, pr.conds, pr.lang_id, hkv)
    else:
        g.prefill_after(pr.text_tokens, pr.conds, pr.lang_id, np.asarray(ref[: i - 1], np.int32), hkv)
        hrow = g.step(hkv, int(ref[i - 1]), i + 1)
    err = float(np.abs(hrow - row).max())
    m = _margin(row, ref[:i], sp)
    say(f"[gpu]   first departure at step {i} (of 1500): oracle {int(ref[i])}, HIP {int(codes[i])}; "
        f"oracle top-2 margin {m:.3g}, HIP-vs-oracle logit difference there {err:.3g}")
    assert m <= 4 * err, "the ids part where the oracle's decision is not a near-tie"


def test_short_greedy_bf16(full_model):
    """Config 1 with bf16 caches: every one of the 128 decisions checked."""
    W, g, M = full_model
    say("[gpu] short 32+64, 128 greedy steps, bf16")
    pr = synth.make_prompt(W.cfg, 32, 64, seed=5)
    sp, st0, st_end, codes, kv = _generate(g, pr, 128, GREEDY, H.ITTS_BF16, 0)
    rows = oracle_rows(M, pr, codes, kv_bf16=True)
    worst, _ = _checkpoints(g, H.ITTS_BF16, pr, codes, rows, (40, 120), n_steps=6)
    assert worst < LOGIT_TOL and worst < 5e-3
    _check_stream(rows, codes, sp, st0, st_end, eps=4 * worst, max_mism=3)


def test_batch8_long(full_model):
    """Config 3: eight sentences decoded together (bf16 caches, per-sequence lengths and
    stop); every decision of every sequence checked, and batched steps near each
    sequence's end (contexts of 250-1400 keys) compared with the oracle."""
    W, g, M = full_model
    rng = np.random.default_rng(100)
    n_text = rng.integers(20, 201, 8)
    n_dec = rng.integers(200, 1201, 8)
    say(f"[gpu] batch 8: text {n_text.tolist()}, decode {n_dec.tolist()}")
    prompts, cps, params = [], [], []
    for b in range(8):
        pr = synth.make_prompt(W.cfg, 32, int(n_text[b]), seed=200 + b)
        prompts.append(pr)
        cps.append(H.CodePrompt(pr.text_tokens, pr.conds, pr.lang_id, None, int(n_dec[b])))
        params.append(H.SamplingParams(max_mel_tokens=int(n_dec[b]), **SAMPLED))
    rngs = [H.SamplerRng(b) for b in range(8)]
    st0 = [r.state.value for r in rngs]
    caches = [g.kv_cache(2048, H.ITTS_BF16) for _ in range(8)]
    got = H.generate_codes_batch(g, cps, caches, params, rngs)
    assert [len(c) for c in got] == n_dec.tolist()
    _dump("batch8", **{f"codes{b}": got[b] for b in range(8)})
    rows = []
    for b in range(8):
        rows.append(oracle_rows(M, prompts[b], got[b], kv_bf16=True))
        say(f"[gpu]   oracle rows of sequence {b} ({len(got[b])} codes)")
    # batched steps: every cache holds its prompt and codes[:c_b], then 3 batched steps
    c = [int(n) - 4 for n in n_dec]
    caches = [g.kv_cache(2048, H.ITTS_BF16) for _ in range(8)]
    worst = 0.0
    for b in range(8):
        a = g.prefill_after(prompts[b].text_tokens, prompts[b].conds, prompts[b].lang_id,
                            np.asarray(got[b][:c[b]], np.int32), caches[b])
        worst = max(worst, float(np.abs(a - rows[b][c[b]]).max()))
    for i in range(3):
        toks = [int(got[b][c[b] + i]) for b in range(8)]
        pos = [c[b] + i + 2 for b in range(8)]
        out = H.step_batch(g, caches, toks, pos)
        for b in range(8):
            worst = max(worst, float(np.abs(out[b] - rows[b][c[b] + i + 1]).max()))
    keys = [cc.valid_len() for cc in caches]
    say(f"[gpu]   batched steps at {keys} keys: max |logit diff| {worst:.3g}")
    assert worst < LOGIT_TOL and worst < 5e-3
    for b in range(8):
        _check_stream(rows[b], got[b], params[b], st0[b], rngs[b].state.value, eps=4 * worst, max_mism=10)


def test_prefill_heavy_all_rows(full_model):
    """Config 4: one forward over 4 x (32 cond + 512 text) = 2188 rows, logits of every
    row, against the oracle's all-row logits per prompt (fp32 keys and values)."""
    W, g, M = full_model
    say("[gpu] prefill-heavy 4 x 547 rows, all-row logits")
    prompts, refs = [], []
    for b in range(4):
        pr = synth.make_prompt(W.cfg, 32, 512, seed=10 + b)
        prompts.append(H.CodePrompt(pr.text_tokens, pr.conds, pr.lang_id, None))
        emb = M.sequence_embedding(pr.text_tokens, pr.conds, pr.lang_id)
        refs.append(M.forward_rows(M.kv(2048, kv_bf16=False), emb, 0))
    got = g.forward_logits(prompts)
    ref = np.concatenate(refs)
    err = np.abs(got - ref).max(axis=1)
    say(f"[gpu]   rows {got.shape[0]}: max |logit diff| {err.max():.3g} (median row {np.median(err):.3g})")
    assert got.shape == (4 * 547, 8194)
    assert err.max() < LOGIT_TOL and err.max() < 1e-4


def test_f32_group_params_full_size(full_f32_params):
    """The shipped checkpoint's dtype (F32 scales and biases, loader.rs:927-930) at the real
    shape: a 535-row prefill (the 128 x 128 GEMM tiles), persistent decode steps, and a
    long-context prefill_after with steps to 1734 keys, against the oracle."""
    W, g, M = full_f32_params
    say("[gpu] F32 group params, full size")
    pr = synth.make_prompt(W.cfg, 32, 500, seed=7)
    for kvt in (H.ITTS_F32, H.ITTS_BF16):
        kv, okv = g.kv_cache(2048, kvt), M.kv(2048, kv_bf16=kvt == H.ITTS_BF16)
        a = g.prefill(pr.text_tokens, pr.conds, pr.lang_id, kv)
        b = M.prefill_after(okv, pr.text_tokens, pr.conds, pr.lang_id)
        worst = float(np.abs(a - b).max())
        for i, t in enumerate(np.random.default_rng(8).integers(0, 8192, 6)):
            worst = max(worst, float(np.abs(g.step(kv, int(t), i + 2) - M.step(okv, int(t), i + 2)).max()))
        say(f"[gpu]   kv {kvt}: decode path {kv.decode_path()}, 535-row prefill + 6 steps max |logit diff| {worst:.3g}")
        assert worst < LOGIT_TOL and worst < (1e-4 if kvt == H.ITTS_F32 else 5e-3)
    pr2 = synth.make_prompt(W.cfg, 32, 200, seed=2)
    codes = np.random.default_rng(22).integers(0, 8192, 1500).astype(np.int32)
    rows = oracle_rows(M, pr2, codes, kv_bf16=True)
    worst, keys = _checkpoints(g, H.ITTS_BF16, pr2, codes, rows, (1496,))
    assert keys[-1] == 235 + 1499 and worst < LOGIT_TOL and worst < 5e-3
