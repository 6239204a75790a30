"""Pins the oracle decoder (gpt.rs) with closed forms, invariants and special cases that
a plausible mistake (a dropped term, a wrong index or head, a transposed operand, a
missing mask) would break."""
import copy

import numpy as np
import pytest

import ito
from itts_hip import synth


# ---------------------------------------------------------------- quantizer / QL --

def test_quantizer_constant_group_guard():
    # a constant group has s = 0: every code is 0 and the dequantised value is b
    w = np.zeros((2, 128), np.float32)
    w[0, :64] = 0.25
    w[0, 64:] = np.linspace(-1, 1, 64)
    w[1] = -3.0
    for bits, pd in [(8, 1), (4, 2)]:
        codes, s, b = ito.quantize(w, bits, pd)
        sf = s.view(np.float16).astype(np.float32) if pd == 1 else s
        bf = b.view(np.float16).astype(np.float32) if pd == 1 else b
        assert sf[0, 0] == 0.0 and bf[0, 0] == 0.25 and sf[1, 1] == 0.0 and bf[1, 1] == -3.0
        assert (codes[0, : 64 * bits // 8] == 0).all()
        deq = ito.dequant(synth.QLinear(codes, s, b, np.zeros(2, np.float32), 2, 128), bits, pd)
        assert (deq[0, :64] == 0.25).all() and (deq[1] == -3.0).all()


def test_quantizer_levels_and_extremes():
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((16, 256)) * 0.02).astype(np.float32)
    for bits, pd in [(8, 1), (4, 1), (8, 2), (4, 2)]:
        codes, s, b = ito.quantize(w, bits, pd)
        q = codes if bits == 8 else np.stack([codes & 15, codes >> 4], -1).reshape(16, 256)
        qmax = 255 if bits == 8 else 15
        # every group reaches both ends (min -> 0, max -> qmax) up to param rounding
        qg = q.reshape(16, 4, 64)
        assert (qg.min(-1) <= 1).all() and (qg.max(-1) >= qmax - 1).all()
        # dequantised weights are within half a step (plus param rounding) of w
        deq = ito.dequant(synth.QLinear(codes, s, b, np.zeros(16, np.float32), 16, 256), bits, pd)
        step = np.repeat((s.view(np.float16) if pd == 1 else s).astype(np.float32), 64, axis=1)
        assert np.all(np.abs(deq - w) <= 0.5 * step + 2e-3 * np.abs(w).max())


def test_quantizer_ramp_exact():
    # a ramp whose range is 255 * 2^-8 with min 0: s and b are exact in fp16, so
    # q = round(w / s) reproduces the ramp exactly
    w = (np.arange(64, dtype=np.float32) * 4 / 256.0).reshape(1, 64)
    w = np.tile(w, (1, 1))
    w[0, -1] = 255 / 256.0
    codes, s, b = ito.quantize(w, 8, 1)
    assert s.view(np.float16)[0, 0] == np.float16(1 / 256.0)
    assert b.view(np.float16)[0, 0] == 0
    assert (codes[0, :-1] == np.arange(63) * 4).all() and codes[0, -1] == 255


def test_dequant_two_roundings_vs_numpy():
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((32, 192)) * 0.02).astype(np.float32)
    for bits, pd in [(8, 1), (4, 1), (8, 2), (4, 2)]:
        codes, s, b = ito.quantize(w, bits, pd)
        q = codes if bits == 8 else np.stack([codes & 15, codes >> 4], -1).reshape(32, 192)
        sf = (s.view(np.float16).astype(np.float32) if pd == 1 else s)
        bf = (b.view(np.float16).astype(np.float32) if pd == 1 else b)
        ref = q.astype(np.float32) * np.repeat(sf, 64, 1)     # numpy float32: one rounding
        ref = ref + np.repeat(bf, 64, 1)                     # second rounding
        got = ito.dequant(synth.QLinear(codes, s, b, np.zeros(32, np.float32), 32, 192), bits, pd)
        assert (got.view(np.uint32) == ref.view(np.uint32)).all()


def _rand_ql(rng, N, K, bits=8, pd=1):
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    codes, s, b = ito.quantize(w, bits, pd)
    return synth.QLinear(codes, s, b, (rng.standard_normal(N) * 0.1).astype(np.float32), N, K)


@pytest.mark.parametrize("bits,pd", [(8, 1), (4, 2)])
def test_ql_forward_vs_fp64_bruteforce(bits, pd):
    rng = np.random.default_rng(3)
    q = _rand_ql(rng, 96, 320, bits, pd)
    x = rng.standard_normal((5, 320)).astype(np.float32)
    W = ito.dequant(q, bits, pd).astype(np.float64)
    ref = x.astype(np.float64) @ W.T + q.bias
    for mode in (ito.ITO_F32, ito.ITO_F64):
        got = ito.ql_forward(q, bits, pd, x, mode)
        assert np.abs(got - ref).max() < (1e-5 if mode == ito.ITO_F32 else 1e-6)


def test_ql_one_hot_returns_dequantised_column_plus_bias():
    rng = np.random.default_rng(4)
    q = _rand_ql(rng, 40, 128)
    W = ito.dequant(q, 8, 1)
    for k in (0, 63, 64, 127):
        x = np.zeros((1, 128), np.float32)
        x[0, k] = 1.0
        got = ito.ql_forward(q, 8, 1, x)[0]
        assert np.array_equal(got, W[:, k] + q.bias)


def test_layernorm_and_gelu_closed_forms():
    n = 128
    w = np.linspace(0.5, 1.5, n).astype(np.float32)
    b = np.linspace(-1, 1, n).astype(np.float32)
    y = np.empty(n, np.float32)
    x = np.full(n, 3.0, np.float32)                    # constant row -> beta
    ito.lib.ito_layernorm(ito._p(x), ito._p(w), ito._p(b), n, 1e-5, ito._p(y))
    assert np.array_equal(y, b)
    x = np.random.default_rng(5).standard_normal(n).astype(np.float32)
    ito.lib.ito_layernorm(ito._p(x), ito._p(w), ito._p(b), n, 1e-5, ito._p(y))
    xd = x.astype(np.float64)
    ref = (xd - xd.mean()) / np.sqrt(xd.var() + 1e-5) * w + b
    assert np.abs(y - ref).max() < 1e-5
    g = ito.lib.ito_gelu
    assert g(0.0) == 0.0
    assert abs(g(10.0) - 10.0) < 1e-6 and abs(g(-10.0)) < 1e-6
    assert abs(g(1.0) - 0.8411920071) < 1e-6          # tanh-form GELU at 1


# ---------------------------------------------------------------- decoder --

@pytest.fixture(scope="module")
def tiny():
    W = synth.make_weights(synth.TINY_CONFIG, seed=21, init="rich", quantizer=ito.quantize)
    return W, ito.Model(W)


def test_embedding_layout_closed_form(tiny):
    W, M = tiny
    text = np.array([7, 9, 11], np.int32)
    conds = np.random.default_rng(6).standard_normal((3, 128)).astype(np.float32)
    prior = np.array([4, 5], np.int32)
    e = M.sequence_embedding(text, conds, 2, prior)
    assert e.shape == (3 + 5 + 1 + 2, 128)
    assert np.array_equal(e[:3], conds)
    full = [0, 7, 9, 11, 1]
    for j, u in enumerate(full):
        assert np.array_equal(e[3 + j], (W.text_emb[u] + W.lang_emb[2]) + W.text_pos[j])
    start_mel = W.cfg["mel_vocab"] - 2
    assert np.array_equal(e[8], W.mel_emb[start_mel] + W.mel_pos[0])
    assert np.array_equal(e[9], W.mel_emb[4] + W.mel_pos[2])   # position 1 is never used
    assert np.array_equal(e[10], W.mel_emb[5] + W.mel_pos[3])


def _ln(x, w, b):
    x = x.astype(np.float64)
    return (x - x.mean()) / np.sqrt(x.var() + 1e-5) * w + b


def _gelu(x):
    return 0.5 * x * (1 + np.tanh(0.7978845608028654 * (x + 0.044715 * x ** 3)))


def test_single_row_stack_closed_form(tiny):
    """With one row, attention returns v: block(x) = x1 + mlp(LN2(x1)), x1 = x + proj(v),
    v = the third d-wide slice of c_attn(LN1(x)).  Pins the q|k|v order and the wiring."""
    W, M = tiny
    d = W.cfg["d_model"]
    x = np.random.default_rng(7).standard_normal((1, d)).astype(np.float32)
    kv = M.kv(16, kv_bf16=False, mode=ito.ITO_F64)
    got = M.forward_rows(kv, x)[0]

    def qlf(q, v):
        Wd = ito.dequant(q, 8, 1).astype(np.float64)
        return Wd @ v + q.bias

    h = x[0].astype(np.float64)
    for L in W.layers:
        qkv = qlf(L.c_attn, _ln(h, L.ln1_w, L.ln1_b))
        h = h + qlf(L.c_proj, qkv[2 * d:])
        h = h + qlf(L.mlp_c_proj, _gelu(qlf(L.c_fc, _ln(h, L.ln2_w, L.ln2_b))))
    z = _ln(_ln(h, W.ln_f_w, W.ln_f_b), W.fn_w, W.fn_b)
    ref = qlf(W.head, z)
    assert np.abs(got - ref).max() < 1e-6


def _permute_heads(W, perm):
    """Relabel heads consistently: c_attn rows of q, k, v (64-row blocks) and c_proj's
    input columns (64-wide blocks = whole quantisation groups)."""
    W2 = copy.deepcopy(W)
    d = W.cfg["d_model"]
    H = W.cfg["n_head"]
    rows = np.concatenate([np.arange(64) + 64 * p for p in perm])
    full = np.concatenate([rows, rows + d, rows + 2 * d])
    for L in W2.layers:
        a = L.c_attn
        a.codes, a.scales, a.biases, a.bias = (np.ascontiguousarray(t[full]) for t in
                                               (a.codes, a.scales, a.biases, a.bias))
        p_ = L.c_proj
        p_.codes = np.ascontiguousarray(p_.codes.reshape(d, H, 64)[:, perm].reshape(d, d))
        p_.scales = np.ascontiguousarray(p_.scales[:, perm])
        p_.biases = np.ascontiguousarray(p_.biases[:, perm])
    return W2


def test_head_relabelling_invariance(tiny):
    # fp64 mode: relabelling reorders c_proj's summation, which only fp64 makes exact enough
    W, M = tiny
    pr = synth.make_prompt(W.cfg, 3, 9, seed=8)
    kv = M.kv(64, kv_bf16=False, mode=ito.ITO_F64)
    ref = M.prefill_after(kv, pr.text_tokens, pr.conds, pr.lang_id)
    ref2 = M.step(kv, 17, 2)
    W2 = _permute_heads(W, [1, 0])
    M2 = ito.Model(W2)
    kv2 = M2.kv(64, kv_bf16=False, mode=ito.ITO_F64)
    got = M2.prefill_after(kv2, pr.text_tokens, pr.conds, pr.lang_id)
    got2 = M2.step(kv2, 17, 2)
    assert np.abs(got - ref).max() < 1e-6 and np.abs(got2 - ref2).max() < 1e-6
    # a broken relabelling (q heads swapped, k/v not) must change the result
    W3 = copy.deepcopy(W)
    d = W.cfg["d_model"]
    idx = np.concatenate([np.arange(64, 128), np.arange(64), np.arange(d, 3 * d)])
    for L in W3.layers:
        a = L.c_attn
        a.codes, a.scales, a.biases, a.bias = (np.ascontiguousarray(t[idx]) for t in
                                               (a.codes, a.scales, a.biases, a.bias))
    M3 = ito.Model(W3)
    kv3 = M3.kv(64, kv_bf16=False, mode=ito.ITO_F64)
    assert np.abs(M3.prefill_after(kv3, pr.text_tokens, pr.conds, pr.lang_id) - ref).max() > 1e-3


def test_causal_mask(tiny):
    W, M = tiny
    pr = synth.make_prompt(W.cfg, 2, 6, seed=9)
    emb = M.sequence_embedding(pr.text_tokens, pr.conds, pr.lang_id)
    T = emb.shape[0]
    kv = M.kv(64, kv_bf16=False)
    a = M.forward_rows(kv, emb, 0)
    emb2 = emb.copy()
    emb2[T - 2:] += 1.0
    b = M.forward_rows(kv, emb2, 0)
    assert np.array_equal(a[: T - 2], b[: T - 2])
    assert not np.allclose(a[T - 2:], b[T - 2:])


@pytest.mark.parametrize("kv_bf16", [False, True])
def test_kv_cache_self_consistency(tiny, kv_bf16):
    """prefill(T+m) last-row logits == prefill(T) then m steps at positions 2.. (exact:
    both paths perform the same operations on the last row)."""
    W, M = tiny
    pr = synth.make_prompt(W.cfg, 3, 8, seed=10)
    prior = [5, 77, 130]
    kv = M.kv(64, kv_bf16=kv_bf16)
    M.prefill_after(kv, pr.text_tokens, pr.conds, pr.lang_id)
    for i, c in enumerate(prior):
        stepped = M.step(kv, c, i + 2)
    kv2 = M.kv(64, kv_bf16=kv_bf16)
    whole = M.prefill_after(kv2, pr.text_tokens, pr.conds, pr.lang_id, prior)
    assert np.array_equal(stepped, whole)
    assert kv.valid_len() == kv2.valid_len() == 3 + 8 + 3 + 3
    for l in range(W.cfg["n_layer"]):
        assert np.array_equal(kv.read(l, 0), kv2.read(l, 0))
        assert np.array_equal(kv.read(l, 1), kv2.read(l, 1))


def test_f32_and_f64_modes_agree(tiny):
    W, M = tiny
    pr = synth.make_prompt(W.cfg, 3, 8, seed=12)
    a = M.prefill_after(M.kv(64, False, ito.ITO_F32), pr.text_tokens, pr.conds, pr.lang_id)
    b = M.prefill_after(M.kv(64, False, ito.ITO_F64), pr.text_tokens, pr.conds, pr.lang_id)
    assert np.abs(a - b).max() < 1e-4


def test_validation_errors(tiny):
    W, M = tiny
    pr = synth.make_prompt(W.cfg, 3, 8, seed=13)
    kv = M.kv(32, kv_bf16=True)
    cases = [
        (lambda: M.prefill_after(kv, [], pr.conds, 1), "text_tokens"),
        (lambda: M.prefill_after(kv, np.arange(2, 2 + 63), pr.conds, 1), "text_tokens"),
        (lambda: M.prefill_after(kv, pr.text_tokens, pr.conds, 99), "lang_id"),
        (lambda: M.prefill_after(kv, [W.cfg["text_vocab"]], pr.conds, 1), "text_tokens"),
        (lambda: M.step(kv, W.cfg["mel_vocab"], 2), "mel_token_id"),
        (lambda: M.step(kv, 3, W.cfg["mel_pos_len"]), "pos_idx"),
    ]
    for fn, field in cases:
        with pytest.raises(ito.OracleError) as e:
            fn()
        assert e.value.status == ito.ITO_E_VALIDATION and e.value.message.startswith(field)
    with pytest.raises(ito.OracleError) as e:
        M.prefill_after(kv, np.arange(2, 30), pr.conds, 1)     # 3 + 28 + 3 = 34 > 32
    assert e.value.status == ito.ITO_E_CAPACITY and kv.valid_len() == 0


def test_generate_min_codes_and_stop(tiny):
    """A head biased towards STOP: greedy stops at once unless min_codes masks it."""
    W, _ = tiny
    W2 = copy.deepcopy(W)
    stop = W.cfg["mel_vocab"] - 1
    W2.head.bias[stop] = 100.0
    M2 = ito.Model(W2)
    pr = synth.make_prompt(W.cfg, 3, 8, seed=14)
    from itts_hip import SamplingParams
    p = SamplingParams(greedy=True, max_mel_tokens=50)
    codes, _, _ = M2.generate_codes_after(M2.kv(256), pr.text_tokens, pr.conds, pr.lang_id, p, 0)
    assert len(codes) == 0
    codes, _, _ = M2.generate_codes_after(M2.kv(256), pr.text_tokens, pr.conds, pr.lang_id, p, 0,
                                          min_codes=7)
    assert len(codes) == 7 and stop not in codes


def test_generate_max_steps_clamp(tiny):
    W, M = tiny
    from itts_hip import SamplingParams
    pr = synth.make_prompt(W.cfg, 3, 8, seed=15)
    prior = list(range(2, 2 + W.cfg["mel_pos_len"] - 3 - 4))   # leaves room for 4 codes
    p = SamplingParams(greedy=True, max_mel_tokens=1000)
    kv = M.kv(512)
    codes, _, _ = M.generate_codes_after(kv, pr.text_tokens, pr.conds, pr.lang_id, p, 0,
                                         prior=prior, min_codes=1000)
    assert len(codes) == 4
    prior = list(range(2, 2 + W.cfg["mel_pos_len"] - 3))       # no room
    with pytest.raises(ito.OracleError) as e:
        M.generate_codes_after(kv, pr.text_tokens, pr.conds, pr.lang_id, p, 0, prior=prior)
    assert e.value.message.startswith("max_mel_tokens")


def test_generate_matches_manual_loop(tiny):
    """generate_codes_after == prefill, then sample/step by hand (sampler.rs:371-389)."""
    W, M = tiny
    from itts_hip import SamplingParams
    pr = synth.make_prompt(W.cfg, 3, 8, seed=16)
    p = SamplingParams(temperature=0.8, top_k=30, top_p=0.8, repetition_penalty=10.0,
                       max_mel_tokens=40)
    seed_state = ito.lib.ito_rng_init(1234)
    codes, st_end, _ = M.generate_codes_after(M.kv(256), pr.text_tokens, pr.conds, pr.lang_id, p,
                                              seed_state, min_codes=40)
    kv = M.kv(256)
    logits = M.prefill_after(kv, pr.text_tokens, pr.conds, pr.lang_id)
    seen = ito.seen_init(W.cfg["mel_vocab"] - 2)
    state = seed_state
    out = []
    for s in range(40):
        logits[W.cfg["mel_vocab"] - 1] = -np.inf
        tok, state = ito.sample_next_token(logits, seen, p, state)
        out.append(tok)
        ito.lib.ito_seen_insert(ito._p(seen), tok)
        if s + 1 < 40:
            logits = M.step(kv, tok, s + 2)
    assert out == codes.tolist() and state == st_end
