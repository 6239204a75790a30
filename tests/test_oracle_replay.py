"""Pins the oracle's replay (gpt.rs:391-422 head_attention, 797-858 replay): all-row
logits against the pinned prefill path, attention probes against their definition
(rows are distributions over the visible keys, masked keys are zero) and against an
independent evaluation of layer 0 from the separately pinned LayerNorm and QuantizedLinear
primitives."""
import numpy as np
import pytest

import ito
from itts_hip import synth


@pytest.fixture(scope="module")
def tiny():
    W = synth.make_weights(synth.TINY_CONFIG, seed=21, init="rich")
    return W, ito.Model(W)


def _ln(x, w, b):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    ito.lib.ito_layernorm(ito._p(x), ito._p(w), ito._p(b), x.shape[0], 1e-5, ito._p(y))
    return y


def _prompt(W, n_text=10, seed=1):
    return synth.make_prompt(W.cfg, 3, n_text, seed=seed)


def test_replay_logits_are_prefill_logits_of_each_prefix(tiny):
    """Row text_hi + i of the replay predicts codes[i]: it equals prefill_after(codes[:i])."""
    W, M = tiny
    pr = _prompt(W)
    codes = [5, 77, 130, 9, 44, 200]
    emb = M.sequence_embedding(pr.text_tokens, pr.conds, pr.lang_id, codes[:-1])
    text_hi = 3 + len(pr.text_tokens) + 2
    lg, _ = M.replay(M.kv(256, kv_bf16=False), emb, row0=text_hi)
    assert lg.shape == (len(codes), W.cfg["mel_vocab"])
    for i in range(len(codes)):
        ref = M.prefill_after(M.kv(256, kv_bf16=False), pr.text_tokens, pr.conds, pr.lang_id, codes[:i])
        assert np.array_equal(ref, lg[i])


def test_probe_rows_are_causal_distributions(tiny):
    W, M = tiny
    pr = _prompt(W)
    emb = M.sequence_embedding(pr.text_tokens, pr.conds, pr.lang_id, [3, 4, 5, 6])
    T = emb.shape[0]
    q0 = 7
    _, (p0, p1) = M.replay(M.kv(256, kv_bf16=False), emb, n_layers=2,
                           probes=[(0, 1, q0, 0, T), (1, 0, q0, 0, T)])
    for p in (p0, p1):
        assert p.shape == (T - q0, T)
        assert np.allclose(p.sum(1), 1.0, atol=1e-6)
        for r in range(T - q0):
            assert (p[r, q0 + r + 1:] == 0).all() and (p[r, : q0 + r + 1] > 0).all()
    # the two heads of layer 0 and layer 1 differ (the probe reads its own head and layer)
    assert not np.allclose(p0, p1)


def test_probe_layer0_matches_independent_evaluation(tiny):
    """Layer 0's block input is the embedding: LN1 -> c_attn (pinned primitives) -> one head's
    softmax(q k^T / 8) with the causal mask, sliced to [k0, k1)."""
    W, M = tiny
    c = W.cfg
    d, H = c["d_model"], c["n_head"]
    pr = _prompt(W, n_text=12, seed=3)
    emb = M.sequence_embedding(pr.text_tokens, pr.conds, pr.lang_id, [11, 12, 13])
    T = emb.shape[0]
    q0, k0, k1 = 17, 3, 17
    for head in range(H):
        _, (p,) = M.replay(M.kv(256, kv_bf16=False), emb, n_layers=1, probes=[(0, head, q0, k0, k1)])
        L = W.layers[0]
        h = np.stack([_ln(emb[t], L.ln1_w, L.ln1_b) for t in range(T)]).astype(np.float64)
        Wq = ito.dequant(L.c_attn, c["quant_bits"], c["param_dtype"]).astype(np.float64)
        qkv = h @ Wq.T + L.c_attn.bias
        q = qkv[:, head * 64:(head + 1) * 64]
        k = qkv[:, d + head * 64:d + (head + 1) * 64]
        s = (q @ k.T) * 0.125
        s = np.where(np.tril(np.ones((T, T), bool)), s, -np.inf)
        s = np.exp(s - s.max(1, keepdims=True))
        s /= s.sum(1, keepdims=True)
        assert np.allclose(p, s[q0:, k0:k1], atol=2e-6), head


def test_replay_validation(tiny):
    W, M = tiny
    emb = M.sequence_embedding(*(lambda p: (p.text_tokens, p.conds, p.lang_id))(_prompt(W)), [1])
    T = emb.shape[0]
    with pytest.raises(ito.OracleError):
        M.replay(M.kv(256), emb, n_layers=1, row0=0)          # logits need the whole stack
    with pytest.raises(ito.OracleError):
        M.replay(M.kv(256), emb, probes=[(0, 9, 0, 0, T)])    # head outside the model
    with pytest.raises(ito.OracleError):
        M.replay(M.kv(8), emb, row0=0)                        # capacity
