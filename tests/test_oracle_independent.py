"""An independent float64 numpy evaluation of the whole decoder (gpt.rs:325-384 per block,
gpt.rs:673-692 for the head) over a multi-row causal prompt, against the oracle's float64
mode: the oracle's multi-key attention (softmax over every earlier key, P.V, division by
the denominator), its residual wiring and its head are pinned by a second implementation
that shares nothing with it but the weights and the (separately pinned) embedding rows.
Planted mistakes in the numpy evaluation (no division by the softmax denominator, keys
used as values, the causal mask dropped) must each move the logits far beyond the
agreement the correct evaluation reaches."""
import numpy as np
import pytest

import ito
from itts_hip import synth


def _params(a):
    return a.view(np.float16).astype(np.float64) if a.dtype == np.uint16 else a.astype(np.float64)


def _dequant(q, bits):
    """W[o, k] = s[o, k/64] * code[o, k] + b[o, k/64] (QuantizedLinear, gpt.rs:221-264)."""
    if bits == 8:
        codes = q.codes.astype(np.float64)
    else:
        lo, hi = q.codes & 0xF, q.codes >> 4
        codes = np.stack([lo, hi], axis=-1).reshape(q.N, q.K).astype(np.float64)
    s = np.repeat(_params(q.scales), 64, axis=1)
    b = np.repeat(_params(q.biases), 64, axis=1)
    return s * codes + b


def _ln(x, w, b):
    m = x.mean(axis=-1, keepdims=True)
    v = ((x - m) ** 2).mean(axis=-1, keepdims=True)
    return (x - m) / np.sqrt(v + 1e-5) * w.astype(np.float64) + b.astype(np.float64)


def _gelu(x):
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


def numpy_forward(W, emb, mistake=None):
    """Logits of every row of emb [T][d] through all blocks and the head, float64."""
    cfg = W.cfg
    bits, d, H = cfg["quant_bits"], cfg["d_model"], cfg["n_head"]
    x = emb.astype(np.float64)
    T = x.shape[0]
    causal = np.tril(np.ones((T, T), dtype=bool))
    for L in W.layers:
        h = _ln(x, L.ln1_w, L.ln1_b)
        qkv = h @ _dequant(L.c_attn, bits).T + L.c_attn.bias
        a = np.empty((T, d))
        for j in range(H):
            q = qkv[:, 64 * j:64 * j + 64]
            k = qkv[:, d + 64 * j:d + 64 * j + 64]
            v = qkv[:, 2 * d + 64 * j:2 * d + 64 * j + 64]
            s = q @ k.T * 0.125
            if mistake != "no_mask":
                s = np.where(causal, s, -np.inf)
            p = np.exp(s - s.max(axis=1, keepdims=True))
            if mistake != "no_den":
                p = p / p.sum(axis=1, keepdims=True)
            a[:, 64 * j:64 * j + 64] = p @ (k if mistake == "k_as_v" else v)
        x = x + a @ _dequant(L.c_proj, bits).T + L.c_proj.bias
        h = _ln(x, L.ln2_w, L.ln2_b)
        f = _gelu(h @ _dequant(L.c_fc, bits).T + L.c_fc.bias)
        x = x + f @ _dequant(L.mlp_c_proj, bits).T + L.mlp_c_proj.bias
    z = _ln(_ln(x, W.ln_f_w, W.ln_f_b), W.fn_w, W.fn_b)
    return z @ _dequant(W.head, bits).T + W.head.bias


@pytest.mark.parametrize("cfg,bits,pd", [(synth.TINY_CONFIG, 8, 1), (synth.SMALL_CONFIG, 8, 2),
                                         (synth.TINY_CONFIG, 4, 1)])
def test_oracle_matches_independent_float64(cfg, bits, pd):
    W = synth.make_weights(dict(cfg, quant_bits=bits, param_dtype=pd), seed=17, init="rich")
    M = ito.Model(W)
    pr = synth.make_prompt(W.cfg, 3, 20, seed=4)
    prior = (np.arange(25, dtype=np.int32) * 7) % (W.cfg["mel_vocab"] - 2)
    emb = M.sequence_embedding(pr.text_tokens, pr.conds, pr.lang_id, prior)
    T = emb.shape[0]
    got = M.forward_rows(M.kv(256, kv_bf16=False, mode=ito.ITO_F64), emb, 0)
    ref = numpy_forward(W, emb)
    scale = float(np.abs(ref).max())
    err = float(np.abs(got - ref).max())
    # the oracle's float64 mode differs from numpy only in summation order and in its
    # float32 embedding/logit storage
    assert err < 1e-5 * scale, (err, scale)
    for mistake in ("no_den", "k_as_v", "no_mask"):
        bad = numpy_forward(W, emb, mistake)
        assert float(np.abs(got - bad).max()) > 1e3 * max(err, 1e-9 * scale), mistake
    assert T == 3 + 22 + 1 + 25
