"""Pins the oracle's CFM DiT estimator and Euler solver (cfm.rs).

The reference's own check, CP-13 (cfm.rs:763-814), needs the absent cfm_estimator checkpoint
and returns early without it; its fixture inputs (cat_condition [1, 282, 512], ref_mel
[1, 80, 172], style, cfm_noise_z) fix the shapes used below.  What pins the oracle here:
  * rope: the complex-rotation form of rope(traditional=true) (pairs as complex numbers
    times e^{i t theta_k}), norm preservation, the identity at t = 0 and the relative-position
    property <R_m q, R_n k> = <R_{m+s} q, R_{n+s} k>;
  * TimestepEmbedder: the closed form at t = 0 (cos = 1, sin = 0) and an evaluation in
    float64 numpy;
  * forward_merged: an independent float64 numpy evaluation of the whole estimator, written
    with vectorised operations (einsum attention, complex rope, a padded-window convolution);
  * solve_euler: the one-step solve against the oracle's forward on CFG inputs assembled in
    numpy from the reference's concatenation rules (cfm.rs:682-742), cfg_rate 0, and the
    reference's validation errors.
"""
import numpy as np
import pytest

import ito
from itts_hip import synth
from itts_hip.cfm import FREQ_DIM, SMALL_CONFIG, merged_dim

CFG = dict(SMALL_CONFIG)


@pytest.fixture(scope="module")
def model():
    W = synth.make_cfm_weights(CFG, seed=3)
    return W, ito.CfmModel(W, CFG)


def test_rope_complex_form_and_invariants():
    rng = np.random.default_rng(0)
    T, H = 40, 2
    x = rng.standard_normal((T, H * 64)).astype(np.float32)
    y = ito.cfm_rope(x, H)
    z = (x[:, 0::2] + 1j * x[:, 1::2]).astype(np.complex128).reshape(T, H, 32)
    theta = 1.0 / 10000.0 ** (np.arange(32) * 2 / 64.0)
    rot = z * np.exp(1j * np.arange(T)[:, None, None] * theta[None, None, :])
    ref = np.empty_like(x, dtype=np.float64)
    ref[:, 0::2] = rot.real.reshape(T, -1)
    ref[:, 1::2] = rot.imag.reshape(T, -1)
    assert np.abs(y - ref).max() < 2e-5 * max(1.0, np.abs(ref).max())
    assert np.array_equal(y[0], x[0])                                   # t = 0: identity
    n_in = np.hypot(x[:, 0::2], x[:, 1::2])
    n_out = np.hypot(y[:, 0::2], y[:, 1::2])
    assert np.allclose(n_in, n_out, rtol=1e-5, atol=1e-6)               # rotations
    q = np.tile(rng.standard_normal(64).astype(np.float32), (T, 1))
    k = np.tile(rng.standard_normal(64).astype(np.float32), (T, 1))
    rq, rk = ito.cfm_rope(q, 1), ito.cfm_rope(k, 1)
    dots = rq.astype(np.float64) @ rk.T.astype(np.float64)
    for s in (1, 7):
        assert np.allclose(dots[3 + s, 10 + s], dots[3, 10], rtol=1e-4, atol=1e-4)
        assert np.allclose(dots[20 + s, 2 + s], dots[20, 2], rtol=1e-4, atol=1e-4)


def _silu(x):
    return x / (1.0 + np.exp(-x))


def _temb(W, p, t):
    k = np.arange(FREQ_DIM // 2)
    f = 1000.0 * np.exp(-np.log(10000.0) * k / (FREQ_DIM // 2))
    emb = np.concatenate([np.cos(t * f), np.sin(t * f)])
    h = _silu(W[f"{p}.mlp.layers.0.weight"].astype(np.float64) @ emb + W[f"{p}.mlp.layers.0.bias"])
    return W[f"{p}.mlp.layers.2.weight"].astype(np.float64) @ h + W[f"{p}.mlp.layers.2.bias"]


def test_timestep_embedder(model):
    W, M = model
    for t in (0.0, 0.04, 0.52, 0.96):
        for which, p in ((1, "t_embedder"), (2, "t_embedder2")):
            got = M.timestep(which, t)
            ref = _temb(W, p, t)
            assert np.abs(got - ref).max() < 1e-4 * max(1.0, np.abs(ref).max()), (t, p)
    # t = 0: the frequency embedding is 128 ones then 128 zeros
    h = _silu(W["t_embedder.mlp.layers.0.weight"][:, :128].astype(np.float64).sum(1) + W["t_embedder.mlp.layers.0.bias"])
    ref0 = W["t_embedder.mlp.layers.2.weight"].astype(np.float64) @ h + W["t_embedder.mlp.layers.2.bias"]
    assert np.allclose(M.timestep(1, 0.0), ref0, rtol=1e-4, atol=1e-4)


def numpy_forward(W, cfg, x_t, x_merged, t, skip_fifo=False, rope_halves=False):
    """Independent float64 evaluation of forward_merged (cfm.rs:545-617).  skip_fifo and
    rope_halves plant two plausible mistakes (skips taken in push order; rope rotating the
    two halves of a head instead of adjacent pairs) to show the comparison detects them."""
    d, H, L = cfg["dim"], cfg["n_heads"], cfg["n_layers"]
    g = lambda n: W[n].astype(np.float64)
    B, T, _ = x_t.shape
    t1 = np.stack([_temb(W, "t_embedder", tb) for tb in t])      # [B, d]
    t2 = np.stack([_temb(W, "t_embedder2", tb) for tb in t])

    def adaln(x, p, c):
        wb = c @ g(f"{p}.project_layer.weight").T + g(f"{p}.project_layer.bias")
        w, b = wb[:, None, :d], wb[:, None, d:]
        rms = np.sqrt((x * x).mean(-1, keepdims=True) + 1e-5)
        return w * (x / rms * g(f"{p}.norm.weight")) + b

    theta = 1.0 / 10000.0 ** (np.arange(32) * 2 / 64.0)
    phase = np.exp(1j * np.arange(T)[:, None] * theta[None, :])   # [T, 32]

    def rope(x):   # [B, T, H, 64]
        if rope_halves:
            z = (x[..., :32] + 1j * x[..., 32:]) * phase[None, :, None, :]
            return np.concatenate([z.real, z.imag], -1)
        z = x[..., 0::2] + 1j * x[..., 1::2]
        z = z * phase[None, :, None, :]
        out = np.empty_like(x)
        out[..., 0::2], out[..., 1::2] = z.real, z.imag
        return out

    h = x_merged.astype(np.float64) @ g("cond_x_merge_linear.weight").T + g("cond_x_merge_linear.bias")
    skips = []
    for i in range(L):
        p = f"transformer.layers.{i}"
        if i > L // 2:
            cat = np.concatenate([h, skips.pop(0) if skip_fifo else skips.pop()], -1)
            x_in = cat @ g(f"{p}.skip_in_linear.weight").T + g(f"{p}.skip_in_linear.bias")
        else:
            x_in = h
        n1 = adaln(x_in, f"{p}.attention_norm", t1)
        qkv = n1 @ g(f"{p}.attention.wqkv.weight").T
        q, k, v = (qkv[..., j * d:(j + 1) * d].reshape(B, T, H, 64) for j in range(3))
        q, k = rope(q), rope(k)
        s = np.einsum("bqhe,bkhe->bhqk", q, k) * 0.125
        s = np.exp(s - s.max(-1, keepdims=True))
        s /= s.sum(-1, keepdims=True)
        att = np.einsum("bhqk,bkhe->bqhe", s, v).reshape(B, T, d)
        hid = x_in + att @ g(f"{p}.attention.wo.weight").T
        n2 = adaln(hid, f"{p}.ffn_norm", t1)
        ff = (_silu(n2 @ g(f"{p}.feed_forward.w1.weight").T) * (n2 @ g(f"{p}.feed_forward.w3.weight").T))
        h = hid + ff @ g(f"{p}.feed_forward.w2.weight").T
        if i < L // 2:
            skips.append(h)
    h = adaln(h, "transformer.norm", t1)
    x_res = np.concatenate([h, x_t], -1) @ g("skip_linear.weight").T + g("skip_linear.bias")
    hw = x_res @ g("conv1.weight").T + g("conv1.bias")
    # WaveNet: conv1d over a zero-padded window, gated tanh * sigmoid, residual/skip split
    NL, K = cfg["wn_layers"], cfg["wn_kernel"]
    gall = t2 @ g("wavenet.cond_layer.weight")[:, 0, :].T + g("wavenet.cond_layer.bias")
    out = np.zeros_like(hw)
    for l in range(NL):
        w = g(f"wavenet.in_layers.{l}.weight")                      # [2d, K, d]
        pad = np.pad(hw, ((0, 0), (K // 2, K // 2), (0, 0)))
        win = np.stack([pad[:, j:j + T] for j in range(K)], 2)      # [B, T, K, d]
        acts = np.einsum("btkc,okc->bto", win, w) + g(f"wavenet.in_layers.{l}.bias")
        acts = acts + gall[:, None, l * 2 * d:(l + 1) * 2 * d]
        act = np.tanh(acts[..., :d]) * (1.0 / (1.0 + np.exp(-acts[..., d:])))
        rs = act @ g(f"wavenet.res_skip_layers.{l}.weight")[:, 0, :].T + g(f"wavenet.res_skip_layers.{l}.bias")
        if l + 1 == NL:
            out = out + rs
        else:
            hw = hw + rs[..., :d]
            out = out + rs[..., d:]
    h = out + x_res @ g("res_projection.weight").T + g("res_projection.bias")
    mod = _silu(t1) @ g("final_layer.adaLN_modulation.layers.1.weight").T + g("final_layer.adaLN_modulation.layers.1.bias")
    shift, scale = mod[:, None, :d], mod[:, None, d:]
    mu = h.mean(-1, keepdims=True)
    nrm = (h - mu) / np.sqrt(((h - mu) ** 2).mean(-1, keepdims=True) + 1e-6)
    fh = (nrm * (1.0 + scale) + shift) @ g("final_layer.linear.weight").T + g("final_layer.linear.bias")
    o = fh @ g("conv2.weight")[:, 0, :].T + g("conv2.bias")
    return o.transpose(0, 2, 1)


def test_forward_matches_independent_numpy(model):
    W, M = model
    rng = np.random.default_rng(1)
    B, T = 2, 19
    x_t = rng.standard_normal((B, T, CFG["in_ch"])).astype(np.float32)
    x_m = rng.standard_normal((B, T, merged_dim(CFG))).astype(np.float32)
    x_m[..., :CFG["in_ch"]] = x_t
    t = np.array([0.0, 0.36], np.float32)
    got = M.forward_merged(x_t, x_m, t)
    ref = numpy_forward(W, CFG, x_t, x_m, t)
    assert got.shape == (B, CFG["in_ch"], T)
    err = np.abs(got - ref).max() / np.abs(ref).max()
    assert err < 1e-4, err
    # the comparison is sensitive to plausible mistakes
    for kw in (dict(skip_fifo=True), dict(rope_halves=True)):
        bad = numpy_forward(W, CFG, x_t, x_m, t, **kw)
        assert np.abs(got - bad).max() / np.abs(bad).max() > 100 * max(err, 1e-7), kw


def _cfg_inputs(W, cfg, x, inp):
    """The CFG pair of forward inputs of one Euler step, assembled in numpy (cfm.rs:682-742)."""
    d, C, T = cfg["dim"], cfg["in_ch"], x.shape[1]
    Tr = inp["ref_mel"].shape[2]
    x_t = np.stack([x.T, x.T])                                          # [2, T, C]
    prompt = np.zeros((2, T, C), np.float32)
    prompt[0, :Tr] = inp["ref_mel"][0].T
    cond = np.concatenate([inp["cat_condition"], np.zeros_like(inp["cat_condition"])])
    cp = cond.astype(np.float64) @ W["cond_projection.weight"].T.astype(np.float64) + W["cond_projection.bias"]
    style = np.concatenate([inp["style"], np.zeros_like(inp["style"])])[:, None, :].repeat(T, 1)
    merged = np.concatenate([x_t, prompt, cp.astype(np.float32), style], -1)
    return x_t, merged


@pytest.mark.parametrize("cfg_rate", [0.7, 0.0])
def test_one_step_solve_matches_forward(model, cfg_rate):
    W, M = model
    inp = synth.make_cfm_inputs(CFG, 30, 11, seed=2)
    out = M.solve_euler(inp["cat_condition"], inp["ref_mel"], inp["style"], inp["noise_z"], 1, cfg_rate)
    x = inp["noise_z"][0].copy()
    x[:, :11] = 0.0
    x_t, merged = _cfg_inputs(W, CFG, x, inp)
    v = M.forward_merged(x_t, merged, np.zeros(2, np.float32))
    guided = v[0] * (1 + cfg_rate) - v[1] * cfg_rate if cfg_rate > 0 else v[0]
    ref = (x + guided * 1.0)[:, 11:]
    assert out.shape == (1, CFG["in_ch"], 19)
    assert np.abs(out[0] - ref).max() < 1e-4 * max(1.0, np.abs(ref).max())


def test_two_step_solve_and_prompt_independence(model):
    W, M = model
    inp = synth.make_cfm_inputs(CFG, 24, 6, seed=4)
    a = M.solve_euler(inp["cat_condition"], inp["ref_mel"], inp["style"], inp["noise_z"], 2, 0.7)
    # the noise over the prompt frames is masked before every step: changing it changes nothing
    nz = inp["noise_z"].copy()
    nz[:, :, :6] += 5.0
    b = M.solve_euler(inp["cat_condition"], inp["ref_mel"], inp["style"], nz, 2, 0.7)
    assert np.array_equal(a, b)
    # second step input: x1 = x0 + dt * guided(t = 0), evaluated at t = 0.5
    x = inp["noise_z"][0].copy()
    x[:, :6] = 0.0
    for step in range(2):
        x[:, :6] = 0.0
        x_t, merged = _cfg_inputs(W, CFG, x, inp)
        v = M.forward_merged(x_t, merged, np.full(2, step * 0.5, np.float32))
        x = x + (v[0] * 1.7 - v[1] * 0.7) * 0.5
    assert np.abs(a[0] - x[:, 6:]).max() < 1e-4 * max(1.0, np.abs(x).max())


def test_solve_validation(model):
    W, M = model
    inp = synth.make_cfm_inputs(CFG, 10, 4, seed=0)
    with pytest.raises(ito.OracleError):
        M.solve_euler(inp["cat_condition"], inp["ref_mel"], inp["style"], inp["noise_z"], 0, 0.7)
    big = synth.make_cfm_inputs(CFG, 10, 10, seed=0)
    with pytest.raises(ito.OracleError):
        M.solve_euler(big["cat_condition"], big["ref_mel"], big["style"], big["noise_z"], 2, 0.7)
