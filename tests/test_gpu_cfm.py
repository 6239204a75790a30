"""CFM DiT estimator and Euler / CFG solver on the HIP path, through the C ABI, against the
oracle's restatement of cfm.rs (forward_merged 545-617, solve_euler 619-760).

The HIP path keeps fp32 activations and contracts on fp16 hi/lo split MFMA products (~22-bit
operands, fp32 accumulation, its own summation order) against the oracle's double
accumulation, so the bar is relative: max |gpu - oracle| / max |oracle| below 2e-4
for one forward and 1e-3 after several Euler steps."""
import sys

import numpy as np
import pytest

import ito
import itts_hip as H
from itts_hip import synth
from itts_hip.cfm import FULL_CONFIG, SMALL_CONFIG, CfmDit, merged_dim, tensor_shapes

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def rel(a, b):
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


@pytest.fixture(scope="module")
def small():
    say("[gpu] small CFM estimator")
    W = synth.make_cfm_weights(SMALL_CONFIG, seed=5)
    m = CfmDit(W, SMALL_CONFIG)
    yield W, m, ito.CfmModel(W, SMALL_CONFIG)
    m.close()


@pytest.mark.parametrize("T", [1, 19, 64, 150])
def test_forward_matches_oracle(small, T):
    W, m, M = small
    say(f"[gpu] cfm forward T={T}")
    rng = np.random.default_rng(T)
    B = 2
    x_t = rng.standard_normal((B, T, SMALL_CONFIG["in_ch"])).astype(np.float32)
    x_m = rng.standard_normal((B, T, merged_dim(SMALL_CONFIG))).astype(np.float32)
    x_m[..., :SMALL_CONFIG["in_ch"]] = x_t
    t = np.array([0.12, 0.88], np.float32)
    got = m.forward_merged(x_t, x_m, t)
    ref = M.forward_merged(x_t, x_m, t)
    assert got.shape == ref.shape == (B, SMALL_CONFIG["in_ch"], T)
    assert rel(got, ref) < 2e-4


@pytest.mark.parametrize("cfg_rate,steps", [(0.7, 3), (0.0, 2)])
def test_solve_euler_matches_oracle(small, cfg_rate, steps):
    W, m, M = small
    say(f"[gpu] cfm solve cfg={cfg_rate} steps={steps}")
    inp = synth.make_cfm_inputs(SMALL_CONFIG, 90, 31, seed=7)
    args = (inp["cat_condition"], inp["ref_mel"], inp["style"], inp["noise_z"], steps, cfg_rate)
    got = m.solve_euler(*args)
    ref = M.solve_euler(*args)
    assert got.shape == ref.shape == (1, SMALL_CONFIG["in_ch"], 59)
    assert rel(got, ref) < 1e-3
    assert m.last_timing_ms() > 0


def test_solve_ignores_noise_over_prompt(small):
    W, m, M = small
    inp = synth.make_cfm_inputs(SMALL_CONFIG, 40, 12, seed=9)
    a = m.solve_euler(inp["cat_condition"], inp["ref_mel"], inp["style"], inp["noise_z"], 2, 0.7)
    nz = inp["noise_z"].copy()
    nz[:, :, :12] = 100.0
    b = m.solve_euler(inp["cat_condition"], inp["ref_mel"], inp["style"], nz, 2, 0.7)
    assert np.array_equal(a, b)


def test_validation(small):
    W, m, M = small
    inp = synth.make_cfm_inputs(SMALL_CONFIG, 20, 8, seed=1)
    with pytest.raises(H.ValidationError) as e:
        m.solve_euler(inp["cat_condition"], inp["ref_mel"], inp["style"], inp["noise_z"], 0, 0.7)
    assert e.value.message.startswith("n_timesteps")
    big = synth.make_cfm_inputs(SMALL_CONFIG, 20, 20, seed=1)
    with pytest.raises(H.ValidationError) as e:
        m.solve_euler(big["cat_condition"], big["ref_mel"], big["style"], big["noise_z"], 2, 0.7)
    assert e.value.message.startswith("ref_mel")
    with pytest.raises(H.ValidationError):
        m.solve_euler(inp["cat_condition"], inp["ref_mel"], inp["style"], inp["noise_z"][:, :, :-1], 2, 0.7)
    missing = dict(W)
    del missing["transformer.layers.2.attention.wo.weight"]
    with pytest.raises(H.WeightLoadError) as e:
        CfmDit(missing, SMALL_CONFIG)
    assert "transformer.layers.2.attention.wo.weight" in e.value.message
    wrong = dict(W)
    wrong["conv2.bias"] = np.zeros(3, np.float32)
    with pytest.raises(H.WeightLoadError):
        CfmDit(wrong, SMALL_CONFIG)


# dim 256 (the one-wave AdaLN with 4 values per lane), and channel counts that are not
# multiples of 4: the merge and skip products then take the few-row fp32 product's scalar
# loads at every row count
MID_CONFIG = dict(dim=256, n_layers=3, n_heads=4, inter=384, in_ch=18, style_dim=30, wn_layers=2, wn_kernel=3)


@pytest.mark.parametrize("T", [7, 100])
def test_forward_d256_unaligned_channels(T):
    say(f"[gpu] cfm forward dim 256, in_ch 18, T={T}")
    W = synth.make_cfm_weights(MID_CONFIG, seed=3)
    m = CfmDit(W, MID_CONFIG)
    try:
        rng = np.random.default_rng(40 + T)
        C = MID_CONFIG["in_ch"]
        x_t = rng.standard_normal((2, T, C)).astype(np.float32)
        x_m = rng.standard_normal((2, T, merged_dim(MID_CONFIG))).astype(np.float32)
        x_m[..., :C] = x_t
        t = np.array([0.3, 0.7], np.float32)
        got = m.forward_merged(x_t, x_m, t)
        ref = ito.CfmModel(W, MID_CONFIG).forward_merged(x_t, x_m, t)
        assert got.shape == ref.shape == (2, C, T)
        assert rel(got, ref) < 2e-4
    finally:
        m.close()


@pytest.mark.parametrize("T", [96, 1033])
def test_full_size_forward_matches_oracle(T):
    """The reference's shape (dim 512, 13 layers, 8 heads, WaveNet 8 x kernel 5) at 96 frames
    and at the 1033 frames of the benchmarked solve (10 s of audio)."""
    say(f"[gpu] full-size CFM forward T={T}")
    W = synth.make_cfm_weights(FULL_CONFIG, seed=11)
    assert set(W) == set(tensor_shapes(FULL_CONFIG))
    m = CfmDit(W, FULL_CONFIG)
    try:
        rng = np.random.default_rng(2)
        x_t = rng.standard_normal((2, T, 80)).astype(np.float32)
        x_m = rng.standard_normal((2, T, merged_dim(FULL_CONFIG))).astype(np.float32)
        x_m[..., :80] = x_t
        t = np.array([0.4, 0.4], np.float32)
        got = m.forward_merged(x_t, x_m, t)
        ref = ito.CfmModel(W, FULL_CONFIG).forward_merged(x_t, x_m, t)
        assert rel(got, ref) < 2e-4
    finally:
        m.close()
