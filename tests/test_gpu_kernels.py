"""Kernel-level parity of the HIP path against the oracle, through the C ABI:
dequantisation bit-exact, GEMV / MFMA GEMM within fp32 rounding of an fp64 reference,
and the device sampler bit-exact (token, penalised logits and RNG state)."""
import sys

import numpy as np
import pytest

import ito
import itts_hip as H
from itts_hip import synth

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def gpt():
    say("[gpu] creating tiny decoder for kernel tests")
    W = synth.make_weights(synth.TINY_CONFIG, seed=3, init="rich")
    g = H.Gpt(W)
    yield g
    g.close()


def _ql(rng, N, K, bits, pd):
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    codes, s, b = H.quantize(w, bits, pd)
    bias = (rng.standard_normal(N) * 0.05).astype(np.float32)
    return synth.QLinear(codes, s, b, bias, N, K)


@pytest.mark.parametrize("bits,pd", [(8, H.ITTS_F16), (4, H.ITTS_F16), (8, H.ITTS_F32), (4, H.ITTS_F32)])
@pytest.mark.parametrize("N,K", [(37, 192), (1280, 1280), (640, 5120)])
def test_dequant_bit_exact(gpt, bits, pd, N, K):
    say(f"[gpu] dequant bits={bits} pd={pd} N={N} K={K}")
    q = _ql(np.random.default_rng(N + K + bits), N, K, bits, pd)
    got = gpt.dequantize(q.codes, q.scales, q.biases, N, K, bits, pd)
    ref = ito.dequant(q, bits, pd)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def _check_linear(got, q, bits, pd, x, tol):
    W = ito.dequant(q, bits, pd).astype(np.float64)
    xd = x.astype(np.float64)
    ref = xd @ W.T + q.bias
    bound = np.abs(xd) @ np.abs(W).T + np.abs(q.bias)
    err = np.abs(got - ref)
    assert np.all(err <= tol * bound + 1e-7), float((err / bound).max())


@pytest.mark.parametrize("bits,pd", [(8, H.ITTS_F16), (4, H.ITTS_F16), (8, H.ITTS_F32)])
@pytest.mark.parametrize("N,K", [(37, 192), (3840, 1280), (1280, 5120), (8194, 1280)])
def test_gemv_vs_fp64(gpt, bits, pd, N, K):
    say(f"[gpu] gemv bits={bits} pd={pd} N={N} K={K}")
    rng = np.random.default_rng(N * 7 + K)
    q = _ql(rng, N, K, bits, pd)
    x = rng.standard_normal((1, K)).astype(np.float32)
    got = gpt.qlinear_forward(q.codes, q.scales, q.biases, q.bias, x, N, K, bits, pd)
    _check_linear(got, q, bits, pd, x, 2e-6)


# Shapes cover: the few-row kernel (M <= 8: one K split, several, a ragged last column
# tile), the 64 x 64 tile with and without split-K, ragged N and M, the 128 x 128 tile
# (M > 512) with and without split-K, the head's N = 8194, and the 4 x 547-row QKV product
# (540 tiles, a ragged last M tile of 12 rows).
@pytest.mark.parametrize("bits,pd", [(8, H.ITTS_F16), (4, H.ITTS_F16), (8, H.ITTS_F32), (4, H.ITTS_F32)])
@pytest.mark.parametrize("M,N,K", [(2, 37, 192), (8, 3840, 1280), (5, 1280, 5120), (7, 8194, 1280), (3, 96, 128),
                                   (99, 3840, 1280), (130, 1280, 5120), (64, 8194, 1280),
                                   (235, 1280, 1280), (600, 1280, 1280), (700, 384, 5120),
                                   (2188, 3840, 1280)])
def test_mfma_gemm_vs_fp64(gpt, bits, pd, M, N, K):
    say(f"[gpu] gemm bits={bits} pd={pd} M={M} N={N} K={K}")
    rng = np.random.default_rng(M + N + K)
    q = _ql(rng, N, K, bits, pd)
    x = rng.standard_normal((M, K)).astype(np.float32)
    got = gpt.qlinear_forward(q.codes, q.scales, q.biases, q.bias, x, N, K, bits, pd)
    # activations enter the MFMA as an fp16 hi/lo pair: ~2^-22 relative per element
    _check_linear(got, q, bits, pd, x, 4e-6)
    # split-K partials are added in split order: repeated calls are bit-identical
    again = gpt.qlinear_forward(q.codes, q.scales, q.biases, q.bias, x, N, K, bits, pd)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))


def _logits_case(rng, n, kind):
    if kind == "normal":
        return (rng.standard_normal(n) * 2).astype(np.float32)
    if kind == "ties":
        return np.round(rng.standard_normal(n) * 2).astype(np.float32)
    raw = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32).view(np.float32)
    pick = rng.random(n) < (0.02 if kind == "special" else 0.5)
    return np.where(pick, raw, (rng.standard_normal(n) * 3).astype(np.float32)).astype(np.float32)


CASES = []
for kind in ("normal", "ties", "special", "raw"):
    for greedy, k, p_, t, pen in [(True, 3, 0.8, 0.8, 10.0), (False, 30, 0.8, 0.8, 10.0),
                                  (False, 3, 0.8, 0.8, 10.0), (False, 1, 0.5, 1.0, 1.0),
                                  (False, 500, 0.95, 1.3, 2.0), (False, 0, 1.0, 0.7, 1.5),
                                  (False, 8194, 0.3, 0.05, 50.0), (False, 4096, 0.9, 2.0, 1.0),
                                  (False, 64, 0.9, 0.8, 10.0), (False, 33, 0.99, 1.0, 1.0), (False, 65, 0.9, 0.8, 2.0)]:
        CASES.append((kind, greedy, k, p_, t, pen))


@pytest.mark.parametrize("kind,greedy,k,top_p,temp,pen", CASES)
def test_sampler_bit_exact(gpt, kind, greedy, k, top_p, temp, pen):
    say(f"[gpu] sampler kind={kind} greedy={greedy} k={k} p={top_p} T={temp} pen={pen}")
    rng = np.random.default_rng(hash((kind, greedy, k, top_p)) & 0xffffffff)
    params = H.SamplingParams(greedy=greedy, top_k=k, top_p=top_p, temperature=temp,
                              repetition_penalty=pen, max_mel_tokens=10)
    for trial in range(6):
        n = 8194 if trial < 4 else int(rng.integers(1, 3000))
        lg = _logits_case(rng, n, kind)
        seen = H.SeenTokenBitSet()
        for t_ in rng.integers(0, n, 40):
            seen.insert(int(t_))
        seed = int(rng.integers(0, 2**63))
        a = lg.copy()
        r = H.SamplerRng(seed)
        tok = H.sample_next_token(gpt, a, seen, params, r)
        b = lg.copy()
        tok_ref, st_ref = ito.sample_next_token(b, seen.words, params, ito.lib.ito_rng_init(seed))
        assert tok == tok_ref, (trial, n)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        assert r.state.value == st_ref


def test_sampler_reference_doctest(gpt):
    say("[gpu] sampler doctest")
    logits = np.full(8194, -10.0, np.float32)
    logits[42] = 25.0
    assert H.sample_next_token(gpt, logits, H.SeenTokenBitSet(), H.SamplingParams(), H.SamplerRng(7)) == 42
