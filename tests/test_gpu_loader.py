"""Gpt::load_from_path on the device: a checkpoint written in the reference's tensor layout
(U32 code words, F32 or F16 group params) loads into the same decoder as the host-tensor
path (logits bit-identical) and matches the oracle.  F32 params are the shipped
checkpoint's dtype (crates/core/src/models/loader.rs:927-930)."""
import sys

import numpy as np
import pytest

import ito
import itts_hip as H
from itts_hip import synth

pytestmark = pytest.mark.gpu

TIGHT_TOL = 2e-4


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("bits,pd", [(8, H.ITTS_F32), (8, H.ITTS_F16), (4, H.ITTS_F32)])
def test_loaded_checkpoint_matches_host_path_and_oracle(tmp_path, bits, pd):
    say(f"[gpu] loader bits={bits} pd={pd}")
    cfg = dict(synth.TINY_CONFIG, quant_bits=bits, param_dtype=pd)
    W = synth.make_weights(cfg, seed=5, init="rich")
    path = tmp_path / "gpt_int8.safetensors"
    synth.save_safetensors(W, str(path))
    g_file = H.Gpt.load_from_path(str(path))
    g_host = H.Gpt(W)
    assert g_file.cfg == {k: v for k, v in W.cfg.items()}
    pr = synth.make_prompt(cfg, 3, 12, seed=2)
    kv_f, kv_h = g_file.kv_cache(128), g_host.kv_cache(128)
    assert kv_f.decode_path() == kv_h.decode_path()
    a = g_file.prefill(pr.text_tokens, pr.conds, pr.lang_id, kv_f)
    b = g_host.prefill(pr.text_tokens, pr.conds, pr.lang_id, kv_h)
    assert np.array_equal(a, b)
    M = ito.Model(W)
    okv = M.kv(128, kv_bf16=True)
    ref = M.prefill_after(okv, pr.text_tokens, pr.conds, pr.lang_id)
    assert np.abs(a - ref).max() < TIGHT_TOL
    for i, t in enumerate([7, 3, 200, 41]):
        a = g_file.step(kv_f, t, i + 2)
        b = g_host.step(kv_h, t, i + 2)
        r = M.step(okv, t, i + 2)
        assert np.array_equal(a, b), i
        assert np.abs(a - r).max() < TIGHT_TOL, i
    p = H.SamplingParams(greedy=True, max_mel_tokens=40)
    ca = H.generate_codes(g_file, pr.text_tokens, pr.conds, pr.lang_id, kv_f, p, H.SamplerRng(0))
    cb = H.generate_codes(g_host, pr.text_tokens, pr.conds, pr.lang_id, kv_h, p, H.SamplerRng(0))
    assert ca.tolist() == cb.tolist()
    g_file.close()
    g_host.close()
